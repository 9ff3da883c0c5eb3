"""Golden fixtures: the reference's known answers (reference_kats.json) through
the oracle, the library's host code and — marked gpu — the HIP path; and the
oracle's greedy streams (oracle_streams.json, written by make_golden.py)
reproduced by the oracle and by the device decoder."""
import json
import math
import os

import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import DecoderConfig

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Q8, Q4, Q6 = 1000, 1001, 1002
QT = {"q8": Q8, "q4": Q4, "q6": Q6}


def _load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


KAT = _load("reference_kats.json")
STREAMS = _load("oracle_streams.json")["cases"]


def _num(v):
    return 2 * math.log(3) if v == "2ln3" else float(v)


# ---------------------------------------------------------------- formats

def test_round_to_int(orc):
    for x, want in KAT["round_to_int"]["cases"]:
        assert orc.round_to_int(x) == want


@pytest.mark.parametrize("impl", ["oracle", "library"])
def test_q8_q4_rows(orc, impl):
    quant = orc.quantize_row if impl == "oracle" else (lambda q, w: _lib_quant_row(q, w))
    k8, k4 = KAT["q8_row"], KAT["q4_row"]
    s, row = quant(Q8, np.array(k8["w"], np.float32))
    assert s == np.float32(k8["scale_num"]) / np.float32(k8["scale_den"])
    assert list(np.asarray(row).view(np.int8)) == k8["codes"]
    s, row = quant(Q4, np.array(k4["w"], np.float32))
    assert s == np.float32(k4["scale_num"]) / np.float32(k4["scale_den"])
    assert list(np.asarray(row)) == k4["bytes"]


def _lib_quant_row(qtype, w):
    s, p = lib.quantize_rows(qtype, w[None, :])
    return s[0], p[0]


def test_q6_values_and_zero_rows(orc):
    for code, want in KAT["q6_values"]["cases"]:
        row = np.array([code], np.uint8)
        assert orc.unpack_row(Q6, row, 1)[0] == want
        assert lib.unpack_rows(Q6, row[None, :], 1)[0, 0] == want
    for name, want in KAT["zero_row"]["decoded"].items():
        for quant, unpack in ((lambda q, w: orc.quantize_row(q, w), lambda q, r: orc.unpack_row(q, r, 9)),
                              (_lib_quant_row, lambda q, r: lib.unpack_rows(q, r[None, :], 9)[0])):
            s, row = quant(QT[name], np.zeros(9, np.float32))
            assert s == 1.0 and not np.asarray(row).any()
            assert (unpack(QT[name], np.asarray(row)) == want).all()


# ---------------------------------------------------------------- ops (oracle)

def _closed_forms():
    for c in KAT["matvec_closed_form"]["cases"]:
        yield np.array(c["w"], np.float32), np.array(c["x"], np.float32)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6])
def test_matvec_closed_forms_oracle(orc, qtype):
    # dequantised weights times x in f64 is what the f32 kernel must reproduce
    for w, x in _closed_forms():
        sc, data = orc.quantize_matrix(qtype, w)
        codes = orc.unpack_matrix(qtype, data, w.shape[1]).astype(np.float64)
        want = (codes @ x.astype(np.float64)) * sc.astype(np.float64)
        assert np.allclose(orc.matvec(qtype, sc, data, x), want, rtol=1e-6, atol=1e-6)


def test_argmax_ties(orc):
    k = KAT["argmax_ties"]
    assert orc.argmax(np.array(k["scores"], np.float32)) == k["index"]


def test_rope_first_token_k(orc):
    k = KAT["rope_first_token_k"]
    got = orc.apply_rope(np.array(k["k"], np.float32), k["cos"], k["sin"], 1, len(k["k"]))
    assert list(got) == k["rotated"]


def _wvs():
    k = KAT["weighted_value_sum"]
    q = np.array(k["q"], np.float32)
    kc = np.array([[_num(v) for v in row] for row in k["k"]], np.float32)
    vc = np.array(k["v"], np.float32)
    return k, q, kc, vc


def test_weighted_value_sum_oracle(orc):
    k, q, kc, vc = _wvs()
    out = orc.cache_attention(q, kc, vc, k["len"], k["heads"], k["kv_heads"], k["head_dim"])
    assert np.max(np.abs(out[4:] - np.array(k["out_head1"]))) < 2e-5


@pytest.mark.parametrize("impl", ["oracle", "library"])
def test_positions(orc, impl):
    fn = orc.mm_positions if impl == "oracle" else lib.mm_positions
    for c in KAT["positions"]["cases"]:
        pos, delta = fn(c["ids"], c["image_token"], tuple(c["grid"]))
        assert np.asarray(pos).tolist() == c["pos"] and delta == c["delta"]


def test_vnni_core(orc):
    # ones against xq = 129 on n columns, plus one column of weight 0 that sets
    # the x scale: x = c, …, c, 127c → scaleX = c, xq = 129, …, 129, 255.
    # (core − 128·rowSum)·scaleX·scale = (core − 128n)·c.
    c = 1.0 / 64
    for n, core in KAT["vnni_core"]["cases"]:
        data = np.array([[1] * n + [0]], np.int8).view(np.uint8)
        x = np.array([c] * n + [127 * c], np.float32)
        out = orc.matvec(Q8, np.array([1.0], np.float32), data, x, vnni=True)
        assert out[0] == np.float32((core - 128 * n) * c)


# ---------------------------------------------------------------- streams (oracle)

def _cfg(rec):
    d = dict(rec["config"])
    d["mrope_section"] = tuple(d["mrope_section"])
    return DecoderConfig(**d)


def _stream_inputs(rec):
    ids = np.array(rec["ids"], np.int32)
    kw = {}
    if "image_rows" in rec:
        kw = dict(image_embeds=synth.image_embeds(rec["image_rows"], rec["config"]["hidden"], seed=rec["image_seed"]),
                  image_token_id=rec["image_token_id"], grid=tuple(rec["grid"]))
    return ids, kw


TINY_CASES = sorted(k for k in STREAMS if k.startswith("tiny"))
ERNIE_CASES = sorted(k for k in STREAMS if k.startswith("ernie"))


@pytest.mark.parametrize("name", TINY_CASES)
def test_oracle_reproduces_tiny_streams(orc, name):
    rec = STREAMS[name]
    cfg = _cfg(rec)
    w = synth.make_weights(cfg, rec["qtype"], seed=rec["weight_seed"])
    m = orc.Model(cfg)
    m.load_weights(w)
    m.set_quirk(rec["quirk"])
    ids, kw = _stream_inputs(rec)
    assert list(m.generate(ids, rec["max_new"], eos=(), **kw)) == rec["tokens"]


# ---------------------------------------------------------------- HIP path

@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [Q8, Q4, Q6])
def test_gpu_matvec_closed_forms(ctx, qtype):
    for w, x in _closed_forms():
        q = lib.QMatrix.quantize(w, qtype)
        codes = lib.unpack_rows(qtype, q.packed, w.shape[1]).astype(np.float64)
        want = (codes @ x.astype(np.float64)) * q.scales.astype(np.float64)
        dw = ctx.upload(q)
        try:
            assert np.allclose(ctx.matvec(dw, x), want, rtol=1e-5, atol=1e-5)
        finally:
            dw.close()


@pytest.mark.gpu
def test_gpu_argmax_ties(ctx):
    # rows whose scores repeat the KAT's: row r of the identity picks x[r]
    k = KAT["argmax_ties"]
    n = len(k["scores"])
    q = lib.QMatrix.quantize(np.eye(n, dtype=np.float32), Q8)
    dw = ctx.upload(q)
    try:
        idx, _ = ctx.matvec_argmax(dw, np.array(k["scores"], np.float32))
    finally:
        dw.close()
    assert idx == k["index"]


@pytest.mark.gpu
def test_gpu_rope_first_token_k(ctx):
    k = KAT["rope_first_token_k"]
    q = np.array(k["k"], np.float32)
    kk = np.array(k["k"], np.float32)
    qo, ko = ctx.mrope_pair(q, kk, np.array(k["cos"], np.float32), np.array(k["sin"], np.float32), 1, 1, 4)
    assert list(ko) == k["rotated"] and list(qo) == k["rotated"]


@pytest.mark.gpu
def test_gpu_weighted_value_sum(ctx):
    k, q, kc, vc = _wvs()
    out = ctx.text_attention(q, kc, vc, k["len"], k["heads"], k["kv_heads"], k["head_dim"])
    assert np.max(np.abs(out[4:] - np.array(k["out_head1"]))) < 2e-5


def _gpu_stream(ctx, rec, use_prefill=False):
    cfg = _cfg(rec)
    w = synth.make_weights(cfg, rec["qtype"], seed=rec["weight_seed"])
    m = lib.Model(ctx, cfg)
    m.load_weights(w)
    m.set_residual_quirk(rec["quirk"])
    ids, kw = _stream_inputs(rec)
    s = m.seq(len(ids) + rec["max_new"] + 4)
    got = s.generate(ids, rec["max_new"], eos=(), use_prefill=use_prefill, **kw)
    s.close()
    m.close()
    return got


@pytest.mark.gpu
@pytest.mark.parametrize("use_prefill", [False, True], ids=["steps", "prefill"])
@pytest.mark.parametrize("name", TINY_CASES + ERNIE_CASES)
def test_gpu_matches_golden_streams(ctx, name, use_prefill):
    rec = STREAMS[name]
    assert list(_gpu_stream(ctx, rec, use_prefill)) == rec["tokens"], name
