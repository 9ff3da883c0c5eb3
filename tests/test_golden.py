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


def _vnni_kat_core(orc, n, core):
    """A Q6 row that takes the VNNI branch (>= 32 columns) and whose integer
    core over its first n columns is the KAT's: n ones against xq = 129, a
    code-31 column against x = 0 (xq = 128, sets the row scale to exactly 1),
    zero codes elsewhere and one x = 127c in a zero column (sets scaleX = c).
    dot = core + 31·128 and rowSum = n + 31, so the finalize leaves
    (core − 128n)·c."""
    cols = 40
    c = 1.0 / 64
    w = np.zeros((1, cols), np.float32)
    w[0, :n] = 1.0
    w[0, n] = 31.0
    x = np.zeros(cols, np.float32)
    x[:n] = c
    x[cols - 1] = 127 * c
    sc, data = orc.quantize_matrix(Q6, w)
    assert sc[0] == 1.0
    assert list(orc.unpack_matrix(Q6, data, cols)[0, :n + 1]) == [1] * n + [31]
    out = orc.matvec(Q6, sc, data, x, vnni=True)
    return out[0], np.float32((core - 128 * n) * c)


def test_vnni_core(orc):
    # vnni_test.go:8-25: all-ones codes against xq = 129
    for n, core in KAT["vnni_core"]["cases"]:
        assert orc.vnni_core([1] * n, [129] * n) == core
        got, want = _vnni_kat_core(orc, n, core)
        assert got == want


def _finalize_case(form, n):
    i = np.arange(n)
    if form.startswith("dots=i*100+128"):
        return (i * 100 + 128).astype(np.int32), i.astype(np.int32), np.float32(i + 1) * np.float32(0.1)
    assert form.startswith("dots=i*37-128*(i%5)")
    return (i * 37 - 128 * (i % 5)).astype(np.int32), (i % 5).astype(np.int32), np.float32(i + 1) * np.float32(0.003)


def _round_each_step(v, sx, s):
    """f32(f32(v·sx)·s) with each product formed exactly in f64 (24-bit by
    24-bit mantissas fit its 53 bits) and rounded once to f32."""
    t = (np.asarray(v, np.float64) * np.float64(sx)).astype(np.float32)
    return (t.astype(np.float64) * np.asarray(s, np.float64)).astype(np.float32)


def test_vnni_finalize_reference_vectors(orc):
    """finalize_test.go:7-58 at the reference's bar (0.001), then exactly:
    the asm multiplies by scaleX first, then by scale[i]
    (dot_vnni_amd64.s:1062-1065), each an f32 rounding."""
    rec = KAT["vnni_finalize"]
    order_seen = False
    for case in rec["cases"]:
        sx = np.float32(case["scale_x"])
        for n in case["ns"]:
            dots, rs, sc = _finalize_case(case["form"], n)
            out = orc.finalize_vnni(dots, rs, sc, sx)
            v = dots.astype(np.int64) - 128 * rs.astype(np.int64)
            ref = (v.astype(np.float32) * sx) * sc
            assert np.all(np.abs(out - ref) <= rec["tolerance"]), (n, out, ref)
            assert np.array_equal(out, _round_each_step(v, sx, sc)), n
            # the other multiplication order rounds differently somewhere,
            # so the exact check above fixes the order
            other = (v.astype(np.float64) * (np.float64(sx) * sc.astype(np.float64)).astype(np.float32)
                     .astype(np.float64)).astype(np.float32)
            order_seen |= not np.array_equal(other, out)
    assert order_seen


def test_vnni_finalize_block_and_tail_forms(orc):
    """The 16-row blocks subtract in f32 after converting dot and 128·rowSum,
    the tail subtracts in int32 and converts once. dot = 2^25 + 3 converts to
    2^25 + 4 (spacing 4, nearest), 128·rowSum = 2^25 exactly: the blocks give
    4, the tail 3."""
    for n in (1, 15, 16, 17, 33):
        dots = np.full(n, (1 << 25) + 3, np.int32)
        rs = np.full(n, 1 << 18, np.int32)
        out = orc.finalize_vnni(dots, rs, np.ones(n, np.float32), 1.0)
        blocks = (n // 16) * 16
        assert list(out) == [4.0] * blocks + [3.0] * (n - blocks), n
    # int32 wrap in the tail (IMULL/SUBL): -2^31 - 128 wraps to 2^31 - 128
    out = orc.finalize_vnni(np.array([-(1 << 31)], np.int32), np.array([1], np.int32), np.ones(1, np.float32), 1.0)
    assert out[0] == np.float32((1 << 31) - 128)


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
@pytest.mark.parametrize("cols", [32, 96, 1024])
def test_vnni_matvec_closed_form(orc, qtype, cols):
    """Power-of-two scales make every step exact: with codes q (one ±qmax per
    row, so scale = 2^m exactly) and x = k·2^j (one |k| = 127, so scaleX =
    2^j and xq = k + 128 exactly), the VNNI result must equal
    Σ q·k · 2^(j+m) computed in integers — a wrong byte offset, a missing
    128·rowSum term or a lost scale fails it."""
    rng = np.random.default_rng(cols + qtype)
    qmax = 7 if qtype == Q4 else 31
    rows = 37
    codes = rng.integers(-qmax, qmax + 1, size=(rows, cols))
    codes[np.arange(rows), rng.integers(0, cols, rows)] = qmax * rng.choice([-1, 1], rows)
    m = rng.integers(-12, 4, size=rows)
    w = (codes * np.exp2(m)[:, None]).astype(np.float32)
    k = rng.integers(-127, 128, size=cols)
    k[rng.integers(0, cols)] = -127
    j = -5
    x = (k * 2.0 ** j).astype(np.float32)
    sc, data = orc.quantize_matrix(qtype, w)
    assert np.array_equal(sc, np.exp2(m).astype(np.float32))
    want = ((codes @ k).astype(np.float64) * np.exp2(m + j)).astype(np.float32)
    assert np.array_equal(orc.matvec(qtype, sc, data, x, vnni=True), want)
    assert np.array_equal(orc.matvec(qtype, sc, data, x), want)


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_vnni_correctness_reference(orc, qtype):
    """vnni_test.go:27-60 on a Q4/Q6 row (>= 32 columns, so the VNNI branch
    runs): within 5 % (or 0.01) of the f32 dot times the row scale. The
    reference draws codes i%17-8; Q4 codes stop at ±7, so its row uses
    i%15-7."""
    rec = KAT["vnni_correctness"]
    for n in rec["ns"]:
        i = np.arange(n)
        a = (i % 17 - 8) if qtype == Q6 else (i % 15 - 7)
        x = (np.float32(1) * (i % rec["x_mod"] - rec["x_off"]).astype(np.float32)) / np.float32(rec["x_den"])
        sc, data = orc.quantize_matrix(qtype, a.astype(np.float32)[None, :])
        vn = orc.matvec(qtype, sc, data, x, vnni=True)[0]
        ref = orc.matvec(qtype, sc, data, x)[0]
        assert abs(vn - ref) <= max(rec["rel_tol"] * abs(ref), rec["abs_tol"]), (n, vn, ref)


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
