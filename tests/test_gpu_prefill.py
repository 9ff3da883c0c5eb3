"""Batched prompt prefill (MFMA GEMMs, causal attention) against the oracle's
token-by-token steps: last-token logits, every K/V row, and the streams that
follow."""
import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
TINY = DecoderConfig(hidden=128, inter=192, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=300, eps=1e-5,
                     rope_theta=500000.0)
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)


def assert_same_choice(gt, ot, gl, ol):
    """Greedy tokens agree, unless the oracle's scores of the two picks are
    closer than twice the measured logit error (each pick's logit then moved
    by at most that error: the flip is the logit bar's, not a new one)."""
    err = float(np.max(np.abs(np.asarray(gl, np.float64) - ol)))
    assert gt == ot or float(ol[ot]) - float(ol[gt]) <= 2 * err, (gt, ot, err)


def _pair(orc, ctx, cfg, qtype, seed=3, quirk=True):
    w = synth.make_weights(cfg, qtype, seed=seed)
    om = orc.Model(cfg)
    om.load_weights(w)
    om.set_quirk(quirk)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    gm.set_residual_quirk(quirk)
    return w, om, gm


def _check_logits(gl, ol):
    # the path's bar: 1e-2 max-abs and 1e-3 relative RMS
    assert np.max(np.abs(gl - ol)) < 1e-2
    assert np.sqrt(np.mean((gl - ol) ** 2)) <= 1e-3 * np.sqrt(np.mean(ol ** 2))


def _check_kv(gs, os_, cfg, rows, rel=2e-4):
    for li in range(cfg.layers):
        gk, gv = gs.read_kv(li)
        ok, ov = os_.kv(li)
        for g, o in ((gk, ok), (gv, ov)):
            g, o = g.reshape(rows, -1), o.reshape(rows, -1)
            scale = max(1.0, float(np.max(np.abs(o))))
            assert float(np.max(np.abs(g - o))) <= rel * scale, li


def _oracle_steps(os_, w, ids, pos, start=0):
    ol = ot = None
    for i in range(start, len(ids)):
        last = i == len(ids) - 1
        ot, ol, _ = os_.step(w["embed"][ids[i]], tuple(pos[i]), need_logits=last)
    return ot, ol


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("cfg", [TINY, MID], ids=["tiny", "mid"])
@pytest.mark.parametrize("quirk", [True, False], ids=["quirk", "noquirk"])
def test_prefill_matches_token_steps(orc, ctx, cfg, qtype, quirk):
    w, om, gm = _pair(orc, ctx, cfg, qtype, quirk=quirk)
    n = 10  # first-token, 1..5 and >= 6 branches of the residual behaviour
    ids = [(7 * p + 3) % cfg.vocab for p in range(n)]
    pos = np.array([[p, p, p] for p in range(n)], np.int32)
    os_, gs = om.seq(16), gm.seq(16)
    ot, ol = _oracle_steps(os_, w, ids, pos)
    gt, gl = gs.prefill(w["embed"][ids], pos, want_logits=True)
    _check_logits(gl, ol)
    assert gt == int(np.argmax(gl))
    assert_same_choice(gt, ot, gl, ol)
    assert len(gs) == n
    _check_kv(gs, os_, cfg, n)


@pytest.mark.parametrize("qtype", [Q4, Q8], ids=["q4", "q8"])
def test_prefill_after_cached_rows(orc, ctx, qtype):
    # 5 tokens by steps, then 37 by one prefill: positions and cache rows continue
    w, om, gm = _pair(orc, ctx, MID, qtype)
    ids = synth.prompt_ids(42, seed=11, high=MID.vocab)
    pos = np.array([[p, p, p] for p in range(42)], np.int32)
    os_, gs = om.seq(48), gm.seq(48)
    ot, ol = _oracle_steps(os_, w, ids, pos)
    for i in range(5):
        gs.step(w["embed"][ids[i]], tuple(pos[i]), need_logits=False)
    gt, gl = gs.prefill(w["embed"][ids[5:]], pos[5:], want_logits=True)
    _check_logits(gl, ol)
    assert_same_choice(gt, ot, gl, ol)
    _check_kv(gs, os_, MID, 42)


@pytest.mark.parametrize("n", [1, 2, 33, 130, 270, 300])
def test_prefill_lengths(orc, ctx, n):
    # 270 and 300 tokens: several 32-token tiles, the last one partly padding
    w, om, gm = _pair(orc, ctx, MID, Q4)
    ids = synth.prompt_ids(n, seed=n, high=MID.vocab)
    pos = np.array([[p, p, p] for p in range(n)], np.int32)
    os_, gs = om.seq(n + 4), gm.seq(n + 4)
    ot, ol = _oracle_steps(os_, w, ids, pos)
    gt, gl = gs.prefill(w["embed"][ids], pos, want_logits=True)
    _check_logits(gl, ol)
    _check_kv(gs, os_, MID, n)


def test_prefill_image_generation_ernie(orc, ctx):
    # the OCR shape in small: 5 ids + a 12×16 merged grid (192 visual rows) + 8 ids,
    # multimodal positions, batched prefill, then 12 greedy tokens on the device
    cfg = ERNIE_0P3B
    w, om, gm = _pair(orc, ctx, cfg, Q4, seed=0)
    img_tok = 100295
    ids = np.concatenate([synth.prompt_ids(5, seed=0), np.full(192, img_tok, np.int32),
                          synth.prompt_ids(8, seed=1)]).astype(np.int32)
    img = synth.image_embeds(192, cfg.hidden, seed=0)
    orc.set_threads(16)
    want = om.generate(ids, 12, eos=(), image_embeds=img, image_token_id=img_tok, grid=(1, 24, 32))
    s = gm.seq(ids.size + 16)
    got = s.generate(ids, 12, eos=(), image_embeds=img, image_token_id=img_tok, grid=(1, 24, 32), use_prefill=True)
    assert list(got) == list(want)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("m", [4, 16, 33, 100, 256, 270, 513])
def test_batched_matvec_mfma_shapes(ctx, orc, rng, qtype, m):
    # the MFMA batched GEMV at the decoder's shapes; 1088 rows leave idle waves
    # in the last workgroup, 320 columns are not whole 256-column LDS stages
    for rows, cols in ((2560, 1024), (1024, 2048), (1024, 3072), (1088, 1024), (256, 320)):
        w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        q = lib.QMatrix.quantize(w, qtype)
        x = rng.standard_normal((m, cols)).astype(np.float32)
        dw = ctx.upload(q)
        got = ctx.matvec(dw, x)
        dw.close()
        for i in range(m):
            want = orc.matvec(qtype, q.scales, q.packed, x[i])
            assert np.max(np.abs(got[i] - want)) <= 5e-5 * max(1.0, float(np.max(np.abs(want))))


@pytest.mark.parametrize("qtype", [Q4, Q6, Q8], ids=["q4", "q6", "q8"])
def test_prefill_gemm_layouts_agree(ctx, qtype, monkeypatch):
    """The LDS-ring GEMM reads the digit planes in its tile layout and the
    weights' tile images; the register-operand GEMM (POCR_PREFILL_GEMM=d)
    reads row-major planes and weights.  Both sum the same exact int32
    products, so a prefill gives the same bits either way: logits of the last
    token and every K/V row."""
    w = synth.make_weights(MID, qtype, seed=21)
    gm = lib.Model(ctx, MID)
    gm.load_weights(w)
    ids = synth.prompt_ids(45, seed=22, high=MID.vocab)
    embs = w["embed"][ids]
    pos = np.array([[p, p, p] for p in range(ids.size)], np.int32)

    def run():
        s = gm.seq(64)
        tok, lg = s.prefill(embs, pos, want_logits=True)
        kv = [s.read_kv(li) for li in range(MID.layers)]
        s.close()
        return tok, lg, kv

    tt, lt, kvt = run()
    monkeypatch.setenv("POCR_PREFILL_GEMM", "d")
    tr, lr, kvr = run()
    monkeypatch.delenv("POCR_PREFILL_GEMM")
    assert tt == tr and np.array_equal(lt, lr)
    for (a, b), (c, d) in zip(kvt, kvr):
        assert np.array_equal(a, c) and np.array_equal(b, d)
    gm.close()
