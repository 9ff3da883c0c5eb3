"""The reference's VNNI activation mode on the GPU (pocr_matvec_vnni,
pocr_model_set_vnni) against the oracle's VNNI mode.

The mode quantizes x once per matvec to u8 with one scale (quant.go:2087-2115,
dot_amd64.go:228-252) and finishes each row from exact int32 sums
(dot_vnni_amd64.s:1043-1080).  Every step is exact or one IEEE operation, so a
matvec must equal the oracle bit for bit.  In this mode the step also sums
RMSNorm's squares and the attention in the oracle's order (the reference's
portable scalar sums, sumSquaresScalar and dotF32's running sums), so whole
decode steps (logits, K/V rows) and greedy streams are bit-identical to the
oracle's VNNI mode too: an ulp of difference upstream of a matvec would move
an activation byte, and with it a whole row, by a step of the weights."""
import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)


def _qmat(rng, rows, cols, qtype, std=0.02):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    return lib.QMatrix.quantize(w, qtype)


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
@pytest.mark.parametrize("shape", [(3072, 1024), (1024, 3072), (2560, 1024), (103424, 1024)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_matvec_vnni_bit_exact_decoder_shapes(ctx, orc, rng, qtype, shape):
    q = _qmat(rng, *shape, qtype)
    x = rng.standard_normal(shape[1]).astype(np.float32)
    got = ctx.matvec_vnni(ctx.upload(q), x)
    want = orc.matvec(qtype, q.scales, q.packed, x, vnni=True)
    assert np.array_equal(got, want)
    # the mode is really a different arithmetic from plain mode
    plain = orc.matvec(qtype, q.scales, q.packed, x)
    assert not np.array_equal(want, plain)


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
@pytest.mark.parametrize("shape", [(7, 33), (130, 100), (65, 96), (40, 4000), (17, 48), (9, 8192)])
def test_matvec_vnni_bit_exact_odd_shapes(ctx, orc, rng, qtype, shape):
    """Columns off the 32/16-column chunks take the code-at-a-time rows; both
    loops produce the same integers."""
    q = _qmat(rng, *shape, qtype, std=1.0)
    x = (rng.standard_normal(shape[1]) * 3).astype(np.float32)
    got = ctx.matvec_vnni(ctx.upload(q), x)
    assert np.array_equal(got, orc.matvec(qtype, q.scales, q.packed, x, vnni=True))


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_matvec_vnni_rows_and_special_vectors(ctx, orc, rng, qtype):
    q = _qmat(rng, 300, 1024, qtype)
    w = ctx.upload(q)
    xs = np.stack([
        np.zeros(1024, np.float32),                          # m = 0: every byte 128, scaleX 1
        rng.standard_normal(1024).astype(np.float32),
        np.where(np.arange(1024) == 5, 7.5, 0.0).astype(np.float32),  # one spike: other bytes 128
        (rng.standard_normal(1024) * 1e-30).astype(np.float32),       # tiny scale
        np.full(1024, -2.0, np.float32),                     # |x| = max everywhere: bytes 1
    ])
    got = ctx.matvec_vnni(w, xs)
    for i in range(xs.shape[0]):
        assert np.array_equal(got[i], orc.matvec(qtype, q.scales, q.packed, xs[i], vnni=True)), i


def test_matvec_vnni_plain_for_q8_and_narrow_inputs(ctx, orc, rng):
    """Q8 has no row sums in the reference and keeps plain mode, as do inputs
    of fewer than 32 columns."""
    q = _qmat(rng, 512, 1024, Q8)
    w = ctx.upload(q)
    x = rng.standard_normal(1024).astype(np.float32)
    assert np.array_equal(ctx.matvec_vnni(w, x), ctx.matvec(w, x))
    for qt in (Q4, Q6):
        q = _qmat(rng, 64, 31, qt, std=1.0)
        w = ctx.upload(q)
        x = rng.standard_normal(31).astype(np.float32)
        assert np.array_equal(ctx.matvec_vnni(w, x), ctx.matvec(w, x))


def _pair(orc, ctx, cfg, qtype, seed=3):
    w = synth.make_weights(cfg, qtype, seed=seed)
    om = orc.Model(cfg)
    om.load_weights(w)
    om.set_vnni(True)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    gm.set_vnni(True)
    return w, om, gm


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
@pytest.mark.parametrize("seed", [3, 4])
def test_vnni_steps_match_oracle(orc, ctx, qtype, seed):
    w, om, gm = _pair(orc, ctx, MID, qtype, seed=seed)
    os_, gs = om.seq(16), gm.seq(16)
    for p in range(10):  # first-token, 1..5 and >= 6 branches
        emb = w["embed"][(7 * p + 3) % MID.vocab]
        ot, ol, _ = os_.step(emb, (p, p, p))
        gt, gl = gs.step(emb, (p, p, p))
        # bit-identical logits: rows 1..10 of the cache cover the single row,
        # the pair form, the 3-8 row trees and the running sum of Softmax
        assert np.array_equal(gl, ol), (p, float(np.max(np.abs(gl - ol))))
        assert gt == ot
    for li in range(MID.layers):
        gk, gv = gs.read_kv(li)
        ok, ov = os_.kv(li)
        assert np.array_equal(gk.reshape(10, -1), ok.reshape(10, -1))
        assert np.array_equal(gv.reshape(10, -1), ov.reshape(10, -1))
    gs.close()
    gm.close()


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_vnni_generation_ernie(orc, ctx, qtype):
    """The 0.3B decoder, 64 prompt ids from [0, 100000) with seed 0, 16 greedy
    tokens in VNNI mode: the oracle's stream in the same mode (the prompt
    through the mode's batched prefill)."""
    cfg = ERNIE_0P3B
    w, om, gm = _pair(orc, ctx, cfg, qtype, seed=0)
    ids = synth.prompt_ids(64, seed=0)
    want = om.generate(ids, 16, eos=())
    s = gm.seq(96)
    got = s.generate(ids, 16, eos=(), use_prefill=True)
    assert list(got) == list(want)
    assert len(s) == 64 + 15
    s.close()
    gm.close()


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_vnni_batched_prefill_bit_exact(orc, ctx, qtype):
    """The VNNI mode's batched prompt (one plane of activation bytes per token,
    the mode's integer finish in the MFMA GEMMs, the ordered attention per
    head and token) against the oracle's VNNI token steps: the last token's
    logits and every K/V row to the bit, through the first-token, 1..5 and >= 6
    residual branches, then a second prompt on top of the cache (rows from
    clen0 = 13)."""
    w, om, gm = _pair(orc, ctx, MID, qtype, seed=5)
    os_, gs = om.seq(40), gm.seq(40)
    embs = w["embed"][[(11 * p + 2) % MID.vocab for p in range(21)]]
    pos = np.array([[p, p, p] for p in range(21)], np.int32)
    for lo, hi in ((0, 13), (13, 21)):
        for p in range(lo, hi):
            ot, ol, _ = os_.step(embs[p], tuple(pos[p]))
        gt, gl = gs.prefill(embs[lo:hi], pos[lo:hi], want_logits=True)
        assert gt == ot
        assert np.array_equal(gl, ol), (lo, float(np.max(np.abs(gl - ol))))
    assert len(gs) == 21
    for li in range(MID.layers):
        gk, gv = gs.read_kv(li)
        ok, ov = os_.kv(li)
        assert np.array_equal(gk.reshape(21, -1), ok.reshape(21, -1)), li
        assert np.array_equal(gv.reshape(21, -1), ov.reshape(21, -1)), li
    gs.close()
    gm.close()


def test_vnni_batched_prefill_runs_batched(ctx, monkeypatch):
    """A 256-row VNNI prompt through the batched prefill and through token
    steps (POCR_BATCHED_PREFILL=0): the same bits, and the batched form is
    the fast one (tens of launches per layer instead of 256 token steps)."""
    import time
    cfg = ERNIE_0P3B
    w = synth.make_weights(cfg, Q4, seed=2)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    gm.set_vnni(True)
    embs = w["embed"][synth.prompt_ids(256, seed=3)]
    pos = np.array([[p, p, p] for p in range(256)], np.int32)

    def run():
        s = gm.seq(260)
        s.prefill(embs[:8], pos[:8])  # warm-up: buffers and first launches
        t0 = time.perf_counter()
        tok, lg = s.prefill(embs[8:], pos[8:], want_logits=True)
        dt = time.perf_counter() - t0
        kv = s.read_kv(cfg.layers - 1)
        s.close()
        return tok, lg, kv, dt

    tb, lb, kvb, dtb = run()
    monkeypatch.setenv("POCR_BATCHED_PREFILL", "0")
    tt, lt, kvt, dtt = run()
    monkeypatch.delenv("POCR_BATCHED_PREFILL")
    assert tb == tt and np.array_equal(lb, lt)
    assert np.array_equal(kvb[0], kvt[0]) and np.array_equal(kvb[1], kvt[1])
    assert dtb * 5 < dtt, (dtb, dtt)
    gm.close()


def test_vnni_mode_rules(ctx, rng):
    cfg = DecoderConfig(hidden=128, inter=192, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=300, eps=1e-5,
                        rope_theta=500000.0)
    w = synth.make_weights(cfg, Q4, seed=1)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    gm.set_vnni(True)
    s = gm.seq(16)
    # fixed before the first sequence
    with pytest.raises(lib.PocrError) as e:
        gm.set_vnni(False)
    assert e.value.code == lib.POCR_ERR_ARG
    s2 = gm.seq(16)
    # 192 intermediate columns are off the batched prefill's 128-column tiles:
    # pocr_prefill takes these rows as token steps, the same cache and logits
    pos = np.array([[p, p, p] for p in range(3)], np.int32)
    tok, lp = s.prefill(w["embed"][[5, 6, 7]], pos, want_logits=True)
    for p in range(3):
        ts, ls = s2.step(w["embed"][5 + p], pos[p])
    assert tok == ts and np.array_equal(lp, ls)
    for li in range(cfg.layers):
        for a, b in zip(s.read_kv(li), s2.read_kv(li)):
            assert np.array_equal(a, b)
    s.close()
    s2.close()
    gm.close()


def _prefilled(gm, ids, budget):
    """A sequence holding the prompt, and the first token the prompt chose."""
    s = gm.seq(ids.size + budget)
    first = int(s.generate(ids, 1, eos=(), use_prefill=True)[0])
    return s, first


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_vnni_decode_batch(orc, ctx, qtype):
    """pocr_decode_batch in the VNNI mode: four sequences, each stream
    bit-identical to the oracle's VNNI-mode stream of that sequence alone
    (the reference serves each request on its own), one of them cut by an
    EOS id."""
    w, om, gm = _pair(orc, ctx, MID, qtype, seed=9)
    prompts = [synth.prompt_ids(n, seed=90 + n, high=MID.vocab) for n in (13, 27, 8, 20)]
    full = [list(om.generate(ids, 14, eos=())) for ids in prompts]
    stop = full[2][6]
    want = [f[: f.index(stop) + 1] if stop in f else f for f in full]
    seqs = [_prefilled(gm, ids, 14) for ids in prompts]
    got = [list(t) for t in lib.decode_batch([s for s, _ in seqs], [f for _, f in seqs],
                                             [ids.size for ids in prompts], 14, eos=(stop,))]
    assert got == want
    for (s, _), ids, g in zip(seqs, prompts, got):
        assert len(s) == ids.size + len(g) - 1
        s.close()
    gm.close()


def test_vnni_continuous_batch(orc, ctx):
    """Continuous batching in the VNNI mode: members join at different token
    steps with different budgets and leave when done; every stream is the
    oracle's VNNI-mode stream of that sequence alone."""
    w, om, gm = _pair(orc, ctx, MID, Q4, seed=11)
    lens, budgets = [11, 26, 7, 19], [12, 7, 15, 9]
    prompts = [synth.prompt_ids(n, seed=70 + i, high=MID.vocab) for i, n in enumerate(lens)]
    want = [list(om.generate(ids, bud, eos=())) for ids, bud in zip(prompts, budgets)]
    b = lib.Batch(gm)
    seqs = [_prefilled(gm, ids, bud) for ids, bud in zip(prompts, budgets)]
    b.join(seqs[0][0], seqs[0][1], lens[0], budgets[0], eos=())
    assert b.step(3) == 1
    b.join(seqs[1][0], seqs[1][1], lens[1], budgets[1], eos=())
    b.join(seqs[2][0], seqs[2][1], lens[2], budgets[2], eos=())
    assert b.step(2) == 3
    b.join(seqs[3][0], seqs[3][1], lens[3], budgets[3], eos=())
    got, pending = {}, [0, 1, 2, 3]
    for _ in range(100):
        b.step(4)
        for i in list(pending):
            n, done = b.poll(seqs[i][0])
            if done:
                got[i] = list(b.leave(seqs[i][0]))
                pending.remove(i)
        if not pending:
            break
    assert [got[i] for i in range(4)] == want
    for i in range(4):
        assert len(seqs[i][0]) == lens[i] + budgets[i] - 1
        seqs[i][0].close()
    b.close()
    gm.close()


@pytest.mark.parametrize("top_k", [40, 0, 200], ids=["top40", "full", "top200"])
def test_vnni_sampled_generation_ernie(orc, ctx, top_k):
    """Sampled decoding in the VNNI mode: the logits are the oracle's to the
    bit, so the candidate sets and draws (top-k ≤ 64, every logit, and the
    wide sorted set) give the oracle's stream."""
    cfg = ERNIE_0P3B
    w, om, gm = _pair(orc, ctx, cfg, Q4, seed=0)
    orc.set_threads(16)
    ids = synth.prompt_ids(21, seed=10)
    want = list(om.generate(ids, 16, eos=(), temperature=0.8, top_k=top_k, seed=5))
    s = gm.seq(ids.size + 16)
    s.set_sampling(0.8, top_k, 5)
    got = list(s.generate(ids, 16, eos=(), use_prefill=True))
    s.close()
    gm.close()
    assert got == want
