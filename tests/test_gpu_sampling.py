"""Sampling LM head on the device against the oracle, at op level and inside
generation: top-k candidates and the draw among them (topKSelectWithWork +
sampleCandidateScoresScratch with fastRNG) for any 1 < k < n, and the draw
over every logit (sampleFullLogitsScratch) for top_k 0 or >= vocab."""
import json
import os

import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
KAT = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")))
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)


def _exact_q8(rng, rows, cols):
    """Q8 rows whose scale is a power of two and codes integers, with integer
    x: every score is exact in f32 on both sides, so ids must match exactly,
    ties included."""
    codes = rng.integers(-20, 21, (rows, cols)).astype(np.float32)
    codes[:, 0] = 127  # max |w| = 127·2^e → scale 2^e exactly
    e = rng.integers(-3, 2, rows).astype(np.float32)
    return codes * (2.0 ** e)[:, None]


@pytest.mark.parametrize("k", [1, 2, 7, 50, 64, 65, 300, 9000])
def test_matvec_topk_exact_scores_with_ties(ctx, orc, k):
    rng = np.random.default_rng(k)
    w = _exact_q8(rng, 9000, 256)
    w[[100, 4000, 8999]] = w[50]  # identical rows: exact ties, lower row first
    x = rng.integers(-3, 4, 256).astype(np.float32)
    x[0] = 0.0
    q = lib.QMatrix.quantize(w, Q8)
    logits = orc.matvec(Q8, q.scales, q.packed, x)
    want_ids, want_sc = orc.topk(logits, k)
    ids, sc = ctx.matvec_topk(ctx.upload(q), x, k)
    assert list(ids) == list(want_ids)
    assert np.array_equal(sc, want_sc)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_matvec_topk_planted_rows(ctx, orc, qtype):
    # the reference's own top-k test shape (270 rows × 5 columns, k = 50)
    k = KAT["topk_planted"]
    rows, cols = k["rows"], k["cols"]
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    w = (((r % 17) - 8) * 0.125 + ((r + c) % 7 - 3) * 0.25).astype(np.float32)
    for row, vals in k["planted"].items():
        w[int(row)] = vals
    x = np.asarray(k["x"], np.float32)
    q = lib.QMatrix.quantize(w, qtype)
    logits = orc.matvec(qtype, q.scales, q.packed, x)
    ids, sc = ctx.matvec_topk(ctx.upload(q), x, k["k"])
    assert len(ids) == k["k"]
    # scores to 1e-4 (the reference's bar); order by score, then lower row
    assert np.max(np.abs(sc - logits[ids])) <= 1e-4
    key = [(-float(s), int(i)) for s, i in zip(sc, ids)]
    assert key == sorted(key)
    # the set is the oracle's top-k up to scores within 1e-4 of the k-th
    kth = np.sort(logits)[::-1][k["k"] - 1]
    want, _ = orc.topk(logits, k["k"])
    sure = {int(i) for i in want if logits[i] > kth + 1e-4}
    assert sure <= set(int(i) for i in ids)
    assert ids[0] == 269


def test_matvec_topk_lm_head(ctx, orc):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((103424, 1024)) * 0.02).astype(np.float32)
    q = lib.QMatrix.quantize(w, Q4)
    wd = ctx.upload(q)
    for seed in range(3):
        x = np.random.default_rng(seed).standard_normal(1024).astype(np.float32)
        logits = orc.matvec(Q4, q.scales, q.packed, x)
        ids, sc = ctx.matvec_topk(wd, x, 64)
        want, wsc = orc.topk(logits, 64)
        assert np.max(np.abs(sc - logits[ids])) <= 1e-4 * max(1.0, float(np.max(np.abs(wsc))))
        gaps = np.diff(np.sort(logits)[::-1][:65])
        if np.min(np.abs(gaps)) > 1e-5:  # no near-ties: the same ids in the same order
            assert list(ids) == list(want)


@pytest.mark.parametrize("k", [2, 3, 4, 5, 8, 9, 20, 64])
@pytest.mark.parametrize("temp", [1.0, 0.7, 2.5, 0.04])
def test_sample_topk_matches_oracle(ctx, orc, k, temp):
    # same logits on both sides: candidates, draw and generator state are
    # bit-identical (temperature 0.04 reaches FastExp's wrap below −88.7)
    rng = np.random.default_rng(k * 100 + int(temp * 100))
    logits = (rng.standard_normal(50000) * 3).astype(np.float32)
    logits[rng.integers(0, 50000, 8)] = logits.max()  # ties at the top
    state = 0x1234_5678_9ABC_DEF0 + k
    r = orc.Rng(state)
    for _ in range(12):
        want_ids, want_sc = orc.topk(logits, k)
        want_tok = orc.sample_candidates(want_ids, want_sc, temp, r)
        tok, state, ids, sc = ctx.sample_topk(logits, k, temp, state)
        assert list(ids) == list(want_ids) and np.array_equal(sc, want_sc)
        assert tok == want_tok
        assert state == r.state.value
        logits = np.roll(logits, 977)


def test_sample_topk_rejects_bad_arguments(ctx):
    logits = np.zeros(100, np.float32)
    for k, temp in ((1, 1.0), (100, 1.0), (4, 0.0), (4, -1.0), (4, float("nan"))):
        with pytest.raises(lib.PocrError):
            ctx.sample_topk(logits, k, temp, 1)
    for temp in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(lib.PocrError) as e:
            ctx.sample_full(logits, temp, 1)
        assert e.value.code == lib.POCR_ERR_ARG
    with pytest.raises(lib.PocrError):
        ctx.sample_full(np.zeros(0, np.float32), 1.0, 1)


@pytest.mark.parametrize("n", [1, 3, 7, 4095, 4096, 4097, 103424])
@pytest.mark.parametrize("temp", [1.0, 0.8, 1.7, 0.05])
def test_sample_full_matches_oracle(ctx, orc, n, temp):
    # every logit: the weights, the f32 running sums in the reference's order
    # (CumulativeSum's four blocks from 4096 on), the pick and the binary
    # search are bit-identical, so token and generator state are too
    # (temperature 0.05 reaches FastExp's wrap below −88.7 for most logits)
    rng = np.random.default_rng(n * 10 + int(temp * 100))
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    state = 0x0DDB_A11_5EED + n
    r = orc.Rng(state)
    for _ in range(10):
        want = orc.sample_full(logits, temp, r)
        tok, state = ctx.sample_full(logits, temp, state)
        assert tok == want and state == r.state.value
        logits = np.roll(logits, 977)


def test_sample_full_two_logits(ctx, orc):
    state = 99
    r = orc.Rng(state)
    for a, b, temp in ((2.0, 1.0, 0.7), (1.0, 2.0, 1.0), (0.5, 0.5, 1.3), (-300.0, 0.0, 1.0)):
        for _ in range(20):
            want = orc.sample_full(np.array([a, b], np.float32), temp, r)
            tok, state = ctx.sample_full(np.array([a, b], np.float32), temp, state)
            assert tok == want and state == r.state.value


def test_sample_full_lm_head_shapes(ctx, orc):
    # 103,424 logits shaped like an LM head's (a few dominant rows, a long
    # tail, exact ties at the top), 40 consecutive draws per temperature
    rng = np.random.default_rng(77)
    logits = (rng.standard_normal(103424) * 2.5).astype(np.float32)
    logits[rng.integers(0, 103424, 6)] = logits.max() + 4.0
    logits[rng.integers(0, 103424, 200)] -= 60.0
    for temp in (1.0, 0.7, 1.3):
        state = 12345
        r = orc.Rng(state)
        for _ in range(40):
            want = orc.sample_full(logits, temp, r)
            tok, state = ctx.sample_full(logits, temp, state)
            assert tok == want and state == r.state.value


@pytest.mark.parametrize("k", [65, 100, 1000, 49999])
@pytest.mark.parametrize("temp", [1.0, 0.7, 0.04])
def test_sample_topk_wide_matches_oracle(ctx, orc, k, temp):
    # more than 64 candidates: every score sorted on the device, the draw's
    # running sums (f32 at temperature 1, f64 otherwise) in candidate order
    rng = np.random.default_rng(k * 10 + int(temp * 100))
    logits = (rng.standard_normal(50000) * 3).astype(np.float32)
    logits[rng.integers(0, 50000, 8)] = logits.max()  # ties at the top
    logits[rng.integers(0, 50000, 400)] = np.float32(0.25)  # ties inside
    state = 0x1234_5678_9ABC_DEF0 + k
    r = orc.Rng(state)
    for _ in range(6):
        want_ids, want_sc = orc.topk(logits, k)
        want_tok = orc.sample_candidates(want_ids, want_sc, temp, r)
        tok, state, ids, sc = ctx.sample_topk(logits, k, temp, state)
        assert np.array_equal(ids, want_ids) and np.array_equal(sc, want_sc)
        assert tok == want_tok
        assert state == r.state.value
        logits = np.roll(logits, 977)


def _models(orc, ctx, cfg, qtype, seed):
    w = synth.make_weights(cfg, qtype, seed=seed)
    om = orc.Model(cfg)
    om.load_weights(w)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    return om, gm


@pytest.mark.parametrize("qtype", [Q4, Q8], ids=["q4", "q8"])
@pytest.mark.parametrize("temp,top_k", [(0.8, 20), (1.0, 3), (1.0, 64), (1.7, 9)])
def test_generate_sampled_matches_oracle(orc, ctx, qtype, temp, top_k):
    om, gm = _models(orc, ctx, MID, qtype, seed=9)
    ids = synth.prompt_ids(23, seed=4, high=MID.vocab)
    for seed in (1, 2024):
        want = list(om.generate(ids, 24, eos=(), temperature=temp, top_k=top_k, seed=seed))
        s = gm.seq(ids.size + 24)
        s.set_sampling(temp, top_k, seed)
        assert list(s.generate(ids, 24, eos=(), use_prefill=True)) == want
        # the generator restarts at the seed for every generation
        assert list(s.generate(ids, 24, eos=(), use_prefill=True)) == want
        s.close()


def test_generate_sampled_ernie_image(orc, ctx):
    cfg = ERNIE_0P3B
    om, gm = _models(orc, ctx, cfg, Q4, seed=0)
    orc.set_threads(16)
    img_tok = 100295
    ids = np.concatenate([synth.prompt_ids(5, seed=10), np.full(24, img_tok, np.int32),
                          synth.prompt_ids(8, seed=20)]).astype(np.int32)
    img = synth.image_embeds(24, cfg.hidden, seed=1)
    kw = dict(image_embeds=img, image_token_id=img_tok, grid=(1, 8, 12))
    want = list(om.generate(ids, 12, eos=(), temperature=0.9, top_k=40, seed=77, **kw))
    s = gm.seq(ids.size + 12)
    s.set_sampling(0.9, 40, 77)
    assert list(s.generate(ids, 12, eos=(), use_prefill=True, **kw)) == want


def _oracle_draw(orc, logits, temp, top_k, state):
    """The oracle's token for one draw over a logits row at generator state."""
    r = orc.Rng(state)
    if top_k <= 0 or top_k >= logits.size:
        return orc.sample_full(logits, temp, r)
    ids, sc = orc.topk(logits, top_k)
    return orc.sample_candidates(ids, sc, temp, r)


def _check_sampled_stream(orc, om, gm, w, ids, got, want, temp, top_k, seed):
    """A device sampled stream against the oracle's.  Where they split, the
    split must come from the logits alone: at the first differing draw m, the
    device's logits row for that draw (the prefill's last row, then one step
    per token, the sampling head's own scores) and the oracle's row give
    their own tokens through the oracle sampler at the generator state before
    draw m, and the two rows agree to 2e-4 of the largest logit.  The sampler
    itself is bit-exact on equal rows (the op-level tests above); with
    thousands of comparable weights a pick lands within the rows' last-bit
    differences of a cumulative boundary every few hundred draws."""
    m = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    if m is None:
        assert len(got) == len(want)
        return None
    cfg = gm.cfg
    n = ids.size
    state = orc.Rng(seed)
    for _ in range(m):
        state.float64()
    st = state.state.value
    s = gm.seq(n + m + 2)
    s.set_sampling(temp, top_k, seed)
    _, dl = s.prefill(w["embed"][ids], np.repeat(np.arange(n, dtype=np.int32)[:, None], 3, axis=1), True)
    for j in range(m):
        _, dl = s.step(w["embed"][want[j]], (n + j,) * 3)
    s.close()
    os_ = om.seq(n + m + 2)
    for p in range(n):
        _, ol, _ = os_.step(w["embed"][ids[p]], (p, p, p), need_logits=p == n - 1, want_logits=p == n - 1)
    for j in range(m):
        _, ol, _ = os_.step(w["embed"][want[j]], (n + j,) * 3)
    scale = max(1.0, float(np.max(np.abs(ol))))
    diff = float(np.max(np.abs(dl.astype(np.float64) - ol)))
    assert _oracle_draw(orc, ol, temp, top_k, st) == want[m]
    assert _oracle_draw(orc, dl, temp, top_k, st) == got[m], f"draw {m}: device token not the sampler's on its logits"
    assert diff <= 2e-4 * scale, f"draw {m}: logits differ by {diff}"
    return m


@pytest.mark.parametrize("qtype", [Q4, Q8], ids=["q4", "q8"])
@pytest.mark.parametrize("temp,top_k", [(0.8, 0), (1.0, 0), (0.9, 300), (1.0, 4999), (1.2, 5000)])
def test_generate_sampled_wide_matches_oracle(orc, ctx, qtype, temp, top_k):
    # top_k 0 and top_k >= vocab (5000) draw from every logit, 300 and 4999
    # from sorted candidates: the stream equals the oracle's up to a split
    # that the logits rows explain
    w = synth.make_weights(MID, qtype, seed=9)
    om = orc.Model(MID)
    om.load_weights(w)
    gm = lib.Model(ctx, MID)
    gm.load_weights(w)
    ids = synth.prompt_ids(23, seed=4, high=MID.vocab)
    for seed in (1, 2024):
        want = list(om.generate(ids, 24, eos=(), temperature=temp, top_k=top_k, seed=seed))
        s = gm.seq(ids.size + 24)
        s.set_sampling(temp, top_k, seed)
        got = list(s.generate(ids, 24, eos=(), use_prefill=True))
        s.close()
        _check_sampled_stream(orc, om, gm, w, ids, got, want, temp, top_k, seed)


def test_generate_full_vocabulary_ernie(orc, ctx):
    cfg = ERNIE_0P3B
    om, gm = _models(orc, ctx, cfg, Q4, seed=0)
    orc.set_threads(16)
    ids = synth.prompt_ids(21, seed=10)
    want = list(om.generate(ids, 16, eos=(), temperature=0.8, top_k=0, seed=5))
    s = gm.seq(ids.size + 16)
    s.set_sampling(0.8, 0, 5)
    assert list(s.generate(ids, 16, eos=(), use_prefill=True)) == want


def test_greedy_settings_stay_greedy(orc, ctx):
    om, gm = _models(orc, ctx, MID, Q4, seed=3)
    ids = synth.prompt_ids(17, seed=8, high=MID.vocab)
    want = list(om.generate(ids, 12, eos=()))
    s = gm.seq(ids.size + 12)
    for temp, top_k in ((0.0, 40), (1.3, 1)):
        s.set_sampling(temp, top_k, 5)
        assert list(s.generate(ids, 12, eos=(), use_prefill=True)) == want
    # back from sampling to greedy: the captured step is rebuilt
    s.set_sampling(0.8, 10, 5)
    s.generate(ids, 12, eos=(), use_prefill=True)
    s.set_sampling(0.0, 0, 0)
    assert list(s.generate(ids, 12, eos=(), use_prefill=True)) == want


def test_sampling_settings_errors(ctx):
    gm = lib.Model(ctx, MID)
    gm.load_weights(synth.make_weights(MID, Q4, seed=1))
    s = gm.seq(16)
    for temp, top_k in ((float("nan"), 4), (float("inf"), 4), (-0.5, 4), (1.0, -2)):
        with pytest.raises(lib.PocrError) as e:
            s.set_sampling(temp, top_k, 0)
        assert e.value.code == lib.POCR_ERR_ARG
    # a sampling sequence decodes in a batch too (its own generator), with
    # any candidate width
    for top_k in (8, 0, 65, MID.vocab):
        s.set_sampling(0.7, top_k, 0)
        s.reset()
        assert len(lib.decode_batch([s], [1], [0], 2, eos=())[0]) == 2


def _tie_prone_logit(orc):
    """A logit whose FastExp weight ends its mantissa in 1 and nine zeros: once
    a running sum of such weights reaches the binade where the grid is
    2^10 weight-ulps, every add of it is a rounding tie."""
    import struct
    for i in range(200000):
        v = float(np.float32(-0.7 + i * 1e-6))
        m = struct.unpack("<I", struct.pack("<f", np.float32(orc.fast_exp(v))))[0] & 0x7FFFFF
        if m and (m & -m).bit_length() - 1 >= 9:
            return v
    raise AssertionError("no tie-prone logit found")


def _chain_logits(orc, case, n, rng):
    if case == "normal":
        return (rng.standard_normal(n) * 3).astype(np.float32)
    if case == "peaked":
        x = (rng.standard_normal(n) * 2).astype(np.float32)
        x[rng.integers(0, n, 3)] += 25.0
        return x
    if case == "flat":
        x = np.zeros(n, np.float32)
        x[n // 3] = 0.5
        return x
    if case == "coarse":
        return (np.round(rng.standard_normal(n) * 4) / 2).astype(np.float32)
    if case == "ties":
        x = np.full(n, _tie_prone_logit(orc), np.float32)
        x[0] = 0.0
        return x
    if case == "tiny":  # weights near the bottom of the normal range first
        x = (rng.standard_normal(n) * 0.5).astype(np.float32)
        x[: n // 8] -= 80.0
        return x
    raise ValueError(case)


@pytest.mark.parametrize("n", [5000, 103424])
@pytest.mark.parametrize("case", ["normal", "peaked", "flat", "coarse", "ties", "tiny"])
def test_parallel_running_sums_equal_one_by_one(ctx, orc, monkeypatch, case, n):
    # POCR_CHAIN=check: every draw also evaluates its running sums one add
    # after another and the call fails if any sum differs in any bit; the
    # draws equal the oracle's
    monkeypatch.setenv("POCR_CHAIN", "check")
    rng = np.random.default_rng(n + len(case))
    logits = _chain_logits(orc, case, n, rng)
    for temp in (1.0, 0.8, 2.0):
        state = 5 + n
        r = orc.Rng(state)
        for _ in range(3):
            want = orc.sample_full(logits, temp, r)
            tok, state = ctx.sample_full(logits, temp, state)
            assert tok == want and state == r.state.value
        k = min(n - 1, 3000)
        for _ in range(2):  # f32 (temperature 1) or f64 candidate sums
            want_ids, want_sc = orc.topk(logits, k)
            want = orc.sample_candidates(want_ids, want_sc, temp, r)
            tok, state, ids, _ = ctx.sample_topk(logits, k, temp, state)
            assert tok == want and state == r.state.value
