"""The sampling LM head's checker: SplitMix64 draws, top-k selection and the
candidate sampler of the oracle, pinned by the reference's known answers, the
published SplitMix64 outputs and what the mathematics fixes (the sampled
distribution is softmax(score / temperature) over the candidates; equal
weights split [0, 1) evenly; a single candidate draws nothing)."""
import json
import math
import os

import numpy as np
import pytest

import oracle

KAT = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")))


def test_splitmix64_published_outputs():
    k = KAT["splitmix64"]
    r = oracle.Rng(k["seed"])
    for h in k["outputs"]:
        assert r.float64() == (int(h, 16) >> 11) * 2.0 ** -53


def test_rng_state_is_the_seed_plus_golden_gamma():
    r = oracle.Rng(12345)
    r.float64()
    assert r.state.value == (12345 + 0x9E3779B97F4A7C15) % (1 << 64)


def test_topk_reference_kats():
    k = KAT["topk_sorted"]
    ids, sc = oracle.topk(k["logits"], k["k"])
    assert list(ids) == k["ids"]
    k = KAT["topk_sort_small"]
    ids, _ = oracle.topk(k["scores"], len(k["scores"]))
    assert list(ids) == k["ids"]
    k = KAT["topk_pairs"]
    scores = np.full(100, -np.inf, np.float32)
    for s, t in k["pairs"]:
        if t >= 0:
            scores[t] = s
    ids, sc = oracle.topk(scores, k["k"])
    assert [[int(i), float(v)] for i, v in zip(ids, sc)] == k["want"]


def planted_logits():
    k = KAT["topk_planted"]
    rows, cols = k["rows"], k["cols"]
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    w = (((r % 17) - 8) * 0.125 + ((r + c) % 7 - 3) * 0.25).astype(np.float32)
    for row, vals in k["planted"].items():
        w[int(row)] = vals
    x = np.asarray(k["x"], np.float32)
    return w, x, (w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)


def test_topk_planted_rows():
    k = KAT["topk_planted"]
    _, _, logits = planted_logits()
    for row, v in k["planted_scores"].items():
        assert logits[int(row)] == v
    ids, sc = oracle.topk(logits, k["k"])
    assert ids[0] == 269 and list(ids[1:3]) == [k["tie_first"], 256]
    order = np.lexsort((np.arange(logits.size), -logits))[: k["k"]]
    assert list(ids) == list(order)


@pytest.mark.parametrize("seed", range(6))
def test_topk_brute_force_with_ties(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 400))
    scores = rng.integers(-6, 6, n).astype(np.float32) * np.float32(0.5)  # many ties
    k = int(rng.integers(1, 70))
    ids, sc = oracle.topk(scores, k)
    order = np.lexsort((np.arange(n), -scores))[:k]
    assert list(ids) == list(order)
    assert np.array_equal(sc, scores[order])


def test_single_candidate_draws_nothing():
    r = oracle.Rng(7)
    assert oracle.sample_candidates([42], [1.0], 0.7, r) == 42
    assert r.state.value == 7


@pytest.mark.parametrize("n", [2, 3, 4, 5, 8, 9, 64])
@pytest.mark.parametrize("temp", [1.0, 0.5])
def test_equal_scores_split_the_unit_interval(n, temp):
    # all weights 1: the pick u·n lands in candidate ceil(u·n) − 1
    ids = np.arange(100, 100 + n, dtype=np.int32)
    scores = np.full(n, 0.25, np.float32)
    r = oracle.Rng(3)
    for _ in range(200):
        probe = oracle.Rng(r.state.value)
        u = probe.float64()
        got = oracle.sample_candidates(ids, scores, temp, r)
        if n == 2:  # u·(1 + w1) <= 1 with w1 = 1
            want = 0 if u * 2 <= 1 else 1
        elif temp == 1.0:  # f32 draw and sums
            want = math.ceil(float(np.float32(np.float32(u) * np.float32(n)))) - 1
        else:  # f64 draw and sums
            want = math.ceil(u * n) - 1
        assert got == 100 + min(max(want, 0), n - 1), (u, n, temp)


@pytest.mark.parametrize("n", [2, 3, 4, 6, 16])
@pytest.mark.parametrize("temp", [1.0, 0.7, 1.6])
def test_sampled_frequencies_follow_softmax(n, temp):
    # P(c_i) = exp(s_i / T) / Σ exp(s_j / T): chi-square over 20k draws
    rng = np.random.default_rng(n * 10 + int(temp * 10))
    scores = np.sort(rng.normal(0, 1.0, n).astype(np.float32))[::-1].copy()
    ids = np.arange(n, dtype=np.int32)
    p = np.exp((scores.astype(np.float64) - scores.max()) / temp)
    p /= p.sum()
    r = oracle.Rng(2024)
    draws = 20000
    counts = np.bincount([oracle.sample_candidates(ids, scores, temp, r) for _ in range(draws)], minlength=n)
    expect = p * draws
    chi2 = float(((counts - expect) ** 2 / expect).sum())
    # 99.9 % quantile of chi-square with n-1 degrees of freedom is below 3·(n−1)+20
    assert chi2 < 3 * (n - 1) + 20, (counts, expect)


def test_sampling_is_monotone_in_the_draw():
    # a larger draw never picks an earlier candidate
    scores = np.array([2.0, 1.5, 1.0, 0.2, -0.3, -1.0, -2.0], np.float32)
    ids = np.arange(7, dtype=np.int32)
    for temp in (1.0, 0.8):
        pairs = []
        r = oracle.Rng(99)
        for _ in range(400):
            u = oracle.Rng(r.state.value).float64()
            pairs.append((u, oracle.sample_candidates(ids, scores, temp, r)))
        pairs.sort()
        picks = [p for _, p in pairs]
        assert picks == sorted(picks)


# ---- full-vocabulary draw (sampleFullLogitsScratch, CumulativeSum,
# pickCumulativeFloat32)

def test_pick_cumulative_reference_kat():
    # internal/model/sampling_test.go:118-134
    cdf = [0.25, 0.75, 1.0]
    for pick, want in ((0.01, 0), (0.25, 0), (0.26, 1), (0.75, 1), (0.90, 2)):
        assert oracle.pick_cumulative(cdf, pick) == want
    assert oracle.pick_cumulative(cdf, 1.1) == -1


@pytest.mark.parametrize("n", [1, 7, 4095, 4096, 5001])
def test_cumsum_of_ones_is_exact(n):
    out, tot = oracle.cumsum(np.ones(n, np.float32))
    assert np.array_equal(out, np.arange(1, n + 1, dtype=np.float32)) and tot == n


def test_cumsum_blocks_sum_from_zero():
    # 2^24 then ones: a single running sum never moves (2^24 + 1 rounds back
    # to 2^24), but from 4096 entries on CumulativeSum sums each quarter from
    # zero and shifts it by the block totals before it, so block b ≥ 1 holds
    # fl(2^24 + 2048·(b−1) + j), j = 1..2048: even j exact, odd j to the even
    # neighbour (4·⌊(j+1)/4⌋)
    n, bs = 8192, 2048
    x = np.ones(n, np.float32)
    x[0] = 2.0 ** 24
    out, tot = oracle.cumsum(x)
    assert np.all(out[:bs] == 2.0 ** 24)
    j = np.arange(1, bs + 1)
    inc = np.where(j % 2 == 0, j, 4 * ((j + 1) // 4))
    for b in (1, 2, 3):
        assert np.array_equal(out[b * bs:(b + 1) * bs], 2.0 ** 24 + 2048 * (b - 1) + inc), b
    assert tot == 2.0 ** 24 + 3 * 2048
    small, _ = oracle.cumsum(x[:4095])  # below 4096: one running sum
    assert np.all(small == 2.0 ** 24)


def test_sample_full_reference_kat():
    # sampling_test.go:108-116: [-100, -100, 0] at temperature 1 gives a valid
    # id for seeds 0..7.  Here −100 is past FastExp's wrap (the weights come
    # out near −1.66·2^111), the running sum is negative, no cumulative entry
    # reaches the pick and the search runs off the end: the last id, 2
    for seed in range(8):
        assert oracle.sample_full(np.array([-100, -100, 0], np.float32), 1.0, oracle.Rng(seed)) == 2
    # sampling_test.go:136-146
    for temp in (0.5, 0.8, 1.5):
        r = oracle.Rng(3)
        for _ in range(8):
            assert 0 <= oracle.sample_full(np.array([-4, 0.5, 3, -2], np.float32), temp, r) < 4


def test_sample_full_two_logits_is_sample_two():
    # sampleTwoLogits (model.go:2309-2324): s0 ≥ s1 draws 0 when u·(1+w1) ≤ 1
    r = oracle.Rng(11)
    for _ in range(100):
        u = oracle.Rng(r.state.value).float64()
        w1 = float(oracle.fast_exp(float(np.float32(np.float32(-1.0) * np.float32(1.0 / np.float32(0.7))))))
        got = oracle.sample_full(np.array([2.0, 1.0], np.float32), 0.7, r)
        assert got == (0 if u * (1 + w1) <= 1 else 1)


def test_sample_full_equal_logits_split_the_unit_interval():
    # all weights 1: cdf[i] = i + 1 (exact), sum = n, pick = f32(u)·n →
    # index ceil(pick) − 1
    for n in (3, 10, 5000):
        r = oracle.Rng(n)
        for _ in range(50):
            u = oracle.Rng(r.state.value).float64()
            pick = float(np.float32(np.float32(u) * np.float32(n)))
            want = max(math.ceil(pick) - 1, 0)
            assert oracle.sample_full(np.full(n, 0.5, np.float32), 0.9, r) == want


@pytest.mark.parametrize("temp", [1.0, 0.6, 2.0])
def test_sample_full_frequencies_follow_softmax(temp):
    # P(i) = exp(x_i / T) / Σ exp(x_j / T): chi-square over 20k draws
    rng = np.random.default_rng(int(temp * 10))
    x = rng.normal(0, 1.0, 12).astype(np.float32)
    p = np.exp((x.astype(np.float64) - x.max()) / temp)
    p /= p.sum()
    r = oracle.Rng(7)
    draws = 20000
    counts = np.bincount([oracle.sample_full(x, temp, r) for _ in range(draws)], minlength=12)
    expect = p * draws
    chi2 = float(((counts - expect) ** 2 / expect).sum())
    assert chi2 < 3 * 11 + 20, (counts, expect)


def test_sample_full_monotone_in_the_draw():
    x = np.random.default_rng(4).normal(0, 2, 6000).astype(np.float32)  # four blocks
    pairs = []
    r = oracle.Rng(5)
    for _ in range(300):
        u = oracle.Rng(r.state.value).float64()
        pairs.append((u, oracle.sample_full(x, 1.0, r)))
    pairs.sort()
    picks = [p for _, p in pairs]
    assert picks == sorted(picks)


@pytest.mark.parametrize("seed", range(4))
def test_topk_wide_k_brute_force_with_ties(seed):
    # k > 64 sorts under the selection sort's order: score descending, lower
    # index first among equal scores
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(70, 3000))
    scores = rng.integers(-20, 20, n).astype(np.float32) * np.float32(0.25)
    k = int(rng.integers(65, n + 1))
    ids, sc = oracle.topk(scores, k)
    order = np.lexsort((np.arange(n), -scores))[:k]
    assert list(ids) == list(order) and np.array_equal(sc, scores[order])


@pytest.mark.parametrize("temp", [1.0, 0.5])
def test_wide_candidates_split_the_unit_interval(temp):
    # 300 equal candidates: the f32 (temperature 1) or f64 sums are exact
    n = 300
    ids = np.arange(n, dtype=np.int32)
    scores = np.full(n, 1.5, np.float32)
    r = oracle.Rng(21)
    for _ in range(100):
        u = oracle.Rng(r.state.value).float64()
        got = oracle.sample_candidates(ids, scores, temp, r)
        if temp == 1.0:
            want = math.ceil(float(np.float32(np.float32(u) * np.float32(n)))) - 1
        else:
            want = math.ceil(u * n) - 1
        assert got == min(max(want, 0), n - 1)
