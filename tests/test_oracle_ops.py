"""Oracle vector ops, matvec, RoPE, attention and positions, pinned by the
reference's known answers, closed forms and f64 brute force."""
import math

import numpy as np
import pytest

from rapidocrvl_amd import lib

Q8, Q4, Q6 = 1000, 1001, 1002


def test_fast_exp_against_libm(orc):
    assert orc.fast_exp(0.0) == 1.0  # poly(0) = 1, n = 0
    xs = np.linspace(-80, 80, 4001, dtype=np.float32)
    got = np.array([orc.fast_exp(float(x)) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    # 5th-degree 2^f polynomial error (≤3.4e-6 on |f|≤0.5) plus the f32 rounding
    # of t = x·log2e, whose ulp grows with |x|; dropping the f^5 term alone
    # would cost ~4e-5
    assert np.all(np.abs(got / want - 1) < 4e-6 + np.abs(xs) * 5e-8)
    # integer multiples of ln2 land on powers of two up to polynomial error
    for k in (-20, -3, 1, 7, 30):
        assert abs(orc.fast_exp(k * math.log(2)) / 2.0**k - 1) < 4e-6


def test_fast_rsqrt_and_silu(orc):
    for x in [1e-6, 0.3, 1.0, 2.0, 17.5, 1e4]:
        # two Newton steps from 0x5f3759df: ≤4.7e-6 (one step would be 1.8e-3)
        assert abs(orc.fast_rsqrt(x) * math.sqrt(x) - 1) < 5e-6
    for x in [-30.0, -5.0, -1.0, 0.0, 0.5, 3.0, 40.0]:
        assert abs(orc.silu(x) - x / (1 + math.exp(-x))) <= 1e-6 * max(1.0, abs(x))


@pytest.mark.parametrize("vals", [
    [42.0], [3.0, 1.0], [3, 1, -2], [1.25, -0.75, 0.5, 2], [1.25, -0.75, 0.5, 2, -1],
    [1.25, -0.75, 0.5, 2, -1, 0.25], [1.25, -0.75, 0.5, 2, -1, 0.25, 1],
    [1.25, -0.75, 0.5, 2, -1, 0.25, 1, -0.5], [-2, 0, 3, 1, -1, 2, 4, 0.5, -0.5],
])
def test_softmax_lengths(orc, vals):
    # quant_test.go:379-444
    x = np.array(vals, np.float64)
    got = orc.softmax(x)
    want = np.exp(x - x.max()) / np.exp(x - x.max()).sum()
    assert np.max(np.abs(got - want)) < 1e-6
    assert abs(got.sum() - 1) < 1e-5


def test_softmax_long(orc, rng):
    x = rng.standard_normal(1500) * 3
    got = orc.softmax(x)
    want = np.exp(x - x.max()) / np.exp(x - x.max()).sum()
    assert np.all(np.abs(got - want) <= 1e-5 * want + 1e-9)  # FastExp relative error ≤ 4e-6


def test_argmax_ties(orc):
    # quant_test.go:448-456
    assert orc.argmax([-1, 0.5, 2, 1.9, 3, 2.5, 3.1, 0]) == 6
    assert orc.argmax([-1, 4, 2, 4, 3, 4]) == 1


def test_rmsnorm_family(orc):
    # quant_test.go:457-488
    x = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9], np.float32)
    w = np.array([1, 0.5, 1.5, 2, 0.25, 1.25, 0.75, 1, 1.1], np.float32)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(orc.rmsnorm(x, w, 1e-6) - want)) < 1e-5
    dst = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9], np.float32)
    add = np.array([0.5, 1, -1.5, 2, -2.5, 3, -3.5, 4, -4.5], np.float32)
    w2 = np.array([1, 1.1, 0.9, 1.2, 0.8, 1.3, 0.7, 1.4, 0.6], np.float32)
    out, dst_after = orc.add_rmsnorm(dst, add, w2, 1e-6)
    assert (dst_after == dst + add).all()
    assert np.max(np.abs(out - orc.rmsnorm(dst + add, w2, 1e-6))) < 1e-6
    out2 = orc.add_rmsnorm_out_only(dst, add, w2, 1e-6)
    assert np.array_equal(out2, out)


def _closed_form_matvec(orc, qtype, w, x):
    sc, data = orc.quantize_matrix(qtype, w)
    codes = orc.unpack_matrix(qtype, data, w.shape[1]).astype(np.float64)
    return sc, data, (codes @ x.astype(np.float64)) * sc.astype(np.float64)


@pytest.mark.parametrize("qtype,tol", [(Q8, 0.05), (Q4, 0.5), (Q6, 0.12)])
def test_matvec_small_known_answers(orc, qtype, tol):
    # quant_test.go:9-85 (approximation vs f32 matvec) and the 4x5 closed-form
    # inputs of internal/backend/vulkan_exec_test.go:1938-2160
    w = np.array([[1, -2, 3], [0.5, 0.25, -0.75]], np.float32)
    x = np.array([2, -1, 0.5], np.float32)
    sc, data, _ = _closed_form_matvec(orc, qtype, w, x)
    assert np.max(np.abs(orc.matvec(qtype, sc, data, x) - w @ x)) <= tol
    for w, x in [
        (np.array([[1, 0, 0, 0, 0], [0, 1, 2, 0, 0], [-1, 0, 0, 0.25, 1], [0.5] * 5], np.float32),
         np.array([2, -1, 0.5, 4, -3], np.float32)),
        (np.array([[1] * 5, [1, 0, 0, 0, -1], [0, 2, 0, -1, 0], [-1] * 5], np.float32),
         np.array([1, 2, 3, 4, 5], np.float32)),
        (np.array([[1, 2, 0], [-1, 0, 1]], np.float32), np.array([3, -2, 5], np.float32)),
    ]:
        sc, data, want = _closed_form_matvec(orc, qtype, w, x)
        assert np.allclose(orc.matvec(qtype, sc, data, x), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("qtype,qmax", [(Q8, 127), (Q4, 7), (Q6, 31)])
def test_matvec_exact_arithmetic(orc, rng, qtype, qmax):
    # power-of-two scale (maxAbs = qmax/8) and integer x: every f32 op is exact
    rows, cols = 37, 96
    codes = rng.integers(-qmax, qmax + 1, size=(rows, cols))
    codes[:, 0] = qmax
    w = (codes / 8.0).astype(np.float32)
    x = rng.integers(-3, 4, size=cols).astype(np.float32)
    sc, data = orc.quantize_matrix(qtype, w)
    assert (sc == np.float32(0.125)).all()
    want = (codes @ x.astype(np.int64)) * 0.125
    assert np.array_equal(orc.matvec(qtype, sc, data, x), want.astype(np.float32))


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6])
def test_matvec_random_vs_f64(orc, rng, qtype):
    w = (rng.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    x = rng.standard_normal(1024).astype(np.float32)
    sc, data, want = _closed_form_matvec(orc, qtype, w, x)
    got = orc.matvec(qtype, sc, data, x)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_vnni_core_and_mode(orc, rng):
    # vnni_test.go:8-25: all-ones weights against xq=129 → 8·129 = 1032, 3·129 = 387;
    # the finalize subtracts 128·rowSum, so x = 1/127-scaled ones give dot = n
    for n, core in [(8, 1032), (3, 387)]:
        assert n * 129 == core
    # x quantisation: RNE, +128 offset, zeros → 128
    s, xq = orc.quantize_x_vnni(np.array([0.0] * 4, np.float32))
    assert s == 1.0 and (xq == 128).all()
    x = np.array([1.0, -1.0, 0.5, -0.25, 127.0 / 254.0], np.float32)
    s, xq = orc.quantize_x_vnni(x)
    assert s == np.float32(1.0) / np.float32(127)
    assert list(xq) == [255, 1, 128 + 64, 128 - 32, 128 + 64]  # 63.5 → 64 (RNE)
    # vnni_test.go:27-60: VNNI result within 5% of the f32 matvec
    for n in (32, 64, 128, 256, 1024):
        a = np.array([i % 17 - 8 for i in range(n)], np.float32)
        xx = np.array([(i % 13 - 6) / 13 for i in range(n)], np.float32)
        sc, data = orc.quantize_matrix(Q4, (a / 8 * 7)[None, :])
        plain = orc.matvec(Q4, sc, data, xx)
        vn = orc.matvec(Q4, sc, data, xx, vnni=True)
        assert abs(vn[0] - plain[0]) <= 0.05 * max(abs(plain[0]), 1e-3)


def test_rope_init_and_tables(orc):
    freq, axis = orc.rope_init(500000.0, 128)
    assert np.allclose(freq, 500000.0 ** (-np.arange(0, 128, 2) / 128.0), rtol=1e-15, atol=0)
    assert list(axis) == [0] * 16 + [1] * 24 + [2] * 24
    c, s = orc.rope_table(freq, axis, 0, 0, 0)
    assert (c == 1).all() and (s == 0).all()  # attention_bench_test.go:181-204
    c, s = orc.rope_table(freq, axis, 7, 7, 7)
    assert np.max(np.abs(c - np.cos(7 * freq))) < 1e-6 and np.max(np.abs(s - np.sin(7 * freq))) < 1e-6
    c, s = orc.rope_table(freq, axis, 7, 3, 11)
    p = np.array([7, 3, 11])[axis]
    assert np.array_equal(c, np.cos(p * freq).astype(np.float32))
    assert np.array_equal(s, np.sin(p * freq).astype(np.float32))


def test_mrope_matches_scalar_reference(orc):
    # model/rope_test.go:10-35: in[i] = sin(0.17 i), 2 heads of 128, theta 1e4, pos (7,3,11)
    x = np.sin(np.arange(256) * 0.17).astype(np.float32)
    freq, axis = orc.rope_init(10000.0, 128)
    c, s = orc.rope_table(freq, axis, 7, 3, 11)
    got = orc.apply_rope(x, c, s, 2, 128)
    want = x.astype(np.float64).copy()
    sections = [16, 24, 24]
    for h in range(2):
        b = h * 128
        for i in range(64):
            ax = 0 if i < 16 else (1 if i < 40 else 2)
            p = (7, 3, 11)[ax]
            ang = p * 10000.0 ** (-2 * i / 128)
            a, bb = x[b + i], x[b + 64 + i]
            want[b + i] = a * math.cos(ang) - bb * math.sin(ang)
            want[b + 64 + i] = bb * math.cos(ang) + a * math.sin(ang)
    assert np.max(np.abs(got - want)) < 1e-6
    assert sum(sections) == 64
    # rotation keeps each (i, i+64) pair's norm
    n0 = x[:64] ** 2 + x[64:128] ** 2
    n1 = got[:64] ** 2 + got[64:128] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


def test_first_token_k_rotation_known_answer(orc):
    # vulkan_fallback_test.go:1066-1119: k=[1,2,3,4] with cos [0,.5] sin [1,.5] → [-3,-1,1,3]
    got = orc.apply_rope(np.array([1, 2, 3, 4], np.float32), [0, 0.5], [1, 0.5], 1, 4)
    assert list(got) == [-3, -1, 1, 3]


def test_weighted_value_sum_known_answer(orc):
    # scratch_test.go:236-248: head 1 of kvDim 8, weights .25/.75 → [40,50,60,70].
    # Scores are chosen so softmax gives exactly those weights: dim 4 → scale .5,
    # s0 = 0, s1 = ln 3.
    k = np.zeros((2, 8), np.float32)
    k[1, 4] = 2 * math.log(3)
    v = np.array([[1, 2, 3, 4, 10, 20, 30, 40], [5, 6, 7, 8, 50, 60, 70, 80]], np.float32)
    q = np.zeros(8, np.float32)
    q[4] = 1
    out = orc.cache_attention(q, k, v, 2, 2, 2, 4)
    assert np.max(np.abs(out[4:] - np.array([40, 50, 60, 70]))) < 2e-5


def _attention_f64(q, kc, vc, L, heads, kvh, dim):
    out = np.zeros(heads * dim)
    g = heads // kvh
    kc = kc.reshape(L, kvh, dim).astype(np.float64)
    vc = vc.reshape(L, kvh, dim).astype(np.float64)
    for h in range(heads):
        s = kc[:, h // g] @ q[h * dim:(h + 1) * dim].astype(np.float64) * np.float32(1 / math.sqrt(dim))
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * dim:(h + 1) * dim] = p @ vc[:, h // g]
    return out


@pytest.mark.parametrize("L", [1, 2, 5, 6, 7, 64, 300])
def test_attention_vs_f64(orc, rng, L):
    heads, kvh, dim = 16, 2, 128
    q = rng.standard_normal(heads * dim).astype(np.float32)
    kc = rng.standard_normal(L * kvh * dim).astype(np.float32)
    vc = rng.standard_normal(L * kvh * dim).astype(np.float32)
    got = orc.cache_attention(q, kc, vc, L, heads, kvh, dim)
    want = _attention_f64(q, kc, vc, L, heads, kvh, dim)
    assert np.max(np.abs(got - want)) < 2e-5
    if L == 1:  # a single cached row returns V exactly (model.go:3980-3983)
        v = vc.reshape(kvh, dim)
        assert np.array_equal(got.reshape(heads, dim), v[np.arange(heads) // 8])


def test_positions_known_answers(orc):
    # model/position_test.go:10-62
    ids = [10, 101305, 100295, 100295, 100295, 100295, 11]
    pos, delta = orc.mm_positions(ids, 100295, (1, 4, 4))
    assert pos.tolist() == [[0, 0, 0], [1, 1, 1], [2, 2, 2], [2, 2, 3], [2, 3, 2], [2, 3, 3], [4, 4, 4]]
    assert delta == -2
    ids = [1, 7, 7, 7, 7, 2, 3, 7, 7, 7, 7, 4]
    pos, delta = orc.mm_positions(ids, 7, (1, 4, 4))
    assert pos.tolist() == [[0, 0, 0], [1, 1, 1], [1, 1, 2], [1, 2, 1], [1, 2, 2], [3, 3, 3], [4, 4, 4],
                            [5, 5, 5], [5, 5, 6], [5, 6, 5], [5, 6, 6], [7, 7, 7]]
    assert delta == -4
    # the library's host copy agrees
    for ids, tok in [([10, 101305, 100295, 100295, 100295, 100295, 11], 100295),
                     ([1, 7, 7, 7, 7, 2, 3, 7, 7, 7, 7, 4], 7)]:
        p2, d2 = lib.mm_positions(ids, tok, (1, 4, 4))
        p1, d1 = orc.mm_positions(ids, tok, (1, 4, 4))
        assert np.array_equal(p1, p2) and d1 == d2


def test_positions_config4_grid(orc):
    # 5 ids + 36×37 merged image rows + 8 ids: text 0..4, image (5, 5+h, 5+w), text 42..49
    img = 100295
    ids = [1, 2, 3, 4, 5] + [img] * 1332 + list(range(10, 18))
    pos, delta = orc.mm_positions(ids, img, (1, 72, 74))
    assert pos[:5].tolist() == [[i] * 3 for i in range(5)]
    h, w = np.meshgrid(np.arange(36), np.arange(37), indexing="ij")
    assert np.array_equal(pos[5:1337], np.stack([np.full(1332, 5), 5 + h.ravel(), 5 + w.ravel()], 1))
    assert pos[1337:].tolist() == [[i] * 3 for i in range(42, 50)]
    assert delta == 50 - 1345
    p2, d2 = lib.mm_positions(ids, img, (1, 72, 74))
    assert np.array_equal(pos, p2) and d2 == delta


@pytest.mark.parametrize("x", [-88.0, -100.0, -150.0, -300.0])
def test_fast_exp_exponent_wrap(orc, x):
    # ops.go:1099-1112 adds n<<23 to the bits of the 2^f polynomial in uint32
    # arithmetic: below n = -126 the exponent field runs out and the carry
    # lands in the sign bit.  The wrapped value follows from 2^f alone: sign
    # and exponent field from (bits(2^f) + n·2^23) mod 2^32, the mantissa of
    # 2^f (to the polynomial's 4e-6).  A clamp or an ldexp would give a tiny
    # positive number instead.
    import struct
    t = float(np.float32(np.float32(x) * np.float32(1.4426950408889634)))
    n = int(np.rint(t))
    p = float(np.float32(2.0 ** (t - n)))
    bits = (struct.unpack("<I", struct.pack("<f", p))[0] + (n << 23)) % (1 << 32)
    got = orc.fast_exp(x)
    gbits = struct.unpack("<I", struct.pack("<f", np.float32(got)))[0]
    assert gbits >> 23 == bits >> 23  # sign and exponent field
    if (bits >> 23) & 0xFF not in (0, 0xFF):
        want = struct.unpack("<f", struct.pack("<I", bits))[0]
        assert abs(got / want - 1) < 4e-6
    if x <= -100.0 and x > -260.0:
        assert got < 0  # the carry reached the sign bit


@pytest.mark.parametrize("qtype", [1000, 1001, 1002], ids=["q8", "q4", "q6"])
def test_prepared_matvec_equals_matvec(orc, qtype):
    # the timing entry (matrix unpacked once) computes the same plain matvec
    from rapidocrvl_amd import lib

    rng = np.random.default_rng(9)
    q = lib.QMatrix.quantize((rng.standard_normal((700, 96)) * 0.02).astype(np.float32), qtype)
    p = orc.Prepared(qtype, q.scales, q.packed, 96)
    for _ in range(3):
        x = rng.standard_normal(96).astype(np.float32)
        assert np.array_equal(p.matvec(x), orc.matvec(qtype, q.scales, q.packed, x))
    p.close()
