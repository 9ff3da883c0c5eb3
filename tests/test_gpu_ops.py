"""Op-level parity of the HIP kernels against the oracle (through the C ABI)."""
import math

import numpy as np
import pytest

from rapidocrvl_amd import lib

import digit_model as dm

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
SHAPES = [(3072, 1024), (1024, 3072), (2560, 1024), (1024, 2048), (103424, 1024)]


def _qmat(rng, rows, cols, qtype, std=0.02):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    return lib.QMatrix.quantize(w, qtype)


def _close(got, want, rel=2e-5):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert err <= rel * scale, f"max err {err} vs scale {scale}"


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_matvec_decoder_shapes(ctx, orc, rng, qtype, shape):
    q = _qmat(rng, *shape, qtype)
    x = rng.standard_normal(shape[1]).astype(np.float32)
    w = ctx.upload(q)
    got = ctx.matvec(w, x)
    want = orc.matvec(qtype, q.scales, q.packed, x)
    _close(got, want)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (7, 33), (130, 100), (65, 96), (4, 5), (2, 3), (40, 4000)])
def test_matvec_odd_shapes(ctx, orc, rng, qtype, shape):
    q = _qmat(rng, *shape, qtype, std=1.0)
    x = rng.standard_normal(shape[1]).astype(np.float32)
    got = ctx.matvec(ctx.upload(q), x)
    _close(got, orc.matvec(qtype, q.scales, q.packed, x))


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_matvec_closed_form_known_answers(ctx, orc, qtype):
    # internal/backend/vulkan_exec_test.go:1938-2160 inputs, tol 1e-4
    cases = [
        (np.array([[1, 0, 0, 0, 0], [0, 1, 2, 0, 0], [-1, 0, 0, 0.25, 1], [0.5] * 5], np.float32),
         np.array([2, -1, 0.5, 4, -3], np.float32)),
        (np.array([[1] * 5, [1, 0, 0, 0, -1], [0, 2, 0, -1, 0], [-1] * 5], np.float32),
         np.array([1, 2, 3, 4, 5], np.float32)),
        (np.array([[1, 2, 0], [-1, 0, 1]], np.float32), np.array([3, -2, 5], np.float32)),
    ]
    for w, x in cases:
        q = lib.QMatrix.quantize(w, qtype)
        got = ctx.matvec(ctx.upload(q), x)
        assert np.max(np.abs(got - orc.matvec(qtype, q.scales, q.packed, x))) <= 1e-4


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("m", [2, 3, 4, 16])
def test_batched_matvec(ctx, orc, rng, qtype, m):
    q = _qmat(rng, 3072, 1024, qtype)
    x = rng.standard_normal((m, 1024)).astype(np.float32)
    got = ctx.matvec(ctx.upload(q), x)
    for i in range(m):
        _close(got[i], orc.matvec(qtype, q.scales, q.packed, x[i]), rel=5e-5)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_matvec_vectors_per_pass(ctx, orc, rng, qtype, shape):
    # M = 2 and 4 share each weight pass of the GEMV (the LM head included)
    q = _qmat(rng, *shape, qtype)
    w = ctx.upload(q)
    for m in (2, 4):
        x = rng.standard_normal((m, shape[1])).astype(np.float32)
        got = ctx.matvec(w, x)
        for i in range(m):
            _close(got[i], orc.matvec(qtype, q.scales, q.packed, x[i]))


# f32 steps after the exact integer plane sums: the MFMA head combines three
# planes (2 fma) and applies two scales (+2 spare)
F32_STEPS = {Q4: 6 * 2.0 ** -24, Q8: 6 * 2.0 ** -24, Q6: 6 * 2.0 ** -24}


def head_model(qtype, codes, scales, x):
    """What the device greedy head computes, exactly, and its f32 magnitude:
    the MFMA head's whole-vector digit planes, for every code width."""
    return dm.head_scores(codes, scales, x)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_matvec_argmax(ctx, orc, rng, qtype):
    """The greedy head computes codes · digits of x (three byte planes under
    one power-of-two scale for the vector, on the matrix cores for Q4, Q8 and
    Q6; restated in tests/digit_model.py) up to its f32 steps;
    its choice is the exact argmax unless the exact top scores lie within the
    digits' actual deviation plus those f32 steps."""
    q = _qmat(rng, 103424, 1024, qtype)
    w = ctx.upload(q)
    codes = lib.unpack_rows(qtype, q.packed, q.cols)
    for seed in range(3):
        x = np.random.default_rng(seed).standard_normal(1024).astype(np.float32)
        exact, _ = dm.scores(qtype, codes, q.scales, x)
        dig, mag = head_model(qtype, codes, q.scales, x)
        f32b = F32_STEPS[qtype] * mag
        dev = np.abs(dig - exact)  # the digit planes' own deviation, per row
        # about 2^-21 of the largest |x|: 1e-6 of the largest score
        assert dev.max() <= 1e-6 * np.abs(exact).max()
        idx, score = ctx.matvec_argmax(w, x)
        assert abs(score - dig[idx]) <= f32b[idx]
        best = int(np.argmax(exact))
        assert exact[best] - exact[idx] <= dev[best] + dev[idx] + f32b[best] + f32b[idx]
        logits = orc.matvec(qtype, q.scales, q.packed, x)
        assert idx == int(np.argmax(logits)) or exact[best] - exact[idx] <= dev[best] + dev[idx] + f32b[best] + f32b[idx]


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_matvec_argmax_planted_near_tie(ctx, orc, qtype):
    """Rows 100 and 200 differ in one code, at a column whose activation is
    2.2e-5 of the vector's maximum: row 200 wins by ~3e-6, below what a head
    reading x to 2^-14.5 (four nibble planes) or 2^-14 (two byte planes)
    resolves (it would see a tie and take row 100) and far above the head's
    2^-21 resolution and the f32 rounding of these small scores."""
    rows, cols, j, i0 = 4096, 1024, 64, 65
    rng = np.random.default_rng(7)
    wf = (rng.standard_normal((rows, cols)) * 1e-4).astype(np.float32)
    wf[100] = 0.0
    wf[100, i0] = 0.875
    wf[200] = wf[100]
    wf[200, j] = 0.125
    q = lib.QMatrix.quantize(wf, qtype)
    codes = lib.unpack_rows(qtype, q.packed, cols)
    assert q.scales[100] == q.scales[200] and codes[200, j] > 0 and codes[100, j] == 0
    x = rng.uniform(-0.9, 0.9, cols).astype(np.float32)
    x[i0] = 1.0
    x[j] = 2.2e-5
    exact, _ = dm.scores(qtype, codes, q.scales, x)
    assert int(np.argmax(exact)) == 200 and exact[200] - exact[100] > 1e-6
    assert int(np.argmax(orc.matvec(qtype, q.scales, q.packed, x))) == 200
    idx, score = ctx.matvec_argmax(ctx.upload(q), x)
    assert idx == 200
    dig, mag = head_model(qtype, codes[[200]], q.scales[[200]], x)
    assert abs(score - dig[0]) <= F32_STEPS[qtype] * mag[0]


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 6, 16, 17])
def test_lm_head_rows_on_matrix_cores(ctx, orc, qtype, m):
    """M rows of x against the 103424×1024 LM head: up to 16 rows per weight
    pass on the matrix cores.  Each row's scores are what the MFMA greedy head
    computes for that row alone (one power-of-two digit scale per row, exact
    plane sums: tests/digit_model.py) up to the f32 steps, within the f32
    matvec tolerance of the oracle, and each row's best score and row are
    pocr_matvec_argmax's for that row, to the bit.  A 17th row goes through
    the single-vector GEMV."""
    rng = np.random.default_rng(40 + m)
    q = _qmat(rng, 103424, 1024, qtype)
    w = ctx.upload(q)
    codes = lib.unpack_rows(qtype, q.packed, q.cols)
    x = rng.standard_normal((m, 1024)).astype(np.float32)
    x[1] *= np.float32(1e-3)  # rows of different magnitude: each its own digit scale
    got = ctx.matvec(w, x)
    nw = min(m, 16)
    dig, mag = dm.head_scores_rows(codes, q.scales, x[:nw])
    for i in range(m):
        _close(got[i], orc.matvec(qtype, q.scales, q.packed, x[i]))
        if i >= 16:
            continue
        assert np.all(np.abs(got[i] - dig[i]) <= F32_STEPS[qtype] * mag[i]), i
        idx, score = ctx.matvec_argmax(w, x[i])
        assert int(np.argmax(got[i])) == idx, i
        assert got[i][idx] == np.float32(score), i


@pytest.mark.parametrize("m", [2, 4, 16, 17])
def test_lm_head_rows_q6(ctx, orc, m):
    """The Q6 103424×1024 LM head at M rows of x (config 2's Q6 head cells):
    every row's scores against the oracle at the f32 matvec bar, and every
    row's greedy pick (pocr_matvec_argmax: the MFMA head, one vector) is that
    row's best exact score up to the digits' and f32 steps' bounds."""
    rng = np.random.default_rng(70 + m)
    q = _qmat(rng, 103424, 1024, Q6)
    w = ctx.upload(q)
    codes = lib.unpack_rows(Q6, q.packed, q.cols)
    x = rng.standard_normal((m, 1024)).astype(np.float32)
    x[1] *= np.float32(1e-3)
    got = ctx.matvec(w, x)
    for i in range(m):
        _close(got[i], orc.matvec(Q6, q.scales, q.packed, x[i]))
    for i in (0, 1, m - 1):
        exact, _ = dm.scores(Q6, codes, q.scales, x[i])
        dig, mag = head_model(Q6, codes, q.scales, x[i])
        f32b = F32_STEPS[Q6] * mag
        dev = np.abs(dig - exact)
        idx, score = ctx.matvec_argmax(w, x[i])
        assert abs(score - dig[idx]) <= f32b[idx], i
        best = int(np.argmax(exact))
        assert exact[best] - exact[idx] <= dev[best] + dev[idx] + f32b[best] + f32b[idx], i


@pytest.mark.parametrize("cols", [1024, 2048])
@pytest.mark.parametrize("m", [1, 5])
def test_q6_head_image_ragged_rows(ctx, orc, cols, m):
    """Q6 matrices of LM-head size are read through the head image (rows in
    the heads' load order, built at upload).  16,421 rows leave a partial last
    block of 16 and a partial last workgroup of blocks: every row's scores are
    the digit model's up to the f32 steps and within the oracle's f32 bar, and
    every vector's greedy pick is that of the one-vector head, to the bit."""
    rows = 16421
    rng = np.random.default_rng(cols + m)
    q = _qmat(rng, rows, cols, Q6)
    w = ctx.upload(q)
    codes = lib.unpack_rows(Q6, q.packed, q.cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    if m > 1:
        x[1] *= np.float32(1e-3)
    got = ctx.matvec(w, x if m > 1 else x[0])
    got = got.reshape(m, rows)
    dig, mag = dm.head_scores_rows(codes, q.scales, x)
    for i in range(m):
        _close(got[i], orc.matvec(Q6, q.scales, q.packed, x[i]))
        assert np.all(np.abs(got[i] - dig[i]) <= F32_STEPS[Q6] * mag[i]), i
        idx, score = ctx.matvec_argmax(w, x[i])
        assert int(np.argmax(got[i])) == idx, i
        assert got[i][idx] == np.float32(score), i
    # the last rows (the partial block) are scored like every other row
    assert np.all(np.isfinite(got[:, -5:]))


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("m", [3, 5, 16])
def test_lm_head_rows_2048_columns(ctx, orc, qtype, m):
    """The M-row heads at 2,048 columns (the 16-vector tiles and, up to 5
    rows, the packed one): every row within the oracle's f32 bar, each row's
    best score and row those of the single-vector head to the bit, and, where
    the digit model's f32 plane sums are exact (Q4, Q6), the scores it gives."""
    rng = np.random.default_rng(90 + m)
    q = _qmat(rng, 16400, 2048, qtype)
    w = ctx.upload(q)
    x = rng.standard_normal((m, 2048)).astype(np.float32)
    x[1] *= np.float32(1e-3)
    got = ctx.matvec(w, x)
    codes = lib.unpack_rows(qtype, q.packed, q.cols)
    exact_model = qtype != Q8
    if exact_model:
        dig, mag = dm.head_scores_rows(codes, q.scales, x)
    for i in range(m):
        _close(got[i], orc.matvec(qtype, q.scales, q.packed, x[i]))
        if exact_model:
            assert np.all(np.abs(got[i] - dig[i]) <= F32_STEPS[qtype] * mag[i]), i
        idx, score = ctx.matvec_argmax(w, x[i])
        assert int(np.argmax(got[i])) == idx, i
        assert got[i][idx] == np.float32(score), i


def test_q6_head_image_matches_rows(ctx, monkeypatch):
    """The Q6 heads read the same bytes from the upload-time image as from the
    rows (POCR_HEAD_IMAGE=0 uploads without the image): scores and greedy picks
    at M = 1, 4 and 16 agree to the bit, for 1024 and 2048 columns."""
    for cols in (1024, 2048):
        rng = np.random.default_rng(cols)
        q = _qmat(rng, 16400, cols, Q6)
        x = rng.standard_normal((16, cols)).astype(np.float32)
        monkeypatch.setenv("POCR_HEAD_IMAGE", "0")
        w_rows = ctx.upload(q)
        monkeypatch.delenv("POCR_HEAD_IMAGE")
        w_img = ctx.upload(q)
        for m in (1, 4, 16):
            a = ctx.matvec(w_rows, x[:m])
            b = ctx.matvec(w_img, x[:m])
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (cols, m)
        for i in range(2):
            assert ctx.matvec_argmax(w_rows, x[i]) == ctx.matvec_argmax(w_img, x[i]), (cols, i)


def test_argmax_ties_pick_lowest_index(ctx):
    # identical rows give bit-identical scores: ties → lowest index
    w = np.zeros((64, 32), np.float32)
    w[:, 0] = -1
    w[[9, 17, 40], 0] = 1
    x = np.ones(32, np.float32)
    for qtype in (Q8, Q4, Q6):
        idx, _ = ctx.matvec_argmax(ctx.upload(lib.QMatrix.quantize(w, qtype)), x)
        assert idx == 9


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_fused_qkv_and_mrope(ctx, orc, rng, qtype):
    a, b, c = (_qmat(rng, r, 1024, qtype) for r in (2048, 256, 256))
    x = rng.standard_normal(1024).astype(np.float32)
    wa, wb, wc = (ctx.upload(m) for m in (a, b, c))
    oa, ob, oc = ctx.fused_matvec3(wa, wb, wc, x)
    ra = orc.matvec(qtype, a.scales, a.packed, x)
    rb = orc.matvec(qtype, b.scales, b.packed, x)
    rc = orc.matvec(qtype, c.scales, c.packed, x)
    _close(oa, ra), _close(ob, rb), _close(oc, rc)
    freq, axis = orc.rope_init(500000.0, 128)
    cos_t, sin_t = orc.rope_table(freq, axis, 9, 4, 13)
    ma, mb, mc = ctx.fused_matvec3_mrope(wa, wb, wc, x, cos_t, sin_t, 16, 2, 128)
    _close(ma, orc.apply_rope(ra, cos_t, sin_t, 16, 128))
    _close(mb, orc.apply_rope(rb, cos_t, sin_t, 2, 128))
    _close(mc, rc)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_swiglu_gate_up(ctx, orc, rng, qtype):
    g, u = _qmat(rng, 3072, 1024, qtype), _qmat(rng, 3072, 1024, qtype)
    x = rng.standard_normal(1024).astype(np.float32)
    got = ctx.swiglu_gate_up(ctx.upload(g), ctx.upload(u), x)
    gg = orc.matvec(qtype, g.scales, g.packed, x)
    uu = orc.matvec(qtype, u.scales, u.packed, x)
    want = np.array([orc.silu(float(a)) for a in gg], np.float32) * uu
    _close(got, want)


def test_swiglu_fast_exp_wrap(ctx, orc):
    """SiLU is x / (1 + FastExp(-x)) with the reference's FastExp, whose
    exponent add wraps below about -88.7 (ops.go:1099-1112): for a gate of 90
    FastExp(-90) is -9.5e37, so SiLU(90) is about -9.5e-37, not 90. The
    device reproduces that bit for bit. Inputs are exact (integer x, scales
    of 1), so gate and up are exact integers on both sides:
    gate_r = 2·g_r, up = 2·3."""
    gs = [3, 40, 43, 44, 45, 50, 60, 100, 127, -20, -44, -45, -50, -127]
    cols = 64
    wg = np.zeros((len(gs), cols), np.float32)
    wu = np.zeros((len(gs), cols), np.float32)
    wg[:, 0] = wu[:, 0] = 127.0
    wg[:, 1] = gs
    wu[:, 1] = 3.0
    x = np.zeros(cols, np.float32)
    x[1] = 2.0
    g, u = lib.QMatrix.quantize(wg, Q8), lib.QMatrix.quantize(wu, Q8)
    assert np.all(g.scales == 1.0) and np.all(u.scales == 1.0)
    got = ctx.swiglu_gate_up(ctx.upload(g), ctx.upload(u), x)
    gate = np.float32(2) * np.array(gs, np.float32)
    want = np.array([orc.silu(float(a)) for a in gate], np.float32) * np.float32(6)
    assert np.array_equal(got, want)
    # what the wrap gives: gates 90, 100, 120 come out as tiny negatives
    # (FastExp(-g) negative and huge), gates -90 and -100 as the gate itself
    # (FastExp(g) wraps to about 0), while 200 and 254 land back in range;
    # below |g| = 88 it is the textbook SiLU
    by_gate = dict(zip(gate.tolist(), got.tolist()))
    for gv in (90.0, 100.0, 120.0):
        assert -1e-20 < by_gate[gv] <= 0.0
    for gv in (-90.0, -100.0):
        assert by_gate[gv] == gv * 6
    silu64 = gate.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64))) * 6
    small = np.abs(gate) < 88
    assert np.all(np.abs(got[small] - silu64[small]) <= 1e-5 * np.maximum(np.abs(silu64[small]), 1e-30))


def test_attention_score_gap_beyond_fast_exp_range(ctx, orc):
    """A score gap above 88 is where the reference's one-pass softmax takes
    FastExp into its wrap: with row 0 at score 0 and rows 1..63 at -100, each
    far row's weight is FastExp(-100) = -4.3e33, the sum is negative and huge,
    and the normalised weights become ≈ 0 for row 0 and 1/63 for each far row:
    the reference returns the mean of the far rows' values. The split decode
    attention cannot form those weights (it rescales per-split sums by
    exp(m_split - m), which the reference never computes), so it clamps
    FastExp's input at -87 and returns the softmax itself: row 0's values.
    Both behaviours are stated here; the greedy streams never reach such
    gaps (scores of |q·k|/√128 ≤ 88 hold for every test model)."""
    L, heads, kvh, dim = 64, 16, 2, 128
    q = np.zeros((heads, dim), np.float32)
    q[:, 0] = 40.0
    kc = np.zeros((L, kvh, dim), np.float32)
    # score = 40·k0 / sqrt(128): -100 at k0 = -100·sqrt(128)/40
    kc[1:, :, 0] = np.float32(-100.0 * math.sqrt(128.0) / 40.0)
    rng = np.random.default_rng(5)
    vc = rng.standard_normal((L, kvh, dim)).astype(np.float32)
    got = ctx.text_attention(q.ravel(), kc.ravel(), vc.ravel(), L, heads, kvh, dim).reshape(heads, dim)
    ref = orc.cache_attention(q.ravel(), kc.ravel(), vc.ravel(), L, heads, kvh, dim).reshape(heads, dim)
    grp = np.arange(heads) // (heads // kvh)
    assert np.max(np.abs(got - vc[0, grp])) < 1e-6
    assert np.max(np.abs(ref - vc[1:, :, :].mean(axis=0)[grp])) < 1e-4
    assert np.max(np.abs(ref - vc[0, grp])) > 0.1
    # up to a gap of 87 both sides are the softmax
    kc[1:, :, 0] = np.float32(-80.0 * math.sqrt(128.0) / 40.0)
    got = ctx.text_attention(q.ravel(), kc.ravel(), vc.ravel(), L, heads, kvh, dim)
    ref = orc.cache_attention(q.ravel(), kc.ravel(), vc.ravel(), L, heads, kvh, dim)
    assert np.max(np.abs(got - ref)) < 2e-5


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("in_place", [True, False])
def test_matvec_add_rmsnorm(ctx, orc, rng, qtype, in_place):
    q = _qmat(rng, 1024, 3072, qtype)
    x = rng.standard_normal(3072).astype(np.float32)
    res = rng.standard_normal(1024).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    out, res_after = ctx.matvec_add_rmsnorm(ctx.upload(q), x, res, nw, 1e-5, in_place)
    mv = orc.matvec(qtype, q.scales, q.packed, x)
    want_out, want_res = orc.add_rmsnorm(res, mv, nw, 1e-5)
    _close(out, want_out)
    _close(res_after, want_res if in_place else res)


def test_rmsnorm_and_rope_known_answers(ctx, orc):
    x = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9], np.float32)
    w = np.array([1, 0.5, 1.5, 2, 0.25, 1.25, 0.75, 1, 1.1], np.float32)
    want = orc.rmsnorm(x, w, 1e-6)
    assert np.max(np.abs(ctx.rmsnorm(x, w, 1e-6) - want)) <= 2e-6 * np.max(np.abs(want))
    q, k = ctx.mrope_pair(np.array([1, 2, 3, 4], np.float32), np.array([1, 2, 3, 4], np.float32),
                          [0, 0.5], [1, 0.5], 1, 1, 4)
    assert list(k) == [-3, -1, 1, 3] and list(q) == [-3, -1, 1, 3]


# lengths cover both rows-per-wave kernels (≤ 2048 rows: 8, above: 16)
@pytest.mark.parametrize("L", [1, 2, 6, 7, 33, 300, 1024, 2049, 4096, 8193])
def test_text_attention_head128(ctx, orc, rng, L):
    q = rng.standard_normal(16 * 128).astype(np.float32)
    kc = rng.standard_normal(L * 256).astype(np.float32)
    vc = rng.standard_normal(L * 256).astype(np.float32)
    got = ctx.text_attention(q, kc, vc, L, 16, 2, 128)
    want = orc.cache_attention(q, kc, vc, L, 16, 2, 128)
    assert np.max(np.abs(got - want)) < 2e-5
    if L == 1:
        assert np.array_equal(got.reshape(16, 128), vc.reshape(2, 128)[np.arange(16) // 8])


def test_text_attention_small_head_known_answer(ctx):
    # scratch_test.go:236-248 weighted value sum through softmax weights .25/.75
    k = np.zeros((2, 8), np.float32)
    k[1, 4] = 2 * math.log(3)
    v = np.array([[1, 2, 3, 4, 10, 20, 30, 40], [5, 6, 7, 8, 50, 60, 70, 80]], np.float32)
    q = np.zeros(8, np.float32)
    q[4] = 1
    out = ctx.text_attention(q, k, v, 2, 2, 2, 4)
    assert np.max(np.abs(out[4:] - np.array([40, 50, 60, 70]))) < 2e-5
