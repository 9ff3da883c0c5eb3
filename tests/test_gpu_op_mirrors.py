"""Op-level mirrors of the fused sublayer functions the reference's Vulkan
backend exposes (internal/backend/vulkan_exec_stub.go) against the oracle's
CPU composition of the same steps, at the decoder's shapes: SwiGLU-down
(+AddRMSNorm, in place and OutOnly), attention-out (+AddRMSNorm), the
first-token value-out branch, AddRMSNorm and single-tensor MRoPE."""
import numpy as np
import pytest

from rapidocrvl_amd import lib

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
QT = [Q8, Q4, Q6]
QID = ["q8", "q4", "q6"]
H, F, HEADS, KVH, HD = 1024, 3072, 16, 2, 128
EPS = 1e-5


def _qmat(rng, rows, cols, qtype, std=0.02):
    return lib.QMatrix.quantize((rng.standard_normal((rows, cols)) * std).astype(np.float32), qtype)


def _close(got, want, rel=2e-5):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert err <= rel * scale, f"max err {err} vs scale {scale}"


def _mv(orc, q, x):
    return orc.matvec(q.qtype, q.scales, q.packed, x)


def _swiglu(orc, g, u, x):
    a, b = _mv(orc, g, x), _mv(orc, u, x)
    return np.array([orc.silu(float(v)) for v in a], np.float32) * b


@pytest.mark.parametrize("qtype", QT, ids=QID)
def test_swiglu_down(ctx, orc, rng, qtype):
    g, u, d = _qmat(rng, F, H, qtype), _qmat(rng, F, H, qtype), _qmat(rng, H, F, qtype)
    x = rng.standard_normal(H).astype(np.float32)
    got = ctx.swiglu_down(ctx.upload(g), ctx.upload(u), ctx.upload(d), x)
    _close(got, _mv(orc, d, _swiglu(orc, g, u, x)))


@pytest.mark.parametrize("in_place", [True, False], ids=["in-place", "out-only"])
@pytest.mark.parametrize("qtype", QT, ids=QID)
def test_swiglu_down_add_rmsnorm(ctx, orc, rng, qtype, in_place):
    g, u, d = _qmat(rng, F, H, qtype), _qmat(rng, F, H, qtype), _qmat(rng, H, F, qtype)
    x = rng.standard_normal(H).astype(np.float32)
    res = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    out, res_after = ctx.swiglu_down_add_rmsnorm(ctx.upload(g), ctx.upload(u), ctx.upload(d), x, res, nw, EPS,
                                                 in_place)
    want, want_res = orc.add_rmsnorm(res, _mv(orc, d, _swiglu(orc, g, u, x)), nw, EPS)
    _close(out, want)
    if in_place:
        _close(res_after, want_res)
    else:
        assert np.array_equal(res_after, res)


def _attn_inputs(rng, L):
    q = rng.standard_normal(HEADS * HD).astype(np.float32)
    kc = rng.standard_normal(L * KVH * HD).astype(np.float32)
    vc = rng.standard_normal(L * KVH * HD).astype(np.float32)
    return q, kc, vc


@pytest.mark.parametrize("L", [1, 7, 1345])
@pytest.mark.parametrize("qtype", QT, ids=QID)
def test_text_attention_out(ctx, orc, rng, qtype, L):
    wo = _qmat(rng, H, HEADS * HD, qtype)
    q, kc, vc = _attn_inputs(rng, L)
    got = ctx.text_attention_out(q, kc, vc, L, HEADS, KVH, HD, ctx.upload(wo))
    _close(got, _mv(orc, wo, orc.cache_attention(q, kc, vc, L, HEADS, KVH, HD)))


@pytest.mark.parametrize("in_place", [True, False], ids=["in-place", "out-only"])
@pytest.mark.parametrize("qtype", QT, ids=QID)
def test_text_attention_out_add_rmsnorm(ctx, orc, rng, qtype, in_place):
    L = 300
    wo = _qmat(rng, H, HEADS * HD, qtype)
    q, kc, vc = _attn_inputs(rng, L)
    res = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    out, res_after = ctx.text_attention_out_add_rmsnorm(q, kc, vc, L, HEADS, KVH, HD, ctx.upload(wo), res, nw, EPS,
                                                        in_place)
    attn = orc.cache_attention(q, kc, vc, L, HEADS, KVH, HD)
    want, want_res = orc.add_rmsnorm(res, _mv(orc, wo, attn), nw, EPS)
    _close(out, want)
    if in_place:
        _close(res_after, want_res)
    else:
        assert np.array_equal(res_after, res)


@pytest.mark.parametrize("in_place", [True, False], ids=["in-place", "out-only"])
@pytest.mark.parametrize("qtype", QT, ids=QID)
def test_first_token_value_out_add_rmsnorm(ctx, orc, rng, qtype, in_place):
    wo = _qmat(rng, H, HEADS * HD, qtype)
    kc = rng.standard_normal(KVH * HD).astype(np.float32)
    vc = rng.standard_normal(KVH * HD).astype(np.float32)
    res = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    # expandValueHeads (model.go:4603-4621): q head h takes kv head h / group
    head_out = np.concatenate([vc[(h // (HEADS // KVH)) * HD:(h // (HEADS // KVH) + 1) * HD] for h in range(HEADS)])
    # the device attention over one row returns that V row exactly
    assert np.array_equal(ctx.text_attention(rng.standard_normal(HEADS * HD), kc, vc, 1, HEADS, KVH, HD), head_out)
    out, res_after = ctx.first_token_value_out_add_rmsnorm(kc, vc, HEADS, KVH, HD, ctx.upload(wo), res, nw, EPS,
                                                           in_place)
    want, want_res = orc.add_rmsnorm(res, _mv(orc, wo, head_out), nw, EPS)
    _close(out, want)
    if in_place:
        _close(res_after, want_res)
    else:
        assert np.array_equal(res_after, res)


@pytest.mark.parametrize("n", [1, 5, 1024, 3000])
def test_add_rmsnorm(ctx, orc, rng, n):
    dst = rng.standard_normal(n).astype(np.float32)
    add = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    out, dst_after = ctx.add_rmsnorm(dst, add, w, EPS, True)
    want, want_dst = orc.add_rmsnorm(dst, add, w, EPS)
    assert np.array_equal(dst_after, want_dst)  # one f32 add per element, as the reference
    _close(out, want, 1e-6)
    out2, dst2 = ctx.add_rmsnorm(dst, add, w, EPS, False)
    assert np.array_equal(dst2, dst)
    _close(out2, orc.add_rmsnorm_out_only(dst, add, w, EPS), 1e-6)


@pytest.mark.parametrize("heads,dim", [(16, 128), (2, 128), (3, 64)])
def test_mrope(ctx, orc, rng, heads, dim):
    freq, axis = orc.rope_init(500000.0, dim, [16, 24, 24] if dim == 128 else None)
    cos_t, sin_t = orc.rope_table(freq, axis, 5, 9, 13)
    x = rng.standard_normal(heads * dim).astype(np.float32)
    # the same two products and one add/sub per element, uncontracted: bit-exact
    assert np.array_equal(ctx.mrope(x, cos_t, sin_t, heads, dim), orc.apply_rope(x, cos_t, sin_t, heads, dim))


def test_mirror_argument_errors(ctx, rng):
    g, u = ctx.upload(_qmat(rng, 64, 32, Q4)), ctx.upload(_qmat(rng, 64, 32, Q4))
    bad_down = ctx.upload(_qmat(rng, 32, 48, Q4))  # takes 48 columns, SwiGLU gives 64
    with pytest.raises(lib.PocrError) as e:
        ctx.swiglu_down(g, u, bad_down, np.zeros(32, np.float32))
    assert e.value.code == lib.POCR_ERR_ARG
    wo = ctx.upload(_qmat(rng, 32, 100, Q4))  # not heads·dim columns
    with pytest.raises(lib.PocrError) as e:
        ctx.text_attention_out(np.zeros(256, np.float32), np.zeros(256, np.float32), np.zeros(256, np.float32), 1,
                               2, 1, 128, wo)
    assert e.value.code == lib.POCR_ERR_ARG
    with pytest.raises(lib.PocrError) as e:
        ctx.mrope(np.zeros(10, np.float32), np.zeros(2, np.float32), np.zeros(2, np.float32), 2, 5)
    assert e.value.code == lib.POCR_ERR_ARG
