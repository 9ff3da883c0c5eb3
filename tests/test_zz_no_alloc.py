"""pocr_text_attention_noalloc: decode attention over caller-owned device
buffers with its split records in a fixed device array (no allocation).
Checked against pocr_text_attention on the same inputs, twice in a row (the
second call smaller: the array keeps the first call's records), and its size
limit."""
import ctypes as C

import numpy as np
import pytest

from rapidocrvl_amd import lib

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class _Hip:
    """Device buffers for the test (the entry under test allocates nothing),
    from the HIP runtime the library itself links: symbols resolved through
    its handle, so a second runtime in the process (torch's) is never used."""

    def __init__(self):
        self.rt = lib.load()
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.bufs = []

    def upload(self, a):
        a = np.ascontiguousarray(a, np.float32)
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), C.c_size_t(max(a.nbytes, 4))) == 0
        self.bufs.append(p)
        assert self.rt.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), H2D) == 0
        return p.value

    def empty(self, n):
        return self.upload(np.full(n, np.nan, np.float32))

    def download(self, ptr, n):
        out = np.zeros(n, np.float32)
        assert self.rt.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(out.nbytes), D2H) == 0
        return out

    def close(self):
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(16, 2, 128), (4, 2, 64)], ids=["gqa8-d128", "d64"])
def test_noalloc_attention_matches_pocr_text_attention(ctx, heads, kv_heads, head_dim):
    hip = _Hip()
    try:
        rng = np.random.default_rng(17)
        lens = (1500, 300) if head_dim == 128 else (900, 40)  # the second call smaller
        for L in lens:
            q = rng.standard_normal(heads * head_dim).astype(np.float32)
            kc = rng.standard_normal(L * kv_heads * head_dim).astype(np.float32)
            vc = rng.standard_normal(L * kv_heads * head_dim).astype(np.float32)
            want = ctx.text_attention(q, kc, vc, L, heads, kv_heads, head_dim)
            out = hip.empty(heads * head_dim)
            ctx.text_attention_noalloc(hip.upload(q), hip.upload(kc), hip.upload(vc), L, heads, kv_heads, head_dim, out)
            got = hip.download(out, heads * head_dim)
            assert np.array_equal(got, want), (L, float(np.max(np.abs(got - want))))
    finally:
        hip.close()


def test_noalloc_attention_rejects_more_records_than_the_array(ctx):
    hip = _Hip()
    try:
        L = 16385  # 2 kv heads x 257 splits of 64 rows > 512 records
        kc = hip.empty(1)  # never read: the size check comes first
        out = hip.empty(1)
        with pytest.raises(lib.PocrError) as e:
            ctx.text_attention_noalloc(kc, kc, kc, L, 16, 2, 128, out)
        assert e.value.code == lib.POCR_ERR_ARG and "512" in str(e.value)
        # the largest accepted size still runs
        L = 16384
        rng = np.random.default_rng(3)
        q = rng.standard_normal(16 * 128).astype(np.float32)
        kv = rng.standard_normal(L * 256).astype(np.float32)
        want = ctx.text_attention(q, kv, kv, L, 16, 2, 128)
        o = hip.empty(16 * 128)
        kd = hip.upload(kv)
        ctx.text_attention_noalloc(hip.upload(q), kd, kd, L, 16, 2, 128, o)
        assert np.array_equal(hip.download(o, 16 * 128), want)
    finally:
        hip.close()
