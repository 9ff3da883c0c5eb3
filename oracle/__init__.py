"""ctypes view of the CPU oracle (oracle/pocr_oracle.c).

Test infrastructure only: tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py use it, to check results and to time the CPU
baseline.  The HIP product path never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# POCR_ORACLE_LIB names another build of the same sources (the sanitizer
# build of tests/sanitize.py)
LIB_PATH = os.environ.get("POCR_ORACLE_LIB") or os.path.join(HERE, "_build", "libpocr_oracle.so")

Q8, Q4, Q6 = 1000, 1001, 1002
TIE_HALF_AWAY, TIE_AMD64 = 0, 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_row_bytes.restype = C.c_size_t
        L.orc_row_bytes.argtypes = [C.c_int, C.c_int]
        L.orc_quantize_row.restype = C.c_float
        L.orc_quantize_row.argtypes = [C.c_int, C.c_int, _f32p, C.c_int, C.c_void_p]
        L.orc_unpack_row.argtypes = [C.c_int, C.c_void_p, C.c_int, _i8p]
        L.orc_round_to_int.argtypes = [C.c_float]
        L.orc_matvec.argtypes = [C.c_void_p, _f32p, _f32p]
        L.orc_matvec_vnni.argtypes = [C.c_void_p, _f32p, _f32p]
        L.orc_quantize_x_vnni.restype = C.c_float
        L.orc_vnni_core.restype = C.c_int32
        L.orc_vnni_core.argtypes = [_i8p, _u8p, C.c_int]
        L.orc_finalize_vnni.argtypes = [_i32p, _i32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_quantize_x_vnni.argtypes = [_f32p, C.c_int, _u8p]
        for fn in ("orc_fast_exp", "orc_fast_rsqrt", "orc_silu"):
            getattr(L, fn).restype = C.c_float
            getattr(L, fn).argtypes = [C.c_float]
        L.orc_softmax.argtypes = [_f32p, C.c_int]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_add_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_add_rmsnorm_out_only.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_argmax.argtypes = [_f32p, C.c_int]
        L.orc_rope_init.argtypes = [C.c_double, C.c_int, C.c_void_p, C.c_int, _f64p, _u8p]
        L.orc_rope_table.argtypes = [_f64p, _u8p, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.orc_apply_rope.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.orc_cache_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_mm_positions.argtypes = [_i32p, C.c_int, C.c_int, _i32p, C.c_int, _i32p, C.POINTER(C.c_int)]
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_create.argtypes = [C.c_int] * 7 + [C.c_float, C.c_double]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_set_matrix.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_void_p, C.c_void_p]
        L.orc_model_set_norm.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        L.orc_model_set_embed.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_model_set_quirk.argtypes = [C.c_void_p, C.c_int]
        L.orc_model_set_vnni.argtypes = [C.c_void_p, C.c_int]
        L.orc_seq_create.restype = C.c_void_p
        L.orc_seq_create.argtypes = [C.c_void_p, C.c_int]
        L.orc_seq_free.argtypes = [C.c_void_p]
        L.orc_seq_reset.argtypes = [C.c_void_p]
        L.orc_seq_len.argtypes = [C.c_void_p]
        L.orc_seq_k.restype = C.POINTER(C.c_float)
        L.orc_seq_k.argtypes = [C.c_void_p, C.c_int]
        L.orc_seq_v.restype = C.POINTER(C.c_float)
        L.orc_seq_v.argtypes = [C.c_void_p, C.c_int]
        L.orc_seq_load.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p, C.c_int]
        L.orc_step.argtypes = [C.c_void_p, C.c_void_p, _f32p, _i32p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_generate.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_void_p, C.c_int, C.c_int, _i32p, C.c_int,
                                   C.c_int, _i32p, C.c_int, _i32p]
        L.orc_generate_sampled.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_void_p, C.c_int, C.c_int, _i32p,
                                           C.c_int, C.c_int, _i32p, C.c_int, C.c_double, C.c_int, C.c_uint64,
                                           _i32p]
        L.orc_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_gelu_tanh.restype = C.c_float
        L.orc_gelu_tanh.argtypes = [C.c_float]
        L.orc_project_image.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_void_p, _f32p,
                                        C.c_void_p, _f32p, C.c_float, _f32p]
        L.orc_rng_float64.restype = C.c_double
        L.orc_rng_float64.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_topk.argtypes = [_f32p, C.c_int, C.c_int, _i32p, _f32p]
        L.orc_sample_candidates.restype = C.c_int32
        L.orc_sample_candidates.argtypes = [_i32p, _f32p, C.c_int, C.c_double, C.POINTER(C.c_uint64)]
        L.orc_cumsum.restype = C.c_float
        L.orc_cumsum.argtypes = [_f32p, _f32p, C.c_int]
        L.orc_pick_cumulative.argtypes = [_f32p, C.c_int, C.c_float]
        L.orc_sample_full.restype = C.c_int32
        L.orc_sample_full.argtypes = [_f32p, C.c_int, C.c_double, C.POINTER(C.c_uint64)]
        L.orc_prepare.restype = C.c_void_p
        L.orc_prepare.argtypes = [C.c_void_p]
        L.orc_prepared_matvec.argtypes = [C.c_void_p, _f32p, _f32p]
        L.orc_prepared_free.argtypes = [C.c_void_p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def layernorm(x, w, b, eps=1e-5):
    """LayerNorm (ops.go:1060-1097), scalar-path order."""
    x = _f32(x)
    out = np.zeros_like(x)
    lib().orc_layernorm(out, x, _f32(w), _f32(b), x.size, eps)
    return out


def gelu_tanh(x):
    """GELUTanh (ops.go:1140-1164) elementwise."""
    return np.array([lib().orc_gelu_tanh(float(v)) for v in np.ravel(_f32(x))], np.float32).reshape(np.shape(x))


def project_image(x, grid, norm_w, norm_b, q1, b1, q2, b2, eps=1e-5):
    """projectImageRows (vision.go:1066-1108) with Q8 matrices q = (scales, packed)."""
    x = _f32(x)
    t, h, w = grid
    vd = _f32(norm_w).size
    K = 4 * vd
    s1, d1 = _f32(q1[0]), np.ascontiguousarray(q1[1], np.uint8)
    s2, d2 = _f32(q2[0]), np.ascontiguousarray(q2[1], np.uint8)
    m1 = _QMat(Q8, s1.size, K, s1.ctypes.data, d1.ctypes.data)
    m2 = _QMat(Q8, s2.size, K, s2.ctypes.data, d2.ctypes.data)
    rows = t * (h // 2) * (w // 2)
    out = np.zeros((max(rows, 1), s2.size), np.float32)
    n = lib().orc_project_image(x, t, h, w, vd, _f32(norm_w), _f32(norm_b), C.byref(m1), _f32(b1), C.byref(m2),
                                _f32(b2), eps, out)
    return out[:n]


class Rng:
    """fastRNG (model.go:1829-1840): SplitMix64 state, Float64 draws."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed & ((1 << 64) - 1))

    def float64(self) -> float:
        return float(lib().orc_rng_float64(C.byref(self.state)))


def topk(scores, k):
    """topKSelectWithWork (topk.go:322-345): ids and scores of the min(k, n)
    best, score descending, equal scores by lower index."""
    scores = _f32(scores)
    ids = np.zeros(max(k, 1), np.int32)
    sc = np.zeros(max(k, 1), np.float32)
    n = lib().orc_topk(scores, scores.size, k, ids, sc)
    return ids[:n], sc[:n]


def sample_candidates(ids, scores, temperature, rng: Rng) -> int:
    """sampleCandidateScoresScratch (model.go:1950-1990) on sorted candidates."""
    ids = np.ascontiguousarray(ids, np.int32)
    return int(lib().orc_sample_candidates(ids, _f32(scores), ids.size, temperature, C.byref(rng.state)))


def cumsum(x):
    """CumulativeSum (cumsum.go:9-58): (prefix array, running block total)."""
    x = _f32(x)
    out = np.zeros_like(x)
    tot = lib().orc_cumsum(out, x, x.size)
    return out, np.float32(tot)


def pick_cumulative(cdf, pick) -> int:
    """pickCumulativeFloat32 (model.go:2326-2340)."""
    cdf = _f32(cdf)
    return int(lib().orc_pick_cumulative(cdf, cdf.size, float(np.float32(pick))))


def sample_full(logits, temperature, rng: Rng) -> int:
    """sampleFullLogitsScratch (model.go:2215-2307): one draw over every logit."""
    logits = _f32(logits)
    return int(lib().orc_sample_full(logits, logits.size, float(temperature), C.byref(rng.state)))


def row_bytes(qtype: int, cols: int) -> int:
    return int(lib().orc_row_bytes(qtype, cols))


def quantize_row(qtype: int, w, tie: int = TIE_HALF_AWAY):
    w = _f32(w)
    out = np.zeros(row_bytes(qtype, w.size), np.uint8)
    s = lib().orc_quantize_row(qtype, tie, w, w.size, out.ctypes.data)
    return np.float32(s), out


def quantize_matrix(qtype: int, w, tie: int = TIE_HALF_AWAY):
    """Encode a [rows, cols] f32 matrix → (scales f32[rows], data u8[rows, row_bytes])."""
    w = _f32(w)
    rows, cols = w.shape
    rb = row_bytes(qtype, cols)
    data = np.zeros((rows, rb), np.uint8)
    scales = np.zeros(rows, np.float32)
    L = lib()
    for r in range(rows):
        scales[r] = L.orc_quantize_row(qtype, tie, w[r], cols, data[r].ctypes.data)
    return scales, data


def unpack_row(qtype: int, row, cols: int):
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(cols, np.int8)
    lib().orc_unpack_row(qtype, row.ctypes.data, cols, out)
    return out


def unpack_matrix(qtype: int, data, cols: int):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    return np.stack([unpack_row(qtype, data[r], cols) for r in range(data.shape[0])])


def round_to_int(x: float) -> int:
    return int(lib().orc_round_to_int(x))


class _QMat(C.Structure):
    _fields_ = [("qtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int),
                ("scale", C.c_void_p), ("data", C.c_void_p)]


def matvec(qtype, scales, data, x, cols=None, vnni=False):
    scales = _f32(scales)
    data = np.ascontiguousarray(data, dtype=np.uint8)
    x = _f32(x)
    rows = scales.size
    cols = x.size if cols is None else cols
    q = _QMat(qtype, rows, cols, scales.ctypes.data, data.ctypes.data)
    out = np.zeros(rows, np.float32)
    (lib().orc_matvec_vnni if vnni else lib().orc_matvec)(C.byref(q), x, out)
    return out


class Prepared:
    """A matrix unpacked once for repeated plain matvecs (timing the CPU path
    the way the model runs it, without the per-call unpack of matvec)."""

    def __init__(self, qtype, scales, data, cols):
        self._scales = _f32(scales)
        self._data = np.ascontiguousarray(data, dtype=np.uint8)
        self.rows = self._scales.size
        q = _QMat(qtype, self.rows, cols, self._scales.ctypes.data, self._data.ctypes.data)
        self.h = lib().orc_prepare(C.byref(q))
        if not self.h:
            raise MemoryError("orc_prepare")

    def matvec(self, x, out=None):
        out = np.zeros(self.rows, np.float32) if out is None else out
        lib().orc_prepared_matvec(self.h, _f32(x), out)
        return out

    def close(self):
        if self.h:
            lib().orc_prepared_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


def quantize_x_vnni(x):
    x = _f32(x)
    xq = np.zeros(x.size, np.uint8)
    s = lib().orc_quantize_x_vnni(x, x.size, xq)
    return np.float32(s), xq


def vnni_core(a, xq) -> int:
    a = np.ascontiguousarray(a, dtype=np.int8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    return int(lib().orc_vnni_core(a, xq, min(a.size, xq.size)))


def finalize_vnni(dots, rowsum, scale, scale_x):
    dots = np.ascontiguousarray(dots, dtype=np.int32)
    rowsum = np.ascontiguousarray(rowsum, dtype=np.int32)
    scale = _f32(scale)
    out = np.zeros(dots.size, np.float32)
    lib().orc_finalize_vnni(dots, rowsum, scale, out, dots.size, np.float32(scale_x))
    return out


def fast_exp(x: float) -> np.float32:
    return np.float32(lib().orc_fast_exp(x))


def fast_rsqrt(x: float) -> np.float32:
    return np.float32(lib().orc_fast_rsqrt(x))


def silu(x: float) -> np.float32:
    return np.float32(lib().orc_silu(x))


def softmax(x):
    x = _f32(x).copy()
    lib().orc_softmax(x, x.size)
    return x


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(out, x, w, x.size, eps)
    return out


def add_rmsnorm(dst, add, w, eps):
    """Returns (out, dst_after) — the in-place AddRMSNorm."""
    dst = _f32(dst).copy()
    out = np.zeros_like(dst)
    lib().orc_add_rmsnorm(out, dst, _f32(add), _f32(w), dst.size, eps)
    return out, dst


def add_rmsnorm_out_only(dst, add, w, eps):
    dst = _f32(dst)
    out = np.zeros_like(dst)
    lib().orc_add_rmsnorm_out_only(out, dst, _f32(add), _f32(w), dst.size, eps)
    return out


def argmax(x) -> int:
    x = _f32(x)
    return int(lib().orc_argmax(x, x.size))


def rope_init(theta: float, head_dim: int, sections=None):
    half = head_dim // 2
    freq = np.zeros(half, np.float64)
    axis = np.zeros(half, np.uint8)
    if sections is None:
        lib().orc_rope_init(theta, head_dim, None, 0, freq, axis)
    else:
        sec = np.ascontiguousarray(sections, dtype=np.int32)
        lib().orc_rope_init(theta, head_dim, sec.ctypes.data, sec.size, freq, axis)
    return freq, axis


def rope_table(freq, axis, t, h, w):
    half = freq.size
    c = np.zeros(half, np.float32)
    s = np.zeros(half, np.float32)
    lib().orc_rope_table(freq, axis, half, t, h, w, c, s)
    return c, s


def apply_rope(x, cos_t, sin_t, heads, dim):
    x = _f32(x).copy()
    lib().orc_apply_rope(x, _f32(cos_t), _f32(sin_t), heads, dim)
    return x


def cache_attention(q, kcache, vcache, length, heads, kv_heads, dim):
    out = np.zeros(heads * dim, np.float32)
    lib().orc_cache_attention(out, _f32(q), _f32(kcache), _f32(vcache), length, heads, kv_heads, dim)
    return out


def mm_positions(ids, image_token_id, grid, merge=2):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    pos = np.zeros((ids.size, 3), np.int32)
    delta = C.c_int(0)
    n = lib().orc_mm_positions(ids, ids.size, image_token_id, np.asarray(grid, np.int32), merge, pos,
                               C.byref(delta))
    if n < 0:
        raise ValueError("positions overflow")
    return pos[:n], int(delta.value)


def set_threads(n: int):
    lib().orc_set_threads(int(n))


class Model:
    """Oracle decoder; weights are borrowed numpy arrays kept alive here."""

    WHICH = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6}

    def __init__(self, cfg):
        self.cfg = cfg
        self._keep = []
        self.h = lib().orc_model_create(cfg.hidden, cfg.inter, cfg.layers, cfg.heads, cfg.kv_heads,
                                        cfg.head_dim, cfg.vocab, cfg.eps, cfg.rope_theta)
        if not self.h:
            raise ValueError("bad config")

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_matrix(self, layer, which, qtype, scales, data, cols):
        scales = _f32(scales)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        self._keep += [scales, data]
        w = 7 if which == "lm_head" else self.WHICH[which]
        rc = lib().orc_model_set_matrix(self.h, layer, w, qtype, scales.size, cols, scales.ctypes.data,
                                        data.ctypes.data)
        assert rc == 0

    def set_norm(self, layer, which, w):
        w = _f32(w)
        self._keep.append(w)
        lib().orc_model_set_norm(self.h, layer, 0 if which == "ln1" else 1, w.ctypes.data)

    def set_embed(self, e):
        e = _f32(e)
        self._keep.append(e)
        lib().orc_model_set_embed(self.h, e.ctypes.data)

    def set_quirk(self, on):
        lib().orc_model_set_quirk(self.h, int(on))

    def set_vnni(self, on):
        lib().orc_model_set_vnni(self.h, int(on))

    def load_weights(self, weights):
        """weights: dict produced by tests/golden synth (see synth.py)."""
        cfg = self.cfg
        for li, lw in enumerate(weights["layers"]):
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                qt, sc, data, cols = lw[name]
                self.set_matrix(li, name, qt, sc, data, cols)
            self.set_norm(li, "ln1", lw["ln1"])
            self.set_norm(li, "ln2", lw["ln2"])
        qt, sc, data, cols = weights["lm_head"]
        self.set_matrix(-1, "lm_head", qt, sc, data, cols)
        self.set_norm(-1, "final", weights["final_norm"])
        self.set_embed(weights["embed"])

    def seq(self, capacity):
        return Seq(self, capacity)

    def generate(self, ids, max_new, eos=(2,), image_embeds=None, image_token_id=-1, grid=(1, 1, 1), merge=2,
                 temperature=0.0, top_k=0, seed=0):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros(max_new, np.int32)
        eos = np.ascontiguousarray(list(eos) if eos else [-(1 << 30)], dtype=np.int32)
        if image_embeds is not None:
            img = _f32(image_embeds)
            n_img = img.shape[0]
            ptr = img.ctypes.data
        else:
            img, n_img, ptr = None, 0, None
        n = lib().orc_generate_sampled(self.h, ids, ids.size, ptr, n_img, image_token_id,
                                       np.asarray(grid, np.int32), merge, max_new, eos, eos.size,
                                       float(temperature), int(top_k), seed & ((1 << 64) - 1), out)
        if n < 0:
            raise RuntimeError(f"orc_generate failed: {n}")
        return out[:n]


class Seq:
    def __init__(self, model: Model, capacity: int):
        self.m = model
        self.h = lib().orc_seq_create(model.h, capacity)
        self.capacity = capacity

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_seq_free(self.h)
            self.h = None

    def __len__(self):
        return int(lib().orc_seq_len(self.h))

    def load(self, layer, k, v, length):
        assert lib().orc_seq_load(self.h, layer, _f32(k), _f32(v), length) == 0

    def kv(self, layer):
        n = len(self) * self.m.cfg.kv_heads * self.m.cfg.head_dim
        k = np.ctypeslib.as_array(lib().orc_seq_k(self.h, layer), shape=(max(n, 1),))[:n].copy()
        v = np.ctypeslib.as_array(lib().orc_seq_v(self.h, layer), shape=(max(n, 1),))[:n].copy()
        return k, v

    def step(self, emb, pos3, need_logits=True, want_logits=True):
        cfg = self.m.cfg
        logits = np.zeros(cfg.vocab, np.float32) if (need_logits and want_logits) else None
        fnorm = np.zeros(cfg.hidden, np.float32) if need_logits else None
        tok = np.zeros(1, np.int32)
        rc = lib().orc_step(self.m.h, self.h, _f32(emb), np.asarray(pos3, np.int32), int(need_logits),
                            logits.ctypes.data if logits is not None else None,
                            tok.ctypes.data if need_logits else None,
                            fnorm.ctypes.data if fnorm is not None else None)
        if rc != 0:
            raise RuntimeError(f"orc_step failed: {rc}")
        return (int(tok[0]) if need_logits else None), logits, fnorm
