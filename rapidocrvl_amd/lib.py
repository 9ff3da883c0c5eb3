"""ctypes binding of libpocr_hip.so (include/pocr_hip.h).

This is the host-side mirror of the reference's ``internal/backend`` hip
implementation: a thin wrapper that converts numpy arrays to pointers and
status codes to exceptions.  Loading fails loudly if the native library is
missing — there is no CPU fallback in this package.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libpocr_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pocr_hip.h")
# POCR_HOST_LIB names a build of the host-only sources (quant_host.cpp,
# gguf.cpp) whose functions then replace the library's own: the sanitizer
# build of tests/sanitize.py
HOST_LIB_PATH = os.environ.get("POCR_HOST_LIB")

POCR_OK = 0
POCR_ERR_ARG = -1
POCR_ERR_DEVICE = -2
POCR_ERR_NOMEM = -3
POCR_ERR_UNSUPPORTED = -4
POCR_ERR_INJECTED = -5

F32, Q8, Q4, Q6 = 0, 1000, 1001, 1002
TIE_HALF_AWAY, TIE_AMD64 = 0, 1
W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN, W_LM_HEAD = range(8)
N_LN1, N_LN2, N_FINAL = 0, 1, 2


class PocrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class PocrConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("intermediate", C.c_int32), ("layers", C.c_int32),
        ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("vocab", C.c_int32), ("rms_norm_eps", C.c_float), ("rope_theta", C.c_double),
        ("mrope_section", C.c_int32 * 3),
    ]


_vp = C.c_void_p
_i = C.c_int
_SIGS = {
    "pocr_abi_version": (_i, []),
    "pocr_last_error": (C.c_char_p, []),
    "pocr_ctx_create": (_i, [_i, C.POINTER(_vp)]),
    "pocr_ctx_destroy": (None, [_vp]),
    "pocr_device_count": (_i, []),
    "pocr_row_bytes": (C.c_size_t, [_i, _i]),
    "pocr_quantize_rows": (_i, [_i, _i, _vp, _i, _i, _vp, _vp]),
    "pocr_unpack_rows": (_i, [_i, _vp, _i, _i, _vp]),
    "pocr_weight_upload": (_i, [_vp, _i, _i, _i, _vp, _vp, C.POINTER(_vp)]),
    "pocr_weight_free": (None, [_vp]),
    "pocr_matvec": (_i, [_vp, _vp, _vp, _i, _vp]),
    "pocr_matvec_vnni": (_i, [_vp, _vp, _vp, _i, _vp]),
    "pocr_matvec_argmax": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "pocr_matvec_topk": (_i, [_vp, _vp, _vp, _i, _vp, _vp]),
    "pocr_sample_topk": (_i, [_vp, _vp, _i, _i, C.c_double, C.POINTER(C.c_uint64), _vp, _vp, _vp]),
    "pocr_sample_full": (_i, [_vp, _vp, _i, C.c_double, C.POINTER(C.c_uint64), _vp]),
    "pocr_fused_matvec3": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "pocr_fused_matvec3_mrope": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "pocr_swiglu_gate_up": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "pocr_matvec_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _vp, C.c_float, _i, _vp]),
    "pocr_rmsnorm": (_i, [_vp, _vp, _vp, _i, C.c_float, _vp]),
    "pocr_mrope_pair": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "pocr_text_attention": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pocr_text_attention_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pocr_text_attention_out": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "pocr_text_attention_out_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, C.c_float, _i,
                                                 _vp]),
    "pocr_first_token_value_out_add_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, C.c_float, _i, _vp]),
    "pocr_swiglu_down": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "pocr_swiglu_down_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _i, _vp]),
    "pocr_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, C.c_float, _i, _vp]),
    "pocr_mrope": (_i, [_vp, _vp, _vp, _vp, _i, _i]),
    "pocr_model_create": (_i, [_vp, C.POINTER(PocrConfig), C.POINTER(_vp)]),
    "pocr_model_destroy": (None, [_vp]),
    "pocr_model_set_weight": (_i, [_vp, _i, _i, _vp]),
    "pocr_model_set_norm": (_i, [_vp, _i, _i, _vp]),
    "pocr_model_set_embed": (_i, [_vp, _vp]),
    "pocr_model_set_residual_quirk": (_i, [_vp, _i]),
    "pocr_model_set_vnni": (_i, [_vp, _i]),
    "pocr_seq_create": (_i, [_vp, _i, C.POINTER(_vp)]),
    "pocr_seq_destroy": (None, [_vp]),
    "pocr_seq_reset": (_i, [_vp]),
    "pocr_seq_set_sampling": (_i, [_vp, C.c_double, _i, C.c_uint64]),
    "pocr_projector_create": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, C.POINTER(_vp)]),
    "pocr_projector_destroy": (None, [_vp]),
    "pocr_project_image": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "pocr_generate_vision": (_i, [_vp, _vp, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp]),
    "pocr_time_project": (_i, [_vp, _i, _i, _i, _i, _vp]),
    "pocr_seq_len": (_i, [_vp]),
    "pocr_seq_device_tokens": (_i, [_vp]),
    "pocr_seq_read_kv": (_i, [_vp, _i, _vp, _vp]),
    "pocr_seq_truncate": (_i, [_vp, _i]),
    "pocr_time_matvec": (_i, [_vp, _vp, _i, _vp, _i, _vp]),
    "pocr_time_matvec_argmax": (_i, [_vp, _vp, _i, _vp, _i, _vp]),
    "pocr_time_matvec_batched": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp]),
    "pocr_time_attention": (_i, [_vp, _i, _i, _i, _i, _i, _i, _vp]),
    "pocr_time_stream_read": (_i, [_vp, C.c_int64, _i, _i, _vp]),
    "pocr_seq_write_kv": (_i, [_vp, _i, _vp, _vp, _i]),
    "pocr_step": (_i, [_vp, _vp, _vp, _i, _vp, _vp]),
    "pocr_prefill": (_i, [_vp, _i, _vp, _vp, _vp, _vp]),
    "pocr_decode_greedy": (_i, [_vp, C.c_int32, C.c_int32, _i, _vp, _i, _vp]),
    "pocr_decode_batch": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _vp, _vp]),
    "pocr_generate": (_i, [_vp, _vp, _i, _vp, _i, C.c_int32, _vp, C.c_int32, _i, _vp, _i, _i, _vp]),
    "pocr_mm_positions": (_i, [_vp, _i, C.c_int32, _vp, C.c_int32, _vp, _vp]),
    "pocr_gguf_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "pocr_gguf_close": (None, [_vp]),
    "pocr_gguf_tensor_count": (_i, [_vp]),
    "pocr_gguf_find": (_i, [_vp, C.c_char_p]),
    "pocr_gguf_tensor_info": (_i, [_vp, _i, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32), C.POINTER(_i), _vp,
                                   C.POINTER(C.c_int64)]),
    "pocr_gguf_read": (_i, [_vp, _i, _vp, C.c_int64]),
    "pocr_gguf_meta_count": (_i, [_vp]),
    "pocr_gguf_meta": (_i, [_vp, _i, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                            C.POINTER(C.c_char_p)]),
    "pocr_model_load_gguf": (_i, [_vp, C.POINTER(PocrConfig), C.c_char_p, C.POINTER(_vp)]),
    "pocr_batch_create": (_i, [_vp, C.POINTER(_vp)]),
    "pocr_batch_destroy": (None, [_vp]),
    "pocr_batch_join": (_i, [_vp, _vp, C.c_int32, C.c_int32, _i, _vp, _i]),
    "pocr_batch_step": (_i, [_vp, _i]),
    "pocr_batch_poll": (_i, [_vp, _vp, C.POINTER(_i)]),
    "pocr_batch_leave": (_i, [_vp, _vp, _vp, _i]),
}

_lib = None


# the entry points implemented by the host-only sources
HOST_SYMBOLS = frozenset(["pocr_row_bytes", "pocr_quantize_rows", "pocr_unpack_rows", "pocr_mm_positions",
                          "pocr_gguf_open", "pocr_gguf_close", "pocr_gguf_tensor_count", "pocr_gguf_find",
                          "pocr_gguf_tensor_info", "pocr_gguf_read", "pocr_gguf_meta_count", "pocr_gguf_meta"])


def header_symbols(path: str = HEADER):
    """Function names declared in include/pocr_hip.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"\b(pocr_[a-z0-9_]+)\s*\(", text)))


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing; run __graft_entry__.build() (or python rapidocrvl_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if HOST_LIB_PATH:
            _use_host_lib(L, C.CDLL(HOST_LIB_PATH))
        _lib = L
    return _lib


_host_error = None  # the host library's message after its last failed call


def _use_host_lib(L, H):
    """Route the host-only entry points to H; a failure there keeps H's
    last-error text for check()."""
    H.pocr_last_error.restype = C.c_char_p
    H.pocr_last_error.argtypes = []

    def route(fn):
        def call(*a):
            global _host_error
            rc = fn(*a)
            _host_error = H.pocr_last_error() if isinstance(rc, int) and rc < 0 else None
            return rc
        return call

    for name in HOST_SYMBOLS:
        res, args = _SIGS[name]
        fn = getattr(H, name)
        fn.restype = res
        fn.argtypes = args
        setattr(L, name, route(fn))


def _ptr(a):
    return None if a is None else a.ctypes.data


def check(rc: int):
    global _host_error
    if rc < 0:
        msg, _host_error = _host_error or load().pocr_last_error(), None
        raise PocrError(rc, msg.decode(errors="replace"))
    return rc


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def row_bytes(qtype: int, cols: int) -> int:
    return int(load().pocr_row_bytes(qtype, cols))


def quantize_rows(qtype: int, w, tie: int = TIE_HALF_AWAY):
    """QuantizeQ*Row over a [rows, cols] f32 matrix → (scales, packed[rows, row_bytes])."""
    w = _f32(w)
    rows, cols = w.shape
    scales = np.zeros(rows, np.float32)
    packed = np.zeros((rows, row_bytes(qtype, cols)), np.uint8)
    check(load().pocr_quantize_rows(qtype, tie, _ptr(w), rows, cols, _ptr(scales), _ptr(packed)))
    return scales, packed


def unpack_rows(qtype: int, packed, cols: int):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = packed.shape[0]
    out = np.zeros((rows, cols), np.int8)
    check(load().pocr_unpack_rows(qtype, _ptr(packed), rows, cols, _ptr(out)))
    return out


def mm_positions(ids, image_token_id: int, grid, merge: int = 2):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    pos = np.zeros((max(ids.size, 1), 3), np.int32)
    delta = np.zeros(1, np.int32)
    g = np.ascontiguousarray(grid, dtype=np.int32)
    n = check(load().pocr_mm_positions(_ptr(ids), ids.size, image_token_id, _ptr(g), merge, _ptr(pos), _ptr(delta)))
    return pos[:n], int(delta[0])


def _eos_list(eos):
    """EOS ids as int32 (an empty list passes a count of zero; the library
    rejects negative ids and more than 1,024, as ValidateGenerateOptions
    does, internal/model/model.go:461-467)."""
    return np.ascontiguousarray(list(eos) if eos else [], dtype=np.int32)


def decode_batch(seqs, first_tokens, first_positions, max_new: int, eos=(2,)):
    """Decode of 1..16 sequences of one model together (pocr_decode_batch):
    returns one token array per sequence, first token first."""
    n = len(seqs)
    handles = (C.c_void_p * n)(*[s.h for s in seqs])
    ft = np.ascontiguousarray(first_tokens, dtype=np.int32)
    fp = np.ascontiguousarray(first_positions, dtype=np.int32)
    eos = _eos_list(eos)
    out = np.zeros((n, max(max_new, 1)), np.int32)
    counts = np.zeros(n, np.int32)
    check(load().pocr_decode_batch(C.cast(handles, C.c_void_p), n, _ptr(ft), _ptr(fp), max_new,
                                   _ptr(eos) if eos.size else None, eos.size, _ptr(out), _ptr(counts)))
    return [out[i, :counts[i]] for i in range(n)]


class Batch:
    """Continuous batching (pocr_batch_*): prefilled sequences of one model
    join and leave between token steps; up to 16 decode together."""

    def __init__(self, model: "Model"):
        h = _vp()
        check(load().pocr_batch_create(model.h, C.byref(h)))
        self.h, self.model = h, model
        self._budget = {}

    def close(self):
        if getattr(self, "h", None):
            load().pocr_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def join(self, seq: "Sequence", first_token: int, first_pos: int, max_new: int, eos=(2,)):
        e = np.ascontiguousarray(list(eos), dtype=np.int32)
        check(load().pocr_batch_join(self.h, seq.h, first_token, first_pos, max_new, _ptr(e) if e.size else None,
                                     e.size))
        self._budget[seq.h.value] = max_new

    def step(self, max_steps: int = 16) -> int:
        """Runs up to max_steps token steps; returns the members still decoding."""
        return check(load().pocr_batch_step(self.h, max_steps))

    def poll(self, seq: "Sequence"):
        done = C.c_int()
        n = check(load().pocr_batch_poll(self.h, seq.h, C.byref(done)))
        return n, bool(done.value)

    def leave(self, seq: "Sequence") -> np.ndarray:
        cap = self._budget.pop(seq.h.value, 0)
        out = np.zeros(max(cap, 1), np.int32)
        n = check(load().pocr_batch_leave(self.h, seq.h, _ptr(out), cap))
        return out[:min(n, cap)]


def device_count() -> int:
    return int(load().pocr_device_count())


class QMatrix:
    """Host copy of one Q*_ROW tensor (tensor.Q8Matrix/Q4Matrix/Q6Matrix, quant.go:5-29)."""

    def __init__(self, qtype: int, rows: int, cols: int, scales, packed):
        self.qtype, self.rows, self.cols = qtype, rows, cols
        self.scales = _f32(scales)
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(rows, row_bytes(qtype, cols))

    @classmethod
    def quantize(cls, w, qtype: int, tie: int = TIE_HALF_AWAY):
        w = _f32(w)
        s, p = quantize_rows(qtype, w, tie)
        return cls(qtype, w.shape[0], w.shape[1], s, p)


class Weight:
    def __init__(self, ctx: "Context", q: QMatrix):
        self.ctx, self.q = ctx, q
        self.rows, self.cols, self.qtype = q.rows, q.cols, q.qtype
        h = _vp()
        check(load().pocr_weight_upload(ctx.h, q.qtype, q.rows, q.cols, _ptr(q.scales), _ptr(q.packed), C.byref(h)))
        self.h = h
        ctx._children.add(self)

    def close(self):
        if getattr(self, "h", None):
            load().pocr_weight_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Context:
    """One device context: the op-level mirror of backend.Vulkan* calls.

    Closing releases dependents first (sequences, models, weights), so the
    native objects are freed child-before-parent whatever order Python's
    garbage collector finalises them in."""

    def __init__(self, device: int = 0):
        self._children = weakref.WeakSet()
        h = _vp()
        check(load().pocr_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            for obj in [o for o in self._children if isinstance(o, Model)]:
                obj.close()
            for obj in list(self._children):
                obj.close()
            load().pocr_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def upload(self, q: QMatrix) -> Weight:
        return Weight(self, q)

    # -- op level ---------------------------------------------------------
    def matvec(self, w: Weight, x):
        x = _f32(x)
        m = 1 if x.ndim == 1 else x.shape[0]
        out = np.zeros((m, w.rows), np.float32)
        check(load().pocr_matvec(self.h, w.h, _ptr(x), m, _ptr(out)))
        return out[0] if x.ndim == 1 else out

    def matvec_vnni(self, w: Weight, x):
        """W·x in the reference's VNNI activation mode (Q8: plain)."""
        x = _f32(x)
        m = 1 if x.ndim == 1 else x.shape[0]
        out = np.zeros((m, w.rows), np.float32)
        check(load().pocr_matvec_vnni(self.h, w.h, _ptr(x), m, _ptr(out)))
        return out[0] if x.ndim == 1 else out

    def matvec_argmax(self, w: Weight, x):
        x = _f32(x)
        idx = np.zeros(1, np.int32)
        sc = np.zeros(1, np.float32)
        check(load().pocr_matvec_argmax(self.h, w.h, _ptr(x), _ptr(idx), _ptr(sc)))
        return int(idx[0]), float(sc[0])

    def matvec_topk(self, w: Weight, x, k: int):
        """The k best rows of W·x (score descending, equal scores by lower row)."""
        x = _f32(x)
        ids = np.zeros(max(k, 1), np.int32)
        sc = np.zeros(max(k, 1), np.float32)
        n = check(load().pocr_matvec_topk(self.h, w.h, _ptr(x), k, _ptr(ids), _ptr(sc)))
        return ids[:n], sc[:n]

    def sample_topk(self, logits, k: int, temperature: float, rng_state: int):
        """One draw from the top k of logits with the fastRNG state rng_state;
        returns (token, advanced state, candidate ids, candidate scores)."""
        logits = _f32(logits)
        st = C.c_uint64(rng_state & ((1 << 64) - 1))
        tok = np.zeros(1, np.int32)
        ids = np.zeros(k, np.int32)
        sc = np.zeros(k, np.float32)
        check(load().pocr_sample_topk(self.h, _ptr(logits), logits.size, k, float(temperature), C.byref(st),
                                      _ptr(tok), _ptr(ids), _ptr(sc)))
        return int(tok[0]), int(st.value), ids, sc

    def sample_full(self, logits, temperature: float, rng_state: int):
        """One draw over every logit (sampleFullLogitsScratch) with the
        fastRNG state rng_state; returns (token, advanced state)."""
        logits = _f32(logits)
        st = C.c_uint64(rng_state & ((1 << 64) - 1))
        tok = np.zeros(1, np.int32)
        check(load().pocr_sample_full(self.h, _ptr(logits), logits.size, float(temperature), C.byref(st), _ptr(tok)))
        return int(tok[0]), int(st.value)

    def fused_matvec3(self, a: Weight, b: Weight, c: Weight, x):
        x = _f32(x)
        oa, ob, oc = (np.zeros(w.rows, np.float32) for w in (a, b, c))
        check(load().pocr_fused_matvec3(self.h, a.h, b.h, c.h, _ptr(x), _ptr(oa), _ptr(ob), _ptr(oc)))
        return oa, ob, oc

    def fused_matvec3_mrope(self, a, b, c, x, cos_t, sin_t, q_heads, kv_heads, head_dim):
        x, cos_t, sin_t = _f32(x), _f32(cos_t), _f32(sin_t)
        oa, ob, oc = (np.zeros(w.rows, np.float32) for w in (a, b, c))
        check(load().pocr_fused_matvec3_mrope(self.h, a.h, b.h, c.h, _ptr(x), _ptr(cos_t), _ptr(sin_t), q_heads,
                                              kv_heads, head_dim, _ptr(oa), _ptr(ob), _ptr(oc)))
        return oa, ob, oc

    def swiglu_gate_up(self, gate: Weight, up: Weight, x):
        x = _f32(x)
        out = np.zeros(gate.rows, np.float32)
        check(load().pocr_swiglu_gate_up(self.h, gate.h, up.h, _ptr(x), _ptr(out)))
        return out

    def matvec_add_rmsnorm(self, w: Weight, x, residual, norm_w, eps, in_place=True):
        """Returns (norm_out, residual_after)."""
        x, norm_w = _f32(x), _f32(norm_w)
        res = _f32(residual).copy()
        out = np.zeros(w.rows, np.float32)
        check(load().pocr_matvec_add_rmsnorm(self.h, w.h, _ptr(x), _ptr(res), _ptr(norm_w), eps, int(in_place),
                                             _ptr(out)))
        return out, res

    def rmsnorm(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        out = np.zeros_like(x)
        check(load().pocr_rmsnorm(self.h, _ptr(x), _ptr(w), x.size, eps, _ptr(out)))
        return out

    def mrope_pair(self, q, k, cos_t, sin_t, q_heads, kv_heads, head_dim):
        q, k = _f32(q).copy(), _f32(k).copy()
        cos_t, sin_t = _f32(cos_t), _f32(sin_t)  # keep the arrays alive across the call
        check(load().pocr_mrope_pair(self.h, _ptr(q), _ptr(k), _ptr(cos_t), _ptr(sin_t), q_heads, kv_heads, head_dim))
        return q, k

    def time_matvec(self, weights, x, iters):
        """Average µs per launch of the M=1 GEMV rotating over `weights`."""
        x = _f32(x)
        arr = (_vp * len(weights))(*[w.h for w in weights])
        us = np.zeros(1, np.float32)
        check(load().pocr_time_matvec(self.h, arr, len(weights), _ptr(x), iters, _ptr(us)))
        return float(us[0])

    def time_matvec_argmax(self, weights, x, iters):
        """Average µs per greedy LM-head launch (argmax only) rotating over `weights`."""
        x = _f32(x)
        arr = (_vp * len(weights))(*[w.h for w in weights])
        us = np.zeros(1, np.float32)
        check(load().pocr_time_matvec_argmax(self.h, arr, len(weights), _ptr(x), iters, _ptr(us)))
        return float(us[0])

    def time_matvec_batched(self, weights, x, iters):
        """Average µs per batched GEMV (x: [m][cols]) rotating over `weights`."""
        x = _f32(x)
        arr = (_vp * len(weights))(*[w.h for w in weights])
        us = np.zeros(1, np.float32)
        check(load().pocr_time_matvec_batched(self.h, arr, len(weights), _ptr(x), x.shape[0], iters, _ptr(us)))
        return float(us[0])

    def time_attention(self, heads, kv_heads, head_dim, cache_len, n_layers, iters):
        """Average µs of one decode-attention call over cache_len rows."""
        us = np.zeros(1, np.float32)
        check(load().pocr_time_attention(self.h, heads, kv_heads, head_dim, cache_len, n_layers, iters, _ptr(us)))
        return float(us[0])

    def time_stream_read(self, nbytes, n_buffers, iters):
        """Average µs of a plain streaming read of nbytes, rotating over n_buffers buffers."""
        us = np.zeros(1, np.float32)
        check(load().pocr_time_stream_read(self.h, nbytes, n_buffers, iters, _ptr(us)))
        return float(us[0])

    def text_attention(self, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim):
        q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
        out = np.zeros(heads * head_dim, np.float32)
        check(load().pocr_text_attention(self.h, _ptr(q), _ptr(kc), _ptr(vc), cache_len, heads, kv_heads, head_dim,
                                         _ptr(out)))
        return out

    def text_attention_out(self, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim, wo):
        q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
        out = np.zeros(wo.rows, np.float32)
        check(load().pocr_text_attention_out(self.h, _ptr(q), _ptr(kc), _ptr(vc), cache_len, heads, kv_heads, head_dim,
                                             wo.h, _ptr(out)))
        return out

    def text_attention_out_add_rmsnorm(self, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim, wo, residual,
                                       norm_w, eps, in_place):
        """Returns (norm_out, residual after)."""
        q, kc, vc, nw = _f32(q), _f32(k_cache), _f32(v_cache), _f32(norm_w)
        res = _f32(residual).copy()
        out = np.zeros(wo.rows, np.float32)
        check(load().pocr_text_attention_out_add_rmsnorm(self.h, _ptr(q), _ptr(kc), _ptr(vc), cache_len, heads,
                                                         kv_heads, head_dim, wo.h, _ptr(res), _ptr(nw), eps,
                                                         int(in_place), _ptr(out)))
        return out, res

    def first_token_value_out_add_rmsnorm(self, k_cache, v_cache, heads, kv_heads, head_dim, wo, residual, norm_w,
                                          eps, in_place):
        """Returns (norm_out, residual after)."""
        kc, vc, nw = _f32(k_cache), _f32(v_cache), _f32(norm_w)
        res = _f32(residual).copy()
        out = np.zeros(wo.rows, np.float32)
        check(load().pocr_first_token_value_out_add_rmsnorm(self.h, _ptr(kc), _ptr(vc), heads, kv_heads, head_dim,
                                                            wo.h, _ptr(res), _ptr(nw), eps, int(in_place),
                                                            _ptr(out)))
        return out, res

    def swiglu_down(self, gate, up, down, x):
        x = _f32(x)
        out = np.zeros(down.rows, np.float32)
        check(load().pocr_swiglu_down(self.h, gate.h, up.h, down.h, _ptr(x), _ptr(out)))
        return out

    def swiglu_down_add_rmsnorm(self, gate, up, down, x, residual, norm_w, eps, in_place):
        """Returns (norm_out, residual after)."""
        x, nw = _f32(x), _f32(norm_w)
        res = _f32(residual).copy()
        out = np.zeros(down.rows, np.float32)
        check(load().pocr_swiglu_down_add_rmsnorm(self.h, gate.h, up.h, down.h, _ptr(x), _ptr(res), _ptr(nw), eps,
                                                  int(in_place), _ptr(out)))
        return out, res

    def add_rmsnorm(self, dst, add, w, eps, in_place):
        """Returns (out, dst after)."""
        d = _f32(dst).copy()
        a, ww = _f32(add), _f32(w)
        out = np.zeros(d.size, np.float32)
        check(load().pocr_add_rmsnorm(self.h, _ptr(d), _ptr(a), _ptr(ww), d.size, eps, int(in_place), _ptr(out)))
        return out, d

    def mrope(self, x, cos_t, sin_t, heads, head_dim):
        x = _f32(x).copy()
        check(load().pocr_mrope(self.h, _ptr(x), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), heads, head_dim))
        return x

    def text_attention_noalloc(self, q_dev, k_dev, v_dev, cache_len, heads, kv_heads, head_dim, out_dev):
        """pocr_text_attention_noalloc over device addresses (ints) the caller owns."""
        check(load().pocr_text_attention_noalloc(self.h, C.c_void_p(q_dev), C.c_void_p(k_dev), C.c_void_p(v_dev),
                                                 cache_len, heads, kv_heads, head_dim, C.c_void_p(out_dev)))


class Model:
    """Device-resident decoder (weights borrowed, norms/embedding copied)."""

    def __init__(self, ctx: Context, cfg, gguf_path: str | None = None):
        self.ctx, self.cfg = ctx, cfg
        c = PocrConfig(cfg.hidden, cfg.inter, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab,
                       cfg.eps, cfg.rope_theta, (C.c_int32 * 3)(*cfg.mrope_section))
        self._seqs = weakref.WeakSet()
        h = _vp()
        if gguf_path is None:
            check(load().pocr_model_create(ctx.h, C.byref(c), C.byref(h)))
        else:
            check(load().pocr_model_load_gguf(ctx.h, C.byref(c), os.fsencode(gguf_path), C.byref(h)))
        self.h = h
        self._weights = []
        ctx._children.add(self)

    def close(self):
        for s in list(getattr(self, "_seqs", ())):
            s.close()
        if getattr(self, "h", None):
            load().pocr_model_destroy(self.h)
            self.h = None
        for w in getattr(self, "_weights", []):
            w.close()
        self._weights = []

    def __del__(self):
        self.close()

    def set_weight(self, layer: int, role: int, q: QMatrix):
        w = self.ctx.upload(q)
        self._weights.append(w)
        check(load().pocr_model_set_weight(self.h, layer, role, w.h))
        return w

    def set_norm(self, layer: int, role: int, w):
        w = _f32(w)
        check(load().pocr_model_set_norm(self.h, layer, role, _ptr(w)))

    def set_embed(self, e):
        e = _f32(e)
        check(load().pocr_model_set_embed(self.h, _ptr(e)))

    def set_residual_quirk(self, on: bool):
        check(load().pocr_model_set_residual_quirk(self.h, int(on)))

    def set_vnni(self, on: bool):
        """Q4/Q6 matvecs in the reference's VNNI activation mode (before any sequence)."""
        check(load().pocr_model_set_vnni(self.h, int(on)))

    def load_weights(self, weights):
        roles = {"q": W_Q, "k": W_K, "v": W_V, "o": W_O, "gate": W_GATE, "up": W_UP, "down": W_DOWN}
        for li, lw in enumerate(weights["layers"]):
            for name, role in roles.items():
                qt, sc, data, cols = lw[name]
                self.set_weight(li, role, QMatrix(qt, sc.size, cols, sc, data))
            self.set_norm(li, N_LN1, lw["ln1"])
            self.set_norm(li, N_LN2, lw["ln2"])
        qt, sc, data, cols = weights["lm_head"]
        self.set_weight(-1, W_LM_HEAD, QMatrix(qt, sc.size, cols, sc, data))
        self.set_norm(-1, N_FINAL, weights["final_norm"])
        self.set_embed(weights["embed"])

    @classmethod
    def from_gguf(cls, ctx: Context, cfg, path: str) -> "Model":
        """All decoder tensors from a GGUF checkpoint (pocr_model_load_gguf)."""
        return cls(ctx, cfg, gguf_path=path)

    def seq(self, capacity: int) -> "Sequence":
        return Sequence(self, capacity)


class GgufFile:
    """A GGUF checkpoint opened by the native reader (gguf.Open,
    internal/gguf/gguf.go:111-251): ``tensors`` maps name → (type, shape,
    payload bytes), ``metadata`` key → int or str."""

    def __init__(self, path: str):
        h = _vp()
        check(load().pocr_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h
        L = load()
        self.tensors = {}
        dims = (C.c_int64 * 8)()
        for i in range(check(L.pocr_gguf_tensor_count(h))):
            name, typ, nd, nb = C.c_char_p(), C.c_uint32(), C.c_int(), C.c_int64()
            check(L.pocr_gguf_tensor_info(h, i, C.byref(name), C.byref(typ), C.byref(nd), dims, C.byref(nb)))
            self.tensors[name.value.decode()] = (typ.value, tuple(dims[j] for j in range(nd.value)), nb.value)
        self.metadata = {}
        for i in range(check(L.pocr_gguf_meta_count(h))):
            key, typ, val, sval = C.c_char_p(), C.c_uint32(), C.c_uint64(), C.c_char_p()
            check(L.pocr_gguf_meta(h, i, C.byref(key), C.byref(typ), C.byref(val), C.byref(sval)))
            self.metadata[key.value.decode()] = sval.value.decode() if typ.value == 8 else val.value

    def close(self):
        if getattr(self, "h", None):
            load().pocr_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def raw(self, name: str) -> np.ndarray:
        typ, shape, nb = self.tensors[name]
        out = np.empty(nb, np.uint8)
        i = check(load().pocr_gguf_find(self.h, name.encode()))
        check(load().pocr_gguf_read(self.h, i, _ptr(out), nb))
        return out

    def float32(self, name: str) -> np.ndarray:
        """File.Float32 (gguf.go:313-327): an F32 tensor in its shape."""
        typ, shape, _ = self.tensors[name]
        if typ != F32:
            raise ValueError(f"{name} has type {typ}, not F32")
        return self.raw(name).view(np.float32).reshape(shape)

    def qrows(self, name: str) -> "QMatrix":
        """File.Q8Row / Q4Row / Q6Row (gguf.go:435-569): scales and packed rows."""
        typ, shape, _ = self.tensors[name]
        if typ not in (Q8, Q4, Q6):
            raise ValueError(f"{name} has type {typ}, not a Q*_ROW")
        rows, cols = shape
        raw = self.raw(name)
        return QMatrix(typ, rows, cols, raw[:rows * 4].view(np.float32).copy(),
                       raw[rows * 4:].reshape(rows, row_bytes(typ, cols)).copy())


class Projector:
    """The vision projector (mlp_AR, vision.go:224-302) with Q8 matrices on the device."""

    def __init__(self, ctx: "Context", norm_w, norm_b, w1, b1, w2, b2, eps: float = 1e-5):
        norm_w, norm_b, w1, b1, w2, b2 = (_f32(a) for a in (norm_w, norm_b, w1, b1, w2, b2))
        self.vd = norm_w.size
        self.td = w2.shape[0]
        h = _vp()
        check(load().pocr_projector_create(ctx.h, self.vd, self.td, _ptr(norm_w), _ptr(norm_b), _ptr(w1), _ptr(b1),
                                           _ptr(w2), _ptr(b2), float(eps), C.byref(h)))
        self.h = h

    @classmethod
    def from_gguf(cls, ctx: "Context", gguf: "GgufFile", eps: float = 1e-5) -> "Projector":
        """The mlp_AR tensors of a checkpoint (cacheVisionWeights, vision.go:224-302):
        pre_norm weight/bias, linear_1 and linear_2 weights and biases, all F32."""
        t = {n: gguf.float32("mlp_AR." + n) for n in ("pre_norm.weight", "pre_norm.bias", "linear_1.weight",
                                                       "linear_1.bias", "linear_2.weight", "linear_2.bias")}
        return cls(ctx, t["pre_norm.weight"], t["pre_norm.bias"], t["linear_1.weight"], t["linear_1.bias"],
                   t["linear_2.weight"], t["linear_2.bias"], eps=eps)

    def close(self):
        if getattr(self, "h", None):
            load().pocr_projector_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def time_project(self, grid, iters=20):
        """Average µs of one device projection of a T·H·W grid."""
        us = np.zeros(1, np.float32)
        check(load().pocr_time_project(self.h, grid[0], grid[1], grid[2], iters, _ptr(us)))
        return float(us[0])

    def project(self, vision_rows, grid):
        """vision rows [T·H·W][vd] → [T·(H/2)·(W/2)][td]."""
        x = _f32(vision_rows)
        t, h, w = grid
        if x.ndim != 2 or x.shape[0] < t * h * w or x.shape[1] != self.vd:
            raise ValueError(f"vision rows {x.shape}: need [{t * h * w}][{self.vd}]")
        out = np.zeros((t * (h // 2) * (w // 2), self.td), np.float32)
        n = check(load().pocr_project_image(self.h, _ptr(x), t, h, w, _ptr(out)))
        return out[:n]


class Sequence:
    def __init__(self, model: Model, capacity: int):
        self.model = model
        h = _vp()
        check(load().pocr_seq_create(model.h, capacity, C.byref(h)))
        self.h = h
        self.capacity = capacity
        model._seqs.add(self)

    def close(self):
        if getattr(self, "h", None):
            load().pocr_seq_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __len__(self):
        return check(load().pocr_seq_len(self.h))

    def device_tokens(self) -> int:
        """Tokens the device decode loop took in the last greedy decode."""
        return check(load().pocr_seq_device_tokens(self.h))

    def reset(self):
        check(load().pocr_seq_reset(self.h))

    def set_sampling(self, temperature: float, top_k: int, seed: int = 0):
        """Token choice of generate/decode: greedy (temperature <= 0 or
        top_k == 1) or draws from the top_k candidates (1 < top_k <= 64)."""
        check(load().pocr_seq_set_sampling(self.h, float(temperature), int(top_k), seed & ((1 << 64) - 1)))

    def read_kv(self, layer: int):
        cfg = self.model.cfg
        n = len(self) * cfg.kv_heads * cfg.head_dim
        k = np.zeros(max(n, 1), np.float32)
        v = np.zeros(max(n, 1), np.float32)
        check(load().pocr_seq_read_kv(self.h, layer, _ptr(k), _ptr(v)))
        return k[:n], v[:n]

    def truncate(self, length: int):
        check(load().pocr_seq_truncate(self.h, length))

    def write_kv(self, layer: int, k, v, length: int):
        k, v = _f32(k), _f32(v)
        check(load().pocr_seq_write_kv(self.h, layer, _ptr(k), _ptr(v), length))

    def step(self, emb, pos3, need_logits=True, want_logits=True):
        cfg = self.model.cfg
        emb = _f32(emb)
        pos = np.ascontiguousarray(pos3, dtype=np.int32)
        logits = np.zeros(cfg.vocab, np.float32) if (need_logits and want_logits) else None
        tok = np.zeros(1, np.int32)
        check(load().pocr_step(self.h, _ptr(emb), _ptr(pos), int(need_logits), _ptr(logits),
                               _ptr(tok) if need_logits else None))
        return (int(tok[0]) if need_logits else None), logits

    def prefill(self, emb, pos3, want_logits=False):
        cfg = self.model.cfg
        emb = _f32(emb)
        pos = np.ascontiguousarray(pos3, dtype=np.int32)
        logits = np.zeros(cfg.vocab, np.float32) if want_logits else None
        tok = np.zeros(1, np.int32)
        check(load().pocr_prefill(self.h, emb.shape[0], _ptr(emb), _ptr(pos), _ptr(logits), _ptr(tok)))
        return int(tok[0]), logits

    def generate_vision(self, proj: Projector, ids, vision_rows, image_token_id: int, grid, max_new, eos=(2,)):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        eos = _eos_list(eos)
        out = np.zeros(max(max_new, 1), np.int32)
        x = _f32(vision_rows)
        g = np.ascontiguousarray(grid, dtype=np.int32)
        if x.ndim != 2 or x.shape[0] < int(np.prod(g)) or x.shape[1] != proj.vd:
            raise ValueError(f"vision rows {x.shape}: need [{int(np.prod(g))}][{proj.vd}]")
        n = check(load().pocr_generate_vision(self.h, proj.h, _ptr(ids), ids.size, _ptr(x), image_token_id, _ptr(g),
                                              max_new, _ptr(eos) if eos.size else None, eos.size,
                                              _ptr(out)))
        return out[:n]

    def decode_greedy(self, first_token: int, first_pos: int, max_new: int, eos=(2,)):
        eos = _eos_list(eos)
        out = np.zeros(max(max_new, 1), np.int32)
        n = check(load().pocr_decode_greedy(self.h, first_token, first_pos, max_new,
                                            _ptr(eos) if eos.size else None, eos.size, _ptr(out)))
        return out[:n]

    def generate(self, ids, max_new, eos=(2,), image_embeds=None, image_token_id=-1, grid=(1, 1, 1), merge=2,
                 use_prefill=False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        eos = _eos_list(eos)
        out = np.zeros(max(max_new, 1), np.int32)
        img = _f32(image_embeds) if image_embeds is not None else None
        n_img = 0 if img is None else img.shape[0]
        g = np.ascontiguousarray(grid, dtype=np.int32)
        n = check(load().pocr_generate(self.h, _ptr(ids), ids.size, _ptr(img), n_img, image_token_id, _ptr(g), merge,
                                       max_new, _ptr(eos) if eos.size else None, eos.size, int(use_prefill),
                                       _ptr(out)))
        return out[:n]
