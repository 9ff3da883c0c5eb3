"""The activation digit planes of the device GEMVs, restated in numpy.

A device GEMV never multiplies f32 activations: each chunk of W columns
(32 for Q4 codes, 16 for Q8/Q6) is written as integer digit planes under a
power-of-two chunk scale S, and the weight codes are dotted with the digits
exactly in int32.  ``digitize`` returns the value those planes represent
(float64, exact), so a test can say what the kernel must compute — the
codes times the digitized x, up to the f32 steps after the integer dots —
and how far that is from the exact product with x.

* byte planes (every layer GEMV; the Q8/Q6 greedy LM head): S ≥ max|x|/127,
  x = S·(d0 + d1/2⁷ + d2/2¹⁴) + e, |e| ≤ S/2¹⁵;
* nibble planes (the Q4 greedy LM head): S > max|x|/7,
  x = S·(e0 + e1/15 + … + e5/15⁵) + e, e_k ∈ [−7, 7], |e| ≤ S/(2·15⁵).
"""
import numpy as np

Q8, Q4, Q6 = 1000, 1001, 1002
NIB_PLANES = 6


def chunk_width(qtype):
    return 32 if qtype == Q4 else 16


def _scale(m, div):
    """frexpf(m·(1/div)) → S = 2^ex (1 for an all-zero chunk), f32 steps."""
    q = m.astype(np.float32) * np.float32(1.0 / div)
    ex = np.frexp(q)[1].astype(np.int64)
    return np.where(m > 0, np.ldexp(1.0, ex), 1.0)


def digitize(qtype, x, nibbles=False):
    """x (f32, length a multiple of the chunk width) → the digitized x, float64."""
    x = np.asarray(x, np.float32)
    W = chunk_width(qtype)
    xc = x.reshape(-1, W)
    m = np.abs(xc).max(axis=1)
    if nibbles:
        S = _scale(m, 7.0)[:, None]
        t = (xc.astype(np.float64) / S).astype(np.float32)  # exact: S is a power of two
        out = np.zeros(xc.shape)
        w = 1.0
        for _ in range(NIB_PLANES):
            e = np.clip(np.rint(t), -7, 7).astype(np.float64)
            out += e * w
            w /= 15.0
            # fmaf(t, 15, −15·e): the exact value, rounded once to f32
            t = (t.astype(np.float64) * 15.0 - 15.0 * e).astype(np.float32)
        return (out * S).reshape(-1)
    S = _scale(m, 127.0)[:, None]
    t = (xc.astype(np.float64) / S).astype(np.float32)
    a = np.rint(t)
    t1 = ((t - a) * np.float32(128.0)).astype(np.float32)  # exact: |t − a| ≤ 1/2
    b = np.rint(t1)
    d2 = np.rint((t1 - b) * np.float32(128.0))
    a, b, d2 = (v.astype(np.float64) for v in (a, b, d2))
    return ((a + b / 128.0 + d2 / 16384.0) * S).reshape(-1)


def residual_bound(qtype, x, nibbles=False):
    """Per-column bound on |x − digitize(x)|: S/(2·15⁵) or S/2¹⁵ per chunk
    (the nibble planes' f32 steps add at most S·2⁻²²/14 more)."""
    x = np.asarray(x, np.float32)
    W = chunk_width(qtype)
    m = np.abs(x.reshape(-1, W)).max(axis=1)
    S = _scale(m, 7.0 if nibbles else 127.0)
    r = S / (2 * 15.0 ** (NIB_PLANES - 1)) if nibbles else S / 2.0 ** 15
    return np.repeat(r, W)


def scores(qtype, codes, scales, xv, rows_per_block=4096):
    """scale·(codes · xv) in float64, and scale·Σ over chunks of |chunk dot|:
    the magnitude the kernel's f32 steps after the integer dots round against."""
    W = chunk_width(qtype)
    rows, cols = codes.shape
    nc = cols // W
    xv = np.asarray(xv, np.float64)
    out = np.zeros(rows)
    mag = np.zeros(rows)
    for i in range(0, rows, rows_per_block):
        prod = codes[i:i + rows_per_block].astype(np.float64) * xv[None, :]
        per_chunk = prod[:, : nc * W].reshape(prod.shape[0], nc, W).sum(axis=2)
        out[i:i + rows_per_block] = per_chunk.sum(axis=1)
        mag[i:i + rows_per_block] = np.abs(per_chunk).sum(axis=1)
    sc = np.asarray(scales, np.float64)
    return out * sc, mag * sc
