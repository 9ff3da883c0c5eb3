"""The activation digit planes of the device GEMVs and greedy heads, restated
in numpy.

A device GEMV never multiplies f32 activations: the activation is written as
three int8 digit planes under a power-of-two scale S, and the weight codes
are dotted with the digits exactly in int32,
  x = S·(d0 + d1/2⁷ + d2/2¹⁴) + e,   |e| ≤ S/2¹⁵.
The layer GEMVs take one scale per chunk of W columns (32 for Q4 codes, 16
for Q8/Q6), S ≥ max|x|/127 over the chunk; the MFMA greedy head takes one
scale for the whole vector.  ``digitize`` and ``planes_whole`` return what
the planes represent (float64, exact), so a test can say what a kernel must
compute — the codes times the digitized x, up to the f32 steps after the
integer dots — and how far that is from the exact product with x.
"""
import numpy as np

Q8, Q4, Q6 = 1000, 1001, 1002


def chunk_width(qtype):
    return 32 if qtype == Q4 else 16


def _scale(m, div):
    """frexpf(m·(1/div)) → S = 2^ex (1 for an all-zero chunk), f32 steps."""
    q = m.astype(np.float32) * np.float32(1.0 / div)
    ex = np.frexp(q)[1].astype(np.int64)
    return np.where(m > 0, np.ldexp(1.0, ex), 1.0)


def _planes(xc, S):
    """digits of rows xc (f32) under scales S (one per row): [3, rows, cols]"""
    t = (xc.astype(np.float64) / S).astype(np.float32)  # exact: S is a power of two
    a = np.rint(t)
    t1 = ((t - a) * np.float32(128.0)).astype(np.float32)  # exact: |t − a| ≤ 1/2
    b = np.rint(t1)
    d2 = np.rint((t1 - b) * np.float32(128.0))
    return np.stack([a, b, d2]).astype(np.float64)


def digitize(qtype, x):
    """x (f32, length a multiple of the chunk width) → the value the layer
    GEMVs' digit planes represent, float64."""
    x = np.asarray(x, np.float32)
    xc = x.reshape(-1, chunk_width(qtype))
    S = _scale(np.abs(xc).max(axis=1), 127.0)[:, None]
    d = _planes(xc, S)
    return ((d[0] + d[1] / 128.0 + d[2] / 16384.0) * S).reshape(-1)


def residual_bound(qtype, x):
    """Per-column bound on |x − digitize(x)|: S/2¹⁵ of the column's chunk."""
    x = np.asarray(x, np.float32)
    W = chunk_width(qtype)
    S = _scale(np.abs(x.reshape(-1, W)).max(axis=1), 127.0)
    return np.repeat(S / 2.0 ** 15, W)


def planes_whole(x):
    """The MFMA greedy head's digits: three byte planes under one power-of-two
    scale S ≥ max|x|/127 over the whole vector.  Returns S and the digits
    [3][n] (float64, exact integers), so that x ≈ S·(d0 + d1/2⁷ + d2/2¹⁴)."""
    x = np.asarray(x, np.float32)
    S = float(_scale(np.array([np.abs(x).max()]), 127.0)[0])
    return S, _planes(x[None, :], S)[:, 0, :]


def head_scores(codes, scales, x, rows_per_block=8192):
    """What the MFMA head computes for x (no RMSNorm), exactly: scale·S·
    (A0 + A1/2⁷ + A2/2¹⁴) with A_p = codes·d_p; and the magnitude its f32
    steps round against, scale·S·(|A0| + |A1|/2⁷ + |A2|/2¹⁴)."""
    S, d = planes_whole(x)
    out = np.zeros(codes.shape[0])
    mag = np.zeros(codes.shape[0])
    w = np.array([1.0, 1.0 / 128, 1.0 / 16384])
    for i in range(0, codes.shape[0], rows_per_block):
        A = codes[i:i + rows_per_block].astype(np.float64) @ d.T
        out[i:i + rows_per_block] = A @ w
        mag[i:i + rows_per_block] = np.abs(A) @ w
    sc = np.asarray(scales, np.float64) * S
    return out * sc, mag * sc


def head_scores_rows(codes, scales, X):
    """head_scores for every row of X at once: ([m, rows], [m, rows]).  The
    integer plane sums are formed in f32, exact while |Σ| < 2^24 (codes ≤ 128
    in magnitude, digits ≤ 127, 1024 columns; Q6 codes ≤ 32 also at 2048)."""
    X = np.asarray(X, np.float32)
    m, cols = X.shape
    assert int(np.abs(codes).max()) * 127 * cols < 2 ** 24
    S = np.zeros(m)
    D = np.zeros((cols, 3 * m), np.float32)
    for i in range(m):
        S[i], d = planes_whole(X[i])
        D[:, 3 * i:3 * i + 3] = d.T
    A = (codes.astype(np.float32) @ D).astype(np.float64).reshape(codes.shape[0], m, 3)
    w = np.array([1.0, 1.0 / 128, 1.0 / 16384])
    sc = np.asarray(scales, np.float64)[None, :] * S[:, None]
    return (A @ w).T * sc, (np.abs(A) @ w).T * sc


def scores(qtype, codes, scales, xv, rows_per_block=4096):
    """scale·(codes · xv) in float64 (xv: x or a digitized x)."""
    out = np.zeros(codes.shape[0])
    xv = np.asarray(xv, np.float64)
    for i in range(0, codes.shape[0], rows_per_block):
        out[i:i + rows_per_block] = codes[i:i + rows_per_block].astype(np.float64) @ xv
    return out * np.asarray(scales, np.float64), None


def gemv_scores(qtype, codes, scales, x, rows_per_block=2048):
    """What the byte-plane GEMV computes for x (no RMSNorm), exactly: scale·
    Σ_c S_c·(A0c + A1c/2⁷ + A2c/2¹⁴) over chunks c; and the magnitude its f32
    steps round against, scale·Σ_c S_c·(|A0c| + |A1c|/2⁷ + |A2c|/2¹⁴)."""
    x = np.asarray(x, np.float32)
    W = chunk_width(qtype)
    xc = x.reshape(-1, W)
    S = _scale(np.abs(xc).max(axis=1), 127.0)  # [chunks]
    d = _planes(xc, S[:, None])                # [3, chunks, W]
    w = np.array([1.0, 1.0 / 128, 1.0 / 16384])
    out = np.zeros(codes.shape[0])
    mag = np.zeros(codes.shape[0])
    nc = xc.shape[0]
    for i in range(0, codes.shape[0], rows_per_block):
        c = codes[i:i + rows_per_block].astype(np.float64).reshape(-1, nc, W)
        A = np.einsum("rcw,pcw->rcp", c, d)    # [rows, chunks, planes], exact integers
        out[i:i + rows_per_block] = (A @ w) @ S
        mag[i:i + rows_per_block] = (np.abs(A) @ w) @ S
    sc = np.asarray(scales, np.float64)
    return out * sc, mag * sc
