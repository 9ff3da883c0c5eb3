"""The vision projector's checker: LayerNorm, GELUTanh and projectImageRows
of the oracle, pinned by the exact formulas in float64, the reference's
temporal-frame test and a float64 restatement of the block walk."""
import json
import math
import os

import numpy as np
import pytest

import oracle
from rapidocrvl_amd import lib

KAT = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")))


def gelu64(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def ln64(x, w, b, eps):
    x = np.asarray(x, np.float64)
    m = x.mean()
    return (x - m) / np.sqrt(((x - m) ** 2).mean() + eps) * w + b


def test_gelu_tanh_matches_the_formula():
    x = np.linspace(-8, 8, 2001).astype(np.float32)
    g = oracle.gelu_tanh(x)
    assert np.max(np.abs(g - gelu64(x)) / np.maximum(1, np.abs(x))) < 1e-6
    assert oracle.gelu_tanh(np.float32(0.0)) == 0.0
    # gelu(x) − gelu(−x) = x
    assert np.max(np.abs((g - g[::-1]) - x)) < 4e-6


@pytest.mark.parametrize("n", [5, 8, 13, 1152])
def test_layernorm_matches_float64(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = oracle.layernorm(x, w, b, 1e-5)
    assert np.max(np.abs(got - ln64(x, w, b, 1e-5))) < 2e-5 * max(1.0, float(np.max(np.abs(w))))
    unit = oracle.layernorm(x, np.ones(n, np.float32), np.zeros(n, np.float32), 1e-5)
    assert abs(float(unit.astype(np.float64).mean())) < 1e-5 and abs(float((unit.astype(np.float64) ** 2).mean()) - 1) < 1e-4


def _q8(w):
    s, p = lib.quantize_rows(lib.Q8, w)
    return s, p


def project64(x, grid, vd, nw, nb, q1, b1, q2, b2, eps):
    """float64 restatement with the same Q8 codes: 2×2 blocks in frame, row,
    column order; quarters base, base+1, base+W, base+W+1."""
    t, h, w = grid
    c1 = q1[1].view(np.int8).astype(np.float64) * q1[0][:, None]
    c2 = q2[1].view(np.int8).astype(np.float64) * q2[0][:, None]
    out = []
    for f in range(t):
        for by in range(h // 2):
            for bx in range(w // 2):
                base = f * h * w + by * 2 * w + bx * 2
                m = np.concatenate([ln64(x[i], nw, nb, eps) for i in (base, base + 1, base + w, base + w + 1)])
                hid = gelu64(c1 @ m + b1)
                out.append(c2 @ hid + b2)
    return np.array(out)


@pytest.mark.parametrize("grid", [(2, 4, 6), (1, 5, 7), (1, 2, 2)])
def test_project_image_matches_float64(grid):
    rng = np.random.default_rng(sum(grid))
    vd, td = 8, 16
    t, h, w = grid
    x = rng.standard_normal((t * h * w, vd)).astype(np.float32)
    x += np.arange(t * h * w, dtype=np.float32)[:, None] * 0.1  # every row distinct
    nw = (1 + 0.1 * rng.standard_normal(vd)).astype(np.float32)
    nb = (0.1 * rng.standard_normal(vd)).astype(np.float32)
    w1 = (rng.standard_normal((4 * vd, 4 * vd)) * 0.3).astype(np.float32)
    w2 = (rng.standard_normal((td, 4 * vd)) * 0.3).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(4 * vd)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(td)).astype(np.float32)
    q1, q2 = _q8(w1), _q8(w2)
    got = oracle.project_image(x, grid, nw, nb, q1, b1, q2, b2)
    want = project64(x, grid, vd, nw, nb, q1, b1, q2, b2, 1e-5)
    assert got.shape == (t * (h // 2) * (w // 2), td)
    assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, float(np.max(np.abs(want))))


def test_project_image_reference_temporal_frames():
    k = KAT["project_temporal_frames"]
    vd, td = k["vd"], k["td"]
    x = np.asarray(k["x"], np.float32)
    eye = np.eye(4 * vd, dtype=np.float32)
    q1, q2 = _q8(eye), _q8(eye[:td].copy())
    out = oracle.project_image(x, k["grid"], np.ones(vd, np.float32), np.zeros(vd, np.float32), q1,
                               np.zeros(4 * vd, np.float32), q2, np.zeros(td, np.float32))
    assert out.shape == (k["rows"], td)
    assert np.any(out[1] != 0) and not np.array_equal(out[0], out[1])
