"""The digit-plane model (tests/digit_model.py) the GPU argmax tests measure
the device heads against: its residuals stay inside the stated bounds, which
follow from the construction (a power-of-two chunk scale, round-to-nearest
digits), over random, tiny, zero and power-of-two chunks."""
import numpy as np
import pytest

import digit_model as dm


def _chunks(W, rng):
    out = [rng.standard_normal(W * 4096).astype(np.float32),
           (rng.standard_normal(W * 512) * 1e-30).astype(np.float32),
           np.zeros(W * 4, np.float32),
           np.ldexp(1.0, rng.integers(-20, 20, W * 256)).astype(np.float32) * rng.choice([-1, 1], W * 256),
           rng.uniform(-7, 7, W * 256).astype(np.float32)]
    return np.concatenate(out)


@pytest.mark.parametrize("qtype,nib", [(dm.Q4, True), (dm.Q4, False), (dm.Q8, False), (dm.Q6, False)],
                         ids=["q4-nibbles", "q4-bytes", "q8-bytes", "q6-bytes"])
def test_residual_within_bound(qtype, nib):
    x = _chunks(dm.chunk_width(qtype), np.random.default_rng(3))
    r = np.abs(x.astype(np.float64) - dm.digitize(qtype, x, nib))
    bound = dm.residual_bound(qtype, x, nib)
    # the bound, and for nibble planes one last-place f32 rounding per plane
    # step (t_k ∈ [4, 8): ≤ 2^-22 of S/15^k, k ≥ 1; below 2^-25·S in all)
    slack = dm._scale(np.abs(x.reshape(-1, dm.chunk_width(qtype))).max(axis=1), 7.0 if nib else 127.0)
    assert np.all(r <= bound + np.repeat(slack, dm.chunk_width(qtype)) * 2.0 ** -25)
    # the bound relative to each chunk's maximum m: S < 2m/7 → 2^-22.3 for
    # nibbles; S < 2m/127 → 2^-20.99 for bytes
    m = np.repeat(np.abs(x.reshape(-1, dm.chunk_width(qtype))).max(axis=1), dm.chunk_width(qtype))
    rel = 2 / (7 * 2 * 15.0 ** 5) if nib else 2 / (127 * 2.0 ** 15)
    nz = m > 0
    assert np.all(bound[nz] <= rel * m[nz])


def test_fewer_nibble_planes_break_the_bound():
    """A model with four nibble planes (the head before) leaves residuals
    225× above the six-plane bound: the bound tells the two apart."""
    x = np.random.default_rng(5).standard_normal(32 * 1024).astype(np.float32)
    old = dm.NIB_PLANES
    try:
        dm.NIB_PLANES = 4
        r4 = np.abs(x.astype(np.float64) - dm.digitize(dm.Q4, x, True))
    finally:
        dm.NIB_PLANES = old
    assert r4.max() > 50 * dm.residual_bound(dm.Q4, x, True).max()


def test_exact_on_representable_values():
    # integer multiples of the chunk scale are digitized without residual
    x = np.array([0.25 * k for k in range(-6, 7)] * 3, np.float32)[:32]  # max 1.5 → S = 0.25
    assert np.array_equal(dm.digitize(dm.Q4, x, True), x.astype(np.float64))
    y = (np.arange(16, dtype=np.float32) - 8) / 64  # max 0.125 → S = 2^-9
    assert np.array_equal(dm.digitize(dm.Q8, y), y.astype(np.float64))
