"""The digit-plane model (tests/digit_model.py) the GPU argmax tests measure
the device heads against: its residuals stay inside the stated bounds, which
follow from the construction (a power-of-two scale, round-to-nearest digits),
over random, tiny, zero and power-of-two inputs."""
import numpy as np
import pytest

import digit_model as dm


def _inputs(W, rng):
    out = [rng.standard_normal(W * 4096).astype(np.float32),
           (rng.standard_normal(W * 512) * 1e-30).astype(np.float32),
           np.zeros(W * 4, np.float32),
           np.ldexp(1.0, rng.integers(-20, 20, W * 256)).astype(np.float32) * rng.choice([-1, 1], W * 256),
           rng.uniform(-127, 127, W * 256).astype(np.float32)]
    return np.concatenate(out)


@pytest.mark.parametrize("qtype", [dm.Q4, dm.Q8, dm.Q6], ids=["q4", "q8", "q6"])
def test_chunk_residual_within_bound(qtype):
    x = _inputs(dm.chunk_width(qtype), np.random.default_rng(3))
    r = np.abs(x.astype(np.float64) - dm.digitize(qtype, x))
    bound = dm.residual_bound(qtype, x)
    assert np.all(r <= bound)
    # S < 2m/127 for the chunk maximum m: the bound is below 2^-20.99·m
    m = np.repeat(np.abs(x.reshape(-1, dm.chunk_width(qtype))).max(axis=1), dm.chunk_width(qtype))
    nz = m > 0
    assert np.all(bound[nz] <= 2 / (127 * 2.0 ** 15) * m[nz])


def test_whole_vector_planes():
    rng = np.random.default_rng(4)
    for x in (rng.standard_normal(1024).astype(np.float32), np.zeros(1024, np.float32),
              (rng.standard_normal(2048) * 1e-30).astype(np.float32)):
        S, d = dm.planes_whole(x)
        xt = S * (d[0] + d[1] / 128 + d[2] / 16384)
        assert np.all(np.abs(x.astype(np.float64) - xt) <= S / 2.0 ** 15)
        assert np.abs(d[0]).max() <= 127 and np.abs(d[1:]).max() <= 64
        assert S * 127 >= np.abs(x).max() and (np.abs(x).max() == 0 or S * 63.5 < np.abs(x).max())


def test_two_planes_break_the_bound():
    """Dropping the last plane leaves residuals ~128× above the bound: the
    bound tells a two-plane head from a three-plane one."""
    x = np.random.default_rng(5).standard_normal(16 * 1024).astype(np.float32)
    S = dm._scale(np.abs(x.reshape(-1, 16)).max(axis=1), 127.0)[:, None]
    d = dm._planes(x.reshape(-1, 16), S)
    two = ((d[0] + d[1] / 128.0) * S).reshape(-1)
    assert np.abs(x - two).max() > 50 * dm.residual_bound(dm.Q8, x).max()


def test_exact_on_representable_values():
    # integer multiples of 2^-14·S are digitized without residual
    y = (np.arange(16, dtype=np.float32) - 8) / 64  # max 0.125 → S = 2^-9
    assert np.array_equal(dm.digitize(dm.Q8, y), y.astype(np.float64))
    z = np.float32(2.0 ** -20) * np.arange(-16, 16, dtype=np.float32) + np.float32(0.5)
    S, d = dm.planes_whole(z)
    assert np.array_equal(S * (d[0] + d[1] / 128 + d[2] / 16384), z.astype(np.float64))
