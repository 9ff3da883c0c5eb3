"""Vision projector on the device (pocr_project_image / pocr_generate_vision)
against the oracle's projectImageRows with the same Q8 matrices."""
import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import DecoderConfig

pytestmark = pytest.mark.gpu

MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)
IMG = 100295


def _weights(vd, td, seed):
    rng = np.random.default_rng(seed)
    K = 4 * vd
    return dict(
        norm_w=(1 + 0.1 * rng.standard_normal(vd)).astype(np.float32),
        norm_b=(0.1 * rng.standard_normal(vd)).astype(np.float32),
        w1=(rng.standard_normal((K, K)) * (1.5 / np.sqrt(K))).astype(np.float32),
        b1=(0.1 * rng.standard_normal(K)).astype(np.float32),
        w2=(rng.standard_normal((td, K)) * (1.0 / np.sqrt(K))).astype(np.float32),
        b2=(0.1 * rng.standard_normal(td)).astype(np.float32),
    )


def _oracle(orc, pw, x, grid):
    q1 = lib.quantize_rows(lib.Q8, pw["w1"])
    q2 = lib.quantize_rows(lib.Q8, pw["w2"])
    return orc.project_image(x, grid, pw["norm_w"], pw["norm_b"], q1, pw["b1"], q2, pw["b2"])


def _close(got, want, rel=1e-4):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= rel * scale, f"max err {err} vs scale {scale}"


@pytest.mark.parametrize("vd,td,grid", [(64, 128, (2, 6, 8)), (64, 128, (1, 5, 7)), (32, 64, (1, 2, 2)),
                                        (1152, 1024, (1, 8, 12))])
def test_project_image_matches_oracle(ctx, orc, vd, td, grid):
    pw = _weights(vd, td, seed=vd + sum(grid))
    t, h, w = grid
    x = np.random.default_rng(7).standard_normal((t * h * w, vd)).astype(np.float32)
    x += np.arange(t * h * w, dtype=np.float32)[:, None] * 0.01
    proj = lib.Projector(ctx, **pw)
    got = proj.project(x, grid)
    want = _oracle(orc, pw, x, grid)
    assert got.shape == want.shape == (t * (h // 2) * (w // 2), td)
    _close(got, want)
    # a second call of another shape reuses or regrows the buffers
    x2 = np.random.default_rng(8).standard_normal((2 * 4 * 6, vd)).astype(np.float32)
    _close(proj.project(x2, (2, 4, 6)), _oracle(orc, pw, x2, (2, 4, 6)))
    proj.close()


def test_projector_rejects_unsupported_shapes(ctx):
    for vd, td in ((5, 64), (48, 64), (64, 100)):
        pw = _weights(vd, td, seed=1)
        with pytest.raises(lib.PocrError) as e:
            lib.Projector(ctx, **pw)
        assert e.value.code == lib.POCR_ERR_UNSUPPORTED


def test_generate_vision_matches_oracle(ctx, orc):
    # vision rows → device projection → image rows of the prompt → tokens,
    # against the oracle generating from its own projected rows
    w = synth.make_weights(MID, lib.Q4, seed=12)
    om = orc.Model(MID)
    om.load_weights(w)
    gm = lib.Model(ctx, MID)
    gm.load_weights(w)
    vd, grid = 64, (1, 8, 12)
    pw = _weights(vd, MID.hidden, seed=3)
    x = np.random.default_rng(5).standard_normal((8 * 12, vd)).astype(np.float32)
    rows = _oracle(orc, pw, x, grid)
    ids = np.concatenate([synth.prompt_ids(5, seed=30, high=MID.vocab), np.full(rows.shape[0], IMG, np.int32),
                          synth.prompt_ids(8, seed=31, high=MID.vocab)]).astype(np.int32)
    want = list(om.generate(ids, 16, eos=(), image_embeds=rows, image_token_id=IMG, grid=grid))
    proj = lib.Projector(ctx, **pw)
    s = gm.seq(ids.size + 16)
    assert list(s.generate_vision(proj, ids, x, IMG, grid, 16, eos=())) == want
    # the placeholders must match the projected rows (23 placeholders for 24 rows)
    with pytest.raises(lib.PocrError):
        s.generate_vision(proj, ids[:-9], x, IMG, grid, 4, eos=())
    # the host buffer must hold T·H·W vision rows
    with pytest.raises(ValueError):
        s.generate_vision(proj, ids, x[:-1], IMG, grid, 4, eos=())
