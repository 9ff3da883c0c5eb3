"""A decoder loaded from a converted GGUF checkpoint (pocr_model_load_gguf)
generates the tokens of the same weights handed over tensor by tensor, and
of the oracle."""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from rapidocrvl_amd import convert, lib, synth
from rapidocrvl_amd.config import DecoderConfig, decoder_config, load_config_json

pytestmark = pytest.mark.gpu

MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    with open(d / "config.json", "w") as f:
        json.dump(synth.config_json(MID), f)
    tensors = synth.make_checkpoint(MID, seed=21)
    save_file({k: torch.from_numpy(v).to(torch.bfloat16) for k, v in tensors.items()}, str(d / "model.safetensors"))
    return str(d)


@pytest.mark.parametrize("quant,qt", [("q4", lib.Q4), ("q6", lib.Q6), ("q8", lib.Q8)])
def test_gguf_model_generates_like_direct_upload(ctx, orc, ckpt, quant, qt):
    dst = os.path.join(ckpt, f"model-{quant}.gguf")
    convert.convert(ckpt, dst, ckpt, quant)
    cfg = decoder_config(load_config_json(ckpt))
    assert cfg == MID
    print(f"gguf model {quant}", flush=True)
    gm = lib.Model.from_gguf(ctx, cfg, dst)
    w = synth.make_weights(MID, qt, seed=21, tie=lib.TIE_AMD64)
    dm = lib.Model(ctx, MID)
    dm.load_weights(w)
    om = orc.Model(MID)
    om.load_weights(w)
    ids = synth.prompt_ids(19, seed=40, high=MID.vocab)
    want = list(om.generate(ids, 12, eos=()))
    assert list(gm.seq(64).generate(ids, 12, eos=())) == want
    assert list(gm.seq(64).generate(ids, 12, eos=(), use_prefill=True)) == want
    assert list(dm.seq(64).generate(ids, 12, eos=())) == want
    # the same device logits for one step from either model
    emb = w["embed"][ids[0]]
    a = gm.seq(8).step(emb, (0, 0, 0))[1]
    b = dm.seq(8).step(emb, (0, 0, 0))[1]
    np.testing.assert_array_equal(a, b)
    gm.close()
    dm.close()


def test_gguf_model_rejections(ctx, ckpt, tmp_path):
    cfg = MID
    # F32 matrices are not a device format
    f32 = str(tmp_path / "f32.gguf")
    convert.convert(ckpt, f32, ckpt, "f32")
    with pytest.raises(lib.PocrError) as e:
        lib.Model.from_gguf(ctx, cfg, f32)
    assert e.value.code == lib.POCR_ERR_UNSUPPORTED
    # a configuration that disagrees with the tensors
    q4 = os.path.join(ckpt, "model-q4.gguf")
    if not os.path.exists(q4):
        convert.convert(ckpt, q4, ckpt, "q4")
    wrong = DecoderConfig(hidden=1024, inter=2048, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000)
    with pytest.raises(lib.PocrError):
        lib.Model.from_gguf(ctx, wrong, q4)
    # a missing tensor
    more = DecoderConfig(hidden=1024, inter=3072, layers=4, heads=16, kv_heads=2, head_dim=128, vocab=5000)
    with pytest.raises(lib.PocrError) as e:
        lib.Model.from_gguf(ctx, more, q4)
    assert "model.layers.3" in str(e.value)
    # the model still loads afterwards
    m = lib.Model.from_gguf(ctx, cfg, q4)
    m.close()


def test_projector_from_gguf(ctx, tmp_path):
    # the mlp_AR tensors stay F32 in a converted file; the projector built from
    # them equals the one built from the same arrays
    rng = np.random.default_rng(4)
    vd, td = 64, 1024
    K = 4 * vd
    t = {"mlp_AR.pre_norm.weight": 1 + 0.1 * rng.standard_normal(vd), "mlp_AR.pre_norm.bias": 0.1 * rng.standard_normal(vd),
         "mlp_AR.linear_1.weight": rng.standard_normal((K, K)) / np.sqrt(K), "mlp_AR.linear_1.bias": 0.1 * rng.standard_normal(K),
         "mlp_AR.linear_2.weight": rng.standard_normal((td, K)) / np.sqrt(K), "mlp_AR.linear_2.bias": 0.1 * rng.standard_normal(td)}
    t = {k: np.ascontiguousarray(v, np.float32) for k, v in t.items()}
    path = str(tmp_path / "vision.gguf")
    convert.write_gguf(path, [], [(k, convert.F32, v.shape, v.tobytes()) for k, v in sorted(t.items())])
    with lib.GgufFile(path) as g:
        pg = lib.Projector.from_gguf(ctx, g)
    pd = lib.Projector(ctx, t["mlp_AR.pre_norm.weight"], t["mlp_AR.pre_norm.bias"], t["mlp_AR.linear_1.weight"],
                       t["mlp_AR.linear_1.bias"], t["mlp_AR.linear_2.weight"], t["mlp_AR.linear_2.bias"])
    x = rng.standard_normal((2 * 4 * 6, vd)).astype(np.float32)
    np.testing.assert_array_equal(pg.project(x, (2, 4, 6)), pd.project(x, (2, 4, 6)))
    pg.close()
    pd.close()
