"""GGUF reader (pocr_gguf_*) and the safetensors → GGUF converter, host only.

The rejection cases are those of internal/gguf/gguf_test.go:12-172; the
converter cases those of internal/gguf/convert_test.go:15-403, with the
reference's own tolerances and value tables.
"""
import json
import math
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from rapidocrvl_amd import convert, lib, synth
from rapidocrvl_amd.config import DecoderConfig, decoder_config, load_config_json

MAX_COUNT = 1 << 20
MAX_STRING = 16 << 20
U64_MAX = (1 << 64) - 1
I64_MAX = (1 << 63) - 1


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _head(nt, nkv, version=3, magic=b"GGUF"):
    return magic + struct.pack("<IQQ", version, nt, nkv)


def _tensor_info(name, dims, typ, offset):
    return _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", typ, offset)


def _with_data(head: bytes, data: bytes) -> bytes:
    pad = (-len(head)) % 32
    return head + b"\0" * pad + data


def _write(tmp_path, name, raw):
    p = tmp_path / name
    p.write_bytes(raw)
    return str(p)


def _rejects(path, needle=None):
    with pytest.raises(lib.PocrError) as e:
        lib.GgufFile(path)
    assert e.value.code == lib.POCR_ERR_ARG
    if needle:
        assert needle in str(e.value)


# ---- reader: the reference's rejection tests --------------------------------

@pytest.mark.parametrize("nt,nkv", [(MAX_COUNT + 1, 0), (0, MAX_COUNT + 1)])
def test_open_rejects_huge_counts(tmp_path, nt, nkv):
    _rejects(_write(tmp_path, "c.gguf", _head(nt, nkv)), "count too large")


def test_open_rejects_huge_string(tmp_path):
    raw = _head(0, 1) + struct.pack("<Q", MAX_STRING + 1)
    _rejects(_write(tmp_path, "s.gguf", raw), "string too large")


@pytest.mark.parametrize("meta", [
    [("", 4, struct.pack("<I", 1))],
    [("general.alignment", 4, struct.pack("<I", 32)), ("general.alignment", 4, struct.pack("<I", 16))],
    [("general\nname", 8, _s("bad"))],
    [("general.x\x7f", 10, struct.pack("<Q", 1))],
], ids=["empty-key", "duplicate-key", "control-character-key", "delete-character-key"])
def test_open_rejects_invalid_metadata_keys(tmp_path, meta):
    head = _head(0, len(meta)) + b"".join(_s(k) + struct.pack("<I", t) + v for k, t, v in meta)
    _rejects(_write(tmp_path, "m.gguf", _with_data(head, b"")))


@pytest.mark.parametrize("dims,typ,offset,data", [
    ([1] * 9, 0, 0, b""),
    ([U64_MAX], 0, 0, b""),
    ([1], 0xFFFFFFFF, 0, bytes(4)),
    ([1], 0, 8, bytes(4)),
    ([2], 0, 0, bytes(4)),
    ([I64_MAX, 2], 0, 0, bytes(4)),  # TensorBytes overflow (gguf_test.go:169-172)
    ([2, I64_MAX], lib.Q4, 0, bytes(4)),
    ([2, I64_MAX - 3], lib.Q8, 0, bytes(4)),
    ([2, (I64_MAX - 7) // 6 + 1], lib.Q6, 0, bytes(4)),
    ([4], lib.Q8, 0, bytes(64)),  # a Q*_ROW tensor must be 2-D
    ([0], 0, 0, b""),  # zero bytes is an invalid size
    ([1], 0, 1 << 63, bytes(4)),
    ([1], 0, I64_MAX, bytes(4)),  # data start + offset would overflow int64
    ([1], 0, I64_MAX - 16, bytes(4)),
    ([1], 0, U64_MAX, bytes(4)),
], ids=["too-many-dims", "negative-dim-after-cast", "unknown-type", "offset-exceeds-file", "tensor-exceeds-file",
        "f32-bytes-overflow", "q4-cols-overflow", "q8-cols-overflow", "q6-cols-overflow", "q8-1d", "empty",
        "offset-too-large", "offset-int64-max", "offset-near-int64-max", "offset-u64-max"])
def test_open_rejects_invalid_tensor_metadata(tmp_path, dims, typ, offset, data):
    head = _head(1, 0) + _tensor_info("x.weight", dims, typ, offset)
    _rejects(_write(tmp_path, "t.gguf", _with_data(head, data)))


@pytest.mark.parametrize("tensors", [
    [("", [1], 0, 0)],
    [("x.weight", [1], 0, 0), ("x.weight", [1], 0, 4)],
    [("x\nweight", [1], 0, 0)],
], ids=["empty-name", "duplicate-name", "control-character-name"])
def test_open_rejects_invalid_tensor_names(tmp_path, tensors):
    head = _head(len(tensors), 0) + b"".join(_tensor_info(*t) for t in tensors)
    _rejects(_write(tmp_path, "n.gguf", _with_data(head, bytes(8))))


@pytest.mark.parametrize("raw,needle", [
    (b"GGUX" + bytes(20), "bad magic"),
    (_head(0, 0, version=2), "unsupported version"),
    (_head(0, 1) + _s("k") + struct.pack("<I", 6) + bytes(8), "unsupported metadata type"),
    (_head(1, 0) + _s("x"), "truncated"),
    (b"GG", "bad magic"),
])
def test_open_rejects_malformed_headers(tmp_path, raw, needle):
    _rejects(_write(tmp_path, "h.gguf", raw), needle)


def test_open_missing_file(tmp_path):
    _rejects(str(tmp_path / "absent.gguf"), "open")


# ---- reader/writer round trip -----------------------------------------------

def test_write_read_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    q4 = lib.QMatrix.quantize(rng.standard_normal((6, 33)), lib.Q4)
    q6 = lib.QMatrix.quantize(rng.standard_normal((2, 17)), lib.Q6)
    q8 = lib.QMatrix.quantize(rng.standard_normal((4, 9)), lib.Q8)
    meta = [("general.architecture", convert.META_STRING, "paddleocrvl"), ("n.u32", convert.META_U32, 7),
            ("n.u64", convert.META_U64, 1 << 40), ("empty", convert.META_STRING, "")]
    qm = lambda q: q.scales.tobytes() + q.packed.tobytes()  # noqa: E731
    tensors = [("a", convert.F32, a.shape, a.tobytes()), ("b", convert.F32, b.shape, b.tobytes()),
               ("q4", lib.Q4, (6, 33), qm(q4)), ("q6", lib.Q6, (2, 17), qm(q6)), ("q8", lib.Q8, (4, 9), qm(q8)),
               ("scalar", convert.F32, (), np.float32(2.5).tobytes())]
    path = str(tmp_path / "rt.gguf")
    convert.write_gguf(path, meta, tensors)
    with lib.GgufFile(path) as g:
        assert g.metadata == {"general.architecture": "paddleocrvl", "n.u32": 7, "n.u64": 1 << 40, "empty": ""}
        assert list(g.tensors) == ["a", "b", "q4", "q6", "q8", "scalar"]
        np.testing.assert_array_equal(g.float32("a"), a)
        np.testing.assert_array_equal(g.float32("b"), b)
        assert g.float32("scalar").item() == 2.5
        for name, q in (("q4", q4), ("q6", q6), ("q8", q8)):
            got = g.qrows(name)
            assert (got.qtype, got.rows, got.cols) == (q.qtype, q.rows, q.cols)
            np.testing.assert_array_equal(got.scales, q.scales)
            np.testing.assert_array_equal(got.packed, q.packed)
        assert g.tensors["q4"] == (lib.Q4, (6, 33), 6 * 4 + 6 * 17)
        assert g.tensors["q6"][2] == 2 * 4 + 2 * 13
        with pytest.raises(ValueError):
            g.float32("q4")
        with pytest.raises(ValueError):
            g.qrows("a")
        with pytest.raises(lib.PocrError):  # the reader hands out whole payloads only
            lib.check(lib.load().pocr_gguf_read(g.h, 0, lib._ptr(np.empty(64, np.uint8)), 8))
        with pytest.raises(lib.PocrError):
            lib.check(lib.load().pocr_gguf_find(g.h, b"missing"))
    raw = open(path, "rb").read()
    assert raw[:4] == b"GGUF" and struct.unpack_from("<IQQ", raw, 4) == (3, 6, 4)
    # each payload starts 32-byte aligned in the file
    for _, _, _, payload in tensors:
        assert raw.index(payload) % 32 == 0


def test_empty_file_list_is_aligned(tmp_path):
    path = str(tmp_path / "e.gguf")
    convert.write_gguf(path, [("k", convert.META_U32, 1)], [])
    assert os.path.getsize(path) % 32 == 0
    with lib.GgufFile(path) as g:
        assert g.tensors == {} and g.metadata == {"k": 1}


# ---- converter: the reference's tests ---------------------------------------

SMALL_CFG = {"vocab_size": 2, "hidden_size": 3, "intermediate_size": 4, "num_hidden_layers": 0,
             "num_attention_heads": 1, "num_key_value_heads": 1, "head_dim": 3,
             "vision_config": {"num_hidden_layers": 0}}
VALUES = np.array([1, -2, 3, 0.5, 0.25, -0.75], np.float32)


def _dir(tmp_path, cfg):
    if cfg is not None:
        (tmp_path / "config.json").write_text(json.dumps(cfg))
    return str(tmp_path)


def _st(path, tensors):
    save_file({k: torch.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v
               for k, v in tensors.items()}, path)


def _unpack(q: lib.QMatrix):
    return lib.unpack_rows(q.qtype, q.packed, q.cols).astype(np.float32) * q.scales[:, None]


@pytest.mark.parametrize("quant,qt,tol,nbytes", [("q8", lib.Q8, 0.03, 6), ("q4", lib.Q4, 0.25, 4),
                                                  ("q6", lib.Q6, 0.08, 6)])
def test_convert_quantized_round_trip(tmp_path, quant, qt, tol, nbytes):
    d = _dir(tmp_path, SMALL_CFG)
    src = os.path.join(d, "model.safetensors")
    _st(src, {"lm_head.weight": VALUES.reshape(2, 3)})
    dst = os.path.join(d, f"model-{quant}.gguf")
    convert.convert(src, dst, d, quant)
    with lib.GgufFile(dst) as g:
        q = g.qrows("lm_head.weight")
        assert q.qtype == qt and q.packed.size == nbytes and q.scales.size == 2 and (q.rows, q.cols) == (2, 3)
        assert g.metadata["paddleocrvl.quantized_tensors"] == 1
        assert g.metadata["paddleocrvl.f32_tensors"] == 0
        assert g.metadata["general.file_type"] == {"q8": 7, "q4": 3, "q6": 6}[quant]
        assert g.metadata["paddleocrvl.quantization"] == quant
        assert g.metadata["paddleocrvl.vocab_size"] == 2 and g.metadata["paddleocrvl.hidden_size"] == 3
        np.testing.assert_allclose(_unpack(q).ravel(), VALUES, atol=tol)
        # the converter's encoder is the x86-64 one (QuantizeQ*RowInto)
        ref = lib.QMatrix.quantize(VALUES.reshape(2, 3), qt, lib.TIE_AMD64)
        np.testing.assert_array_equal(q.packed, ref.packed)
        np.testing.assert_array_equal(q.scales, ref.scales)


def test_convert_q4_nibble_layout(tmp_path):
    # convert_test.go:339-352 reads the Q4 rows by hand: low nibble for even
    # columns, high nibble for odd ones, value (nibble-8)·scale
    d = _dir(tmp_path, SMALL_CFG)
    src = os.path.join(d, "model.safetensors")
    _st(src, {"lm_head.weight": VALUES.reshape(2, 3)})
    dst = os.path.join(d, "m.gguf")
    convert.convert(src, dst, d, "q4")
    with lib.GgufFile(dst) as g:
        q = g.qrows("lm_head.weight")
    data = q.packed.ravel()
    for i, want in enumerate(VALUES):
        col, row = i % 3, i // 3
        p = data[row * 2 + col // 2]
        nib = (p >> 4) if col & 1 else (p & 0x0F)
        assert abs((int(nib) - 8) * q.scales[row] - want) <= 0.25


def test_convert_q6_bit_layout(tmp_path):
    # convert_test.go:386-400: 6-bit codes packed LSB first, value (code-32)·scale
    d = _dir(tmp_path, SMALL_CFG)
    src = os.path.join(d, "model.safetensors")
    _st(src, {"lm_head.weight": VALUES.reshape(2, 3)})
    dst = os.path.join(d, "m.gguf")
    convert.convert(src, dst, d, "q6")
    with lib.GgufFile(dst) as g:
        q = g.qrows("lm_head.weight")
    data = q.packed.ravel()
    for i, want in enumerate(VALUES):
        col, row = i % 3, i // 3
        bit = col * 6
        idx = row * 3 + bit // 8
        x = int(data[idx])
        if idx + 1 < (row + 1) * 3:
            x |= int(data[idx + 1]) << 8
        code = (x >> (bit % 8)) & 0x3F
        assert abs((code - 32) * q.scales[row] - want) <= 0.08


def test_convert_f32_round_trip(tmp_path):
    d = _dir(tmp_path, {"vision_config": {}})
    src = os.path.join(d, "model.safetensors")
    vals = np.array([1, -2, 3, 0.5], np.float32)
    _st(src, {"x.weight": vals.reshape(2, 2)})
    dst = os.path.join(d, "model.gguf")
    seen = []
    convert.convert(src, dst, d, progress=lambda done, total, name, typ: seen.append((done, total)))
    assert seen[-1] == (1, 1)
    with lib.GgufFile(dst) as g:
        assert g.metadata["paddleocrvl.quantization"] == "f32"
        assert g.metadata["paddleocrvl.source_tensors"] == 1
        assert g.metadata["paddleocrvl.f32_tensors"] == 1
        assert g.metadata["paddleocrvl.quantized_tensors"] == 0
        got = g.float32("x.weight")
        assert got.shape == (2, 2)
        np.testing.assert_array_equal(got.ravel(), vals)


def test_convert_bf16_widens_exactly(tmp_path):
    d = _dir(tmp_path, {"vision_config": {}})
    vals = (np.arange(256 * 1024 + 5) % 251 - 125).astype(np.float32) / 8
    src = os.path.join(d, "model.safetensors")
    save_file({"x.weight": torch.from_numpy(vals.reshape(1, -1)).to(torch.bfloat16)}, src)
    dst = os.path.join(d, "model.gguf")
    convert.convert(src, dst, d)
    with lib.GgufFile(dst) as g:
        got = g.float32("x.weight")
    assert got.shape == (1, vals.size)
    for idx in (0, 1024, vals.size - 1):
        want = np.array([vals[idx]], np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
        assert got[0, idx] == want.view(np.float32)[0]


def test_convert_sharded_index(tmp_path):
    d = _dir(tmp_path, {"vision_config": {}})
    _st(os.path.join(d, "a.safetensors"), {"a.weight": np.array([7], np.float32)})
    _st(os.path.join(d, "b.safetensors"), {"b.weight": np.array([9], np.float32)})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"a.weight": "a.safetensors", "b.weight": "b.safetensors"}}, f)
    dst = os.path.join(d, "model.gguf")
    convert.convert(d, dst, d)
    with lib.GgufFile(dst) as g:
        assert g.float32("b.weight").tolist() == [9.0]
        assert g.metadata["paddleocrvl.source_shards"] == 2


def test_convert_rejects_escaping_shard(tmp_path):
    d = _dir(tmp_path, {"vision_config": {}})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"x.weight": "../x.safetensors"}}, f)
    with pytest.raises(ValueError):
        convert.convert(d, os.path.join(d, "m.gguf"), d)


def test_convert_without_config_quantizes_nothing(tmp_path):
    # config.Load failing leaves cfg nil: nothing is quantized and the config
    # keys are left out (convert.go:57, 323-330, 403)
    src = str(tmp_path / "w.safetensors")
    _st(src, {"lm_head.weight": VALUES.reshape(2, 3)})
    dst = str(tmp_path / "m.gguf")
    convert.convert(src, dst, str(tmp_path / "nowhere"), "q8")
    with lib.GgufFile(dst) as g:
        assert g.tensors["lm_head.weight"][0] == convert.F32
        assert "paddleocrvl.vocab_size" not in g.metadata
        assert g.metadata["paddleocrvl.quantization"] == "q8"


@pytest.mark.parametrize("inp,want", [("", "f32"), (" F32 ", "f32"), (" Q8 ", "q8"), ("\tQ4\n", "q4")])
def test_normalize_quantization(inp, want):
    assert convert.normalize_quantization(inp) == want


def test_unsupported_quantization(tmp_path):
    with pytest.raises(ValueError):
        convert.convert(str(tmp_path), str(tmp_path / "x.gguf"), str(tmp_path), "q5")


@pytest.mark.parametrize("name,shape,want", [
    ("lm_head.weight", (16, 8), True),
    ("model.layers.0.self_attn.q_proj.weight", (8, 8), True),
    ("model.layers.1.self_attn.k_proj.weight", (4, 8), True),
    ("model.layers.1.self_attn.v_proj.weight", (4, 8), True),
    ("model.layers.1.self_attn.o_proj.weight", (8, 8), True),
    ("model.layers.1.mlp.gate_proj.weight", (32, 8), True),
    ("model.layers.1.mlp.up_proj.weight", (32, 8), True),
    ("model.layers.1.mlp.down_proj.weight", (8, 32), True),
    ("model.layers.2.self_attn.q_proj.weight", (8, 8), False),
    ("model.layers.x.self_attn.q_proj.weight", (8, 8), False),
    ("model.layers.0.self_attn.q_proj.bias", (8,), False),
    ("model.layers.0.self_attn.q_proj.weight", (4, 8), False),
    ("model.layers.+1.mlp.up_proj.weight", (32, 8), True),   # strconv.Atoi takes a sign
    ("model.layers.-1.mlp.up_proj.weight", (32, 8), False),
    ("model.layers.0", (8, 8), False),
    ("model.embed_tokens.weight", (16, 8), False),
])
def test_is_quantized_text_tensor(name, shape, want):
    cfg = {"vocab_size": 16, "hidden_size": 8, "intermediate_size": 32, "num_hidden_layers": 2,
           "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 4}
    assert convert.quantized_text_tensor(name, shape, cfg) is want


def test_replace_overwrites_existing(tmp_path):
    dst = str(tmp_path / "m.gguf")
    open(dst, "w").write("old")
    convert.write_gguf(dst, [], [("x", convert.F32, (1,), np.float32(3).tobytes())])
    assert not os.path.exists(dst + ".tmp")
    with lib.GgufFile(dst) as g:
        assert g.float32("x").tolist() == [3.0]


def test_config_loader_defaults(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 64, "num_attention_heads": 4,
                                                      "intermediate_size": 128, "num_hidden_layers": 2,
                                                      "vocab_size": 10}))
    c = load_config_json(str(tmp_path))
    assert (c["head_dim"], c["num_key_value_heads"], c["rope_theta"], c["rms_norm_eps"]) == (16, 4, 10000.0, 1e-6)
    dc = decoder_config(c)
    assert dc.mrope_section == (16, 24, 24) and dc.kv_heads == 4
    (tmp_path / "config.json").write_text('{"hidden_size": 1, "hidden_size": 2}')
    with pytest.raises(ValueError):
        load_config_json(str(tmp_path))


def test_synthetic_checkpoint_converts_to_the_same_weights(tmp_path):
    # a checkpoint of make_checkpoint converted at q4 holds exactly the
    # matrices make_weights(TIE_AMD64) builds from the same seeds
    cfg = DecoderConfig(hidden=64, inter=128, layers=2, heads=4, kv_heads=2, head_dim=16, vocab=96)
    d = _dir(tmp_path, synth.config_json(cfg))
    ck = synth.make_checkpoint(cfg, seed=3)
    save_file({k: torch.from_numpy(v).to(torch.bfloat16) for k, v in ck.items()}, os.path.join(d, "model.safetensors"))
    dst = os.path.join(d, "model-q4.gguf")
    convert.convert(d, dst, d, "q4")
    w = synth.make_weights(cfg, lib.Q4, seed=3, tie=lib.TIE_AMD64)
    roles = dict(zip(synth.ROLES, ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                                   "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")))
    with lib.GgufFile(d + "/model-q4.gguf") as g:
        assert g.metadata["paddleocrvl.quantized_tensors"] == 1 + 7 * cfg.layers
        assert g.metadata["paddleocrvl.text_layers"] == cfg.layers
        for li, lw in enumerate(w["layers"]):
            for role, name in roles.items():
                q = g.qrows(f"model.layers.{li}.{name}.weight")
                np.testing.assert_array_equal(q.scales, lw[role][1])
                np.testing.assert_array_equal(q.packed, lw[role][2])
            np.testing.assert_array_equal(g.float32(f"model.layers.{li}.input_layernorm.weight"), lw["ln1"])
        np.testing.assert_array_equal(g.qrows("lm_head.weight").packed, w["lm_head"][2])
        np.testing.assert_array_equal(g.float32("model.embed_tokens.weight"), w["embed"])
        np.testing.assert_array_equal(g.float32("model.norm.weight"), w["final_norm"])
        assert not math.isnan(float(g.float32("model.norm.weight").sum()))
