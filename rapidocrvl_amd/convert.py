"""Checkpoint conversion and GGUF writing.

``convert(src, dst, config_dir, quantization)`` turns a Hugging Face
safetensors checkpoint into the GGUF layout the reference writes
(ConvertSafetensorsWithOptions, internal/gguf/convert.go:42-198):

* tensors sorted by name, each payload at a 32-byte aligned offset from the
  aligned end of the header;
* with q8/q6/q4, the text decoder's matrices (isQuantizedTextTensor,
  convert.go:402-433: lm_head and model.layers.N.{self_attn.{q,k,v,o}_proj,
  mlp.{gate,up,down}_proj}.weight with the config's shapes) as Q8_ROW /
  Q6_ROW / Q4_ROW — f32 scales[rows] then the packed rows
  (writeQuantizedRows, convert.go:207-289) — encoded by the library's row
  encoders with the x86-64 converter's rounding (QuantizeQ*RowInto);
* every other tensor as F32 (BF16/F16 sources widened exactly);
* the metadata block of convert.go:302-332, the config keys only when a
  config.json was found (the reference ignores a failed config.Load and
  quantizes nothing then).

The source is resolved as safetensors.OpenModel does
(internal/safetensors/safetensors.go:48-64): a file, else
``model.safetensors`` in the directory, else its
``model.safetensors.index.json`` weight_map.  Tensors are read one at a time,
so a full checkpoint never sits in memory at once.

``write_gguf`` is the container writer (writeHeader, convert.go:436-488);
``pocr_gguf_open`` / ``pocr_model_load_gguf`` read the result.
"""
from __future__ import annotations

import json
import os
import re
import struct

import numpy as np

from . import lib
from .config import load_config_json

ALIGN = 32
VERSION = 3
F32, Q8_ROW, Q4_ROW, Q6_ROW = 0, 1000, 1001, 1002
META_U32, META_U64, META_STRING = 4, 10, 8
FILE_TYPE = {"f32": 0, "q8": 7, "q6": 6, "q4": 3}
QTYPE = {"q8": Q8_ROW, "q6": Q6_ROW, "q4": Q4_ROW}
_WS = " \n\r\t\v\f"


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def normalize_quantization(q: str) -> str:
    """normalizeQuantization (convert.go:342-348): ASCII-trimmed, lower-cased,
    empty → f32."""
    q = (q or "").strip(_WS)
    return q.translate(str.maketrans("ABCDEFGHIJKLMNOPQRSTUVWXYZ", "abcdefghijklmnopqrstuvwxyz")) if q else "f32"


def payload_bytes(typ: int, shape) -> int:
    """Bytes of one tensor's payload (TensorBytes, internal/gguf/gguf.go:586-629)."""
    if typ == F32:
        return int(np.prod(shape, dtype=np.int64)) * 4
    rows, cols = shape
    return rows * 4 + rows * lib.row_bytes(typ, cols)


def write_gguf(path: str, metadata, tensors, progress=None) -> None:
    """metadata: [(key, META_*, value)]; tensors: [(name, type, shape,
    payload)] in file order, payload being bytes or a callable returning them.
    Written to ``path + ".tmp"`` and renamed over ``path`` (replaceFile,
    convert.go:200-205)."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", VERSION, len(tensors), len(metadata)))
    for key, typ, val in metadata:
        head += _string(key) + struct.pack("<I", typ)
        if typ == META_U32:
            head += struct.pack("<I", val)
        elif typ == META_U64:
            head += struct.pack("<Q", val)
        elif typ == META_STRING:
            head += _string(val)
        else:
            raise ValueError(f"metadata type {typ}")
    off = 0
    offsets = []
    for name, typ, shape, payload in tensors:
        off = _align(off)
        offsets.append(off)
        head += _string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", typ, off)
        off += payload_bytes(typ, shape)
    tmp = path + ".tmp"
    try:
        with open(tmp, "wb") as f:
            f.write(head)
            base = _align(len(head))
            for i, ((name, typ, shape, payload), o) in enumerate(zip(tensors, offsets)):
                if progress:
                    progress(i, len(tensors), name, typ)
                f.write(b"\0" * (base + o - f.tell()))
                data = payload() if callable(payload) else payload
                if len(data) != payload_bytes(typ, shape):
                    raise ValueError(f"{name}: payload of {len(data)} bytes, want {payload_bytes(typ, shape)}")
                f.write(data)
            if base > f.tell():  # an empty tensor list still ends aligned
                f.write(b"\0" * (base - f.tell()))
        if progress:
            progress(len(tensors), len(tensors), "", None)
        if os.path.exists(path):
            os.remove(path)
        os.rename(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise


def quantized_text_tensor(name: str, shape, cfg) -> bool:
    """isQuantizedTextTensor (convert.go:402-433) over a loaded config.json."""
    if cfg is None or len(shape) != 2:
        return False
    H, hd = cfg.get("hidden_size", 0), cfg.get("head_dim", 0)
    if name == "lm_head.weight":
        return tuple(shape) == (cfg.get("vocab_size", 0), H)
    if not name.startswith("model.layers."):
        return False
    layer, dot, suffix = name[len("model.layers."):].partition(".")
    if not dot or not re.fullmatch(r"[+-]?[0-9]+", layer):  # strconv.Atoi's syntax
        return False
    li = int(layer)
    if li < 0 or li >= cfg.get("num_hidden_layers", 0):
        return False
    q, kv = cfg.get("num_attention_heads", 0) * hd, cfg.get("num_key_value_heads", 0) * hd
    inter = cfg.get("intermediate_size", 0)
    want = {"self_attn.q_proj.weight": (q, H), "self_attn.k_proj.weight": (kv, H),
            "self_attn.v_proj.weight": (kv, H), "self_attn.o_proj.weight": (H, q),
            "mlp.gate_proj.weight": (inter, H), "mlp.up_proj.weight": (inter, H),
            "mlp.down_proj.weight": (H, inter)}
    return want.get(suffix) == tuple(shape)


class _Source:
    """Tensor name → (file, shape) of a checkpoint, read lazily."""

    def __init__(self, src: str):
        from safetensors import safe_open

        if os.path.isfile(src):
            files = {name: src for name in self._names(safe_open, src)}
        elif os.path.isfile(os.path.join(src, "model.safetensors")):
            single = os.path.join(src, "model.safetensors")
            files = {name: single for name in self._names(safe_open, single)}
        elif os.path.isfile(os.path.join(src, "model.safetensors.index.json")):
            with open(os.path.join(src, "model.safetensors.index.json")) as f:
                wm = json.load(f).get("weight_map") or {}
            if not wm:
                raise ValueError(f"{src}: empty weight_map")
            files = {}
            for name, shard in wm.items():
                if not name or any(ord(c) < 0x20 or ord(c) == 0x7F for c in name):
                    raise ValueError(f"{src}: invalid tensor name {name!r}")
                if os.path.isabs(shard) or ".." in shard.replace("\\", "/").split("/"):
                    raise ValueError(f"{src}: shard path {shard!r} escapes the directory")
                files[name] = os.path.join(src, shard)
        else:
            raise FileNotFoundError(f"no model.safetensors or model.safetensors.index.json in {src}")
        self.files = files
        self.shards = len(set(files.values()))
        self._open = {}
        self._safe_open = safe_open

    @staticmethod
    def _names(safe_open, path):
        with safe_open(path, framework="pt") as f:
            return list(f.keys())

    def _handle(self, name):
        path = self.files[name]
        if path not in self._open:
            self._open[path] = self._safe_open(path, framework="pt").__enter__()
        return self._open[path]

    def shape(self, name):
        return tuple(self._handle(name).get_slice(name).get_shape())

    def f32(self, name) -> np.ndarray:
        t = self._handle(name).get_tensor(name)
        return np.ascontiguousarray(t.float().numpy(), np.float32)  # BF16/F16 → F32 exactly

    def close(self):
        for h in self._open.values():
            h.__exit__(None, None, None)
        self._open.clear()


def convert(src: str, dst: str, config_dir: str = ".", quantization: str = "", progress=None) -> None:
    """ConvertSafetensorsWithOptions (convert.go:42-198)."""
    quant = normalize_quantization(quantization)
    if quant not in FILE_TYPE:
        raise ValueError(f"unsupported quantization {quantization!r}")
    try:
        cfg = load_config_json(config_dir or ".")
    except (OSError, ValueError):
        cfg = None
    sf = _Source(src)
    try:
        entries = []
        n_q = 0
        for name in sorted(sf.files):
            shape = sf.shape(name)
            if quant != "f32" and quantized_text_tensor(name, shape, cfg):
                qt = QTYPE[quant]

                def payload(name=name, qt=qt):
                    scales, packed = lib.quantize_rows(qt, sf.f32(name), lib.TIE_AMD64)
                    return scales.tobytes() + packed.tobytes()

                entries.append((name, qt, shape, payload))
                n_q += 1
            else:
                entries.append((name, F32, shape, lambda name=name: sf.f32(name).tobytes()))
        meta = [("general.architecture", META_STRING, "paddleocrvl"),
                ("general.name", META_STRING, "PaddleOCR-VL-0.9B"),
                ("general.alignment", META_U32, ALIGN), ("general.file_type", META_U32, FILE_TYPE[quant]),
                ("paddleocrvl.gguf_version", META_U32, VERSION), ("paddleocrvl.quantization", META_STRING, quant),
                ("paddleocrvl.source_tensors", META_U64, len(entries)),
                ("paddleocrvl.source_shards", META_U64, sf.shards),
                ("paddleocrvl.f32_tensors", META_U64, len(entries) - n_q),
                ("paddleocrvl.quantized_tensors", META_U64, n_q)]
        if cfg is not None:
            meta += [("paddleocrvl.vocab_size", META_U64, cfg.get("vocab_size", 0)),
                     ("paddleocrvl.text_layers", META_U64, cfg.get("num_hidden_layers", 0)),
                     ("paddleocrvl.hidden_size", META_U64, cfg.get("hidden_size", 0)),
                     ("paddleocrvl.vision_layers", META_U64,
                      (cfg.get("vision_config") or {}).get("num_hidden_layers", 0))]
        write_gguf(dst, meta, entries, progress)
    finally:
        sf.close()
