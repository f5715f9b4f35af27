"""SafeTensors reader over memory maps (``src/pretrained/safetensors.clj``).

A file is an 8-byte little-endian header length, a JSON header mapping each
tensor name to ``{"dtype", "shape", "data_offsets": [begin, end]}`` (offsets
relative to the end of the header; ``"__metadata__"`` is skipped), then the
tensor bytes.  ``tensor_view`` returns the stored elements as a zero-copy view
of the mapped file -- what ``rstr_model_bind_raw`` uploads and widens on the
device -- and ``read_tensor`` / ``load_safetensors`` the f32 conversion of
``read-tensor-floats`` (safetensors.clj:39-78) for host-side use and checks.
"""
from __future__ import annotations

import json
import struct

import numpy as np

# stored element type of each SafeTensors dtype (BF16 kept as its bit patterns)
STORED = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64, "I32": np.int32,
          "I16": np.int16, "I8": np.int8, "U8": np.uint8}


class SafetensorsError(ValueError):
    pass


def read_header(path: str):
    """safetensors.clj:24-37: (header dict, absolute data offset)."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise SafetensorsError(f"truncated SafeTensors file: {path}")
        (n,) = struct.unpack("<Q", raw)
        body = f.read(n)
        if len(body) != n:
            raise SafetensorsError(f"truncated SafeTensors header: {path}")
    return json.loads(body.decode("utf-8")), 8 + n


def load_safetensors_lazy(path: str) -> dict:
    """safetensors.clj:107-130: header only, ``{"path", "data-offset", "tensors":
    {name: {"dtype", "shape", "offset", "end-offset"}}}``."""
    header, data_offset = read_header(path)
    tensors = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        b, e = info["data_offsets"]
        tensors[name] = {"dtype": info["dtype"], "shape": [int(x) for x in info["shape"]],
                         "offset": int(b), "end-offset": int(e)}
    return {"path": path, "data-offset": data_offset, "tensors": tensors, "_map": None}


def _map(lazy: dict) -> np.memmap:
    if lazy.get("_map") is None:
        lazy["_map"] = np.memmap(lazy["path"], dtype=np.uint8, mode="r")
    return lazy["_map"]


def tensor_view(lazy: dict, name: str) -> np.ndarray:
    """The stored elements of one tensor, shaped, as a read-only view of the map."""
    info = lazy["tensors"].get(name)
    if info is None:
        raise SafetensorsError(f"Tensor not found: {name}")
    st = STORED.get(info["dtype"])
    if st is None:
        raise SafetensorsError(f"Unsupported dtype: {info['dtype']}")
    numel = int(np.prod(info["shape"], dtype=np.int64))
    b = lazy["data-offset"] + info["offset"]
    e = lazy["data-offset"] + info["end-offset"]
    if e - b != numel * np.dtype(st).itemsize:
        raise SafetensorsError(f"tensor {name}: {e - b} bytes for {numel} {info['dtype']} elements")
    return _map(lazy)[b:e].view(st).reshape(info["shape"])


def to_f32(stored: np.ndarray, dtype: str) -> np.ndarray:
    """read-tensor-floats (safetensors.clj:39-78): F16 exact, BF16 as the upper
    16 bits of an f32, integers converted."""
    if dtype == "BF16":
        return (np.asarray(stored, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(stored).astype(np.float32)


def read_tensor(lazy: dict, name: str) -> dict:
    """safetensors.clj:132-152."""
    info = lazy["tensors"].get(name)
    if info is None:
        raise SafetensorsError(f"Tensor not found: {name}")
    return {"dtype": info["dtype"], "shape": info["shape"], "data": to_f32(tensor_view(lazy, name), info["dtype"])}


def load_safetensors(path: str) -> dict:
    """safetensors.clj:80-105: every tensor converted to f32."""
    lazy = load_safetensors_lazy(path)
    return {n: read_tensor(lazy, n) for n in lazy["tensors"]}
