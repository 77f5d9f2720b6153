"""Reader for the MMFREE1 weight blob (the reference's model.mmfree).

Layout (cpp/src/io/weights.cpp:3-8 and 191-254; written by tools/provision.py:126-163):
``b"MMFREE1\\n"`` | u64 little-endian header length | JSON header | zero padding to 64 |
data section. The header is ``{"config": {...}, "tensors": {name: {dtype, shape, offset,
nbytes}}}`` with offsets relative to the data section. Unlike the reference loader, this
one validates every offset and size against the file.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"MMFREE1\n"
ALIGN = 64

#: The six ternary projections of a layer, in blob order (tools/provision.py:38-45).
LAYER_PROJS = ("i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj")


@dataclass
class Config:
    """HGRNBitConfig fields the engine reads (cpp/include/mmfree/config.hpp:8-21)."""

    vocab_size: int = 32000
    hidden_size: int = 1024
    num_hidden_layers: int = 24
    num_heads: int = 1
    expand_ratio: int = 1
    intermediate_size: int = 2816
    use_lower_bound: bool = True
    use_short_conv: bool = False
    rms_norm_eps: float = 1e-6


@dataclass
class Blob:
    path: str
    config: Config
    tensors: dict = field(default_factory=dict)  # name -> np.ndarray (read-only memmap)

    def get(self, name: str) -> np.ndarray:
        if name not in self.tensors:
            raise KeyError(f"weights: missing tensor {name}")
        return self.tensors[name]

    def proj(self, tag: str):
        """(wq int8 [N, K], scale_w float, normw float32 [K]) of a BitLinear projection."""
        return (self.get(tag + ".wq"), float(self.get(tag + ".scale_w")[0]),
                self.get(tag + ".normw"))


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


def read_blob(path: str) -> Blob:
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(16)
        if len(head) < 16 or head[:8] != MAGIC:
            raise ValueError(f"weights: bad magic in {path}")
        (hl,) = struct.unpack("<Q", head[8:16])
        if 16 + hl > size:
            raise ValueError(f"weights: header length {hl} exceeds file size {size}")
        header = json.loads(f.read(hl).decode("utf-8"))
    cfg_j = header.get("config")
    if cfg_j is None:
        raise ValueError("weights: no config in header")
    cfg = Config()
    for k in ("vocab_size", "hidden_size", "num_hidden_layers", "num_heads", "expand_ratio",
              "intermediate_size"):
        if k in cfg_j:
            setattr(cfg, k, int(cfg_j[k]))
    for k in ("use_lower_bound", "use_short_conv"):
        if k in cfg_j:
            setattr(cfg, k, bool(cfg_j[k]))
    if "rms_norm_eps" in cfg_j:
        cfg.rms_norm_eps = float(cfg_j["rms_norm_eps"])
    ts = header.get("tensors")
    if not isinstance(ts, dict):
        raise ValueError("weights: no tensors in header")
    data_start = _align(16 + hl)
    blob = Blob(path, cfg)
    for name, meta in ts.items():
        dt = {"f32": np.float32, "i8": np.int8}.get(meta.get("dtype"))
        if dt is None:
            raise ValueError(f"weights: tensor {name} has unknown dtype {meta.get('dtype')!r}")
        shape = tuple(int(s) for s in meta["shape"])
        numel = int(np.prod(shape)) if shape else 0
        nbytes = numel * np.dtype(dt).itemsize
        off = data_start + int(meta["offset"])
        if int(meta.get("nbytes", nbytes)) != nbytes or off + nbytes > size:
            raise ValueError(f"weights: tensor {name} ({shape}, {meta.get('dtype')}) does not fit "
                             f"the file at offset {meta['offset']}")
        blob.tensors[name] = np.memmap(path, dtype=dt, mode="r", offset=off, shape=shape)
    return blob
