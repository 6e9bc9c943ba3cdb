"""Drafter bundle: a flat little-endian file of named arrays plus a JSON header.

Format (``drafting/export_drafter.py:12-31`` of the reference, kept byte-compatible so bundles
exported there load here): magic ``MRBDRFT1``, uint64 header length, UTF-8 JSON header
``{"version", "config", "arrays": {name: {dtype, shape, offset, nbytes}}, "source"}``, then
each array at a 64-byte aligned absolute offset.  ``config`` holds the keys of
``bundle_config`` (``export_drafter.py:212-215``).

bf16 arrays, which numpy has no dtype for, are stored with dtype string ``"bf16"`` as raw
16-bit words and come back as ``torch.bfloat16`` tensors.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

MAGIC = b"MRBDRFT1"
VERSION = 1
ALIGN = 64


def _align(x: int) -> int:
    return -(-x // ALIGN) * ALIGN


@dataclass
class Bundle:
    config: dict
    arrays: dict                       # name -> numpy array (memory-mapped when loaded) or torch tensor
    source: dict = field(default_factory=dict)

    def tensors(self, names=None) -> dict:
        """torch views of the arrays (sketch uint16/uint32 arrays as int32, bf16 words as bfloat16)."""
        out = {}
        for k, a in self.arrays.items():
            if names is not None and k not in names:
                continue
            if isinstance(a, torch.Tensor):
                out[k] = a
                continue
            if a.dtype in (np.uint16, np.uint32):
                a = np.minimum(a.astype(np.int64), np.iinfo(np.int32).max).astype(np.int32)
            out[k] = torch.from_numpy(np.array(a, copy=True))
        return out


def bundle_config(**kw) -> dict:
    """Config dict with the derived keys (``groups``, ``route_token_dim``)."""
    kw["groups"] = kw["q_heads"] // kw["kv_heads"]
    kw["route_token_dim"] = len(kw["ngrams"]) * kw["mem_dim"]
    return kw


def _as_numpy(v) -> tuple[np.ndarray, str]:
    if isinstance(v, torch.Tensor):
        v = v.detach().cpu()
        if v.dtype == torch.bfloat16:
            return v.contiguous().view(torch.int16).numpy().view(np.uint16), "bf16"
        v = v.numpy()
    a = np.ascontiguousarray(v)
    return a, a.dtype.str


def write_bundle(path: str | Path, config: dict, arrays: dict, source: dict | None = None) -> Path:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    data = {k: _as_numpy(v) for k, v in arrays.items()}
    meta = {k: {"dtype": dt, "shape": list(a.shape), "offset": 0, "nbytes": int(a.nbytes)} for k, (a, dt) in data.items()}
    while True:  # offsets depend on the header length, which depends on the offsets
        header = json.dumps({"version": VERSION, "config": config, "arrays": meta, "source": source or {}},
                            sort_keys=True).encode("utf-8")
        off = _align(16 + len(header) + 256)
        new = {}
        for k, (a, _) in data.items():
            new[k] = dict(meta[k], offset=off)
            off = _align(off + a.nbytes)
        if new == meta:
            break
        meta = new
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<Q", len(header)))
        f.write(header)
        for k, (a, _) in data.items():
            f.write(b"\0" * (meta[k]["offset"] - f.tell()))
            a.astype(a.dtype.newbyteorder("<"), copy=False).tofile(f)
    return path


def read_header(path: str | Path) -> dict:
    with open(path, "rb") as f:
        if f.read(8) != MAGIC:
            raise ValueError(f"{path}: not a drafter bundle")
        (n,) = struct.unpack("<Q", f.read(8))
        return json.loads(f.read(n).decode("utf-8"))


def load_bundle(path: str | Path, mmap: bool = True) -> Bundle:
    head = read_header(path)
    if head["version"] != VERSION:
        raise ValueError(f"bundle version {head['version']} != {VERSION}")
    arrays = {}
    for k, m in head["arrays"].items():
        bf16 = m["dtype"] == "bf16"
        dt = np.dtype(np.uint16) if bf16 else np.dtype(m["dtype"])
        shape = tuple(m["shape"])
        if mmap and m["nbytes"]:
            a = np.memmap(path, dtype=dt, mode="r", offset=m["offset"], shape=shape)
        else:
            with open(path, "rb") as f:
                f.seek(m["offset"])
                a = np.frombuffer(f.read(m["nbytes"]), dtype=dt).reshape(shape).copy()
        if bf16:
            a = torch.from_numpy(np.array(a).view(np.int16)).view(torch.bfloat16)
        arrays[k] = a
    return Bundle(head["config"], arrays, head.get("source", {}))
