"""Safetensors files without torch: the header (8-byte little-endian length, JSON) and memory-mapped tensor bytes.

BF16 and F8_E4M3 have no numpy dtype; they come back as ``uint16`` / ``uint8`` arrays with the stored dtype string
kept beside them, which is what the format classes take. The role is the reference's ``formats/safetensors_reader.py``
(checkpoint input of the packer); the code is this backend's own.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterable, List, Mapping, Optional, Tuple

import numpy as np

NP_DTYPES = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "F8_E4M3": np.uint8,
             "U8": np.uint8, "I8": np.int8, "I16": np.int16, "I32": np.int32, "I64": np.int64, "U32": np.uint32,
             "BOOL": np.bool_}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: Tuple[int, ...]
    begin: int            # absolute byte offsets in the file
    end: int
    path: Path


def read_header(path) -> Tuple[Dict[str, TensorInfo], Dict[str, str]]:
    p = Path(path)
    with open(p, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen))
    meta = header.pop("__metadata__", None) or {}
    out = {}
    for name, v in header.items():
        b, e = v["data_offsets"]
        if v["dtype"] not in NP_DTYPES:
            raise ValueError(f"{p.name}: tensor {name} has unsupported dtype {v['dtype']}")
        info = TensorInfo(name, v["dtype"], tuple(int(x) for x in v["shape"]), 8 + hlen + b, 8 + hlen + e, p)
        if info.end - info.begin != int(np.prod(info.shape, dtype=np.int64)) * np.dtype(NP_DTYPES[info.dtype]).itemsize:
            raise ValueError(f"{p.name}: tensor {name}: {info.end - info.begin} bytes for {info.dtype} {info.shape}")
        out[name] = info
    return out, meta


class Checkpoint:
    """The tensors of one safetensors file, every shard of a directory (``model.safetensors.index.json``), or all
    ``*.safetensors`` in it. ``get`` memory-maps (no copy until the caller makes one)."""

    def __init__(self, path) -> None:
        p = Path(path)
        if p.is_file():
            files = [p]
        elif (p / "model.safetensors.index.json").exists():
            with open(p / "model.safetensors.index.json") as f:
                files = sorted({p / fn for fn in json.load(f)["weight_map"].values()})
        else:
            files = sorted(p.glob("*.safetensors"))
        if not files:
            raise FileNotFoundError(f"no safetensors under {p}")
        self.tensors: Dict[str, TensorInfo] = {}
        self.metadata: Dict[str, str] = {}
        for fp in files:
            infos, meta = read_header(fp)
            dup = set(infos) & set(self.tensors)
            if dup:
                raise ValueError(f"{fp.name}: tensors also in another shard: {sorted(dup)[:3]}")
            self.tensors.update(infos)
            self.metadata.update(meta)
        self._maps: Dict[Path, np.memmap] = {}

    def names(self) -> List[str]:
        return sorted(self.tensors)

    def info(self, name: str) -> TensorInfo:
        return self.tensors[name]

    def get(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        mm = self._maps.get(t.path)
        if mm is None:
            mm = self._maps[t.path] = np.memmap(t.path, dtype=np.uint8, mode="r")
        return mm[t.begin: t.end].view(NP_DTYPES[t.dtype]).reshape(t.shape)


def write(path, tensors: Mapping[str, Tuple[np.ndarray, str]], metadata: Optional[Mapping[str, str]] = None) -> None:
    """Write ``{name: (array, safetensors dtype)}`` (BF16 / F8_E4M3 given as their uint16 / uint8 bit patterns)."""
    header: Dict[str, object] = {}
    blobs: List[bytes] = []
    off = 0
    for name, (arr, dtype) in tensors.items():
        a = np.ascontiguousarray(np.asarray(arr).astype(NP_DTYPES[dtype], copy=False))
        b = a.tobytes()
        header[name] = {"dtype": dtype, "shape": [int(x) for x in a.shape], "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = dict(metadata)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
