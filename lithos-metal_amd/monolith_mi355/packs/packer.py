"""Checkpoint → gfx950 weight pack, and the pack reader — this backend's counterpart of the reference's packer /
``PackFile`` (``packs/packer.py:1-277``). Directory layout::

    weights.pack   [slab 0: T16 tiles][row scales f32][pad][slab 1 …][aux 0][pad][aux 1 …]
    manifest.json  per slab: format, N, K, experts, byte offsets, the row-scale table and where the rows came from;
                   per aux / table: dtype, shape, offset, transform

A slab is one matrix the GEMV streams (optionally several checkpoint matrices stacked by rows, row subsets, a row
permutation such as the gate|up interleave, or E equally shaped experts back to back) in the T16 layout of
``formats/pack.py``. Per-tensor scales (NVFP4 ``weight_scale_2``, FP8 ``weight_scale``) become the per-row table, so
every row keeps the scale of the matrix it came from whatever order the rows end up in. Slabs are packed one at a
time: memory is the largest slab, not the checkpoint.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, List, Optional, Sequence

import numpy as np

from ..formats import FORMATS, DequantSpec
from ..formats import pack as T16
from ..formats.fp import bf16_to_f32
from . import transforms
from .checkpoint import group_tensors, logical_shape
from .safetensors_io import NP_DTYPES, Checkpoint

ALIGN = 4096
LAYOUT = "t16"
VERSION = 1
AUX_TRANSFORMS = (None, "f32", "bf16_f32", "one_plus", "neg_exp")


@dataclass(frozen=True)
class Segment:
    """Rows of one checkpoint matrix ``<source>.weight`` — all, or ``rows`` (``rows[new] = old``)."""

    source: str
    rows: Optional[np.ndarray] = None


def _tensor_scale(spec: DequantSpec) -> Optional[float]:
    if spec.format == "nvfp4":
        return float(spec.params["weight_scale_2"])
    if spec.format == "fp8_e4m3":
        return float(spec.params["weight_scale"])
    return None


def _unit_scale(spec: DequantSpec) -> DequantSpec:
    key = {"nvfp4": "weight_scale_2", "fp8_e4m3": "weight_scale"}.get(spec.format)
    return spec if key is None else DequantSpec(spec.format, spec.shape, spec.tensors, dict(spec.params, **{key: 1.0}))


class Packer:
    def __init__(self, checkpoint, out_dir) -> None:
        """``checkpoint``: a safetensors file / directory, or None for a pack written only from already packed slabs
        and computed tables (``add_packed``, ``add_table``)."""
        self.ckpt = Checkpoint(checkpoint) if checkpoint is not None else None
        names = self.ckpt.names() if self.ckpt is not None else []
        self.dtypes = {n: self.ckpt.info(n).dtype for n in names}
        self.shapes = {n: self.ckpt.info(n).shape for n in names}
        self.groups = group_tensors(names, self.dtypes)
        self.out = Path(out_dir)
        self.out.mkdir(parents=True, exist_ok=True)
        self._fh = open(self.out / "weights.pack", "wb")
        self._pos = 0
        self._slabs: List[Dict[str, Any]] = []
        self._aux: List[Dict[str, Any]] = []

    def _align(self) -> None:
        pad = -self._pos % ALIGN
        self._fh.write(b"\0" * pad)
        self._pos += pad

    def _put(self, b: bytes) -> int:
        off = self._pos
        self._fh.write(b)
        self._pos += len(b)
        return off

    def _segment(self, seg: Segment, fmt: str) -> DequantSpec:
        g = self.groups.get(seg.source)
        if g is None:
            raise KeyError(f"pack: no matrix {seg.source!r} ({seg.source}.weight) in the checkpoint")
        shape = logical_shape(g, self.shapes)
        if shape is None or len(shape) != 2:
            raise ValueError(f"pack: {seg.source} is not a matrix ({shape})")
        tensors = {"weight": self.ckpt.get(g.weight)}
        tensors.update({side: self.ckpt.get(full) for side, full in g.sides.items()})
        n = int(shape[0])
        if seg.rows is not None:
            rows = np.asarray(seg.rows, dtype=np.int64)
            tensors = {k: (v[rows] if getattr(v, "ndim", 0) >= 1 and v.shape[0] == n else v) for k, v in tensors.items()}
            n = len(rows)
        if g.format == fmt:
            return FORMATS[fmt].unpack(tensors, shape=(n, int(shape[1])))
        if g.format in ("bf16", "f32"):          # a float matrix quantized at pack time with the format's quantizer
            w = tensors["weight"]
            w32 = bf16_to_f32(w) if g.format == "bf16" else np.asarray(w, np.float32)
            return FORMATS[fmt].quantize(np.ascontiguousarray(w32.reshape(n, int(shape[1]))))
        raise ValueError(f"pack: {seg.source} is stored as {g.format!r}; slab wants {fmt!r} (only BF16 / F32 "
                         f"matrices are quantized at pack time)")

    def add_slab(self, name: str, fmt: str, segments: Sequence[Segment], *, row_perm=None,
                 experts: int = 1) -> Dict[str, Any]:
        if fmt not in FORMATS:
            raise ValueError(f"slab {name}: unknown format {fmt!r}")
        specs = [self._segment(s, fmt) for s in segments]
        k = specs[0].shape[1]
        if any(s.shape[1] != k for s in specs):
            raise ValueError(f"slab {name}: segments differ in K")
        rows = [s.shape[0] for s in specs]
        n = sum(rows)
        stacked = {key: np.concatenate([np.asarray(s.tensors[key]) for s in specs], axis=0) for key in specs[0].tensors}
        scales = [_tensor_scale(s) for s in specs]
        row_scale = None if scales[0] is None else np.repeat(np.array(scales, np.float32), rows)
        if row_perm is not None:
            perm = np.asarray(row_perm, dtype=np.int64)
            if not np.array_equal(np.sort(perm), np.arange(n)):
                raise ValueError(f"slab {name}: row_perm is not a permutation of {n} rows")
            stacked = {key: v[perm] for key, v in stacked.items()}
            row_scale = None if row_scale is None else row_scale[perm]
        if experts < 1 or n % experts or (experts > 1 and (n // experts) % 16):
            raise ValueError(f"slab {name}: {n} rows do not split into {experts} experts of whole 16-row tiles")
        spec = _unit_scale(DequantSpec(fmt, (n, k), stacked, dict(specs[0].params)))
        data, info = T16.pack(spec, row_scale)
        self._align()
        off = self._put(data.tobytes())
        rs_off = self._put(info.row_scale.tobytes()) if info.row_scale is not None else None
        entry = {"name": name, "format": fmt, "n": n // experts, "k": k, "experts": experts, "offset": off,
                 "nbytes": int(data.size), "row_scales_offset": rs_off,
                 "row_scales_len": None if info.row_scale is None else int(info.row_scale.size),
                 "row_perm": row_perm is not None,
                 "segments": [{"source": s.source, "rows": int(r), "row_select": s.rows is not None,
                               "tensor_scale": sc} for s, r, sc in zip(segments, rows, scales)]}
        self._slabs.append(entry)
        return entry

    def add_packed(self, slabs: Sequence[Dict[str, Any]]) -> List[Dict[str, Any]]:
        """Slabs already in the T16 layout (a model's device weights, a re-pack): each ``dict(name, format, n, k,
        data, row_scale=None, experts=1)`` with ``data`` the pack bytes of ``experts`` matrices of ``n`` rows and
        ``row_scale`` their per-row table (padded to whole tiles per expert). The slabs of one call are written back
        to back — their code bytes contiguous, then their row-scale tables contiguous — so an emitter may stream two
        adjacent slabs of one format and K as one stacked matrix (a router and the shared expert's gate, the routed
        experts and the shared expert)."""
        self._align()
        entries = []
        for sl in slabs:
            fmt, n, k, experts = sl["format"], int(sl["n"]), int(sl["k"]), int(sl.get("experts", 1))
            if fmt not in FORMATS:
                raise ValueError(f"slab {sl['name']}: unknown format {fmt!r}")
            data = np.ascontiguousarray(np.asarray(sl["data"]).view(np.uint8).reshape(-1))
            if data.size != experts * T16.pack_bytes(fmt, n, k):
                raise ValueError(f"slab {sl['name']}: {data.size} bytes for {experts} × T16 {fmt} [{n}, {k}] "
                                 f"({T16.pack_bytes(fmt, n, k)} each)")
            entries.append({"name": sl["name"], "format": fmt, "n": n, "k": k, "experts": experts,
                            "offset": self._put(data.tobytes()), "nbytes": int(data.size), "row_scales_offset": None,
                            "row_scales_len": None, "row_perm": bool(sl.get("row_perm", False)), "segments": [],
                            "_rs": sl.get("row_scale")})
        for e in entries:
            rs = e.pop("_rs")
            if rs is not None:
                rs = np.ascontiguousarray(np.asarray(rs, np.float32).reshape(-1))
                if rs.size != e["experts"] * -(-e["n"] // 16) * 16:
                    raise ValueError(f"slab {e['name']}: row-scale table of {rs.size}, expected whole tiles per expert")
                e["row_scales_offset"], e["row_scales_len"] = self._put(rs.tobytes()), int(rs.size)
        self._slabs.extend(entries)
        return entries

    def add_aux(self, name: str, source: str, *, transform: Optional[str] = None, perm=None) -> Dict[str, Any]:
        info = self.ckpt.info(source)
        a = self.ckpt.get(source)
        if transform is None:
            out, dtype = np.ascontiguousarray(a), info.dtype
        elif transform == "f32":
            out, dtype = (bf16_to_f32(a) if info.dtype == "BF16" else np.asarray(a, np.float32)), "F32"
        elif transform == "bf16_f32":
            out, dtype = transforms.bf16_round_f32(a, dtype_in=info.dtype), "F32"
        elif transform == "one_plus":
            out, dtype = transforms.one_plus(a, dtype_in=info.dtype), "F32"
        elif transform == "neg_exp":
            out, dtype = transforms.neg_exp(a, dtype_in=info.dtype), "F32"
        else:
            raise ValueError(f"aux {name}: transform {transform!r} is not one of {AUX_TRANSFORMS}")
        if perm is not None:
            perm = np.asarray(perm, dtype=np.int64)
            if not np.array_equal(np.sort(perm), np.arange(out.shape[0])):
                raise ValueError(f"aux {name}: perm is not a permutation of the leading axis")
            out = out[perm]
        return self._raw(name, np.ascontiguousarray(out), dtype, source, transform)

    def add_table(self, name: str, array: np.ndarray, dtype: str = "F32") -> Dict[str, Any]:
        """A computed constant (RoPE tables …); BF16 given as its uint16 bit pattern."""
        return self._raw(name, np.ascontiguousarray(np.asarray(array).astype(NP_DTYPES[dtype], copy=False)), dtype,
                         None, "table")

    def _raw(self, name, arr, dtype, source, transform) -> Dict[str, Any]:
        self._align()
        off = self._put(arr.tobytes())
        entry = {"name": name, "source": source, "transform": transform, "dtype": dtype,
                 "shape": [int(x) for x in arr.shape], "offset": off, "nbytes": int(arr.nbytes)}
        self._aux.append(entry)
        return entry

    def write(self, extra: Optional[Dict[str, Any]] = None) -> Dict[str, Any]:
        self._align()
        self._fh.close()
        manifest = {"version": VERSION, "layout": LAYOUT, "alignment": ALIGN, "pack": "weights.pack",
                    "nbytes": self._pos, "slabs": self._slabs, "aux": self._aux, **(extra or {})}
        with open(self.out / "manifest.json", "w") as f:
            json.dump(manifest, f, indent=1)
        return manifest


class PackFile:
    """The read side: slabs and aux tensors memory-mapped from ``weights.pack``, uploaded on request."""

    def __init__(self, directory) -> None:
        self.dir = Path(directory)
        with open(self.dir / "manifest.json") as f:
            self.manifest = json.load(f)
        if self.manifest.get("layout") != LAYOUT or self.manifest.get("version") != VERSION:
            raise ValueError(f"{self.dir}: not a {LAYOUT} pack of version {VERSION}")
        self._mm = np.memmap(self.dir / self.manifest["pack"], dtype=np.uint8, mode="r")
        self.slabs = {s["name"]: s for s in self.manifest["slabs"]}
        self.aux = {a["name"]: a for a in self.manifest["aux"]}

    def slab_bytes(self, name: str) -> np.ndarray:
        s = self.slabs[name]
        return self._mm[s["offset"]: s["offset"] + s["nbytes"]]

    def row_scales(self, name: str) -> Optional[np.ndarray]:
        s = self.slabs[name]
        if s["row_scales_offset"] is None:
            return None
        o = s["row_scales_offset"]
        return self._mm[o: o + 4 * s["row_scales_len"]].view(np.float32)

    def aux_array(self, name: str) -> np.ndarray:
        a = self.aux[name]
        return self._mm[a["offset"]: a["offset"] + a["nbytes"]].view(NP_DTYPES[a["dtype"]]).reshape(a["shape"])

    def slab_info(self, name: str, expert: int = 0) -> T16.PackInfo:
        s = self.slabs[name]
        n, k = s["n"], s["k"]
        nt, c = -(-n // 16), k // T16.chunk_cols(s["format"])
        per = s["nbytes"] // s["experts"]
        rs = self.row_scales(name)
        rs = None if rs is None else np.asarray(rs[expert * nt * 16: (expert + 1) * nt * 16])
        return T16.PackInfo(s["format"], n, k, nt, c, per, rs)

    def dequantize_slab(self, name: str, expert: int = 0) -> np.ndarray:
        """The float32 ``[N, K]`` the kernels compute with: rows in pack order, row scales applied."""
        s = self.slabs[name]
        info = self.slab_info(name, expert)
        per = s["nbytes"] // s["experts"]
        data = np.asarray(self.slab_bytes(name)[expert * per: (expert + 1) * per])
        spec = T16.unpack(data, info)
        w = FORMATS[s["format"]].dequantize(_unit_scale(spec))
        if info.row_scale is not None:
            w = (w * info.row_scale[: s["n"], None]).astype(np.float32)
        return w

    def upload(self, name: str, device="cuda"):
        """The slab as a device ``PackedWeight`` (the GEMV's operand)."""
        import torch
        from ..kernels import PackedWeight
        s = self.slabs[name]
        data = torch.from_numpy(np.array(self.slab_bytes(name))).to(device)
        rs = self.row_scales(name)
        rs = None if rs is None else torch.from_numpy(np.array(rs)).to(device)
        return PackedWeight(s["format"], s["n"], s["k"], s["experts"], data, rs)
