"""Group a checkpoint's tensors into matrices with their scale tensors and name each group's storage format from
the stored dtypes — the ModelOpt and MLX conventions the reference recognises (``formats/checkpoint.py:20-63``):

* NVFP4 (ModelOpt): ``weight`` U8 ``[N, K/2]`` + ``weight_scale`` F8_E4M3 ``[N, K/16]`` + ``weight_scale_2`` F32;
* NVFP4 (MLX): ``weight`` U32 ``[N, K/8]`` + ``scales`` U8 ``[N, K/16]``, no tensor scale;
* FP8 E4M3 (ModelOpt): ``weight`` F8_E4M3 ``[N, K]`` + ``weight_scale`` F32;
* affine INT4 (MLX): ``weight`` U32 ``[N, K/8]`` + ``scales`` / ``biases`` F16 or BF16 ``[N, K/64]``;
* BF16 / F32 matrices as stored.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Iterable, Mapping, Optional, Tuple

SIDE_KEYS = ("weight_scale", "weight_scale_2", "input_scale", "scales", "biases")


@dataclass
class Group:
    base: str                              # "<base>.weight" is the matrix
    weight: str
    sides: Dict[str, str] = field(default_factory=dict)
    format: str = ""                       # nvfp4 | fp8_e4m3 | int4_affine | bf16 | f32 | "" (unknown)


def group_tensors(names: Iterable[str], dtypes: Mapping[str, str]) -> Dict[str, Group]:
    names = list(names)
    groups = {n[: -len(".weight")]: Group(n[: -len(".weight")], n) for n in names if n.endswith(".weight")}
    for n in names:
        for side in SIDE_KEYS:
            suffix = "." + side
            if n.endswith(suffix) and n[: -len(suffix)] in groups:
                groups[n[: -len(suffix)]].sides[side] = n
    for g in groups.values():
        g.format = storage_format(g, dtypes)
    return groups


def storage_format(g: Group, dtypes: Mapping[str, str]) -> str:
    wd = dtypes.get(g.weight, "")
    sd = {k: dtypes.get(v, "") for k, v in g.sides.items()}
    if wd == "U8" and sd.get("weight_scale") == "F8_E4M3" and "weight_scale_2" in g.sides:
        return "nvfp4"
    if wd == "F8_E4M3" and sd.get("weight_scale") == "F32":
        return "fp8_e4m3"
    if wd == "U32" and sd.get("scales") in ("F16", "BF16") and "biases" in g.sides:
        return "int4_affine"
    if wd == "U32" and sd.get("scales") == "U8" and "biases" not in g.sides:
        return "nvfp4"
    return {"BF16": "bf16", "F32": "f32"}.get(wd, "")


def logical_shape(g: Group, shapes: Mapping[str, Tuple[int, ...]]) -> Optional[Tuple[int, ...]]:
    """The dequantized ``[N, K]`` of a group: 2 codes per U8 (ModelOpt NVFP4), 8 per U32 (MLX)."""
    sh = tuple(shapes[g.weight])
    if g.format == "nvfp4":
        return sh[:-1] + (sh[-1] * (2 if "weight_scale_2" in g.sides else 8),)
    if g.format == "int4_affine":
        return sh[:-1] + (sh[-1] * 8,)
    return sh
