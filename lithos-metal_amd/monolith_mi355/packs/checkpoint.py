"""Recognise the quantized matrices of a safetensors checkpoint: which tensors belong to one matrix, and in which
storage format the matrix is held.

A matrix ``<base>`` is the tensor ``<base>.weight`` plus the sibling tensors ``<base>.<side>`` that carry its scales
(the ModelOpt and MLX naming the reference reads, ``formats/checkpoint.py:20-63``). Its format is decided by a
signature table: the first signature whose weight dtype and side dtypes all match names the format, and says how
many codes one stored element of the weight holds (so the logical ``[N, K]`` follows from the stored shape):

=================  ============  ====================================================  =======  ===============
format             weight dtype  sides (dtype)                                          absent   codes / element
=================  ============  ====================================================  =======  ===============
nvfp4 (ModelOpt)   U8            weight_scale (F8_E4M3), weight_scale_2 (any)                    2
fp8_e4m3           F8_E4M3       weight_scale (F32)                                               1
int4_affine (MLX)  U32           scales (F16 / BF16), biases (any)                                8
nvfp4 (MLX)        U32           scales (U8)                                            biases   8
bf16 / f32         BF16 / F32    —                                                                1
=================  ============  ====================================================  =======  ===============

Side tensors a format does not use (``input_scale``, an activation scale) still join their group.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Iterable, Mapping, Optional, Tuple

# the suffixes that attach a tensor to the matrix of the same base name
SIDE_KEYS = ("weight_scale", "weight_scale_2", "input_scale", "scales", "biases")


@dataclass(frozen=True)
class Signature:
    format: str
    weight_dtype: str
    sides: Tuple[Tuple[str, Tuple[str, ...]], ...]   # (side, accepted dtypes); () = any dtype
    absent: Tuple[str, ...] = ()
    codes_per_element: int = 1


SIGNATURES = (
    Signature("nvfp4", "U8", (("weight_scale", ("F8_E4M3",)), ("weight_scale_2", ())), codes_per_element=2),
    Signature("fp8_e4m3", "F8_E4M3", (("weight_scale", ("F32",)),)),
    Signature("int4_affine", "U32", (("scales", ("F16", "BF16")), ("biases", ())), codes_per_element=8),
    Signature("nvfp4", "U32", (("scales", ("U8",)),), absent=("biases",), codes_per_element=8),
    Signature("bf16", "BF16", ()),
    Signature("f32", "F32", ()),
)


@dataclass
class Group:
    """One matrix: ``weight`` is the full name of ``<base>.weight``; ``sides`` maps a side key to its full name."""

    base: str
    weight: str
    sides: Dict[str, str] = field(default_factory=dict)
    format: str = ""                       # a Signature's format, or "" when none matches
    codes_per_element: int = 1


def _matches(sig: Signature, g: Group, dtypes: Mapping[str, str]) -> bool:
    if dtypes.get(g.weight) != sig.weight_dtype or any(k in g.sides for k in sig.absent):
        return False
    for side, accepted in sig.sides:
        if side not in g.sides or (accepted and dtypes.get(g.sides[side]) not in accepted):
            return False
    return True


def storage_format(g: Group, dtypes: Mapping[str, str]) -> str:
    """The format of the first matching signature ("" when none does); also records its codes per element."""
    for sig in SIGNATURES:
        if _matches(sig, g, dtypes):
            g.codes_per_element = sig.codes_per_element
            return sig.format
    g.codes_per_element = 1
    return ""


def group_tensors(names: Iterable[str], dtypes: Mapping[str, str]) -> Dict[str, Group]:
    """``{base: Group}`` for every ``<base>.weight`` in ``names``, with its side tensors and its format."""
    by_base: Dict[str, Dict[str, str]] = {}
    for name in names:
        base, dot, suffix = name.rpartition(".")
        if dot and (suffix == "weight" or suffix in SIDE_KEYS):
            by_base.setdefault(base, {})[suffix] = name
    groups: Dict[str, Group] = {}
    for base, members in by_base.items():
        if "weight" not in members:
            continue                       # scales without a matrix (or of one stored under another name)
        g = Group(base, members.pop("weight"), members)
        g.format = storage_format(g, dtypes)
        groups[base] = g
    return groups


def logical_shape(g: Group, shapes: Mapping[str, Tuple[int, ...]]) -> Optional[Tuple[int, ...]]:
    """The dequantized shape of a group: the stored shape with its last axis times the codes each element holds."""
    stored = tuple(shapes[g.weight])
    if not stored:
        return None
    return stored[:-1] + (stored[-1] * g.codes_per_element,)
