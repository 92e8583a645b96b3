"""The operator registry — the reference's plugin interface for the decode hot path (``monolith/ops/registry.py:12-54``,
``monolith/compiler/coverage.py:33-41``), kept with the same names and semantics so the reference's lowering can
target this backend: an :class:`OpDef` per op kind, bound per profile to a :class:`KernelBinding`; a lookup falls
back to the wildcard profile ``"*"``; rebinding a profile to a different kernel is an error.

On this backend a binding names a C-ABI entry point of ``libmi355.so`` (``include/lithos_mi355.h``) and its fixed
parameters (the reference binds MSL kernel names and function constants). The profile key is the GPU architecture,
``"gfx950"``.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import Any, Dict, Generic, Iterator, Mapping, Optional, TypeVar

WILDCARD = "*"
PROFILE = "gfx950"


class OpClass(enum.Enum):
    """How an op's blocks relate (``monolith/core/ir.py``): independent blocks, a reduction, or a serial op."""

    MAP = "map"
    REDUCE = "reduce"
    SERIAL = "serial"


T = TypeVar("T")


class Registry(Generic[T]):
    """Name → item, registered once (``monolith/registry.py``)."""

    def __init__(self, what: str) -> None:
        self.what = what
        self._items: Dict[str, T] = {}

    def register(self, name: str, item: T) -> T:
        if name in self._items and self._items[name] is not item:
            raise ValueError(f"{self.what} {name!r} is already registered")
        self._items[name] = item
        return item

    def resolve(self, name: str) -> Optional[T]:
        return self._items.get(name)

    def __getitem__(self, name: str) -> T:
        if name not in self._items:
            raise KeyError(f"unknown {self.what} {name!r}")
        return self._items[name]

    def __contains__(self, name: str) -> bool:
        return name in self._items

    def __iter__(self) -> Iterator[str]:
        return iter(sorted(self._items))

    def names(self):
        return sorted(self._items)


@dataclass(frozen=True)
class KernelBinding:
    """Which entry point implements an op on a profile, with its fixed parameters and workgroups per CU."""

    kernel: str
    function_constants: Mapping[str, Any] = field(default_factory=dict)
    threadgroups_per_core: int = 1


@dataclass(frozen=True)
class CostModel:
    """Per-block cost the planner reasons with (bytes streamed, ALU work, ALU-bound flag)."""

    bytes_per_block: int = 0
    flops_per_block: int = 0
    alu_bound: bool = False


@dataclass
class OpDef:
    """An op kind: its class, the kind of block domain it partitions over, its cost, and its kernel bindings."""

    name: str
    klass: OpClass
    domain_kind: str
    cost: CostModel = field(default_factory=CostModel)
    kernels: Dict[str, KernelBinding] = field(default_factory=dict)   # profile key -> binding, "*" = any

    def binding_for(self, profile_key: str) -> Optional[KernelBinding]:
        return self.kernels.get(profile_key) or self.kernels.get(WILDCARD)

    def bind(self, profile_key: str, binding: KernelBinding) -> "OpDef":
        if profile_key in self.kernels and self.kernels[profile_key] != binding:
            raise ValueError(f"op {self.name}: profile {profile_key!r} already bound to {self.kernels[profile_key]}")
        self.kernels[profile_key] = binding
        return self


OPS: Registry[OpDef] = Registry("op")


def register_op(opdef: OpDef) -> OpDef:
    return OPS.register(opdef.name, opdef)
