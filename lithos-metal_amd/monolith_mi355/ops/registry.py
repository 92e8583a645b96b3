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
    """A name table whose entries cannot be replaced by a different object (``monolith/registry.py``)."""

    def __init__(self, what: str) -> None:
        self.what = what
        self._items: Dict[str, T] = {}

    def register(self, name: str, item: T) -> T:
        if self._items.get(name, item) is not item:
            raise ValueError(f"{name!r}: another {self.what} holds this name")
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
    """The implementation of an op on one profile: the libmi355 entry point, the descriptor fields it fixes, and
    how many of its workgroups the planner expects per CU."""

    kernel: str
    function_constants: Mapping[str, Any] = field(default_factory=dict)
    threadgroups_per_core: int = 1


@dataclass(frozen=True)
class CostModel:
    """What one block of the op's domain costs: bytes it streams, arithmetic it does, which of the two bounds it."""

    bytes_per_block: int = 0
    flops_per_block: int = 0
    alu_bound: bool = False


@dataclass
class OpDef:
    """One op kind of the IR: how its blocks combine (``klass``), what its domain is split into, its cost, and the
    per-profile implementations (``"*"`` binds every profile)."""

    name: str
    klass: OpClass
    domain_kind: str
    cost: CostModel = field(default_factory=CostModel)
    kernels: Dict[str, KernelBinding] = field(default_factory=dict)   # profile key -> binding, "*" = any

    def binding_for(self, profile_key: str) -> Optional[KernelBinding]:
        return self.kernels.get(profile_key) or self.kernels.get(WILDCARD)

    def bind(self, profile_key: str, binding: KernelBinding) -> "OpDef":
        held = self.kernels.get(profile_key)
        if held is not None and held != binding:
            raise ValueError(f"{self.name} on {profile_key}: bound to {held.kernel} already, not to {binding.kernel}")
        self.kernels[profile_key] = binding
        return self


OPS: Registry[OpDef] = Registry("op")


def register_op(opdef: OpDef) -> OpDef:
    return OPS.register(opdef.name, opdef)
