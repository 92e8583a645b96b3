"""The op graph the backend lowers: values (device tensors of a decode step) and ops over them, with the reference's
IR fields (``monolith/core/ir.py:78-92``: ``Op(kind, inputs, outputs, domain, klass, attrs)``, state written in place
declared through ``updates``, ``:190-195``).

A value here is bound to memory when the graph is built from live layers (``tensor``: the device tensor that holds
it) or names a step-state field (``field``: the program's StepState word it reads or writes). A weight value carries
its T16 pack geometry (format, rows, columns, experts) and its per-row tensor-scale table.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

# a value's role decides the buffer it lives in (BufferSpec.role)
ROLES = ("weights", "state", "arena", "params", "step_state", "ring")


@dataclass(eq=False)
class Value:
    name: str
    shape: Tuple[int, ...]
    dtype: str                             # "bf16" | "f32" | "i32" | "i8" | "f16" | "u8" | "u64"
    role: str = "arena"
    tensor: Any = None                     # the device tensor holding it (bound graphs), or None (the program allocates)
    offset: int = 0                        # bytes into the tensor (a view: z inside the projection output)
    ld: Optional[int] = None               # row stride in elements when it differs from shape[-1]
    field: Optional[str] = None            # a step-state field (role "step_state")
    base: Optional["Value"] = None         # a view of another value: its buffer, at ``offset`` bytes further

    @property
    def itemsize(self) -> int:
        return {"bf16": 2, "f16": 2, "f32": 4, "i32": 4, "i8": 1, "u8": 1, "u64": 8}[self.dtype]

    @property
    def nbytes(self) -> int:
        n = self.itemsize
        for d in self.shape:
            n *= d
        return n

    @property
    def row_stride(self) -> int:
        return self.ld if self.ld is not None else self.shape[-1]


@dataclass(eq=False)
class Weight(Value):
    format: str = "nvfp4"
    n: int = 0
    k: int = 0
    experts: int = 1
    row_scale: Optional[Value] = None


@dataclass(eq=False)
class Op:
    kind: str
    inputs: List[Value]
    outputs: List[Value]
    domain: str = ""
    klass: str = ""
    attrs: Dict[str, Any] = field(default_factory=dict)
    updates: List[Value] = field(default_factory=list)   # state the op writes in place (caches, recurrent states)


@dataclass
class Graph:
    ops: List[Op] = field(default_factory=list)
    t: int = 1                             # tokens per step

    def add(self, kind: str, inputs, outputs, **attrs) -> Op:
        op = Op(kind, list(inputs), list(outputs), attrs=attrs)
        self.ops.append(op)
        return op

    def values(self) -> List[Value]:
        seen: Dict[int, Value] = {}
        for op in self.ops:
            for v in list(op.inputs) + list(op.outputs) + list(op.updates):
                if v is not None:
                    seen.setdefault(id(v), v)
        return list(seen.values())
