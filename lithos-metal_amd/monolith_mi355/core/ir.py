"""The op graph a model lowers to (``monolith/core/ir.py:78-248``): values (tensors of one step) and ops over them.

What the contract fixes, and this module keeps: an op is ``Op(kind, inputs, outputs, domain, klass, attrs)``; a
value is a graph *source* — a step input (``tokens`` reads the step state), a packed weight slab (``format`` names
its storage format), a persistent state (caches, recurrent states, written in place by the ops that list it in
``updates``) or a constant from the pack's aux section — or the output of exactly one earlier op; a row *view*
aliases rows of another value's buffer. Names are unique; ``scope`` prefixes activation names so one module tree
can be lowered several times into a graph.

Nothing here knows a kernel: ops are bound to entry points through the op registry, and the emitter maps values to
buffers (weights and constants to windows of the pack file, by name).
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, Iterable, Iterator, List, Optional, Sequence, Set, Tuple

from .dtypes import DType
from .shapes import Dim, Shape, Sym


class OpClass(Enum):
    MAP = "MAP"          # every block writes its own outputs
    REDUCE = "REDUCE"    # blocks write partials that a follow-up folds in block order
    SERIAL = "SERIAL"    # one wave: the step's serial bookkeeping (advance, accept scan, verify select)


@dataclass(frozen=True)
class BlockDomain:
    kind: str
    n_blocks: Dim

    def __post_init__(self) -> None:
        if isinstance(self.n_blocks, int) and self.n_blocks <= 0:
            raise ValueError(f"BlockDomain({self.kind}): n_blocks must be positive, got {self.n_blocks}")


@dataclass(eq=False)
class Value:
    name: str
    shape: Shape
    dtype: DType
    format: Optional[str] = None
    producer: Optional["Op"] = None
    consumers: List["Op"] = field(default_factory=list)
    is_input: bool = False
    is_weight: bool = False
    is_state: bool = False
    is_const: bool = False
    view_of: Optional[Tuple[str, int]] = None     # (base value, first row)

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def is_view(self) -> bool:
        return self.view_of is not None

    @property
    def is_source(self) -> bool:
        return self.is_input or self.is_weight or self.is_state or self.is_const

    def __repr__(self) -> str:
        fmt = f", format={self.format}" if self.format else ""
        return f"Value({self.name}: {list(self.shape)} {self.dtype}{fmt})"


@dataclass(eq=False)
class Op:
    kind: str
    inputs: List[Value]
    outputs: List[Value]
    domain: BlockDomain
    klass: OpClass
    attrs: Dict[str, Any] = field(default_factory=dict)
    id: int = -1

    def __repr__(self) -> str:
        return f"Op#{self.id}({self.kind}, {self.klass.value}, {self.domain.kind}x{self.domain.n_blocks})"


class Graph:
    """Ops in program order and the values between them."""

    def __init__(self, name: str = "step") -> None:
        self.name = name
        self.ops: List[Op] = []
        self.values: Dict[str, Value] = {}
        self.views: Dict[str, List[Value]] = {}
        self.symbols: Set[Sym] = set()
        self._scope = ""

    # ---- values ---------------------------------------------------------------------------------------------
    @contextmanager
    def scope(self, prefix: str) -> Iterator[None]:
        outer = self._scope
        self._scope = outer + prefix
        try:
            yield
        finally:
            self._scope = outer

    def _new(self, name: str, shape: Sequence[Dim], dtype: DType, fmt: Optional[str], scoped: bool) -> Value:
        full = (self._scope + name) if scoped else name
        if full in self.values:
            raise ValueError(f"graph {self.name}: value name {full!r} is already taken")
        v = Value(full, tuple(shape), dtype, fmt)
        self.values[full] = v
        self.symbols.update(d for d in v.shape if isinstance(d, Sym))
        return v

    def value(self, name: str, shape: Sequence[Dim], dtype: DType, *, format: Optional[str] = None,
              scoped: bool = True) -> Value:
        return self._new(name, shape, dtype, format, scoped)

    def input(self, name: str, shape: Sequence[Dim], dtype: DType) -> Value:
        v = self._new(name, shape, dtype, None, False)
        v.is_input = True
        return v

    def weight(self, name: str, shape: Sequence[int], format: str) -> Value:
        v = self._new(name, shape, DType.U8, format, False)
        v.is_weight = True
        return v

    def state(self, name: str, shape: Sequence[Dim], dtype: DType) -> Value:
        v = self._new(name, shape, dtype, None, False)
        v.is_state = True
        return v

    def const(self, name: str, shape: Sequence[Dim], dtype: DType) -> Value:
        v = self._new(name, shape, dtype, None, False)
        v.is_const = True
        return v

    def view(self, name: str, base: Value, row: int, rows: int = 1) -> Value:
        if self.values.get(base.name) is not base:
            raise ValueError(f"graph {self.name}: {base!r} does not belong to this graph")
        if base.is_source or base.is_view:
            raise ValueError(f"graph {self.name}: cannot view {base!r} (a source or a view)")
        n = base.shape[0] if base.shape else 0
        if not isinstance(n, int) or row < 0 or rows < 1 or row + rows > n:
            raise ValueError(f"graph {self.name}: view rows [{row}, {row + rows}) outside {base!r} (static rows only)")
        v = self.value(name, (rows,) + tuple(base.shape[1:]), base.dtype)
        v.view_of = (base.name, row)
        self.views.setdefault(base.name, []).append(v)
        return v

    # ---- ops ------------------------------------------------------------------------------------------------
    def op(self, kind: str, inputs: Iterable[Value], outputs: Iterable[Value], *, domain: BlockDomain,
           klass: OpClass, **attrs: Any) -> Op:
        ins, outs = list(inputs), list(outputs)
        for v in ins + outs:
            if self.values.get(v.name) is not v:
                raise ValueError(f"graph {self.name}: {v!r} does not belong to this graph")
        for v in outs:
            if v.producer is not None:
                raise ValueError(f"graph {self.name}: {v!r} already has a producer {v.producer!r}")
            if v.is_source:
                raise ValueError(f"graph {self.name}: {v!r} is a graph source and cannot be produced by an op")
        for name in attrs.get("updates", ()):
            sv = self.values.get(name)
            if sv is None or not sv.is_state:
                raise ValueError(f"graph {self.name}: op {kind} updates {name!r}, which is not a state of this graph")
            if sv not in ins:
                raise ValueError(f"graph {self.name}: op {kind} updates {name!r} without reading it")
        op = Op(kind, ins, outs, domain, klass, dict(attrs), id=len(self.ops))
        for v in outs:
            v.producer = op
        for v in ins:
            v.consumers.append(op)
        self.ops.append(op)
        return op

    # ---- structure ------------------------------------------------------------------------------------------
    def producers(self, op: Op) -> List[Op]:
        found = {v.producer.id: v.producer for v in op.inputs if v.producer is not None}
        return [found[i] for i in sorted(found)]

    def states(self) -> List[Value]:
        return [v for v in self.values.values() if v.is_state]

    def check(self) -> None:
        """Every op has an output; every non-source input was produced earlier — as a whole value, or, for a row
        view, every row it reads by earlier writes of its base or of sibling views."""
        for op in self.ops:
            if not op.outputs:
                raise ValueError(f"graph {self.name}: {op!r} has no outputs")
            for v in op.inputs:
                if v.is_source:
                    continue
                if v.producer is not None:
                    if v.producer.id >= op.id:
                        raise ValueError(f"graph {self.name}: {op!r} reads {v!r} before its producer {v.producer!r}")
                    continue
                base_name, row0 = v.view_of if v.view_of is not None else (v.name, 0)
                base = self.values[base_name]
                rows = v.shape[0] if v.shape and isinstance(v.shape[0], int) else None
                if rows is None or (base.producer is None and base_name not in self.views):
                    raise ValueError(f"graph {self.name}: {op!r} reads {v!r}, which nothing produces")
                written: Set[int] = set()
                if base.producer is not None and base.producer.id < op.id:
                    written.update(range(int(base.shape[0])))
                for w in self.views.get(base_name, ()):
                    if w.producer is not None and w.producer.id < op.id:
                        written.update(range(w.view_of[1], w.view_of[1] + int(w.shape[0])))
                gap = sorted(set(range(row0, row0 + rows)) - written)
                if gap:
                    raise ValueError(f"graph {self.name}: {op!r} reads rows {gap[:4]} of {base!r} before any op "
                                     f"writes them")

    def __len__(self) -> int:
        return len(self.ops)

    def __repr__(self) -> str:
        return f"Graph({self.name}: {len(self.ops)} ops, {len(self.values)} values)"
