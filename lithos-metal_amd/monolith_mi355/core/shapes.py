"""Symbolic row counts (``monolith/core/shapes.py``): ``T`` is the step's tokens; a program binds every row symbol
to its maximum for memory planning (``step_bindings``)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Iterable, Mapping, Optional, Tuple, Union


@dataclass(frozen=True)
class Sym:
    name: str

    def __repr__(self) -> str:
        return self.name


Dim = Union[int, Sym]
Shape = Tuple[Dim, ...]

T = Sym("T")              # tokens of this step (1 for decode, 1 + γ for a verify pass)
N_INJ = Sym("n_inject")   # rows a drafter injects
N_CHAIN = Sym("n_chain")  # an LM drafter's chain rows
N_FIRST = Sym("n_first")  # an LM drafter's first chain step
CTX = Sym("ctx")          # committed context length


def step_bindings(t_max: int) -> Dict[Sym, int]:
    return {T: t_max, N_INJ: t_max, N_CHAIN: 1, N_FIRST: t_max + 1}


def is_static(shape: Iterable[Dim]) -> bool:
    return all(not isinstance(d, Sym) for d in shape)


def _sym_name(d) -> Optional[str]:
    """A symbol's name whatever module defined it (a graph lowered by the reference carries its own ``Sym``)."""
    if isinstance(d, int):
        return None
    return getattr(d, "name", None)


def bind(shape: Iterable[Dim], bindings: Mapping) -> Tuple[int, ...]:
    """Every symbol replaced by its binding (looked up by name, so foreign ``Sym`` objects bind too)."""
    by_name = {getattr(k, "name", k): v for k, v in bindings.items()}
    out = []
    for d in shape:
        name = _sym_name(d)
        if name is None:
            out.append(int(d))
        elif name in by_name:
            out.append(int(by_name[name]))
        else:
            raise KeyError(f"unbound symbolic dimension {name}")
    return tuple(out)


def numel(shape: Iterable[Dim], bindings: Optional[Mapping] = None) -> int:
    n = 1
    for d in bind(shape, bindings or {}):
        n *= d
    return n
