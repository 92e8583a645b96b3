"""Coverage check (``monolith/compiler/coverage.py:33-41``): every op of a program must have a kernel binding for
the profile, or compilation stops with the list of what is missing."""

from __future__ import annotations

from typing import Iterable, List, Optional, Tuple

from .registry import OPS, PROFILE, OpDef


class CoverageError(RuntimeError):
    def __init__(self, profile: str, missing: List[Tuple[str, Optional[OpDef]]]):
        self.profile, self.missing = profile, missing
        names = ", ".join(f"{k} ({'unknown op' if od is None else 'no binding'})" for k, od in missing)
        super().__init__(f"profile {profile}: no kernel for {names}")


def check_coverage(op_kinds: Iterable[str], profile: str = PROFILE) -> None:
    """Raise :class:`CoverageError` unless every op kind has a kernel binding for ``profile``."""
    missing: List[Tuple[str, Optional[OpDef]]] = []
    for kind in op_kinds:
        od = OPS.resolve(kind)
        if od is None or od.binding_for(profile) is None:
            missing.append((kind, od))
    if missing:
        raise CoverageError(profile, missing)
