"""The decode-path operator API (``monolith/ops``): op definitions with their gfx950 bindings and the coverage
check. The compiler side — the backend, the ``handler(ctx, op)`` emitters and the emitted program — is
:mod:`monolith_mi355.compiler`; :mod:`monolith_mi355.kernels` calls each entry point directly.

Op semantics follow the reference's docstrings (``ops/gemv.py:1-12``, ``ops/norm.py:1-6``, ``ops/attention.py:1-15``,
``ops/gdn.py:1-17``, ``ops/moe.py:1-16``). Where this backend fuses two reference ops into one launch (``gqa_merge``
into ``gqa_decode``, ``gdn_norm`` into ``gdn_mixer``) the second op's binding names the fused entry point and
``fused_into`` says which op carries it.
"""

from .coverage import CoverageError, check_coverage
from .registry import OPS, PROFILE, WILDCARD, CostModel, KernelBinding, OpClass, OpDef, Registry, register_op
from . import defs as _defs  # noqa: F401  (registers the ops)

__all__ = ["OPS", "PROFILE", "WILDCARD", "CostModel", "KernelBinding", "OpClass", "OpDef", "Registry", "register_op",
           "CoverageError", "check_coverage"]
