"""The compiler IR in the reference's contract (``monolith/core/{ir,dtypes,shapes}.py``): a graph of ops over
values, built by a model's ``lower``. Kept interface-compatible so a graph lowered by the reference's ``nn`` modules
and one built here both feed :func:`monolith_mi355.compiler.emit_program`."""

from .dtypes import DType
from .ir import BlockDomain, Graph, Op, OpClass, Value
from .shapes import CTX, N_CHAIN, N_FIRST, N_INJ, T, Dim, Shape, Sym, bind, is_static, numel, step_bindings

__all__ = ["DType", "BlockDomain", "Graph", "Op", "OpClass", "Value", "CTX", "N_CHAIN", "N_FIRST", "N_INJ", "T",
           "Dim", "Shape", "Sym", "bind", "is_static", "numel", "step_bindings"]
