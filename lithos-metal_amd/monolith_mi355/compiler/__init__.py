"""The compiler side of the operator API for gfx950: an op graph (``ir``), the backend with its extension points and
the handler context (``context``), one handler per op kind on the library's entry points (``handlers``), lowering of
this package's decode layers (``lower``) and emission into the ``program.json`` format (``emit``)."""

from .context import EmitContext, Gfx950Backend, Profile, current_backend, dispatch, get_backend, register_backend, using_backend
from .emit import compile_program, emit_program, shared_emit
from .handlers import HANDLERS
from .ir import Graph, Op, Value, Weight
from .lower import lower_decoder, lower_layer

__all__ = ["EmitContext", "Gfx950Backend", "Profile", "current_backend", "dispatch", "get_backend",
           "register_backend", "using_backend", "compile_program", "emit_program", "shared_emit", "HANDLERS", "Graph",
           "Op", "Value", "Weight", "lower_decoder", "lower_layer"]
