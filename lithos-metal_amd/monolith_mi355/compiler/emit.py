"""Emission: an op graph to a :class:`~monolith_mi355.runtime.program.Program` through the selected backend's
handlers, and the decode model's compile (the reference's ``compile_program`` path: lowering, then the
``@dispatch("emit")`` entry, ``monolith/backends/metal/context.py:39-53``)."""

from __future__ import annotations

from ..ops.coverage import check_coverage
from ..runtime.program import Program
from .context import EmitContext, Profile, current_backend, dispatch
from .handlers import HANDLERS
from .ir import Graph
from .lower import lower_decoder

# op kinds the graph may hold that are not registered ops: the program's serial tail
_PROGRAM_OPS = ("advance",)


def shared_emit(graph: Graph, profile: Profile) -> Program:
    """Every op through ``backend.handler(kind, HANDLERS)(ctx, op)``, in graph order."""
    check_coverage(sorted({op.kind for op in graph.ops if op.kind not in _PROGRAM_OPS}))
    ctx = EmitContext(profile, t=graph.t)
    backend = current_backend()
    for op in graph.ops:
        backend.handler(op.kind, HANDLERS)(ctx, op)
    program = ctx.program
    program.bound_tensors = dict(ctx.bound)   # memory the program binds but does not allocate (Engine: buffers=)
    return program


@dispatch("emit")
def emit_program(graph: Graph, profile: Profile) -> Program:
    return shared_emit(graph, profile)


def compile_program(model, profile: Profile) -> Program:
    """The one-token decode step of ``model`` (a ``layers.DecoderModel``) as a program for ``profile``'s backend.
    Its weights, norms and states stay the model's tensors: run it with
    ``Engine(program, buffers=engine.bound_buffers(program))``."""
    return emit_program(lower_decoder(model), profile)
