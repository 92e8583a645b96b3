"""The compiler side of the operator API for gfx950: ``emit_program`` / ``compile_program`` take a step graph in the
reference's op contract (``monolith_mi355.core``; built by ``monolith_mi355.nn`` or by the reference's own modules)
and a pack, run the backend's fusion passes (``plan``) and emit a ``program.json`` program of library calls through
one handler per op kind (``handlers``); ``lower`` bridges the hand-built ``layers.DecoderModel`` into those terms."""

from .context import EmitContext, Gfx950Backend, Profile, current_backend, dispatch, get_backend, register_backend, using_backend
from .emit import compile_program, emit_program, lower_round, shared_emit
from .handlers import HANDLERS
from .lower import compile_decoder, describe, load_states, state_images, write_pack
from .plan import PASSES, Plan, run_passes

__all__ = ["EmitContext", "Gfx950Backend", "Profile", "current_backend", "dispatch", "get_backend",
           "register_backend", "using_backend", "compile_program", "emit_program", "lower_round", "shared_emit",
           "HANDLERS", "compile_decoder", "describe", "load_states", "state_images", "write_pack", "PASSES", "Plan",
           "run_passes"]
