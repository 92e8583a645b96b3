"""``emit_program`` / ``compile_program`` for gfx950: a step graph in the reference's op contract → a runtime
:class:`~monolith_mi355.runtime.program.Program` of library calls, weights mapped from the pack file
(``compiler/emit.py:1389-1478, 1567-1620`` — same entry points, argument names and program format).

Pipeline: coverage check on the graph's op kinds → the plan's passes (``plan.py``: the reference's split ops folded
into this backend's fused entry points) → one handler per remaining op → the tail (``advance``) → buffers of
values no op binds dropped. ``T`` is static per program: a speculative (``dynamic_t``) program computes every row of
its ``1 + γ`` verify block each step and its serial ops read the step's own count from the step state, as the
hand-built ``SpecProgram`` does; the reference's per-T predicated variants exist to save ALU work on its GPU and
have no counterpart here.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Sequence, Union

from ..core import BlockDomain, DType, Graph, OpClass
from ..ops.coverage import check_coverage
from ..runtime.program import Program, StepStateLayout
from .context import EmitContext, Profile, current_backend, dispatch, STATE_LAYOUT
from .handlers import HANDLERS, advance
from .plan import PASSES, Plan, run_passes


def shared_emit(g, *, pack=None, profile: Profile, t: Optional[int] = None, dynamic_t: bool = False,
                layout: Optional[StepStateLayout] = None, eos: Union[int, Sequence[int], None] = None,
                ring_capacity: Optional[int] = None, tail: Optional[str] = "advance", token=None,
                speculative: bool = False, passes=PASSES, **_options: Any) -> Program:
    layout = layout or StepStateLayout(*STATE_LAYOUT)
    packs = [] if pack is None else ([pack] if hasattr(pack, "manifest") else list(pack))
    if dynamic_t and t is None:
        raise ValueError("emit_program: a dynamic-T program on gfx950 needs t (its verify block's rows)")
    t = 1 if t is None else int(t)
    if not 1 <= t <= layout.t_max:
        raise ValueError(f"emit_program: T = {t} must be within 1..t_max = {layout.t_max}")
    check_coverage(sorted({op.kind for op in g.ops}), profile.key)
    slabs = {s["name"]: s for pk in packs for s in pk.manifest["slabs"]}
    plan = run_passes(Plan.from_graph(g, t, slabs), passes)
    caps = [c for c in (_context_capacity(plan), profile.ctx_cap) if c]
    ctx = EmitContext(profile, plan, packs, layout=layout, ring_capacity=ring_capacity, ctx_cap=min(caps) if caps else 0)
    ctx.eos = profile.eos if eos is None else eos
    backend = current_backend()
    for op in plan.ops:
        backend.handler(op.kind, HANDLERS)(ctx, op)
    if tail == "advance":
        if token is None:
            raise ValueError("emit_program: the advance needs the sampled token value")
        advance(ctx, token)
    elif tail is not None:
        raise ValueError(f"emit_program: unknown tail {tail!r}")
    program = ctx.program
    bound = {name for op in program.ops for _, name, _ in op.bindings}
    for name in [n for n, spec in program.buffers.items() if spec.role == "arena" and n not in bound]:
        del program.buffers[name]
    program.plan_report = dict(plan.report)
    program.state_names = sorted(n for n, s in program.buffers.items() if s.role == "state")
    return program


def _context_capacity(plan: Plan) -> int:
    """The positions a sequence may occupy: the smallest KV cache of the attention ops less the rows a step appends
    after its first (a verify block of T rows writes positions pos .. pos + T - 1); 0 = unbounded. The serial ops
    stop the program at a step whose position reaches it, so no kernel writes past a cache."""
    caps = [plan.shape(op.inputs[1])[0] - (plan.t - 1) for op in plan.ops if op.kind == "gqa_decode"]
    return min(caps) if caps else 0


@dispatch("emit")
def emit_program(g, *, pack=None, profile: Profile, t: Optional[int] = None, dynamic_t: bool = False,
                 layout: Optional[StepStateLayout] = None, eos=None, ring_capacity: Optional[int] = None,
                 tail: Optional[str] = "advance", token=None, speculative: bool = False, **options: Any) -> Program:
    """The step program of graph ``g`` for ``profile``: weights and constants from ``pack`` (a ``PackFile`` or
    several) by name, ``T = t`` rows (1 by default; a speculative program's verify block with ``dynamic_t``),
    ``tail="advance"`` closing the step on ``token``; ``eos`` and ``ring_capacity`` default to the profile's.
    Accepts the reference's other keyword options (tuning, barriers, attention variant) and ignores them: they
    choose among Metal kernels."""
    return shared_emit(g, pack=pack, profile=profile, t=t, dynamic_t=dynamic_t, layout=layout, eos=eos,
                       ring_capacity=ring_capacity, tail=tail, token=token, speculative=speculative, **options)


def lower_round(g: Graph, token, *, gamma: int, draft_table: str = "draft_table", verify_length: Optional[int] = None,
                threshold: Optional[float] = None, table_shape=None):
    """Append the speculative round to a lowered target step (``compiler/emit.py:1534-1564``): the accept scan on
    the sampled tokens, each mixer's commit pass (``commit_kind``), the draft source and the verify-length select.
    The drafter is out of this build's scope: its stand-in is a table lookup, ``embed`` of the pack constant
    ``draft_table`` (int32 drafts per position, viewed as 16-bit words) at the step state's ``position`` — the
    drafts proposed after the token at that position (``table_shape``: its ``[positions, 16-bit words]`` when the
    graph does not hold it yet). Returns the select's value."""
    acc = g.value("accepted", (1,), DType.U32)
    g.op("accept_scan", [token], [acc], domain=BlockDomain("span", 1), klass=OpClass.SERIAL)
    for op in list(g.ops):
        ck = op.attrs.get("commit_kind")
        if ck:
            attrs = {k: v for k, v in op.attrs.items() if k != "commit_kind"}
            g.op(ck, list(op.inputs), [g.value(f"{op.outputs[0].name}.commit", (1,), DType.U32)], domain=op.domain,
                 klass=op.klass, **attrs)
    table = g.values.get(draft_table)
    if table is None and table_shape is not None:
        table = g.const(draft_table, tuple(int(d) for d in table_shape), DType.BF16)
    if table is None:
        raise ValueError(f"lower_round: the graph has no constant {draft_table!r} (the drafts per position)")
    pos = g.values.get("position") or g.input("position", (1,), DType.U32)
    words = int(table.shape[1])
    drafts = g.value("drafts", (1, words), DType.BF16)
    g.op("embed", [pos, table], [drafts], domain=BlockDomain("rows", 1), klass=OpClass.MAP)
    sel = g.value("verify_len", (1,), DType.U32)
    attrs: Dict[str, Any] = dict(gamma=gamma)
    if verify_length is not None:
        attrs["fixed"] = int(verify_length)
    else:
        attrs["threshold"] = float(0.0 if threshold is None else threshold)
    g.op("verify_select", [drafts], [sel], domain=BlockDomain("span", 1), klass=OpClass.SERIAL, **attrs)
    return sel


@dispatch("compile")
def compile_program(model, pack, profile: Profile, *, t: Optional[int] = None, eos=None,
                    ring_capacity: Optional[int] = None, layout: Optional[StepStateLayout] = None,
                    dynamic_t: bool = False, gamma: int = 0, verify_length: Optional[int] = None,
                    draft_table: str = "draft_table", **options: Any) -> Program:
    """Lower ``model`` (anything with the reference's ``lower(g) -> token`` contract: ``nn.HybridDecoder``, a
    reference model) and emit its step program from ``pack``. ``gamma`` > 0 appends the speculative round
    (``lower_round``; verify block of ``1 + gamma`` rows, ``dynamic_t``) instead of the advance."""
    g = Graph("step")
    token = model.lower(g)
    if not gamma:
        g.check()
        return emit_program(g, pack=pack, profile=profile, t=t, layout=layout, eos=eos, ring_capacity=ring_capacity,
                            tail="advance", token=token, **options)
    aux = next((pk.aux[draft_table] for pk in ([pack] if hasattr(pack, "manifest") else pack)
                if draft_table in pk.aux), None)
    shape = None if aux is None else (aux["shape"][0], aux["nbytes"] // aux["shape"][0] // 2)
    lower_round(g, token, gamma=gamma, draft_table=draft_table, verify_length=verify_length, table_shape=shape)
    g.check()
    return emit_program(g, pack=pack, profile=profile, t=t or gamma + 1, dynamic_t=True, layout=layout, eos=eos,
                        ring_capacity=ring_capacity, tail=None, speculative=True, **options)
