"""``handler(ctx, op)`` emitters of the decode path's op kinds for gfx950: each turns an IR op into one program op on
a typed entry point of libmi355 — the descriptor's scalars in ``meta["desc"]``, its pointers as bindings (the
reference's handler table, ``compiler/emit.py:1381-1386``; the handler contract, ``:97-166``).

The step-state fields the kernels read on the device come from the program's StepState buffer: the GDN step's parity
and stop flag, attention's position, the embedding's pending tokens, the advance's whole state. Workspaces (split-K
partials and fold counters, attention partials, argmax partials) are program buffers sized by the library's own
``*_workspace_bytes`` for the op's shape and zero-initialized (their counters return to zero after every launch).
"""

from __future__ import annotations

import ctypes as C
from typing import Any, Dict, Optional, Sequence, Tuple

from ..runtime import hip
from .context import EmitContext
from .ir import Op, Value, Weight

EPILOGUE = {None: hip.MI_EPI[None], "residual": hip.MI_EPI["residual"], "silu_mul": hip.MI_EPI["silu_mul"],
            "silu_mul_rounded": hip.MI_EPI["silu_mul_rounded"]}


def _field_index(desc_cls, name: str) -> int:
    return [f for f, _ in desc_cls._fields_].index(name)


def _state(ctx: EmitContext, name: str) -> Tuple[str, int]:
    return ctx.program.step_state, ctx.layout.offset(name)


def lib_op(ctx: EmitContext, entry: str, desc_cls, scalars: Dict[str, Any], pointers: Dict[str, Any], name: str,
           writes: Sequence[str] = ()):
    """One program op on the entry point ``entry``: scalar descriptor fields, pointer fields bound to buffers (a
    value, or a ``(buffer, offset)`` pair)."""
    bindings = []
    for fld, where in pointers.items():
        if where is None:
            continue
        bname, off = where if isinstance(where, tuple) else ctx.buf(where)
        bindings.append((_field_index(desc_cls, fld), bname, int(off)))
    return ctx.add(ctx.library(entry), bindings, (0, 0, 0), (0, 0, 0), name,
                   writes=[_field_index(desc_cls, w) for w in writes], desc=dict(scalars), entry=entry)


def _probe(desc_cls, scalars: Dict[str, Any], pointer_fields: Sequence[str]):
    """A descriptor with dummy non-null pointers, for the host-only sizing calls (``*_workspace_bytes``)."""
    d = desc_cls(**{k: v for k, v in scalars.items() if not isinstance(v, (list, tuple))})
    for f in pointer_fields:
        setattr(d, f, 256)
    return d


# ---- GEMV family -------------------------------------------------------------------------------------------------
def _gemv_common(ctx: EmitContext, op: Op, *, out_f32: bool = False, grouped: bool = False):
    x, w = op.inputs[0], op.inputs[1]
    assert isinstance(w, Weight)
    y = op.outputs[0]
    a = op.attrs
    epi = a.get("epilogue")
    residual = a.get("residual")
    norm_w = a.get("norm_w")
    gated = a.get("gated_norm")                     # (w [128] f32 value, z value, eps)
    m = a.get("tokens", x.shape[0])
    scalars = dict(format=hip.MI_FMT[w.format], n=w.n, k=w.k, m=m, ldx=x.row_stride, ldy=y.row_stride,
                   epilogue=EPILOGUE[epi], ldr=residual.row_stride if residual is not None else 0,
                   eps=float(a.get("eps", 1e-6)), out_f32=int(out_f32))
    ptrs: Dict[str, Any] = dict(w=w, row_scale=w.row_scale, x=x, y=y, residual=residual, norm_w=norm_w)
    if gated is not None:
        gw, gz, geps = gated
        scalars.update(ld_gnorm_z=gz.row_stride, gnorm_eps=float(geps))
        ptrs.update(gnorm_w=gw, gnorm_z=gz)
    if grouped:
        groups = op.inputs[2]
        scalars.update(max_groups=groups.shape[0], top_k=a["top_k"], x_per_slot=int(a.get("x_per_slot", False)),
                       shared_expert=int(a.get("shared_expert", 0)),
                       shared_epilogue=EPILOGUE[a.get("shared_epilogue")])
        ptrs["groups"] = groups
        route = a.get("route")
        if route is not None:                       # one token: the launch routes for itself
            scalars.update(route_experts=route["logits"].shape[1], route_top_k=route["top_k"],
                           route_renorm=int(route.get("renorm", True)), route_gate_col=route.get("gate_col", 0),
                           route_ld=route["logits"].row_stride)
            ptrs.update(route_logits=route["logits"], route_ids=route["ids"], route_weights=route["weights"])
    probe = _probe(hip.MiGemvDesc, scalars, [f for f, v in ptrs.items() if v is not None])
    need = int(hip.load().mi_gemv_workspace_bytes(C.byref(probe)))
    if need:
        scalars["workspace_bytes"] = need
        ptrs["workspace"] = (ctx.scratch("gemv", need, shared=True), 0)
    return scalars, ptrs


def gemv(ctx: EmitContext, op: Op):
    """``gemv`` (``ops/gemv.py:1-12``): y = x·Wᵀ, the norm fused on load, residual / silu·mul epilogues."""
    scalars, ptrs = _gemv_common(ctx, op)
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, op.attrs.get("name", "gemv"), writes=("y",))


def lm_head(ctx: EmitContext, op: Op):
    """``lm_head`` (``ops/gemv.py:12``): the GEMV with FP32 output (``out_f32``) unless the op asks for BF16
    logits (``attrs["bf16"]``, what the argmax and sampler read)."""
    scalars, ptrs = _gemv_common(ctx, op, out_f32=not op.attrs.get("bf16", False))
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, op.attrs.get("name", "lm_head"), writes=("y",))


def moe_gemv(ctx: EmitContext, op: Op):
    """``moe_gemv`` (``ops/moe.py``): the grouped GEMV over the experts the route chose."""
    scalars, ptrs = _gemv_common(ctx, op, grouped=True)
    writes = ("y", "groups", "route_ids", "route_weights") if op.attrs.get("route") is not None else ("y",)
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, op.attrs.get("name", "moe_gemv"), writes=writes)


def rmsnorm_stat(ctx: EmitContext, op: Op):
    h, stat = op.inputs[0], op.outputs[0]
    return lib_op(ctx, "mi_rmsnorm_stat", hip.MiNormDesc, dict(t=h.shape[0], k=h.shape[1], ldh=h.row_stride,
                                                               stat_parts=1),
                  dict(h=h, stat=stat), op.attrs.get("name", "rmsnorm_stat"), writes=("stat",))


def norm_apply(ctx: EmitContext, op: Op):
    h, w = op.inputs[0], op.inputs[1]
    stat = op.inputs[2] if len(op.inputs) > 2 else None
    x = op.outputs[0]
    return lib_op(ctx, "mi_norm_apply", hip.MiNormDesc,
                  dict(t=h.shape[0], k=h.shape[1], ldh=h.row_stride, stat_parts=1, ldx=x.row_stride,
                       eps=float(op.attrs.get("eps", 1e-6))),
                  dict(h=h, stat=stat, w=w, x=x), op.attrs.get("name", "norm_apply"), writes=("x",))


# ---- Gated DeltaNet ----------------------------------------------------------------------------------------------
def _gdn(ctx: EmitContext, op: Op, commit: bool):
    proj, conv, rec = op.inputs[0], op.inputs[1], op.inputs[2]
    a = op.attrs
    hk, hv = a["k_heads"], a["v_heads"]
    dk, dv, cw = a.get("dk", 128), a.get("dv", 128), a.get("conv_width", 4)
    kd, vd = hk * dk, hv * dv
    conv_dim = 2 * kd + vd
    offs = a.get("offsets") or (0, vd, vd + kd, vd + 2 * kd, vd + conv_dim, vd + conv_dim + hv)
    scalars = dict(t=proj.shape[0], k_heads=hk, v_heads=hv, dk=dk, dv=dv, conv_width=cw, ld_proj=proj.row_stride,
                   z_off=offs[0], q_off=offs[1], k_off=offs[2], v_off=offs[3], a_off=offs[4], b_off=offs[5],
                   eps=float(a.get("eps", 1e-6)), defer_norm=int(a.get("defer_norm", False)), commit=int(commit))
    rec_out = a.get("rec_out", rec)
    ptrs = dict(proj=proj, conv_w=a["conv_w"], neg_exp_a=a["neg_exp_a"], dt_bias=a["dt_bias"], norm_w=a["norm_w"],
                conv_in=conv, rec_in=rec, rec_out=rec_out, done=_state(ctx, "done"), step=_state(ctx, "step"))
    if commit:
        ptrs["t_dev"] = _state(ctx, "checkpoint_index")
    else:
        ptrs["y"] = op.outputs[0]
        scalars["ld_y"] = op.outputs[0].row_stride
    return lib_op(ctx, "mi_gdn_step", hip.MiGdnDesc, scalars, ptrs, a.get("name", "gdn_commit" if commit else "gdn_mixer"),
                  writes=("conv_in", "rec_out") + (() if commit else ("y",)))


def gdn_mixer(ctx: EmitContext, op: Op):
    """``gdn_mixer`` + ``gdn_norm`` (``ops/gdn.py:1-12``): the conv state in two slots chosen by the step's parity."""
    return _gdn(ctx, op, commit=False)


def gdn_commit(ctx: EmitContext, op: Op):
    """``gdn_commit`` (``ops/gdn.py:13-17``): the accept scan's committed rows replayed into the output slot."""
    return _gdn(ctx, op, commit=True)


# ---- attention ---------------------------------------------------------------------------------------------------
def gqa_decode(ctx: EmitContext, op: Op):
    """``gqa_decode`` + ``gqa_merge`` (``ops/attention.py``) over the int8 KV cache at the step state's position."""
    proj, kc, ks, vc, vs, cos, sin = op.inputs[:7]
    qn = op.inputs[7] if len(op.inputs) > 7 else None
    kn = op.inputs[8] if len(op.inputs) > 8 else None
    y = op.outputs[0]
    a = op.attrs
    d = a.get("head_dim", 128)
    scalars = dict(t=proj.shape[0], heads=a["heads"], kv_heads=a["kv_heads"], head_dim=d, rotary_dim=cos.shape[1],
                   pos=0, ctx_max=a["ctx_max"], gate=int(a.get("gate", True)), qk_norm=int(qn is not None),
                   ld_proj=proj.row_stride, eps=float(a.get("eps", 1e-6)),
                   scaling=float(a.get("scaling", d ** -0.5)), ld_y=y.row_stride,
                   kv_dtype=int(a.get("kv_dtype", hip.MI_KV_INT8)))
    ptrs = dict(proj=proj, rope_cos=cos, rope_sin=sin, q_norm=qn, k_norm=kn, k_codes=kc, k_scales=ks, v_codes=vc,
                v_scales=vs, y=y, pos_dev=_state(ctx, "position"), done=_state(ctx, "done"))
    probe = _probe(hip.MiGqaDesc, scalars, [f for f, v in ptrs.items() if v is not None])
    need = int(hip.load().mi_gqa_workspace_bytes(C.byref(probe)))
    scalars["workspace_bytes"] = need
    ptrs["workspace"] = (ctx.scratch("gqa", need, shared=True), 0)
    return lib_op(ctx, "mi_gqa_decode", hip.MiGqaDesc, scalars, ptrs, a.get("name", "gqa_decode"),
                  writes=("k_codes", "k_scales", "v_codes", "v_scales", "y"))


# ---- MoE ---------------------------------------------------------------------------------------------------------
def moe_route(ctx: EmitContext, op: Op):
    logits = op.inputs[0]
    ids, weights, groups = op.outputs
    a = op.attrs
    scalars = dict(t=logits.shape[0], n_experts=a.get("n_experts", logits.shape[1]), top_k=a["top_k"],
                   renorm=int(a.get("renorm", True)), ld_logits=logits.row_stride,
                   max_groups=groups.shape[0] if groups is not None else 0,
                   shared_expert=int(a.get("shared_expert", 0)), shared_gate_col=int(a.get("shared_gate_col", 0)))
    return lib_op(ctx, "mi_moe_route", hip.MiMoeRouteDesc, scalars,
                  dict(logits=logits, ids=ids, weights=weights, groups=groups), a.get("name", "moe_route"),
                  writes=("ids", "weights", "groups"))


def moe_combine(ctx: EmitContext, op: Op):
    h, weights = op.inputs[0], op.inputs[1]
    a = op.attrs
    shared, gate, residual = a.get("shared"), a.get("shared_gate"), a.get("residual")
    out = op.outputs[0]
    scalars = dict(t=weights.shape[0], hidden=h.shape[1], top_k=a["top_k"], ldh=h.row_stride,
                   ld_shared=shared.row_stride if shared is not None else 0,
                   ld_gate=gate.row_stride if gate is not None else 0,
                   ldr=residual.row_stride if residual is not None else 0, ldo=out.row_stride)
    return lib_op(ctx, "mi_moe_combine", hip.MiMoeCombineDesc, scalars,
                  dict(h=h, weights=weights, shared=shared, shared_gate=gate, residual=residual, out=out),
                  a.get("name", "moe_combine"), writes=("out",))


# ---- the token loop's serial ops ---------------------------------------------------------------------------------
def embed(ctx: EmitContext, op: Op):
    """``embed`` (``ops/embed.py:1-7``) of the step state's pending tokens."""
    table, out = op.inputs[0], op.outputs[0]
    return lib_op(ctx, "mi_embed", hip.MiEmbedDesc,
                  dict(t=out.shape[0], vocab=table.shape[0], hidden=table.shape[1], ldo=out.row_stride),
                  dict(tokens=_state(ctx, "pending_tokens"), table=table, out=out), op.attrs.get("name", "embed"),
                  writes=("out",))


def argmax(ctx: EmitContext, op: Op):
    """``argmax`` (``ops/sample.py:9``): the token per row, ties to the lowest index."""
    logits, ids = op.inputs[0], op.outputs[0]
    scalars = dict(t=logits.shape[0], vocab=logits.shape[1], ld=logits.row_stride, f32=int(logits.dtype == "f32"))
    probe = _probe(hip.MiArgmaxDesc, scalars, ["logits", "ids"])
    need = int(hip.load().mi_argmax_workspace_bytes(C.byref(probe)))
    scalars["workspace_bytes"] = need
    return lib_op(ctx, "mi_argmax", hip.MiArgmaxDesc, scalars,
                  dict(logits=logits, ids=ids, workspace=(ctx.scratch("argmax", need, shared=True), 0)),
                  op.attrs.get("name", "argmax"), writes=("ids",))


def advance(ctx: EmitContext, op: Op):
    """The program tail (``compiler/emit.py:1459-1462``; ``advance.metal:15-37``): the last row's token to the ring,
    position and step forward, the stop rules. The host pump reads done / error from the step state itself."""
    ids = op.inputs[0]
    eos = [int(e) for e in ctx.profile.eos][:8]
    scalars = dict(ring_cap=ctx.profile.ring_capacity, ctx_cap=ctx.profile.ctx_cap, n_eos=len(eos), eos=eos)
    return lib_op(ctx, "mi_advance", hip.MiAdvanceDesc, scalars,
                  dict(state=_state(ctx, "step"), tokens=ids, ring=(ctx.program.ring, 0)), "advance",
                  writes=("state", "ring"))


HANDLERS = {"gemv": gemv, "lm_head": lm_head, "moe_gemv": moe_gemv, "rmsnorm_stat": rmsnorm_stat,
            "norm_apply": norm_apply, "gdn_mixer": gdn_mixer, "gdn_commit": gdn_commit, "gqa_decode": gqa_decode,
            "moe_route": moe_route, "moe_combine": moe_combine, "embed": embed, "argmax": argmax, "advance": advance}
