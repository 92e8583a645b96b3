"""``handler(ctx, op)`` emitters for gfx950 (the reference's handler table, ``compiler/emit.py:1381-1386``; the handler
contract, ``:97-166``): each turns one op of the lowered plan into a program op on a typed entry point of libmi355
— the descriptor's scalars in ``meta["desc"]``, its pointers as bindings ``(field index, buffer, offset)``.

The ops arrive in the reference's contract (input positions and attrs as ``monolith/nn`` lowers them,
``compiler/emit.py:259-1378`` reads them), after the plan's passes fused the split ones (``plan.py``). Weights
resolve by slab name to windows of the pack (``ctx.windows`` / ``ctx.row_scales``); a row range of a slab is an
offset into it (whole 16-row tiles). Step-state fields the kernels read on the device come from the program's step
state: the GDN step's parity and stop flag, attention's position, the embedding's pending tokens, the commit's
accepted count. Workspaces (split-K partials and fold counters, attention partials, argmax partials) are program
buffers sized by the library's own ``*_workspace_bytes`` and zeroed at allocation (their counters return to zero
after every launch).
"""

from __future__ import annotations

import ctypes as C
from typing import Any, Dict, Optional, Sequence, Tuple

from ..formats import pack as T16
from ..runtime import hip
from .context import EmitContext
from .plan import POp

EPILOGUE = {None: hip.MI_EPI[None], "residual": hip.MI_EPI["residual"], "silu_mul": hip.MI_EPI["silu_mul"],
            "silu_mul_rounded": hip.MI_EPI["silu_mul_rounded"]}
GROUP_REC = 18


def _field_index(desc_cls, name: str) -> int:
    return [f for f, _ in desc_cls._fields_].index(name)


def lib_op(ctx: EmitContext, entry: str, desc_cls, scalars: Dict[str, Any], pointers: Dict[str, Any], name: str,
           writes: Sequence[str] = ()):
    """One program op on the entry point ``entry``: scalar descriptor fields, pointer fields bound to buffers (a
    plan value, or a ``(buffer, offset)`` pair)."""
    bindings = []
    for fld, where in pointers.items():
        if where is None:
            continue
        bname, off = ctx.buf(where)
        bindings.append((_field_index(desc_cls, fld), bname, int(off)))
    return ctx.add(ctx.library(entry), bindings, (0, 0, 0), (0, 0, 0), name,
                   writes=[_field_index(desc_cls, w) for w in writes if pointers.get(w) is not None],
                   desc=dict(scalars), entry=entry)


def _probe(desc_cls, scalars: Dict[str, Any], pointer_fields: Sequence[str]):
    """A descriptor with dummy non-null pointers, for the host-only sizing calls (``*_workspace_bytes``)."""
    d = desc_cls(**{k: v for k, v in scalars.items() if not isinstance(v, (list, tuple))})
    for f in pointer_fields:
        setattr(d, f, 256)
    return d


def _rows(ctx: EmitContext, v) -> int:
    return ctx.plan.shape(v)[0]


# ---- weights -----------------------------------------------------------------------------------------------------
def _weight(ctx: EmitContext, w, start: int = 0) -> Tuple[dict, Tuple[str, int], Optional[Tuple[str, int]]]:
    """The slab entry of weight value ``w`` and the (buffer, offset) of its codes and row scales from row ``start``
    (a whole tile)."""
    s = ctx.slab(w.name)
    if start % 16:
        raise ValueError(f"{w.name}: a row range must start on a 16-row tile (row {start})")
    per_tile = T16.pack_bytes(s["format"], 16, s["k"])
    b, off = ctx.windows[w.name]
    codes = (b, off + (start // 16) * per_tile)
    rs = None
    if w.name in ctx.row_scales:
        rb, roff = ctx.row_scales[w.name]
        rs = (rb, roff + 4 * start)
    return s, codes, rs


# ---- GEMV family -------------------------------------------------------------------------------------------------
def _gemv_inputs(op: POp):
    """x, w, (stat, norm_w), residual by the reference's positions (``compiler/emit.py:321-329``)."""
    ins = list(op.inputs)
    x, w, rest = ins[0], ins[1], ins[2:]
    nw = None
    if op.attrs.get("norm"):
        nw, rest = rest[1], rest[2:]
    residual = rest[0] if op.attrs.get("epilogue") == "residual" else None
    return x, w, nw, residual


def _gemv_desc(ctx: EmitContext, op: POp, *, out_f32: bool = False):
    a = op.attrs
    x, w, nw, residual = _gemv_inputs(op)
    if a.get("round_silu") or a.get("round_residual"):
        raise NotImplementedError(f"gemv {w.name}: round_silu / round_residual are not built for gfx950")
    rr = a.get("row_range")
    start = int(rr[0]) if rr is not None else 0
    s, codes, rs = _weight(ctx, w, start)
    n = int(a["n_rows"]) if "n_rows" in a else int(rr[1]) if rr is not None else s["n"] * s["experts"]
    y = op.outputs[0]
    eps = float(a.get("eps", 1e-6))
    if nw is None and a.get("fused_norm") is not None:
        nw, eps = a["fused_norm"]
    scalars = dict(format=hip.MI_FMT[s["format"]], n=n, k=s["k"], m=_rows(ctx, x), ldx=ctx.ld(x), ldy=ctx.ld(y),
                   epilogue=EPILOGUE[a.get("epilogue")], ldr=ctx.ld(residual) if residual is not None else 0,
                   eps=eps, out_f32=int(out_f32))
    ptrs: Dict[str, Any] = dict(w=codes, row_scale=rs, x=x, y=y, residual=residual, norm_w=nw)
    gated = a.get("gated_norm")                                      # (norm_w, z, eps): the GDN norm on load
    if gated is not None:
        gw, gz, geps = gated
        scalars.update(ld_gnorm_z=ctx.ld(gz), gnorm_eps=float(geps))
        ptrs.update(gnorm_w=gw, gnorm_z=gz)
    nn = a.get("next_norm")                                           # (norm_w, x_next, eps): the next RMSNorm
    if nn is not None:
        nnw, nnx, neps = nn
        scalars.update(ld_next_x=ctx.ld(nnx), next_eps=float(neps))
        ptrs.update(next_norm_w=nnw, next_x=nnx)
    conv = a.get("conv")                                              # the GDN short conv in the epilogue
    if conv is not None:
        scalars.update(conv_row0=int(conv["row0"]), conv_channels=int(conv["channels"]), ld_conv=ctx.ld(conv["out"]))
        ptrs.update(conv_w=conv["w"], conv_in=conv["state"], conv_out=conv["out"], conv_step=ctx.field("step"),
                    conv_done=ctx.field("done"))
    return scalars, ptrs


def _workspace(ctx: EmitContext, scalars, ptrs) -> None:
    probe = _probe(hip.MiGemvDesc, scalars, [f for f, v in ptrs.items() if v is not None])
    need = int(hip.load().mi_gemv_workspace_bytes(C.byref(probe)))
    if need:
        scalars["workspace_bytes"] = need
        ptrs["workspace"] = (ctx.scratch("gemv", need, shared=True), 0)


def gemv(ctx: EmitContext, op: POp):
    """``gemv`` (``ops/gemv.py:1-12``): y = x·Wᵀ, the norm fused on load, residual / silu·mul epilogues."""
    scalars, ptrs = _gemv_desc(ctx, op)
    _workspace(ctx, scalars, ptrs)
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, f"gemv:{op.inputs[1].name}",
                  writes=("y", "conv_in", "conv_out", "next_x"))


def lm_head(ctx: EmitContext, op: POp):
    """``lm_head`` (``ops/gemv.py:12``): BF16 logits when the op asks for them (``out="bf16"``, what the argmax and
    sampler read), FP32 otherwise."""
    scalars, ptrs = _gemv_desc(ctx, op, out_f32=op.attrs.get("out") != "bf16")
    _workspace(ctx, scalars, ptrs)
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, "lm_head", writes=("y",))


def moe_gemv(ctx: EmitContext, op: POp):
    """``moe_gemv`` (``ops/moe.py``; ``compiler/emit.py:1329-1353``): the expert projection over the experts the route
    chose — the grouped GEMV over the route's expert groups. Gate|up takes the experts' rounding (gate and up each
    rounded to BF16, ``nn/moe.py:52-62``); the shared expert, when it is a slot of the launch, its own (one
    rounding, ``nn/mlp.py:25-26``)."""
    a = op.attrs
    x, w, _ids = op.inputs
    s, codes, rs = _weight(ctx, w)
    rows = int(a["expert_rows"])
    silu = a.get("epilogue") == "silu_mul"
    slots = int(a.get("slots", a["top_k"]))
    y = op.outputs[0]
    t = _rows(ctx, y)
    eps = 1e-6
    nw = None
    if a.get("fused_norm") is not None:
        nw, eps = a["fused_norm"]
    k_in = s["k"]
    n_out = rows // 2 if silu else rows
    groups = a["groups"]
    scalars = dict(format=hip.MI_FMT[s["format"]], n=rows, k=k_in, m=t,
                   ldx=k_in if a.get("x_per_slot") else ctx.ld(x), ldy=n_out,
                   epilogue=EPILOGUE["silu_mul_rounded" if silu else None], eps=eps,
                   max_groups=ctx.plan.shape(groups)[0], top_k=slots, x_per_slot=int(bool(a.get("x_per_slot"))),
                   shared_expert=int(a.get("shared_expert", 0)),
                   shared_epilogue=EPILOGUE[a.get("shared_epilogue")] if a.get("shared_expert") else 0,
                   group_max_pairs=int(a.get("pairs_per_record", 0)))
    ptrs: Dict[str, Any] = dict(w=codes, row_scale=rs, x=x, y=y, norm_w=nw, groups=groups)
    writes = ["y"]
    route = a.get("route_op")
    if route is not None:                         # one token: the launch routes for itself
        logits = route.inputs[0]
        scalars.update(route_experts=int(route.attrs["n_experts"]), route_top_k=int(route.attrs["top_k"]),
                       route_renorm=int(bool(route.attrs.get("renorm", True))),
                       route_gate_col=int(route.attrs.get("shared_gate_col", 0)), route_ld=ctx.ld(logits))
        ptrs.update(route_logits=logits, route_ids=route.outputs[0], route_weights=route.outputs[1])
        writes += ["groups", "route_ids", "route_weights"]
    _workspace(ctx, scalars, ptrs)
    return lib_op(ctx, "mi_gemv", hip.MiGemvDesc, scalars, ptrs, f"moe_gemv:{w.name.split('.e0.')[0]}",
                  writes=writes)


def rmsnorm_stat(ctx: EmitContext, op: POp):
    h, stat = op.inputs[0], op.outputs[0]
    return lib_op(ctx, "mi_rmsnorm_stat", hip.MiNormDesc, dict(t=_rows(ctx, h), k=ctx.plan.width(h), ldh=ctx.ld(h),
                                                               stat_parts=1),
                  dict(h=h, stat=stat), "rmsnorm_stat", writes=("stat",))


def norm_apply(ctx: EmitContext, op: POp):
    """``norm_apply`` (``ops/norm.py:11-12``): x = bf16(h·rsqrt(stat/K + eps)·(1 + w)); with its statistic's op
    fused away the entry point computes the statistic itself, in the same order."""
    h, stat, w = op.inputs
    x = op.outputs[0]
    if op.attrs.get("stat_computed"):
        stat = None
    return lib_op(ctx, "mi_norm_apply", hip.MiNormDesc,
                  dict(t=_rows(ctx, h), k=ctx.plan.width(h), ldh=ctx.ld(h), stat_parts=1, ldx=ctx.ld(x),
                       eps=float(op.attrs.get("eps", 1e-6))),
                  dict(h=h, stat=stat, w=w, x=x), "norm_apply", writes=("x",))


# ---- Gated DeltaNet ----------------------------------------------------------------------------------------------
def _gdn_layout(ctx: EmitContext, op: POp):
    """The projection the step reads: one buffer holding z | q | k | v (| a | b) at column offsets, a|b possibly in
    a second one (mixed storage formats), from the op's ``proj_segments`` (``nn/gdn.py:95-112``)."""
    a = op.attrs
    ps = a["proj_segments"]
    n_main = 1 + max(idx for idx, _, _ in ps.values())
    mains = op.inputs[:n_main]
    cs, rs, conv_w, nea, dtb = op.inputs[n_main:n_main + 5]
    kd = a["k_heads"] * a["dk"]
    plan = ctx.plan
    root0, c0 = plan.root(mains[ps["in_proj_qkv"][0]])
    q_off = c0 + ps["in_proj_qkv"][1]
    lay = dict(ld_proj=ctx.ld(mains[ps["in_proj_qkv"][0]]), q_off=q_off, k_off=q_off + kd, v_off=q_off + 2 * kd)
    z = a.get("z")
    if z is not None:
        zr, zc = plan.root(z)
        if zr != root0:
            raise NotImplementedError("gdn_mixer: the z rows and the q|k|v rows must come from one slab (the "
                                      "projection's first format group)")
        lay["z_off"] = zc
    ia, ib = ps["in_proj_a"], ps["in_proj_b"]
    ab_val = mains[ia[0]]
    ab_root, ab_c = plan.root(ab_val)
    ab = None
    if ab_root == root0:
        lay.update(a_off=ab_c + ia[1], b_off=ab_c + ib[1], ld_ab=0)
    else:
        ab = (ab_val, ab_c)
        lay.update(a_off=ia[1], b_off=ib[1], ld_ab=ctx.ld(ab_val))
    proj = (plan.values[root0], 0)
    return lay, proj, ab, cs, rs, conv_w, nea, dtb


def _state_slot(ctx: EmitContext, st, slot: int):
    """(buffer, offset) of slot ``slot`` of a two-slot state value ``[2, ...]``."""
    b, off = ctx.buf(st)
    shape = ctx.plan.shape(st)
    if shape[0] != 2:
        raise ValueError(f"{st.name}: a Gated DeltaNet state needs two slots (StateEntry.checkpoints = 2), got {shape}")
    from .context import _itemsize, _numel
    return b, off + slot * _numel(shape[1:]) * _itemsize(st)


def _gdn(ctx: EmitContext, op: POp, commit: bool):
    a = op.attrs
    lay, proj, ab, cs, rs, conv_w, nea, dtb = _gdn_layout(ctx, op)
    pb, poff = ctx.buf(proj[0])
    speculative = any(o.kind == "gdn_commit" for o in ctx.plan.ops)
    t = ctx.plan.shape(op.inputs[0])[0]
    scalars = dict(t=t, k_heads=a["k_heads"], v_heads=a["v_heads"], dk=a["dk"], dv=a["dv"],
                   conv_width=a["conv_width"], eps=float(a.get("norm_eps", a.get("eps", 1e-6))),
                   defer_norm=int(bool(a.get("defer_norm"))), commit=int(commit), z_off=lay.get("z_off", 0),
                   ld_proj=lay["ld_proj"], q_off=lay["q_off"], k_off=lay["k_off"], v_off=lay["v_off"],
                   a_off=lay["a_off"], b_off=lay["b_off"], ld_ab=lay["ld_ab"])
    # the recurrent state stays in slot 0; a verify pass writes its rows' state into slot 1, and the commit replays
    # the accepted rows from slot 0 into slot 0 (in place, as a plain step does)
    slot0 = _state_slot(ctx, rs, 0)
    rec_out = _state_slot(ctx, rs, 1) if (speculative and not commit) else slot0
    ptrs: Dict[str, Any] = dict(proj=(pb, poff), conv_w=conv_w, neg_exp_a=nea, dt_bias=dtb, norm_w=a.get("norm_w"),
                                conv_in=ctx.buf(cs), rec_in=slot0, rec_out=rec_out, done=ctx.field("done"),
                                step=ctx.field("step"))
    if ab is not None:                               # a|b in their own slab's output (a second storage format)
        ptrs["ab"] = ctx.buf(ab[0])
    if a.get("pre") is not None and not commit:       # the conv ran in the input projection
        ptrs["pre"] = a["pre"]
        scalars["ld_pre"] = ctx.ld(a["pre"])
    if commit:
        ptrs["t_dev"] = ctx.field("checkpoint_index")
    else:
        y = op.outputs[0]
        ptrs["y"] = y
        scalars["ld_y"] = ctx.ld(y)
        if a.get("norm_w") is None:
            raise NotImplementedError("gdn_mixer: the read-out must be normed (gdn_norm fused)")
    return lib_op(ctx, "mi_gdn_step", hip.MiGdnDesc, scalars, ptrs, "gdn_commit" if commit else "gdn_mixer",
                  writes=("conv_in", "rec_out", "y"))


def gdn_mixer(ctx: EmitContext, op: POp):
    """``gdn_mixer`` + ``gdn_norm`` (``ops/gdn.py:1-12``): conv state in two slots chosen by the step's parity, the
    recurrent state, the gated norm (or the read-out for the output projection to norm, ``defer_norm``)."""
    return _gdn(ctx, op, commit=False)


def gdn_commit(ctx: EmitContext, op: POp):
    """``gdn_commit`` (``ops/gdn.py:13-17``): the accept scan's committed rows replayed from the step's input state."""
    return _gdn(ctx, op, commit=True)


# ---- attention ---------------------------------------------------------------------------------------------------
def gqa_decode(ctx: EmitContext, op: POp):
    """``gqa_decode`` + ``gqa_merge`` (``ops/attention.py``; ``compiler/emit.py:868-983``): q/k norm, RoPE (the
    reference's permuted layout: full-width pairs over ``[ctx, D]`` tables), the new keys into the cache at the step
    state's position, attention over the cache, the merge and × σ(gate) in one entry point."""
    proj, kc, vc, cos, sin, qn, kn = op.inputs
    y = op.outputs[0]
    a = op.attrs
    d, heads, kv = int(a["head_dim"]), int(a["heads"]), int(a["kv_heads"])
    segs = {name: (off, n) for name, off, n in a["segments"]}
    if segs.get("q", (0,))[0] != 0 or segs["k"][0] != heads * d or segs["v"][0] != (heads + kv) * d:
        raise NotImplementedError(f"gqa_decode: the projection must hold q | k | v in order (segments {a['segments']})")
    ctx_max = ctx.plan.shape(kc)[0]
    rot = d if a.get("rope") == "permuted" else int(a["rotary_dim"])
    gate_v = a.get("gate_value")
    int8 = ctx.profile.kv_cache == "int8"
    scalars = dict(t=_rows(ctx, proj), heads=heads, kv_heads=kv, head_dim=d, rotary_dim=rot, pos=0, ctx_max=ctx_max,
                   gate=int(bool(a.get("gate", gate_v is not None))), qk_norm=int(bool(a.get("qk_norm", True))),
                   ld_proj=ctx.ld(proj), eps=float(a.get("eps", 1e-6)), scaling=float(a.get("scaling", d ** -0.5)),
                   ld_y=ctx.ld(y), kv_dtype=hip.MI_KV_INT8 if int8 else hip.MI_KV_BF16,
                   ld_gate=ctx.ld(gate_v) if gate_v is not None else 0)
    ptrs: Dict[str, Any] = dict(proj=proj, rope_cos=cos, rope_sin=sin, q_norm=qn if scalars["qk_norm"] else None,
                                k_norm=kn if scalars["qk_norm"] else None, k_codes=kc, v_codes=vc, y=y,
                                pos_dev=ctx.field("position"), done=ctx.field("done"), gate_src=gate_v)
    if int8:                                       # per (token, KV head) f16 scales: state buffers of their own
        for side, cache in (("k_scales", kc), ("v_scales", vc)):
            ptrs[side] = (_scales_buffer(ctx, cache, kv * ctx_max * 2), 0)
    probe = _probe(hip.MiGqaDesc, scalars, [f for f, v in ptrs.items() if v is not None])
    need = int(hip.load().mi_gqa_workspace_bytes(C.byref(probe)))
    scalars["workspace_bytes"] = need
    ptrs["workspace"] = (ctx.scratch("gqa", need, shared=True), 0)
    return lib_op(ctx, "mi_gqa_decode", hip.MiGqaDesc, scalars, ptrs, "gqa_decode",
                  writes=("k_codes", "k_scales", "v_codes", "v_scales", "y"))


def _scales_buffer(ctx: EmitContext, cache, nbytes: int) -> str:
    from ..runtime.program import BufferSpec
    name = f"{cache.name}.scales"
    ctx.program.buffers.setdefault(name, BufferSpec(nbytes, None, "state"))
    return name


# ---- MoE ---------------------------------------------------------------------------------------------------------
def moe_route(ctx: EmitContext, op: POp):
    """``moe_route`` (``ops/moe.py``): softmax top-k per token and the expert groups the grouped GEMVs read; at one
    token with the shared expert fused, the gate|up launch routes for itself and this op emits nothing."""
    a = op.attrs
    if a.get("inline"):
        return None
    logits = op.inputs[0]
    ids, weights = op.outputs
    groups = a["groups"]
    scalars = dict(t=_rows(ctx, logits), n_experts=int(a["n_experts"]), top_k=int(a["top_k"]),
                   renorm=int(bool(a.get("renorm", True))), ld_logits=ctx.ld(logits),
                   max_groups=ctx.plan.shape(groups)[0], shared_expert=int(a.get("shared_expert", 0)),
                   shared_gate_col=int(a.get("shared_gate_col", 0)), pairs_per_record=int(a.get("pairs_per_record", 0)))
    return lib_op(ctx, "mi_moe_route", hip.MiMoeRouteDesc, scalars,
                  dict(logits=logits, ids=ids, weights=weights, groups=groups), "moe_route",
                  writes=("ids", "weights", "groups"))


def moe_combine(ctx: EmitContext, op: POp):
    """``moe_combine`` (``ops/moe.py``; ``compiler/emit.py:1356-1378``): Σ w·h over the slots (+ bf16(σ(gate))·shared)
    (+ residual), FP32, one rounding."""
    a = op.attrs
    ins = list(op.inputs)
    h, weights, rest = ins[0], ins[1], ins[2:]
    shared = gate = residual = None
    if a.get("has_shared"):
        shared, gate, rest = rest[0], rest[1], rest[2:]
    if a.get("has_residual"):
        residual = rest[0]
    out = op.outputs[0]
    hidden = ctx.plan.width(out)
    slots = int(a.get("slots", a["top_k"]))
    scalars = dict(t=_rows(ctx, out), hidden=hidden, top_k=slots, ldh=hidden,
                   ld_shared=ctx.ld(shared) if shared is not None else 0,
                   ld_gate=ctx.ld(gate) if gate is not None else 0,
                   ldr=ctx.ld(residual) if residual is not None else 0, ldo=ctx.ld(out))
    ptrs = dict(h=h, weights=weights, shared=shared, shared_gate=gate, residual=residual, out=out)
    nn = a.get("next_norm")                       # (norm_w, x_next, eps): the next RMSNorm, written by the combine
    if nn is not None:
        nnw, nnx, neps = nn
        scalars.update(ld_next_x=ctx.ld(nnx), next_eps=float(neps))
        ptrs.update(next_norm_w=nnw, next_x=nnx)
    return lib_op(ctx, "mi_moe_combine", hip.MiMoeCombineDesc, scalars, ptrs, "moe_combine", writes=("out", "next_x"))


# ---- the token loop's serial ops ---------------------------------------------------------------------------------
def embed(ctx: EmitContext, op: POp):
    """``embed`` (``ops/embed.py:1-7``): rows of the table by token id — the pack's BF16 embedding slab (gathered
    from its tiles) or a row-major constant."""
    tokens, table = op.inputs
    out = op.outputs[0]
    if getattr(table, "is_weight", False):
        s = ctx.slab(table.name)
        if s["format"] != "bf16":
            raise NotImplementedError(f"embed: the embedding slab is {s['format']}; gfx950 gathers BF16 slabs")
        vocab, hidden, t16 = s["n"], s["k"], 1
    else:
        vocab, hidden, t16 = ctx.plan.shape(table)[0], ctx.plan.width(table), 0
    return lib_op(ctx, "mi_embed", hip.MiEmbedDesc,
                  dict(t=_rows(ctx, out), vocab=vocab, hidden=hidden, ldo=ctx.ld(out), t16=t16),
                  dict(tokens=tokens, table=table, out=out), "embed", writes=("out",))


def argmax(ctx: EmitContext, op: POp):
    """``argmax`` (``ops/sample.py:9``): the token per row, ties to the lowest index."""
    logits, ids = op.inputs[0], op.outputs[0]
    f32 = str(getattr(logits.dtype, "short", logits.dtype)) == "f32"
    scalars = dict(t=_rows(ctx, logits), vocab=ctx.plan.width(logits), ld=ctx.ld(logits), f32=int(f32))
    probe = _probe(hip.MiArgmaxDesc, scalars, ["logits", "ids"])
    need = int(hip.load().mi_argmax_workspace_bytes(C.byref(probe)))
    scalars["workspace_bytes"] = need
    return lib_op(ctx, "mi_argmax", hip.MiArgmaxDesc, scalars,
                  dict(logits=logits, ids=ids, workspace=(ctx.scratch("argmax", need, shared=True), 0)),
                  "argmax", writes=("ids",))


def _eos(ctx: EmitContext):
    eos = ctx.eos
    eos = [int(e) for e in ([eos] if isinstance(eos, int) else eos) if e is not None and int(e) >= 0][:8]
    return len(eos), eos


def advance(ctx: EmitContext, token):
    """The program tail (``compiler/emit.py:1459-1462``; ``advance.metal:15-37``): the last row's token to the ring,
    position and step forward, the stop rules. The host pump reads done / error from the step state itself."""
    n_eos, eos = _eos(ctx)
    scalars = dict(ring_cap=ctx.program.ring_capacity, ctx_cap=ctx.program.context_capacity, n_eos=n_eos, eos=eos)
    return lib_op(ctx, "mi_advance", hip.MiAdvanceDesc, scalars,
                  dict(state=ctx.field("step"), tokens=token, ring=(ctx.program.ring, 0)), "advance",
                  writes=("state", "ring"))


def accept_scan(ctx: EmitContext, op: POp):
    """``accept_scan`` (``ops/draft.py:28``): the verified prefix and the bonus token to the ring, the committed
    count into the step state (``checkpoint_index``) for the commit passes, position and stop rules."""
    token = op.inputs[0]
    n_eos, eos = _eos(ctx)
    log = ctx.scratch("accept_log", 64 * 4, shared=True)
    scalars = dict(ring_cap=ctx.program.ring_capacity, ctx_cap=ctx.program.context_capacity,
                   lm=int(bool(op.attrs.get("lm"))), n_eos=n_eos, eos=eos, log_cap=64)
    return lib_op(ctx, "mi_accept_scan", hip.MiAcceptScanDesc, scalars,
                  dict(state=ctx.field("step"), tokens=token, ring=(ctx.program.ring, 0), log=(log, 0)),
                  "accept_scan", writes=("state", "ring", "log"))


def verify_select(ctx: EmitContext, op: POp):
    """``verify_select`` (``ops/draft.py:27``): the next step's verify length and rows from the drafts — a fixed
    length (``fixed``), the confident prefix (``threshold``) or the cost rule (``cost``)."""
    a = op.attrs
    drafts = op.inputs[0]
    conf = op.inputs[1] if len(op.inputs) > 1 else None
    gamma = int(a["gamma"])
    if a.get("fixed") is not None:
        mode, thr = 2, float(int(a["fixed"]))
    elif a.get("cost"):
        mode, thr = 1, float(a.get("threshold", 0.0))
    else:
        mode, thr = 0, float(a.get("threshold", 0.0))
    cost = list(a.get("cost") or [1.0] * 16)[:16]
    cost += [1.0] * (16 - len(cost))
    if conf is None:
        from ..runtime.program import BufferSpec
        ones = ctx.params("verify_select.conf", b"\x00\x00\x80\x3f" * max(gamma, 1))
        conf = (ones, 0)
    return lib_op(ctx, "mi_verify_select", hip.MiVerifySelectDesc,
                  dict(gamma=gamma, t_max=ctx.t, mode=mode, threshold=thr, cost=cost,
                       ctx_cap=ctx.program.context_capacity, lm=int(bool(a.get("lm"))), log_cap=0),
                  dict(state=ctx.field("step"), drafts=drafts, conf=conf), "verify_select", writes=("state",))


HANDLERS = {"gemv": gemv, "lm_head": lm_head, "moe_gemv": moe_gemv, "rmsnorm_stat": rmsnorm_stat,
            "norm_apply": norm_apply, "gdn_mixer": gdn_mixer, "gdn_commit": gdn_commit, "gqa_decode": gqa_decode,
            "moe_route": moe_route, "moe_combine": moe_combine, "embed": embed, "argmax": argmax,
            "accept_scan": accept_scan, "verify_select": verify_select}
