"""Lower the decode layers built from this package (``layers.py``) to the op graph, bound to their live device memory:
the reference's layer ``lower`` methods (``nn/linear.py:63-191``, ``nn/gdn.py``, ``nn/attention.py``, ``nn/mlp.py``,
``nn/decoder.py``) for one token per step.

Weights, norms and states are the layers' own tensors (the program binds them by storage); activations between ops
are values the program allocates. Layer by layer the ops are the ones ``layers.py`` launches eagerly:

* Gated DeltaNet layer: ``gemv`` in_proj (norm fused) → ``gdn_mixer`` (conv state in two slots by the step's parity,
  the recurrent state in place; the gated norm deferred to the next GEMV where ``defers_norm``) → ``gemv`` out_proj
  (+ residual) → the MLP;
* attention layer: ``gemv`` q|gate|k|v (norm fused) → ``gqa_decode`` at the step state's position → ``gemv`` o_proj
  (+ residual) → the MLP;
* MLP: ``gemv`` gate|up (norm fused, silu·mul) → ``gemv`` down (+ residual); a MoE block (``lower_moe``) in its place:
  the shared expert, the router, ``moe_route``, the grouped ``moe_gemv`` pair and ``moe_combine``;
* the token loop: ``embed`` of the pending token → the layers → ``lm_head`` (final norm fused, BF16 logits) →
  ``argmax`` → ``advance``.
"""

from __future__ import annotations

from typing import List

from .ir import Graph, Value, Weight


def _dt(t) -> str:
    import torch
    return {torch.bfloat16: "bf16", torch.float32: "f32", torch.float16: "f16", torch.int8: "i8", torch.uint8: "u8",
            torch.int32: "i32"}[t.dtype]


def bound(name: str, t, role: str) -> Value:
    """A value held by the tensor ``t``."""
    return Value(name, tuple(t.shape), _dt(t), role=role, tensor=t)


def weight(name: str, pw) -> Weight:
    """A packed weight (``kernels.PackedWeight``) as a graph value."""
    rs = bound(f"{name}.row_scale", pw.row_scale, "weights") if pw.row_scale is not None else None
    return Weight(name, (pw.nbytes,), "u8", role="weights", tensor=pw.data, format=pw.format, n=pw.n, k=pw.k,
                  experts=pw.experts, row_scale=rs)


def act(name: str, *shape: int, dtype: str = "bf16") -> Value:
    return Value(name, tuple(shape), dtype)


def lower_moe(g: Graph, moe, h: Value, prefix: str) -> Value:
    """A ``layers.MoeBlock`` (``nn/moe.py``): the router and the shared expert's σ-gate as one BF16 GEMV of E + 1 rows
    into a row padded to 8, the top-k route with its expert groups, the grouped gate|up and down GEMVs, the weighted
    combine with the residual. With the shared expert stacked after the routed ones (``fused_shared``) it is slot k
    of every token inside the grouped launches (its own silu·mul epilogue) and of the combine, and at one token the
    gate|up launch routes for itself (no route op); otherwise the shared expert runs as two dense GEMVs first and
    the combine adds it with its gate. One stream: the ops run in this order."""
    m, e, k = g.t, moe.experts, moe.top_k
    pad = (e + 1 + 7) // 8 * 8
    norm = bound(f"{prefix}.norm", moe.norm_w, "weights")
    fused = getattr(moe, "fused_shared", False)
    s_out = None
    if not fused:
        s_act = act(f"{prefix}.shared_act", m, moe.shared_inter)
        s_out = act(f"{prefix}.shared_out", m, moe.hidden)
        g.add("gemv", [h, weight(f"{prefix}.shared_gate_up", moe.shared_gate_up.packed)], [s_act],
              epilogue="silu_mul", norm_w=norm, eps=moe.eps, name=f"{prefix}.shared_gate_up")
        g.add("gemv", [s_act, weight(f"{prefix}.shared_down", moe.shared_down.packed)], [s_out],
              name=f"{prefix}.shared_down")
    logits = act(f"{prefix}.router_logits", m, pad)
    router_out = Value(f"{prefix}.router_gate", (m, e + 1), "bf16", ld=pad, base=logits)
    route_in = Value(f"{prefix}.route_logits", (m, e), "bf16", ld=pad, base=logits)
    gate = Value(f"{prefix}.shared_gate", (m, 1), "bf16", ld=pad, offset=2 * e, base=logits)
    g.add("gemv", [h, weight(f"{prefix}.router", moe.router_gate)], [router_out], norm_w=norm, eps=moe.eps,
          name=f"{prefix}.router")
    ks = k + (1 if fused else 0)                     # slots per token
    ids = act(f"{prefix}.ids", m, ks, dtype="i32")
    wts = act(f"{prefix}.weights", m, ks, dtype="f32")
    from ..kernels import GROUP_REC
    groups = act(f"{prefix}.groups", min(e, m * k) + (1 if fused else 0), GROUP_REC, dtype="i32")
    shared = dict(shared_expert=e) if fused else {}
    inline = fused and m == 1                        # one token: the gate|up launch routes for itself
    if not inline:
        g.add("moe_route", [route_in], [ids, wts, groups], top_k=k, renorm=True, name=f"{prefix}.route",
              **(dict(shared_expert=e, shared_gate_col=e) if fused else {}))
    a = act(f"{prefix}.expert_act", m * ks, moe.inter)
    hk = act(f"{prefix}.expert_out", m * ks, moe.hidden)
    gu = moe.gate_up_s if fused else moe.gate_up
    dn = moe.down_s if fused else moe.down
    extra = dict(shared, shared_epilogue="silu_mul") if fused else {}
    if inline:
        extra["route"] = dict(logits=route_in, ids=ids, weights=wts, top_k=k, renorm=True, gate_col=e)
    g.add("moe_gemv", [h, weight(f"{prefix}.gate_up", gu), groups], [a], tokens=m, top_k=ks, x_per_slot=False,
          epilogue="silu_mul_rounded", norm_w=norm, eps=moe.eps, name=f"{prefix}.experts_gate_up", **extra)
    g.add("moe_gemv", [a, weight(f"{prefix}.down", dn), groups], [hk], tokens=m, top_k=ks, x_per_slot=True,
          name=f"{prefix}.experts_down", **shared)
    out = act(f"{prefix}.out", m, moe.hidden)
    if fused:
        g.add("moe_combine", [hk, wts], [out], top_k=ks, residual=h, name=f"{prefix}.combine")
    else:
        g.add("moe_combine", [hk, wts], [out], top_k=k, shared=s_out, shared_gate=gate, residual=h,
              name=f"{prefix}.combine")
    return out


def lower_mlp(g: Graph, mlp, h: Value, prefix: str) -> Value:
    if hasattr(mlp, "experts"):
        return lower_moe(g, mlp, h, prefix)
    inter = mlp.inter
    a = act(f"{prefix}.act", g.t, inter)
    out = act(f"{prefix}.out", g.t, h.shape[1])
    g.add("gemv", [h, weight(f"{prefix}.gate_up", mlp.gate_up.packed)], [a], epilogue="silu_mul",
          norm_w=bound(f"{prefix}.norm", mlp.norm_w, "weights"), eps=mlp.eps, name=f"{prefix}.gate_up")
    g.add("gemv", [a, weight(f"{prefix}.down", mlp.down.packed)], [out], epilogue="residual", residual=h,
          name=f"{prefix}.down")
    return out


def lower_gdn_layer(g: Graph, layer, h: Value, prefix: str) -> Value:
    hidden = layer.hidden
    proj = act(f"{prefix}.proj", g.t, layer.n_proj)
    o = act(f"{prefix}.o", g.t, layer.hv * layer.dv)
    h1 = act(f"{prefix}.h1", g.t, hidden)
    g.add("gemv", [h, weight(f"{prefix}.in_proj", layer.w_in.packed)], [proj],
          norm_w=bound(f"{prefix}.norm1", layer.norm_w, "weights"), eps=layer.eps, name=f"{prefix}.in_proj")
    defer = layer.defers_norm(g.t)
    norm_w = bound(f"{prefix}.gdn_norm", layer.gdn_norm_w, "weights")
    g.add("gdn_mixer", [proj, bound(f"{prefix}.conv", layer.conv_state, "state"),
                        bound(f"{prefix}.rec", layer.rec_state, "state")], [o],
          k_heads=layer.hk, v_heads=layer.hv, dk=layer.dk, dv=layer.dv, conv_width=layer.conv, eps=layer.eps,
          defer_norm=defer, conv_w=bound(f"{prefix}.conv_w", layer.conv_w, "weights"),
          neg_exp_a=bound(f"{prefix}.neg_exp_a", layer.neg_exp_a, "weights"),
          dt_bias=bound(f"{prefix}.dt_bias", layer.dt_bias, "weights"), norm_w=norm_w, name=f"{prefix}.gdn")
    gated = None
    if defer:                                      # z = proj[:, :hv·dv], a view with the projection's row stride
        z = Value(f"{prefix}.z", (g.t, layer.hv * layer.dv), "bf16", ld=layer.n_proj, base=proj)
        gated = (norm_w, z, layer.eps)
    g.add("gemv", [o, weight(f"{prefix}.out_proj", layer.w_out.packed)], [h1], epilogue="residual", residual=h,
          gated_norm=gated, name=f"{prefix}.out_proj")
    return lower_mlp(g, layer.mlp, h1, f"{prefix}.mlp")


def lower_attn_layer(g: Graph, layer, h: Value, prefix: str) -> Value:
    c = layer.cache
    proj = act(f"{prefix}.proj", g.t, layer.n_proj)
    o = act(f"{prefix}.o", g.t, layer.heads * layer.d)
    h1 = act(f"{prefix}.h1", g.t, layer.hidden)
    g.add("gemv", [h, weight(f"{prefix}.qkv", layer.w_qkv.packed)], [proj],
          norm_w=bound(f"{prefix}.norm1", layer.norm_w, "weights"), eps=layer.eps, name=f"{prefix}.qkv")
    scales = c.k_scales is not None
    g.add("gqa_decode", [proj, bound(f"{prefix}.k_codes", c.k_codes, "state"),
                         bound(f"{prefix}.k_scales", c.k_scales, "state") if scales else None,
                         bound(f"{prefix}.v_codes", c.v_codes, "state"),
                         bound(f"{prefix}.v_scales", c.v_scales, "state") if scales else None,
                         bound(f"{prefix}.cos", layer.cos, "weights"), bound(f"{prefix}.sin", layer.sin, "weights"),
                         bound(f"{prefix}.q_norm", layer.q_norm, "weights"),
                         bound(f"{prefix}.k_norm", layer.k_norm, "weights")], [o],
          heads=layer.heads, kv_heads=layer.kv, head_dim=layer.d, ctx_max=c.ctx_max, gate=True, eps=layer.eps,
          kv_dtype=c.kv_dtype,
          name=f"{prefix}.gqa")
    g.add("gemv", [o, weight(f"{prefix}.o_proj", layer.w_o.packed)], [h1], epilogue="residual", residual=h,
          name=f"{prefix}.o_proj")
    return lower_mlp(g, layer.mlp, h1, f"{prefix}.mlp")


def lower_layer(g: Graph, layer, h: Value, prefix: str) -> Value:
    if getattr(layer, "ping_pong", False):
        return lower_gdn_layer(g, layer, h, prefix)
    return lower_attn_layer(g, layer, h, prefix)


def lower_decoder(model) -> Graph:
    """The one-token step of a ``layers.DecoderModel``: embed → layers → final norm + lm_head → argmax → advance."""
    g = Graph(t=1)
    vocab, hidden = model.embed_table.shape
    h = act("h0", 1, hidden)
    g.add("embed", [bound("embed_table", model.embed_table, "weights")], [h])
    for i, layer in enumerate(model.layers):
        h = lower_layer(g, layer, h, f"layers.{i}")
    logits = act("logits", 1, vocab)
    ids = act("ids", 16, dtype="i32")
    g.add("lm_head", [h, weight("lm_head", model.lm_head)], [logits], norm_w=bound("norm", model.norm_w, "weights"),
          eps=model.eps, bf16=True)
    g.add("argmax", [logits], [ids])
    g.add("advance", [ids], [])
    return g


def layer_values(g: Graph) -> List[Value]:
    return g.values()
