"""A ``layers.DecoderModel`` (the hand-built decode layers) in the reference's terms: the module tree that lowers to
the same step graph (``nn.HybridDecoder``), the pack of its weights under the names that tree's ops reference
(``Packer.add_packed``: the device bytes as they are, so the program streams the same bits), and the images of its
states in the program's state buffers. ``compile_decoder`` chains them with ``compile_program``.

Pack order is part of the plan: a MoE block's router and shared-expert gate, its routed experts' gate|up and the
shared expert's, and their downs, are written back to back, which lets the emitter stack each pair into one launch
(``plan.merge_adjacent_slabs``, ``plan.fuse_shared_expert``) — the launches the hand-built block makes.
"""

from __future__ import annotations

from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np

from .. import nn as NN


def _np(t) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy()


def _bits(t) -> np.ndarray:
    """A BF16 tensor's bit patterns."""
    import torch
    return _np(t.contiguous().view(torch.int16)).view(np.uint16)


def describe(model) -> NN.HybridDecoder:
    """The module tree of ``model``'s geometry (layer kinds, heads, MoE blocks)."""
    kinds, gdn, attn, moe, moe_layers, inter = [], None, None, None, [], None
    for i, layer in enumerate(model.layers):
        if getattr(layer, "ping_pong", False):
            kinds.append("gdn")
            gdn = dict(k_heads=layer.hk, v_heads=layer.hv, dk=layer.dk, dv=layer.dv, conv_width=layer.conv)
        else:
            if getattr(layer, "layout", "checkpoint") != "packed":
                raise ValueError(f"layer {i}: the reference's graph reads the packed attention layout "
                                 "(AttnDecoderLayer(layout='packed'))")
            kinds.append("attention")
            attn = dict(heads=layer.heads, kv_heads=layer.kv, head_dim=layer.d, rotary_dim=layer.rotary_dim,
                        theta=layer.theta, gate=True)
            ctx = layer.cache.ctx_max
        mlp = layer.mlp
        if hasattr(mlp, "experts"):
            moe_layers.append(i)
            moe = dict(experts=mlp.experts, top_k=mlp.top_k, inter=mlp.inter, shared_inter=mlp.shared_inter)
        else:
            inter = mlp.inter
    ctxs = {l.cache.ctx_max for l in model.layers if not getattr(l, "ping_pong", False)}
    if len(ctxs) > 1:
        raise ValueError("the attention layers must share one context capacity (one RoPE table)")
    return NN.HybridDecoder(vocab=model.vocab, hidden=model.hidden, layer_types=kinds, inter=inter or 1,
                            eps=model.eps, gdn=gdn, attention=attn, moe=moe, moe_layers=moe_layers,
                            max_context=ctxs.pop() if ctxs else 4096)


def _slab(name: str, pw, *, n=None, experts=None) -> dict:
    return dict(name=name, format=pw.format, n=pw.n if n is None else n, k=pw.k,
                experts=pw.experts if experts is None else experts, data=_np(pw.data),
                row_scale=None if pw.row_scale is None else _np(pw.row_scale))


def write_pack(model, out_dir, spec: NN.HybridDecoder = None, tables=None):
    """Write ``model``'s weights as a gfx950 pack under ``spec``'s slab and constant names, plus ``tables``
    (``{name: (array, safetensors dtype)}``, e.g. a speculative program's ``draft_table``); returns the
    ``PackFile``."""
    from ..formats import device as DV
    from ..kernels import PackedWeight
    from ..packs import Packer, PackFile
    spec = spec or describe(model)
    out = Path(out_dir)
    pk = Packer(None, out)                           # no checkpoint: every slab arrives packed

    def f32(name, t):
        pk.add_table(name, _np(t).astype(np.float32), "F32")

    emb = PackedWeight("bf16", model.vocab, model.hidden, 1, DV.pack_bf16(model.embed_table), None)
    pk.add_packed([_slab(spec.embed_tokens.slab_name, emb)])
    for blk, layer in zip(spec.blocks, model.layers):
        f32(f"{blk.input_norm.prefix}weight", layer.norm_w)
        mx = blk.mixer
        if isinstance(mx, NN.GatedDeltaNet):
            pk.add_packed([_slab(mx.in_proj.slab_groups()[0].name, layer.w_in.packed)])
            pk.add_packed([_slab(mx.out_proj.slab_groups()[0].name, layer.w_out.packed)])
            pk.add_table(f"{mx.prefix}conv_w", _bits(layer.conv_w), "BF16")
            f32(f"{mx.prefix}a_log", layer.neg_exp_a)
            f32(f"{mx.prefix}dt_bias", layer.dt_bias)
            f32(f"{mx.prefix}norm_w", layer.gdn_norm_w)
        else:
            pk.add_packed([_slab(mx.qkv.slab_groups()[0].name, layer.w_qkv.packed)])
            pk.add_packed([_slab(mx.o_proj.slab_groups()[0].name, layer.w_o.packed)])
            f32(f"{mx.prefix}q_norm", layer.q_norm)
            f32(f"{mx.prefix}k_norm", layer.k_norm)
        mlp, m = blk.mlp, layer.mlp
        f32(f"{blk.post_norm.prefix}weight", m.norm_w)
        if isinstance(mlp, NN.SparseMoE):
            e = m.experts
            router = PackedWeight("bf16", e, m.hidden, 1, DV.pack_bf16(m.router_w), None)
            pk.add_packed([_slab(mlp.router.slab_groups()[0].name, router),
                           _slab(mlp.shared_gate.slab_groups()[0].name, m.shared_gate)])
            gu_name, dn_name = mlp.gate_up.slab.slab_groups()[0].name, mlp.down.slab.slab_groups()[0].name
            pk.add_packed([_slab(gu_name, m.gate_up), _slab(mlp.shared_gate_up.slab_groups()[0].name,
                                                              m.shared_gate_up.packed)])
            pk.add_packed([_slab(dn_name, m.down), _slab(mlp.shared_down.slab_groups()[0].name,
                                                         m.shared_down.packed)])
        else:
            pk.add_packed([_slab(mlp.gate_up.slab_groups()[0].name, m.gate_up.packed)])
            pk.add_packed([_slab(mlp.down.slab_groups()[0].name, m.down.packed)])
    attn = [l for l in model.layers if not getattr(l, "ping_pong", False)]
    if attn:
        pk.add_table("rope_cos", _bits(attn[0].cos), "BF16")
        pk.add_table("rope_sin", _bits(attn[0].sin), "BF16")
    f32(f"{spec.norm.prefix}weight", model.norm_w)
    pk.add_packed([_slab(spec.lm_head.slab_name, model.lm_head)])
    for name, (arr, dtype) in (tables or {}).items():
        pk.add_table(name, np.asarray(arr), dtype)
    pk.write({"model": "decoder", "layers": [type(l).__name__ for l in model.layers]})
    return PackFile(out)


def state_images(model, spec: NN.HybridDecoder = None) -> Dict[str, bytes]:
    """The bytes to load into the program's state buffers so it continues from ``model``'s states: the GDN conv
    state with the current slot first (the program's step 0 reads slot 0), the recurrent state in slot 0, and the
    KV caches in the backend's layout (int8 codes with their scales in ``<cache>.scales``, or BF16 values)."""
    import torch
    spec = spec or describe(model)
    out: Dict[str, bytes] = {}
    for blk, layer in zip(spec.blocks, model.layers):
        mx = blk.mixer
        if isinstance(mx, NN.GatedDeltaNet):
            cs = layer.conv_state
            cur, other = cs[layer.parity], cs[1 - layer.parity]
            out[f"{mx.prefix}conv_state"] = _np(torch.stack([cur, other]).contiguous().view(torch.int16)).tobytes()
            rec = layer.rec
            out[f"{mx.prefix}rec_state"] = _np(torch.stack([rec, torch.zeros_like(rec)])).tobytes()
        else:
            c = layer.cache
            out[f"{mx.prefix}k_cache"] = _np(c.k_codes.contiguous().view(torch.uint8)).tobytes()
            out[f"{mx.prefix}v_cache"] = _np(c.v_codes.contiguous().view(torch.uint8)).tobytes()
            if c.k_scales is not None:
                out[f"{mx.prefix}k_cache.scales"] = _np(c.k_scales.contiguous().view(torch.uint8)).tobytes()
                out[f"{mx.prefix}v_cache.scales"] = _np(c.v_scales.contiguous().view(torch.uint8)).tobytes()
    return out


def compile_decoder(model, out_dir, profile, *, tables=None, **options) -> Tuple[object, object, Dict[str, bytes]]:
    """``(program, pack, state images)`` of ``model``'s step: its pack written to ``out_dir`` (with ``tables``), its
    module tree lowered to the reference-contract graph and emitted from that pack (``options`` go to
    ``compile_program``: ``t``, ``gamma`` …)."""
    from .emit import compile_program
    spec = describe(model)
    pack = write_pack(model, out_dir, spec, tables)
    return compile_program(spec, pack, profile, **options), pack, state_images(model, spec)


def load_states(engine, images: Dict[str, bytes]) -> None:
    """Write state images into an Engine's buffers (every name must be a state buffer of its program)."""
    for name, data in images.items():
        spec = engine.program.buffers.get(name)
        if spec is None or spec.role != "state":
            raise KeyError(f"{name}: not a state buffer of the program")
        if len(data) > spec.nbytes:
            raise ValueError(f"{name}: {len(data)} bytes for a {spec.nbytes}-byte state")
        engine.buffers[name].write(data, 0)
