"""Decode layers composed from the HIP kernels: ``h += mixer(norm1(h)); h += mlp(norm2(h))`` (``nn/decoder.py:14-26``)
with a Gated DeltaNet (``nn/gdn.py:21-120``) or gated GQA (``nn/attention.py:27-155``) mixer and the gated MLP
(``nn/mlp.py:14-30``), every projection an NVFP4 GEMV with its RMSNorm fused on load and its residual add fused in
the epilogue. A step is 5 launches for the GDN layer and 7 for the attention layer (with MI_LAYER_CHAIN=1 the
one-token projection tail is one persistent GEMV chain launch instead of three); nothing allocates inside
``step`` when ``out`` buffers are given, so a step can be captured into a HIP graph.

Weights are synthetic (N(0, 0.02) quantized on the GPU with the reference NVFP4 rule) — there is no network for
checkpoints; ``export()`` hands the quantized codes to a checker. Each layer owns its state (GDN conv + recurrent
state, attention KV cache), so several instances are several layers of one model.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from . import kernels
from .formats import device as DV


def _torch():
    import torch
    return torch


# MI_LAYER_CHAIN=1: at one token, a layer's projection tail (output projection → gate|up → down) runs as one
# persistent GEMV chain launch (kernels.gemv_chain) instead of one launch per GEMV. Off by default: at the 27B shapes
# the chain measured slower (MLP 46–48 µs against 38–41 µs for the two launches)
CHAIN_TAIL = os.environ.get("MI_LAYER_CHAIN", "0") == "1"
# At one or two tokens the Gated DeltaNet short conv runs in the input projection's epilogue (each projection row of
# the q|k|v channels is convolved where it is produced) and the step reads the convolved values; MI_GDN_FOLD=0 keeps
# the conv inside gdn_step (A/B comparisons)
FOLD_CONV = os.environ.get("MI_GDN_FOLD", "1") != "0"


@dataclass
class QuantizedMatrix:
    """NVFP4 codes as the reference's format holds them (``weight`` [N, K/2] u8, ``weight_scale`` [N, K/16] E4M3,
    per-row tensor scale) plus the packed device weight."""

    codes: "object"
    scales: "object"
    row_scale: "object"
    packed: kernels.PackedWeight


def nvfp4_matrix(n: int, k: int, gen, device, *, gate_up: bool = False, std: float = 0.02) -> QuantizedMatrix:
    """A random N(0, std) matrix quantized to NVFP4 on the device and packed. ``gate_up``: [gate; up] halves of n/2
    rows each (own tensor scales), rows interleaved by 8 for the silu·mul epilogue (``packs/transforms.py:16-24``)."""
    torch = _torch()
    if gate_up:
        half = n // 2
        gc, gs, g2 = DV.nvfp4_quantize(torch.randn(half, k, generator=gen, device=device) * std)
        uc, us, u2 = DV.nvfp4_quantize(torch.randn(half, k, generator=gen, device=device) * std)
        codes, scales = DV.interleave_rows(gc, uc), DV.interleave_rows(gs, us)
        rs = DV.interleave_rows(torch.full((half, 1), g2, device=device),
                                torch.full((half, 1), u2, device=device)).reshape(-1)
    else:
        codes, scales, s2 = DV.nvfp4_quantize(torch.randn(n, k, generator=gen, device=device) * std)
        rs = torch.full((n,), s2, device=device)
    n_pad = -(-n // 16) * 16
    rs_pad = torch.cat([rs, rs.new_ones(n_pad - n)]) if n_pad != n else rs
    packed = kernels.PackedWeight("nvfp4", n, k, 1, DV.pack_nvfp4(codes, scales), rs_pad.contiguous())
    return QuantizedMatrix(codes, scales, rs, packed)


def _gemv_bytes(n: int, k: int, m: int, *, n_out: Optional[int] = None, residual: bool = False) -> int:
    """Algorithmic HBM bytes of one NVFP4 GEMV: codes + block scales (9/16 B per weight), x in, y out (+ residual in)."""
    n_out = n if n_out is None else n_out
    return n * k * 9 // 16 + m * k * 2 + m * n_out * 2 + (m * n_out * 2 if residual else 0)


class GatedMLP:
    """``down(silu(gate·x)·(up·x)) + residual`` with x = RMSNorm(h)(1 + w) fused into the gate|up GEMV."""

    def __init__(self, hidden: int, inter: int, gen, device, eps: float = 1e-6):
        torch = _torch()
        self.hidden, self.inter, self.eps = hidden, inter, eps
        self.norm_w = 1.0 + torch.randn(hidden, generator=gen, device=device) * 0.1     # (1 + w), float32
        self.gate_up = nvfp4_matrix(2 * inter, hidden, gen, device, gate_up=True)
        self.down = nvfp4_matrix(hidden, inter, gen, device)

    def phases(self, h, act, out):
        """The MLP as GEMV-chain phases: gate|up (norm fused, silu·mul) → down (+ residual h)."""
        return [(self.gate_up.packed, h, dict(epilogue="silu_mul", norm_w=self.norm_w, eps=self.eps, out=act)),
                (self.down.packed, act, dict(epilogue="residual", residual=h, out=out))]

    def __call__(self, h, act=None, out=None, next_norm=None, x_in=None):
        """``next_norm = (w, x_next, eps)``: also write the next RMSNorm of the output (see :func:`kernels.gemv`);
        ``x_in``: this MLP's normalized input when the caller has it (M ≥ 3), so its gate|up takes no norm."""
        if CHAIN_TAIL and h.shape[0] == 1 and next_norm is None and x_in is None:
            torch = _torch()
            if act is None:
                act = torch.empty(1, self.inter, dtype=torch.bfloat16, device=h.device)
            if out is None:
                out = torch.empty_like(h)
            return kernels.gemv_chain(self.phases(h, act, out))[1]
        if x_in is not None:
            act = kernels.gemv(self.gate_up.packed, x_in, epilogue="silu_mul", out=act)
        else:
            act = kernels.gemv(self.gate_up.packed, h, epilogue="silu_mul", norm_w=self.norm_w, eps=self.eps, out=act)
        return kernels.gemv(self.down.packed, act, epilogue="residual", residual=h, out=out, next_norm=next_norm)

    def bytes_per_step(self, m: int) -> int:
        return (_gemv_bytes(2 * self.inter, self.hidden, m, n_out=self.inter) + self.hidden * 4
                + _gemv_bytes(self.hidden, self.inter, m, residual=True))


class GdnDecoderLayer:
    """Gated DeltaNet layer (27B geometry by default: hidden 5120, 16 key / 48 value heads of 128, conv 4, MLP
    17408). Projection rows z|q|k|v|a|b (``nn/gdn.py:48-52``)."""

    def __init__(self, *, hidden=5120, k_heads=16, v_heads=48, dk=128, dv=128, conv=4, inter=17408, eps=1e-6,
                 device="cuda", seed=0):
        torch = _torch()
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.hidden, self.hk, self.hv, self.dk, self.dv, self.conv, self.eps = hidden, k_heads, v_heads, dk, dv, conv, eps
        self.conv_dim = 2 * k_heads * dk + v_heads * dv
        self.n_proj = v_heads * dv + self.conv_dim + 2 * v_heads
        self.norm_w = 1.0 + torch.randn(hidden, generator=gen, device=device) * 0.1
        self.w_in = nvfp4_matrix(self.n_proj, hidden, gen, device)
        self.w_out = nvfp4_matrix(hidden, v_heads * dv, gen, device)
        self.conv_w = (torch.randn(self.conv_dim, conv, generator=gen, device=device) * 0.3).to(torch.bfloat16)
        self.a_log = (torch.rand(v_heads, generator=gen, device=device) * 3 - 2).to(torch.bfloat16).float()
        self.neg_exp_a = -torch.exp(self.a_log)
        self.dt_bias = torch.randn(v_heads, generator=gen, device=device).to(torch.bfloat16).float()
        self.gdn_norm_w = (1.0 + torch.randn(dv, generator=gen, device=device) * 0.2).to(torch.bfloat16).float()
        self.mlp = GatedMLP(hidden, inter, gen, device, eps)
        # both conv-state slots in one tensor [2, conv_dim, W-1]: a step reads one and writes the other
        self.conv_state = torch.zeros(2, self.conv_dim, conv - 1, dtype=torch.bfloat16, device=device)
        self.conv_state[0] = (torch.randn(self.conv_dim, conv - 1, generator=gen, device=device) * 0.5).to(torch.bfloat16)
        self.rec_state = torch.randn(v_heads, dk, dv, generator=gen, device=device) * 0.1
        self.rec_slots = [self.rec_state, None]    # the second recurrent-state slot of a speculative verify pass
        self.slot = 0
        self.parity = 0
        self._bufs: Dict[int, tuple] = {}

    def pre(self, m: int):
        """The convolved q|k|v [m, conv_dim] the input projection writes when it runs the conv (m <= 2)."""
        key = ("pre", m)
        if key not in self._bufs:
            self._bufs[key] = _torch().empty(m, self.conv_dim, dtype=_torch().bfloat16, device=self.rec_state.device)
        return self._bufs[key]

    def folds_conv(self, m: int, verify: bool = False) -> bool:
        return FOLD_CONV and m <= 2 and not verify

    def buffers(self, m: int):
        torch = _torch()
        if m not in self._bufs:
            dev = self.rec_state.device
            self._bufs[m] = (torch.empty(m, self.n_proj, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.hv * self.dv, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.hidden, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.mlp.inter, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.hidden, dtype=torch.bfloat16, device=dev))
        return self._bufs[m]

    ping_pong = True          # the conv state alternates between two buffers: a captured program holds step pairs

    def defers_norm(self, m: int) -> bool:
        """Whether a step of ``m`` tokens leaves the gated RMSNorm to the output projection (``o`` then holds the
        BF16 read-out): at M <= 2 (gemv_row stages its input where the norm fits); at M >= 3 its GEMV kernel keeps
        the activations in registers and the norm stays a small kernel of its own. z must be a 16-byte aligned view
        of the projection."""
        return m <= 2 and self.n_proj % 8 == 0

    def _second_slot(self):
        if self.rec_slots[1 - self.slot] is None:
            self.rec_slots[1 - self.slot] = self.rec_slots[self.slot].clone()
        return self.rec_slots[1 - self.slot]

    def commit(self, t_dev, done=None):
        """``gdn_commit`` after a verify pass (``step(..., verify=True)``): replay the first ``t_dev`` (device int32:
        the accept scan's committed rows) tokens of that pass from its input state into the other slots, which
        become the layer's state."""
        kernels.gdn_step(self._verify_proj, self.conv_state[self.parity], self.conv_state[1 - self.parity],
                         self.rec_slots[self.slot], self._second_slot(), conv_w=self.conv_w, neg_exp_a=self.neg_exp_a,
                         dt_bias=self.dt_bias, norm_w=self.gdn_norm_w, k_heads=self.hk, v_heads=self.hv, dk=self.dk,
                         dv=self.dv, conv_width=self.conv, eps=self.eps, commit=True, t_dev=t_dev, done=done)
        self.parity ^= 1
        self.slot ^= 1

    @property
    def rec(self):
        """The current recurrent state."""
        return self.rec_slots[self.slot]

    def step(self, h, out=None, pos=None, verify: bool = False, done=None, x_in=None, next_norm=None):
        """One decode step over ``h [M, hidden]`` bf16 (M ≤ 16 tokens): returns the layer output; advances the state.
        ``pos`` is accepted for a uniform layer interface (the recurrence needs no position). ``verify``: a
        speculative verify pass — the outputs for every row, the state left for :meth:`commit`. ``done``: a step
        program's stop flag; once set the state passes through unchanged. At M ≥ 3 a chain of layers hands the
        input norm over: ``x_in`` = this layer's normalized input (``norm_apply(h, norm_w)``, written by the layer
        before), and ``next_norm = (w, x_next, eps)`` makes this layer write the next one's (inside the MLP's
        split-K reduction): the same values as each layer normalizing its own input, one launch fewer a layer."""
        proj, o, h1, act, h2 = self.buffers(h.shape[0])
        out = h2 if out is None else out
        cin, cout = self.conv_state[self.parity], self.conv_state[1 - self.parity]
        fold = self.folds_conv(h.shape[0], verify)
        pre = self.pre(h.shape[0]) if fold else None
        conv = dict(w=self.conv_w, state=cin, out_state=cout, out=pre, row0=self.hv * self.dv, done=done) if fold else None
        if x_in is not None:
            kernels.gemv(self.w_in.packed, x_in, out=proj, conv=conv)
        else:
            kernels.gemv(self.w_in.packed, h, norm_w=self.norm_w, eps=self.eps, out=proj, conv=conv)
        rec = self.rec_slots[self.slot]
        defer = self.defers_norm(h.shape[0])
        if verify:                              # the verify pass writes the other slots; commit() settles them
            rec_out = self._second_slot()
        else:
            rec_out = rec
        kernels.gdn_step(proj, cin, cout, rec, rec_out, conv_w=self.conv_w, neg_exp_a=self.neg_exp_a,
                         dt_bias=self.dt_bias, norm_w=self.gdn_norm_w, k_heads=self.hk, v_heads=self.hv, dk=self.dk,
                         dv=self.dv, conv_width=self.conv, eps=self.eps, out=o, defer_norm=defer, done=done, pre=pre)
        if verify:
            self._verify_proj = proj
        else:
            self.parity ^= 1
        # the gated RMSNorm (gdn_norm) is applied by the output projection while it stages o; z = proj[:, :hv·dv]
        gated = (self.gdn_norm_w, proj[:, : self.hv * self.dv], self.eps) if defer else None
        if CHAIN_TAIL and h.shape[0] == 1 and next_norm is None:
            kernels.gemv_chain([(self.w_out.packed, o, dict(epilogue="residual", residual=h, out=h1, gated_norm=gated))]
                               + self.mlp.phases(h1, act, out))
            return out
        kernels.gemv(self.w_out.packed, o, epilogue="residual", residual=h, out=h1, gated_norm=gated)
        return self.mlp(h1, act=act, out=out, next_norm=next_norm)

    def mixer_bytes(self, m: int) -> int:
        state = 2 * self.hv * self.dk * self.dv * 4 + 2 * self.conv_dim * (self.conv - 1) * 2
        params = self.conv_dim * self.conv * 2 + 3 * self.hv * 4 + self.dv * 4
        return state + params + m * self.n_proj * 2 + m * self.hv * self.dv * 2

    def bytes_per_step(self, m: int) -> int:
        return (_gemv_bytes(self.n_proj, self.hidden, m) + self.hidden * 4 + self.mixer_bytes(m)
                + _gemv_bytes(self.hidden, self.hv * self.dv, m, residual=True) + self.mlp.bytes_per_step(m))

    def export(self) -> dict:
        """Host copies of everything the checker needs (quantized codes, parameters, state)."""
        def q(mat):
            return {"weight": mat.codes.cpu().numpy(), "weight_scale": mat.scales.cpu().numpy(),
                    "row_scale": mat.row_scale.cpu().numpy()}
        return {"w_in": q(self.w_in), "w_out": q(self.w_out), "gate_up": q(self.mlp.gate_up), "down": q(self.mlp.down),
                "norm1": self.norm_w.cpu().numpy(), "norm2": self.mlp.norm_w.cpu().numpy(),
                "conv_w": self.conv_w.float().cpu().numpy(), "a_log": self.a_log.cpu().numpy(),
                "dt_bias": self.dt_bias.cpu().numpy(), "gdn_norm_w": self.gdn_norm_w.cpu().numpy(),
                "conv_state": self.conv_state[self.parity].float().cpu().numpy(),
                "rec_state": self.rec.cpu().numpy()}


class AttnDecoderLayer:
    """Gated GQA layer (hidden 5120, 24 query / 4 KV heads of 128, partial RoPE 64 at θ = 1e6, q/k norm, output
    gate, KV cache of ``ctx`` tokens — int8, or the reference's BF16 with ``kv_dtype="bf16"`` — MLP 17408; head dim
    128 or 256). Projection rows q|gate per head, then k, v."""

    def __init__(self, *, hidden=5120, heads=24, kv_heads=4, head_dim=128, rotary_dim=64, theta=1e6, ctx=32768,
                 inter=17408, eps=1e-6, device="cuda", seed=0, kv_dtype="int8", layout="checkpoint"):
        """``layout="packed"``: the projection rows in the reference's pack order ``[q | k | v | gate]`` with the
        RoPE head-dim permutation on q and k (``nn/attention.py:52-64``), the permuted full-width RoPE tables and
        norm weights — the same weights and the same attention, laid out as a compiled program holds them."""
        torch = _torch()
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        if layout not in ("checkpoint", "packed"):
            raise ValueError(f"AttnDecoderLayer: layout {layout!r}")
        self.hidden, self.heads, self.kv, self.d, self.eps = hidden, heads, kv_heads, head_dim, eps
        self.layout, self.rotary_dim, self.theta = layout, rotary_dim, theta
        self.n_proj = heads * 2 * head_dim + 2 * kv_heads * head_dim
        self.norm_w = 1.0 + torch.randn(hidden, generator=gen, device=device) * 0.1
        self.w_qkv = nvfp4_matrix(self.n_proj, hidden, gen, device)
        self.w_o = nvfp4_matrix(hidden, heads * head_dim, gen, device)
        self.q_norm = (1.0 + torch.randn(head_dim, generator=gen, device=device) * 0.1).to(torch.bfloat16).float()
        self.k_norm = (1.0 + torch.randn(head_dim, generator=gen, device=device) * 0.1).to(torch.bfloat16).float()
        self.cos, self.sin = kernels.rope_tables(theta, rotary_dim, ctx, device=device)
        if layout == "packed":
            from . import nn as NN
            from .formats.fp import f32_to_bf16
            spec = NN.GQAAttention(hidden, heads, kv_heads, head_dim, rotary_dim, theta, eps, prefix="", max_context=ctx)
            self.row_perm = spec.row_perm()
            self.core_rows = spec.core_rows
            perm = torch.as_tensor(self.row_perm, device=device)
            m = self.w_qkv
            codes, scales, rs = m.codes[perm], m.scales[perm], m.row_scale[perm]
            n_pad = -(-self.n_proj // 16) * 16
            rs_pad = torch.cat([rs, rs.new_ones(n_pad - self.n_proj)]) if n_pad != self.n_proj else rs
            self.w_qkv = QuantizedMatrix(codes, scales, rs, kernels.PackedWeight(
                "nvfp4", self.n_proj, hidden, 1, DV.pack_nvfp4(codes, scales), rs_pad.contiguous()))
            hp = torch.as_tensor(NN.rope_head_perm(head_dim, rotary_dim), device=device)
            self.q_norm, self.k_norm = self.q_norm[hp].contiguous(), self.k_norm[hp].contiguous()
            cos, sin = NN.rope_tables_permuted(theta, head_dim, rotary_dim, ctx)
            self.cos = torch.from_numpy(f32_to_bf16(cos).astype(np.int16)).view(torch.bfloat16).to(device)
            self.sin = torch.from_numpy(f32_to_bf16(sin).astype(np.int16)).view(torch.bfloat16).to(device)
        self.cache = kernels.KVCache(kv_heads, ctx, head_dim, device=device, dtype=kv_dtype)
        self.mlp = GatedMLP(hidden, inter, gen, device, eps)
        self._bufs: Dict[int, tuple] = {}

    def fill_cache(self, n: int, gen=None):
        """The first ``n`` positions: random int8 codes and f16 scales (N(0, 1) K/V quantized per token), or BF16
        N(0, 1) values."""
        torch = _torch()
        c = self.cache
        if c.dtype == "bf16":
            c.k_codes[:, :n] = torch.randn(c.k_codes[:, :n].shape, generator=gen, device=c.k_codes.device).to(
                torch.bfloat16)
            nb = -(-n // 64)
            c.v_codes[:, :nb] = torch.randn(c.v_codes[:, :nb].shape, generator=gen, device=c.v_codes.device).to(
                torch.bfloat16)
            return
        c.k_codes[:, :n].random_(-127, 128, generator=gen)
        c.v_codes[:, : -(-n // 64)].random_(-127, 128, generator=gen)
        c.k_scales[:, :n] = 3.0 / 127
        c.v_scales[:, :n] = 3.0 / 127

    def buffers(self, m: int):
        torch = _torch()
        if m not in self._bufs:
            dev = self.norm_w.device
            self._bufs[m] = (torch.empty(m, self.n_proj, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.heads * self.d, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.hidden, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.mlp.inter, dtype=torch.bfloat16, device=dev),
                             torch.empty(m, self.hidden, dtype=torch.bfloat16, device=dev))
        return self._bufs[m]

    def step(self, h, pos: int, out=None, done=None, x_in=None, next_norm=None):
        """One decode step over ``h [M, hidden]`` at positions ``pos..pos+M-1``; the new k/v enter the cache. ``pos``
        is an int or a one-element device int32 tensor (the step state's position in a captured program); ``done``
        the program's stop flag (once set, nothing enters the cache). ``x_in`` / ``next_norm``: the input norm
        handed over between layers at M ≥ 3, as in :meth:`GdnDecoderLayer.step`."""
        proj, o, h1, act, h2 = self.buffers(h.shape[0])
        out = h2 if out is None else out
        if x_in is not None:
            kernels.gemv(self.w_qkv.packed, x_in, out=proj)
        else:
            kernels.gemv(self.w_qkv.packed, h, norm_w=self.norm_w, eps=self.eps, out=proj)
        gate_src = proj[:, self.core_rows:] if self.layout == "packed" else None
        kernels.gqa_decode(proj, self.cache, pos, heads=self.heads, rope_cos=self.cos, rope_sin=self.sin, gate=True,
                           q_norm=self.q_norm, k_norm=self.k_norm, eps=self.eps, out=o, done=done, gate_src=gate_src)
        if CHAIN_TAIL and h.shape[0] == 1 and next_norm is None:
            kernels.gemv_chain([(self.w_o.packed, o, dict(epilogue="residual", residual=h, out=h1))]
                               + self.mlp.phases(h1, act, out))
            return out
        kernels.gemv(self.w_o.packed, o, epilogue="residual", residual=h, out=h1)
        return self.mlp(h1, act=act, out=out, next_norm=next_norm)

    def mixer_bytes(self, m: int, pos: int) -> int:
        per_key = self.cache.bytes_per_key()
        return (pos + m) * per_key + m * self.n_proj * 2 + m * self.heads * self.d * 2 + m * per_key

    def bytes_per_step(self, m: int, pos: int) -> int:
        return (_gemv_bytes(self.n_proj, self.hidden, m) + self.hidden * 4 + self.mixer_bytes(m, pos)
                + _gemv_bytes(self.hidden, self.heads * self.d, m, residual=True) + self.mlp.bytes_per_step(m))

    def export(self) -> dict:
        def q(mat):
            return {"weight": mat.codes.cpu().numpy(), "weight_scale": mat.scales.cpu().numpy(),
                    "row_scale": mat.row_scale.cpu().numpy()}
        c = self.cache
        return {"w_qkv": q(self.w_qkv), "w_o": q(self.w_o), "gate_up": q(self.mlp.gate_up), "down": q(self.mlp.down),
                "norm1": self.norm_w.cpu().numpy(), "norm2": self.mlp.norm_w.cpu().numpy(),
                "q_norm": self.q_norm.cpu().numpy(), "k_norm": self.k_norm.cpu().numpy(),
                "cos": self.cos.float().cpu().numpy(), "sin": self.sin.float().cpu().numpy(),
                "k_codes": c.k_codes.cpu().numpy(), "k_scales": c.k_scales.cpu().numpy(),
                "v_codes": c.v_codes_token_major().cpu().numpy(), "v_scales": c.v_scales.cpu().numpy()}


class MoeBlock:
    """The hybrid MoE layer's feed-forward (``nn/moe.py``; BASELINE configs[4], 35B-A3B-like): RMSNorm fused into the
    router GEMV (BF16) and the expert GEMVs, softmax top-k routing (renormalized) with the expert groups, the grouped
    gate|up GEMV (silu·mul, rounded as the reference's expert MLP) and down GEMV over the chosen experts only, one
    shared expert with its σ-gate, and the weighted combine plus residual. NVFP4 experts stored back to back."""

    def __init__(self, *, hidden=2048, experts=256, top_k=8, inter=512, shared_inter=512, eps=1e-6, device="cuda",
                 seed=0):
        torch = _torch()
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.hidden, self.experts, self.top_k, self.inter, self.eps = hidden, experts, top_k, inter, eps
        self.norm_w = 1.0 + torch.randn(hidden, generator=gen, device=device) * 0.1
        self.router_w = (torch.randn(experts, hidden, generator=gen, device=device) * 0.02).to(torch.bfloat16)
        self.router = kernels.PackedWeight("bf16", experts, hidden, 1, DV.pack_bf16(self.router_w), None)

        def stack(mats):
            return kernels.PackedWeight("nvfp4", mats[0].packed.n, mats[0].packed.k, len(mats),
                                        torch.cat([m.packed.data for m in mats]),
                                        torch.cat([m.packed.row_scale for m in mats]))
        self.gate_up_q = [nvfp4_matrix(2 * inter, hidden, gen, device, gate_up=True) for _ in range(experts)]
        self.down_q = [nvfp4_matrix(hidden, inter, gen, device) for _ in range(experts)]
        self.shared_gate_up = nvfp4_matrix(2 * shared_inter, hidden, gen, device, gate_up=True)
        self.shared_down = nvfp4_matrix(hidden, shared_inter, gen, device)
        self.shared_gate_w = (torch.randn(1, hidden, generator=gen, device=device) * 0.02).to(torch.bfloat16)
        self.shared_gate = kernels.PackedWeight("bf16", 1, hidden, 1, DV.pack_bf16(self.shared_gate_w), None)
        # the router and the shared expert's gate read the same normed h: one BF16 GEMV of experts + 1 rows
        self.router_gate = kernels.PackedWeight("bf16", experts + 1, hidden, 1,
                                                DV.pack_bf16(torch.cat([self.router_w, self.shared_gate_w])), None)
        self.shared_inter = shared_inter
        # the shared expert stacked after the routed ones (when it has their shape): it then runs inside the grouped
        # expert launches as slot k of every token, weight bf16(σ(gate)) from the router's row E — two launches
        # fewer and no second stream; the combine takes it as one more slot
        self.fused_shared = shared_inter == inter

        def routed(st):                                  # the first E experts of a stack, as views
            nb = st.data.numel() // st.experts
            return kernels.PackedWeight(st.format, st.n, st.k, experts, st.data[: experts * nb],
                                        st.row_scale[: experts * (st.row_scale.numel() // st.experts)])
        if self.fused_shared:
            self.gate_up_s = stack(self.gate_up_q + [self.shared_gate_up])
            self.down_s = stack(self.down_q + [self.shared_down])
            self.gate_up, self.down = routed(self.gate_up_s), routed(self.down_s)
        else:
            self.gate_up, self.down = stack(self.gate_up_q), stack(self.down_q)
        self._bufs: Dict[int, tuple] = {}
        self._xn: Dict[int, object] = {}
        # the shared expert runs on a second stream beside the router → experts chain (default priority), with its
        # own zeroed split-K workspace so the two branches never share partials or fold counters
        on_gpu = torch.device(device).type == "cuda"
        self.side = torch.cuda.Stream(device=device) if on_gpu else None
        self.side_ws = torch.zeros(8 << 20 if on_gpu else 16, dtype=torch.uint8, device=device)

    def buffers(self, m: int):
        torch = _torch()
        if m not in self._bufs:
            sh = 1 if self.fused_shared else 0
            # at M >= 3 the route splits an expert's pairs into records of two (one pass of the grouped GEMV each)
            dev, k = self.norm_w.device, self.top_k + sh
            g = m * k if m > 2 else min(self.experts, m * self.top_k) + sh
            bf = torch.bfloat16
            self._bufs[m] = (torch.empty(m, (self.experts + 1 + 7) // 8 * 8, dtype=bf, device=dev),
                             (torch.empty(m, k, dtype=torch.int32, device=dev),
                              torch.empty(m, k, dtype=torch.float32, device=dev),
                              torch.empty(g, kernels.GROUP_REC, dtype=torch.int32, device=dev)),
                             torch.empty(m * k, self.inter, dtype=bf, device=dev),
                             torch.empty(m * k, self.hidden, dtype=bf, device=dev),
                             torch.empty(m, self.shared_inter, dtype=bf, device=dev),
                             torch.empty(m, self.hidden, dtype=bf, device=dev),
                             torch.empty(m, 1, dtype=bf, device=dev),
                             torch.empty(m, self.hidden, dtype=bf, device=dev))
        return self._bufs[m]

    def _normed(self, m: int):
        if m not in self._xn:
            self._xn[m] = _torch().empty(m, self.hidden, dtype=_torch().bfloat16, device=self.norm_w.device)
        return self._xn[m]

    def __call__(self, h, act=None, out=None, next_norm=None, x_in=None):
        """``h [M, hidden]`` bf16 → the block's output with the residual added (M ≤ 16). ``act`` is accepted so the
        block can stand in for a decoder layer's dense MLP (it keeps its own intermediates). ``next_norm = (w,
        x_next, eps)``: also the next RMSNorm of the output (written by the combine); ``x_in``: the block's
        normalized input when the caller has it (M ≥ 3: the block then takes no norm launch of its own)."""
        y = self._forward(h, out, next_norm, x_in)
        if next_norm is not None and not self.fused_shared:
            nw, nx, neps = next_norm
            kernels.norm_apply(y, nw, eps=neps, out=nx)
        return y

    def _forward(self, h, out, next_norm=None, x_in=None):
        m = h.shape[0]
        logits, route, act, hk, s_act, s_out, s_gate, y = self.buffers(m)
        out = y if out is None else out
        torch = _torch()
        e, k = self.experts, self.top_k
        if self.fused_shared:
            # M >= 3: the input norm once, for the router and the experts (inside each GEMV every workgroup would
            # normalize the whole [M, K] input again); M <= 2: fused into both GEMVs' loads
            x, nw = h, self.norm_w
            if m > 2:
                x, nw = (x_in if x_in is not None
                         else kernels.norm_apply(h, self.norm_w, eps=self.eps, out=self._normed(m))), None
            kernels.gemv(self.router_gate, x, norm_w=nw, eps=self.eps, out=logits[:, :e + 1])
            ids, wts, groups = route
            if m == 1:                  # one token: the expert gate|up launch routes for itself (one launch fewer)
                inline = dict(logits=logits[:, :e], ids=ids, weights=wts, top_k=k, renorm=True, gate_col=e)
            else:
                kernels.moe_route(logits[:, :e], k, renorm=True, out=route, shared_expert=e, shared_gate=e,
                                  pairs_per_record=2 if m > 2 else 0)
                inline = None
            ppr = 2 if m > 2 else 0
            kernels.moe_gemv(self.gate_up_s, x, groups, tokens=m, top_k=k + 1, x_per_slot=False,
                             epilogue="silu_mul_rounded", norm_w=nw, eps=self.eps, out=act,
                             shared_expert=e, shared_epilogue="silu_mul", route=inline, group_max_pairs=ppr)
            kernels.moe_gemv(self.down_s, act, groups, tokens=m, top_k=k + 1, x_per_slot=True, out=hk,
                             group_max_pairs=ppr)
            return kernels.moe_combine(hk, wts, top_k=k + 1, residual=h, out=out, next_norm=next_norm)

        def shared(ws=None):
            kernels.gemv(self.shared_gate_up.packed, h, epilogue="silu_mul", norm_w=self.norm_w, eps=self.eps,
                         out=s_act, workspace=ws)
            kernels.gemv(self.shared_down.packed, s_act, out=s_out, workspace=ws)

        # M >= 3: the shared expert runs beside the router → experts chain (M = 8: 104 → 82 µs); at
        # M <= 2 its kernels are short and the fork / join costs more than it hides (34 → 39 µs), so one stream
        main = torch.cuda.current_stream(h.device)
        concurrent = m > 2
        if concurrent:
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                shared(self.side_ws)
        else:
            shared()
        e = self.experts
        kernels.gemv(self.router_gate, h, norm_w=self.norm_w, eps=self.eps, out=logits[:, :e + 1])
        _, wts, groups = kernels.moe_route(logits[:, :e], self.top_k, renorm=True, out=route)
        kernels.moe_gemv(self.gate_up, h, groups, tokens=m, top_k=self.top_k, x_per_slot=False,
                         epilogue="silu_mul_rounded", norm_w=self.norm_w, eps=self.eps, out=act)
        kernels.moe_gemv(self.down, act, groups, tokens=m, top_k=self.top_k, x_per_slot=True, out=hk)
        if concurrent:
            main.wait_stream(self.side)
        return kernels.moe_combine(hk, wts, top_k=self.top_k, shared=s_out, shared_gate=logits[:, e:e + 1], residual=h,
                                   out=out)

    def bytes_per_step(self, m: int, distinct_experts: int) -> int:
        """Algorithmic HBM bytes of one step with ``distinct_experts`` experts chosen over the M tokens."""
        k = self.top_k
        expert = _gemv_bytes(2 * self.inter, self.hidden, 0) + _gemv_bytes(self.hidden, self.inter, 0)
        return (self.experts * self.hidden * 2 + m * self.hidden * 2 + self.hidden * 4      # router, x, norm w
                + distinct_experts * expert + m * k * (self.inter * 2 * 2 + self.hidden * 2 * 2)
                + _gemv_bytes(2 * self.shared_inter, self.hidden, m, n_out=self.shared_inter)
                + _gemv_bytes(self.hidden, self.shared_inter, m) + self.hidden * 2 + m * self.hidden * 4)


class DecoderModel:
    """Embedding, decoder layers, final RMSNorm and LM head (``nn/decoder.py``, ``models/*``): what a step program
    runs once per token. ``lm_head`` is BF16 (the reference's unquantized head), its RMSNorm fused on load."""

    def __init__(self, layers, *, vocab: int, hidden: int, eps: float = 1e-6, device="cuda", seed=0):
        torch = _torch()
        gen = torch.Generator(device=device)
        gen.manual_seed(seed + 7919)
        self.layers, self.vocab, self.hidden, self.eps = list(layers), vocab, hidden, eps
        self.embed_table = (torch.randn(vocab, hidden, generator=gen, device=device) * 0.5).to(torch.bfloat16)
        self.norm_w = 1.0 + torch.randn(hidden, generator=gen, device=device) * 0.1
        self.lm_w = (torch.randn(vocab, hidden, generator=gen, device=device) * 0.02).to(torch.bfloat16)
        self.lm_head = kernels.PackedWeight("bf16", vocab, hidden, 1, DV.pack_bf16(self.lm_w), None)

    def step_bytes(self, pos: int) -> int:
        """Algorithmic HBM bytes of one token step (M = 1)."""
        total = self.hidden * 2 + self.vocab * self.hidden * 2 + self.hidden * 4 + self.vocab * 2   # BF16 logits
        for layer in self.layers:
            total += layer.bytes_per_step(1) if getattr(layer, "ping_pong", False) else layer.bytes_per_step(1, pos)
        return total
