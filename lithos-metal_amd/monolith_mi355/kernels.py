"""Typed Python entry points over the C ABI, one per op kind of the reference's operator API (``monolith/ops``).

Device memory is torch-ROCm tensors (plumbing only: their ``data_ptr()`` crosses the boundary as a plain pointer);
work goes on torch's current stream unless a stream is passed. Every function checks shapes on the host before
anything is launched, so a kernel never sees operands that do not match its grid.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .formats import DequantSpec
from .formats import pack as _pack
from .runtime import hip


def _torch():
    import torch
    return torch


def _check_flag(flag, name, what="done"):
    torch = _torch()
    if flag is not None and (flag.dtype != torch.int32 or flag.numel() != 1 or flag.device.type != "cuda"):
        raise ValueError(f"{name}: {what} must be a one-element int32 device tensor (a step-state field)")


@dataclass
class PackedWeight:
    """A T16 pack resident in HBM: ``data`` uint8 ``[experts·nbytes]``, NVFP4 / FP8 ``row_scale`` float32
    ``[experts·n_pad]``."""

    format: str
    n: int
    k: int
    experts: int
    data: "object"
    row_scale: Optional["object"]

    @property
    def n_pad(self) -> int:
        return -(-self.n // 16) * 16

    @property
    def nbytes(self) -> int:
        return int(self.data.numel())


def upload(specs, device="cuda", row_scales=None) -> PackedWeight:
    """Pack one matrix (or a list of equally shaped experts, stored back to back) and copy it to ``device``."""
    torch = _torch()
    specs = [specs] if isinstance(specs, DequantSpec) else list(specs)
    fmt, (n, k) = specs[0].format, specs[0].shape
    blobs, scales = [], []
    for i, s in enumerate(specs):
        if s.format != fmt or tuple(s.shape) != (n, k):
            raise ValueError("upload: experts must share format and shape")
        data, info = _pack.pack(s, None if row_scales is None else row_scales[i])
        blobs.append(data)
        if info.row_scale is not None:
            scales.append(info.row_scale)
    data = torch.from_numpy(np.concatenate(blobs)).to(device)
    rs = torch.from_numpy(np.concatenate(scales)).to(device) if scales else None
    return PackedWeight(fmt, n, k, len(specs), data, rs)


def _bf16_2d(t, name, aligned=True):
    torch = _torch()
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name}: expected a row-major 2-D bfloat16 tensor, got {t.dtype} {tuple(t.shape)}")
    if aligned and (t.data_ptr() % 16 or t.stride(0) % 8):
        raise ValueError(f"{name}: needs 16-byte alignment and a row stride multiple of 8")


def gemv(w: PackedWeight, x, *, epilogue=None, residual=None, norm_w=None, eps: float = 1e-6, out=None,
         stream=None, workspace=None, out_f32: bool = False, gated_norm=None, conv=None, next_norm=None):
    """``gemv`` (``ops/gemv.py:1-12``): ``y = x·Wᵀ`` for ``x [M, K]`` bf16, M ≤ 16; ``epilogue`` None | "residual" |
    "silu_mul" (rows gate|up interleaved by 8, output N/2 columns) | "silu_mul_rounded"; ``norm_w`` = the (1 + w)
    float32 weight of a fused input RMSNorm; ``out_f32`` writes the unrounded FP32 result (``lm_head``).
    ``gated_norm = (w [128] float32, z [M, K] bf16 view, eps)`` applies the Gated DeltaNet output norm
    (``gdn_norm``, ``nn/gdn.py:86-93``) to x per 128-column head while staging it. ``conv`` runs the Gated
    DeltaNet short conv in the epilogue (M ≤ 2): ``dict(w=taps [C, 4] bf16, state=…, out=[M, C] bf16, row0=first
    output row of the C channels, out_state=…, step=…, done=…)`` — ``state`` is ``[C, 3]`` with ``out_state`` the
    other slot, or both slots ``[2, C, 3]`` with ``step`` (a one-element device int32) choosing by parity; ``done`` a
    stop flag. ``out`` then feeds :func:`gdn_step` as ``pre``. ``next_norm = (w [N] float32 (1 + w), x_next [M, N]
    bf16 view, eps)`` also writes the next RMSNorm of the output, ``x_next = bf16(y·rsqrt(mean y² + eps)·w)`` — bit
    for bit :func:`norm_apply` of ``out`` — inside the split-K reduction launch where the plan has one (M ≥ 3), else
    with a norm launch after the GEMV."""
    d, out = _gemv_desc(w, x, epilogue=epilogue, residual=residual, norm_w=norm_w, eps=eps, out=out,
                        workspace=workspace, out_f32=out_f32, gated_norm=gated_norm)
    if next_norm is not None:
        _gemv_next_norm(d, next_norm, x.shape[0], w.n)
    if conv is not None:
        _gemv_conv(d, conv, x.shape[0], w)
    hip.call("mi_gemv", C.byref(d), hip.stream_handle(stream))
    return out


def _gemv_next_norm(d, next_norm, m: int, n: int) -> None:
    """The next-norm fields of a GEMV descriptor, checked."""
    torch = _torch()
    nw, nx, neps = next_norm
    if nw.dtype != torch.float32 or nw.numel() != n or not nw.is_contiguous():
        raise ValueError("gemv next_norm: w must be a contiguous float32 [N]")
    _bf16_2d(nx, "gemv next_norm x")
    if nx.shape[0] < m or nx.shape[1] < n:
        raise ValueError("gemv next_norm: x too small")
    d.next_norm_w, d.next_x, d.ld_next_x, d.next_eps = hip.ptr(nw), hip.ptr(nx), nx.stride(0), float(neps)


def _gemv_conv(d, conv, m: int, w) -> None:
    """The conv fields of a GEMV descriptor, checked."""
    torch = _torch()
    taps, state, cout = conv["w"], conv["state"], conv["out"]
    ch = taps.shape[0]
    step, out_state = conv.get("step"), conv.get("out_state")
    if taps.dtype != torch.bfloat16 or tuple(taps.shape) != (ch, 4) or not taps.is_contiguous():
        raise ValueError("gemv conv: w must be contiguous bf16 [C, 4]")
    want = (2, ch, 3) if step is not None else (ch, 3)
    for name, t in (("state", state),) + ((("out_state", out_state),) if step is None else ()):
        if t is None or t.dtype != torch.bfloat16 or tuple(t.shape) != want or not t.is_contiguous():
            raise ValueError(f"gemv conv: {name} must be contiguous bf16 {want}")
    _bf16_2d(cout, "gemv conv out", aligned=False)
    if cout.shape[0] < m or cout.shape[1] < ch:
        raise ValueError("gemv conv: out must be [M, C]")
    _check_flag(step, "gemv conv", "step")
    _check_flag(conv.get("done"), "gemv conv")
    d.conv_w, d.conv_in, d.conv_out = hip.ptr(taps), hip.ptr(state), hip.ptr(cout)
    d.conv_out_state = hip.ptr(out_state) if step is None else 0
    d.conv_row0, d.conv_channels, d.ld_conv = int(conv["row0"]), ch, cout.stride(0)
    d.conv_step, d.conv_done = hip.ptr(step), hip.ptr(conv.get("done"))


def _gemv_desc(w: PackedWeight, x, *, epilogue=None, residual=None, norm_w=None, eps: float = 1e-6, out=None,
               workspace=None, out_f32: bool = False, gated_norm=None):
    """The checked ``mi_gemv_desc`` of one GEMV (and its output tensor, allocated when not given)."""
    torch = _torch()
    _bf16_2d(x, "gemv x")
    m, k = x.shape
    if k != w.k or not 1 <= m <= 16:
        raise ValueError(f"gemv: x {tuple(x.shape)} does not match K={w.k} / M in 1..16")
    n_out = w.n // 2 if epilogue in ("silu_mul", "silu_mul_rounded") else w.n
    odt = torch.float32 if out_f32 else torch.bfloat16
    if out is None:
        out = torch.empty((m, n_out), dtype=odt, device=x.device)
    if out.dtype != odt or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError(f"gemv: out must be a row-major 2-D {odt} tensor")
    if out.shape[0] < m or out.shape[1] < n_out:
        raise ValueError("gemv: out too small")
    if epilogue == "residual":
        _bf16_2d(residual, "gemv residual")
        if residual.shape[0] < m or residual.shape[1] < w.n:
            raise ValueError("gemv: residual too small")
    if norm_w is not None and (norm_w.dtype != torch.float32 or norm_w.numel() != k):
        raise ValueError("gemv: norm_w must be float32 [K]")
    gw, gz, geps = gated_norm if gated_norm is not None else (None, None, 0.0)
    if gated_norm is not None:
        if gw.dtype != torch.float32 or gw.numel() != 128:
            raise ValueError("gemv: gated_norm weight must be float32 [128]")
        _bf16_2d(gz, "gemv gated_norm z")
        if gz.shape[0] < m or gz.shape[1] < k:
            raise ValueError("gemv: gated_norm z too small")
    d = hip.MiGemvDesc(format=hip.MI_FMT[w.format], n=w.n, k=w.k, m=m, w=hip.ptr(w.data),
                       row_scale=hip.ptr(w.row_scale), x=hip.ptr(x), ldx=x.stride(0), y=hip.ptr(out),
                       ldy=out.stride(0), epilogue=hip.MI_EPI[epilogue],
                       residual=hip.ptr(residual) if epilogue == "residual" else 0,
                       ldr=residual.stride(0) if epilogue == "residual" else 0, norm_w=hip.ptr(norm_w), eps=eps,
                       groups=0, max_groups=0, top_k=0, x_per_slot=0,
                       workspace=hip.ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel(),
                       out_f32=int(out_f32), gnorm_w=hip.ptr(gw), gnorm_z=hip.ptr(gz),
                       ld_gnorm_z=gz.stride(0) if gz is not None else 0, gnorm_eps=geps)
    return d, out


def gemv_chain(phases, *, workspace=None, stream=None):
    """A chain of dependent one-token NVFP4 GEMVs in one persistent launch (``mi_gemv_chain``): ``phases`` is a list
    of ``(w, x, kwargs)`` with :func:`gemv`'s keyword arguments (``epilogue``, ``residual``, ``norm_w``, ``eps``,
    ``out``, ``gated_norm``); phase i runs after phase i-1 has finished, so its ``x`` or ``residual`` may be an
    earlier phase's ``out``. The fused counterpart of the reference's MLP / region megakernels
    (``compiler/mlp_fusion.py:103-130``). Returns the outputs."""
    if not 1 <= len(phases) <= 4:
        raise ValueError("gemv_chain: 1..4 phases")
    descs, outs = [], []
    for w, x, kw in phases:
        if w.format != "nvfp4" or x.shape[0] != 1:
            raise ValueError("gemv_chain: NVFP4 weights and one token")
        d, o = _gemv_desc(w, x, **kw)
        descs.append(d)
        outs.append(o)
    arr = (hip.MiGemvDesc * len(descs))(*descs)
    ws = 0 if workspace is None else hip.ptr(workspace)
    nb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    hip.call("mi_gemv_chain", arr, len(descs), ws, nb, hip.stream_handle(stream))
    return outs


def rmsnorm_stat(h, *, out=None, stream=None):
    """``rmsnorm_stat`` (``ops/norm.py:11``): ``stat[i] = Σ_k h[i, k]²`` (float32) over BF16 rows."""
    torch = _torch()
    _bf16_2d(h, "rmsnorm_stat h")
    t, k = h.shape
    if out is None:
        out = torch.empty(t, dtype=torch.float32, device=h.device)
    if out.dtype != torch.float32 or out.numel() < t:
        raise ValueError("rmsnorm_stat: out must be float32 [t]")
    d = hip.MiNormDesc(t=t, k=k, h=hip.ptr(h), ldh=h.stride(0), stat=hip.ptr(out), stat_parts=1)
    hip.call("mi_rmsnorm_stat", C.byref(d), hip.stream_handle(stream))
    return out


def norm_apply(h, w, *, stat=None, eps: float = 1e-6, out=None, stream=None):
    """``norm_apply`` (``ops/norm.py:12``): ``x = bf16(h·rsqrt(s / K + eps)·w)`` with ``w`` the (1 + w) float32
    weight and ``s`` the row's Σh² — the sum of ``stat [t, parts]``'s partials, or computed here when ``stat`` is
    None."""
    torch = _torch()
    _bf16_2d(h, "norm_apply h")
    t, k = h.shape
    if w.dtype != torch.float32 or w.numel() != k or not w.is_contiguous():
        raise ValueError("norm_apply: w must be a contiguous float32 [K]")
    parts = 1
    if stat is not None:
        if stat.dtype != torch.float32 or stat.shape[0] < t or not stat.is_contiguous():
            raise ValueError("norm_apply: stat must be a contiguous float32 [t] or [t, parts]")
        parts = 1 if stat.dim() == 1 else stat.shape[1]
    if out is None:
        out = torch.empty(t, k, dtype=torch.bfloat16, device=h.device)
    _bf16_2d(out, "norm_apply out")
    d = hip.MiNormDesc(t=t, k=k, h=hip.ptr(h), ldh=h.stride(0), stat=hip.ptr(stat), stat_parts=parts, w=hip.ptr(w),
                       x=hip.ptr(out), ldx=out.stride(0), eps=eps)
    hip.call("mi_norm_apply", C.byref(d), hip.stream_handle(stream))
    return out


def dequant(w: PackedWeight, expert: int = 0, stream=None):
    """The packed matrix decoded to float32 ``[N, K]`` by the kernels' own decode (exactness check)."""
    torch = _torch()
    out = torch.empty((w.n, w.k), dtype=torch.float32, device=w.data.device)
    nb = _pack.pack_bytes(w.format, w.n, w.k)
    base = hip.ptr(w.data) + expert * nb
    rs = 0 if w.row_scale is None else hip.ptr(w.row_scale) + 4 * expert * w.n_pad
    hip.call("mi_dequant", hip.MI_FMT[w.format], base, rs, w.n, w.k, hip.ptr(out), hip.stream_handle(stream))
    return out


def gdn_step(proj, conv_in, conv_out, rec_in, rec_out, *, conv_w, neg_exp_a, dt_bias, norm_w, k_heads, v_heads,
             dk=128, dv=128, conv_width=4, eps=1e-6, ab=None, offsets=None, out=None, stream=None,
             defer_norm: bool = False, commit: bool = False, t_dev=None, done=None, step=None, pre=None):
    """``gdn_mixer`` + ``gdn_norm`` (``ops/gdn.py:1-24``) for ``proj [T, N1]`` bf16 in part order
    ``z | q | k | v | a | b`` (``nn/gdn.py:48-52``) unless ``offsets`` (z, q, k, v, a, b) says otherwise.
    Conv state ``[conv_dim, W-1]`` bf16 is read from ``conv_in`` and written to ``conv_out`` (distinct); the FP32
    recurrent state ``[hv, dk, dv]`` is read from ``rec_in`` and written to ``rec_out`` (may be the same tensor).
    Returns ``[T, hv·dv]`` bf16: the gated-norm output, or with ``defer_norm`` the BF16 read-out ``o`` for a
    consumer that applies the norm itself (``gemv(..., gated_norm=...)``). ``commit`` is ``gdn_commit``
    (``ops/gdn.py:13-17``): the speculative commit pass re-runs the first ``t_dev`` (device int32, ≤ T; None = all)
    tokens from the step's input state into ``rec_out`` / ``conv_out`` and returns None (no read-out). ``done``: a
    step program's stop flag (one-element device int32 view of the step state): once set, the step takes no token —
    the states pass through unchanged (``gdn_mixer.metal:281,330`` return at done). ``step``: a step program's step
    counter (one-element device int32): ``conv_in`` is then both conv-state slots ``[2, conv_dim, W-1]`` and
    ``conv_out`` is None — the step reads slot ``step & 1`` and writes the other (the reference's two slots by step
    parity), so one captured step serves every step of a replay. ``pre``: the convolved q|k|v ``[T, conv_dim]``
    bf16 written by the input projection's conv epilogue (``gemv(..., conv=…)``, T ≤ 2); the step then skips the
    conv, and ``conv_in`` / ``conv_out`` may be None."""
    torch = _torch()
    _bf16_2d(proj, "gdn proj", aligned=False)
    t = proj.shape[0]
    kd, vd = k_heads * dk, v_heads * dv
    conv_dim = 2 * kd + vd
    if offsets is None:
        offsets = (0, vd, vd + kd, vd + 2 * kd, vd + conv_dim, vd + conv_dim + v_heads)
    z_off, q_off, k_off, v_off, a_off, b_off = offsets
    if step is not None and conv_out is not None:
        raise ValueError("gdn_step: with step, conv_in holds both slots and conv_out is None")
    conv_shapes = ((("conv_in", conv_in, (2, conv_dim, conv_width - 1), torch.bfloat16),) if step is not None else
                   (("conv_in", conv_in, (conv_dim, conv_width - 1), torch.bfloat16),
                    ("conv_out", conv_out, (conv_dim, conv_width - 1), torch.bfloat16)))
    if pre is not None:
        _bf16_2d(pre, "gdn pre", aligned=False)
        if commit or t > 2 or pre.shape[0] < t or pre.shape[1] < conv_dim:
            raise ValueError("gdn_step: pre is [T, conv_dim] bf16 for a step of T <= 2 (not the commit pass)")
        conv_shapes = tuple(c for c in conv_shapes if c[1] is not None)
    for name, tns, shape, dt in conv_shapes + (
                                 ("rec_in", rec_in, (v_heads, dk, dv), torch.float32),
                                 ("rec_out", rec_out, (v_heads, dk, dv), torch.float32),
                                 ("conv_w", conv_w, (conv_dim, conv_width), torch.bfloat16),
                                 ("neg_exp_a", neg_exp_a, (v_heads,), torch.float32),
                                 ("dt_bias", dt_bias, (v_heads,), torch.float32), ("norm_w", norm_w, (dv,), torch.float32)):
        if tuple(tns.shape) != shape or tns.dtype != dt or not tns.is_contiguous():
            raise ValueError(f"gdn_step: {name} must be a contiguous {dt} {shape}, got {tns.dtype} {tuple(tns.shape)}")
    if max(offsets[:4]) + dk > proj.shape[1] and ab is None:
        raise ValueError("gdn_step: proj is narrower than the z|q|k|v|a|b offsets")
    if t_dev is not None and (t_dev.dtype != torch.int32 or t_dev.numel() != 1):
        raise ValueError("gdn_step: t_dev must be a one-element int32 device tensor")
    _check_flag(done, "gdn_step")
    _check_flag(step, "gdn_step", "step")
    if out is None and not commit:
        out = torch.empty((t, vd), dtype=torch.bfloat16, device=proj.device)
    d = hip.MiGdnDesc(t=t, k_heads=k_heads, v_heads=v_heads, dk=dk, dv=dv, conv_width=conv_width, proj=hip.ptr(proj),
                      ld_proj=proj.stride(0), z_off=z_off, q_off=q_off, k_off=k_off, v_off=v_off, ab=hip.ptr(ab),
                      ld_ab=ab.stride(0) if ab is not None else 0, a_off=a_off, b_off=b_off, conv_w=hip.ptr(conv_w),
                      neg_exp_a=hip.ptr(neg_exp_a), dt_bias=hip.ptr(dt_bias), norm_w=hip.ptr(norm_w),
                      conv_in=hip.ptr(conv_in) if conv_in is not None else 0,
                      conv_out=hip.ptr(conv_out) if conv_out is not None else 0,
                      rec_in=hip.ptr(rec_in),
                      rec_out=hip.ptr(rec_out), y=hip.ptr(out), ld_y=out.stride(0) if out is not None else 0, eps=eps,
                      defer_norm=int(defer_norm), commit=int(commit), t_dev=hip.ptr(t_dev), done=hip.ptr(done),
                      step=hip.ptr(step), pre=hip.ptr(pre), ld_pre=pre.stride(0) if pre is not None else 0)
    hip.call("mi_gdn_step", C.byref(d), hip.stream_handle(stream))
    return out


# ---- GQA decode attention over the int8 KV cache ---------------------------------------------------------------------
def rope_tables(theta: float, rotary_dim: int, ctx: int, device="cuda"):
    """BF16 ``cos``/``sin`` ``[ctx, rotary_dim]`` for positions ``0..ctx-1``, ``cat(freqs, freqs)``, computed in FP32
    the way the reference builds them per step (``nn/oracle.py:49-55``, ``nn/attention.py:230-233``)."""
    torch = _torch()
    inv = 1.0 / (torch.tensor(float(theta), dtype=torch.float32) **
                 (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    freqs = torch.arange(ctx, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(torch.bfloat16).to(device), emb.sin().to(torch.bfloat16).to(device)


def torch_index(a, device):
    return _torch().as_tensor(np.asarray(a), device=device)


class KVCache:
    """One attention layer's KV cache in this backend's layout: ``k_codes [kv, ctx_max, D]`` and ``v_codes
    [kv, ctx_max/64, D, 64]`` (transposed inside blocks of 64 keys — key k of a block at position ``V_POS[k]``, the
    order in which the kernel's score tiles hold the keys — so each block of keys is contiguous). ``dtype="int8"``:
    int8 codes with ``k_scales`` / ``v_scales [kv, ctx_max]`` float16, ``scale = f16(absmax / 127)`` per token and
    KV head; ``dtype="bf16"``: the reference's BF16 values (``nn/attention.py:87-89``, ``[ctx_max, Hkv, D]`` there)
    and no scales. 288 GB of HBM holds a 262 144-token int8 context for all 16 attention layers of the 27B model at
    4 KV heads × 128 dims many times over."""

    BLOCK = 64
    V_POS = np.array([((k & 15) >> 2) * 16 + (k >> 5) * 8 + ((k >> 4) & 1) * 4 + (k & 3) for k in range(64)])

    def __init__(self, kv_heads: int, ctx_max: int, head_dim: int = 128, device="cuda", dtype: str = "int8"):
        torch = _torch()
        if ctx_max % self.BLOCK:
            raise ValueError(f"KVCache: ctx_max must be a multiple of {self.BLOCK}")
        if dtype not in ("int8", "bf16"):
            raise ValueError("KVCache: dtype is 'int8' or 'bf16'")
        self.kv_heads, self.ctx_max, self.head_dim, self.dtype = kv_heads, ctx_max, head_dim, dtype
        el = torch.int8 if dtype == "int8" else torch.bfloat16
        self.k_codes = torch.zeros((kv_heads, ctx_max, head_dim), dtype=el, device=device)
        self.v_codes = torch.zeros((kv_heads, ctx_max // self.BLOCK, head_dim, self.BLOCK), dtype=el, device=device)
        self.k_scales = self.v_scales = None
        if dtype == "int8":
            self.k_scales = torch.zeros((kv_heads, ctx_max), dtype=torch.float16, device=device)
            self.v_scales = torch.zeros((kv_heads, ctx_max), dtype=torch.float16, device=device)

    @property
    def kv_dtype(self) -> int:
        return hip.MI_KV_BF16 if self.dtype == "bf16" else hip.MI_KV_INT8

    def v_codes_token_major(self):
        """``v_codes`` as ``[kv, ctx_max, D]`` (a copy)."""
        torch = _torch()
        kv, nb, d, b = self.v_codes.shape
        idx = torch.as_tensor(self.V_POS, device=self.v_codes.device)
        return self.v_codes.index_select(3, idx).permute(0, 1, 3, 2).reshape(kv, nb * b, d)

    def set_v_token_major(self, codes):
        """Store ``codes [kv, ctx_max, D]`` (int8 codes or BF16 values) into the blocked ``v_codes``."""
        kv, nb, d, b = self.v_codes.shape
        blocks = codes.reshape(kv, nb, b, d).permute(0, 1, 3, 2)           # [kv, nb, D, key]
        self.v_codes[..., torch_index(self.V_POS, self.v_codes.device)] = blocks

    @property
    def nbytes(self) -> int:
        return sum(int(t.numel() * t.element_size()) for t in (self.k_codes, self.v_codes, self.k_scales, self.v_scales)
                   if t is not None)

    def bytes_per_key(self) -> int:
        """HBM bytes one cached key costs a step (its K and V rows and scales, every KV head)."""
        return self.kv_heads * (4 * self.head_dim if self.dtype == "bf16" else 2 * self.head_dim + 4)


def gqa_decode(proj, cache: KVCache, pos, *, heads: int, rope_cos, rope_sin, gate: bool = True,
               q_norm=None, k_norm=None, eps: float = 1e-6, scaling: Optional[float] = None, out=None, stream=None,
               workspace=None, done=None, gate_src=None):
    """``gqa_decode`` + ``gqa_merge`` (``ops/attention.py``; ``GQAAttention.mix``, ``nn/attention.py:215-243``) for
    ``proj [T, N1]`` bf16 (``q|gate`` per head, then ``k``, ``v``): q/k norm (``q_norm``/``k_norm`` = the (1 + w)
    float32 weights, both or neither), partial RoPE from the BF16 tables ``[ctx_max, rotary_dim]``, the new k/v
    appended to ``cache`` (int8: quantized; bf16: as they are) at ``pos..pos+T``, attention over the cache,
    × σ(gate). Head dim 128 or 256. Returns ``[T, heads·D]`` bf16.
    ``pos`` is an int, or a one-element int32 device tensor the kernels read (a step program's StepState position:
    the same launch serves every step of a replayed graph). ``done``: a step program's stop flag (one-element device
    int32): once set, nothing is appended to the cache and ``out`` is not written. ``workspace``: a uint8 tensor of
    ``mi_gqa_workspace_bytes`` (key-range partials, prepared query rows, arrival counters: zeroed once before its
    first use; the counters return to zero after each call), or None for the library's own. ``gate_src``: the
    reference's packed layout (``nn/attention.py:52-64``) — ``proj`` holds ``q | k | v`` and the gate rows are this
    ``[T, heads·D]`` bf16 view; with the RoPE head-dim permutation the tables are ``[ctx_max, D]``."""
    torch = _torch()
    _bf16_2d(proj, "gqa proj", aligned=False)
    t = proj.shape[0]
    d, kv = cache.head_dim, cache.kv_heads
    if gate_src is not None:
        _bf16_2d(gate_src, "gqa gate", aligned=False)
        if not gate or gate_src.shape[0] < t or gate_src.shape[1] < heads * d:
            raise ValueError("gqa_decode: gate_src must be [T, heads·D] bf16 and needs gate=True")
    q_cols = heads * (2 if gate and gate_src is None else 1) * d
    if proj.shape[1] < q_cols + 2 * kv * d:
        raise ValueError(f"gqa_decode: proj has {proj.shape[1]} columns, needs {q_cols + 2 * kv * d}")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("gqa_decode: q_norm and k_norm go together")
    for name, tb in (("rope_cos", rope_cos), ("rope_sin", rope_sin)):
        if tb.dtype != torch.bfloat16 or tb.dim() != 2 or tb.shape[0] < cache.ctx_max or not tb.is_contiguous():
            raise ValueError(f"gqa_decode: {name} must be a contiguous bf16 [ctx_max, rotary_dim] table")
    for name, w in (("q_norm", q_norm), ("k_norm", k_norm)):
        if w is not None and (w.dtype != torch.float32 or w.numel() != d):
            raise ValueError(f"gqa_decode: {name} must be float32 [{d}]")
    if out is None:
        out = torch.empty((t, heads * d), dtype=torch.bfloat16, device=proj.device)
    _bf16_2d(out, "gqa out", aligned=False)
    if out.shape[0] < t or out.shape[1] < heads * d:
        raise ValueError("gqa_decode: out too small")
    pos_dev = None
    if not isinstance(pos, int):
        if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device.type != "cuda":
            raise ValueError("gqa_decode: pos must be an int or a one-element int32 device tensor")
        pos_dev, pos = pos, 0
    _check_flag(done, "gqa_decode")
    desc = hip.MiGqaDesc(t=t, heads=heads, kv_heads=kv, head_dim=d, rotary_dim=rope_cos.shape[1], pos=pos,
                         ctx_max=cache.ctx_max, gate=int(gate), qk_norm=int(q_norm is not None), proj=hip.ptr(proj),
                         ld_proj=proj.stride(0), rope_cos=hip.ptr(rope_cos), rope_sin=hip.ptr(rope_sin),
                         q_norm=hip.ptr(q_norm), k_norm=hip.ptr(k_norm), eps=eps,
                         scaling=d ** -0.5 if scaling is None else scaling, k_codes=hip.ptr(cache.k_codes),
                         k_scales=hip.ptr(cache.k_scales), v_codes=hip.ptr(cache.v_codes),
                         v_scales=hip.ptr(cache.v_scales), y=hip.ptr(out), ld_y=out.stride(0), kv_dtype=cache.kv_dtype,
                         workspace=hip.ptr(workspace),
                         workspace_bytes=0 if workspace is None else workspace.numel() * workspace.element_size(),
                         pos_dev=hip.ptr(pos_dev), done=hip.ptr(done), gate_src=hip.ptr(gate_src),
                         ld_gate=0 if gate_src is None else gate_src.stride(0))
    hip.call("mi_gqa_decode", C.byref(desc), hip.stream_handle(stream))
    return out


# ---- MoE: route (+ expert groups), grouped expert GEMV, combine -------------------------------------------------------
GROUP_REC = 18


def moe_route(logits, top_k: int, *, renorm: bool = True, groups: bool = True, out=None, stream=None,
              shared_expert: int = 0, shared_gate=None, pairs_per_record: int = 0):
    """``moe_route`` (``ops/moe.py``): ``logits [T, E]`` bf16 → ``(ids [T, k] int32, weights [T, k] float32,
    groups [max_groups, 18] int32 or None)``; ``max_groups = min(E, T·k)``. The groups feed ``moe_gemv``. ``out``:
    preallocated ``(ids, weights, groups)`` (a captured step allocates nothing). ``shared_expert`` > 0 (its index in
    the stacked experts, after the routed ones) with ``shared_gate`` = the column of ``logits``' rows that holds the
    shared gate's logit (the logits tensor a view of a wider router output): every token gets slot k = the shared
    expert with weight bf16(σ(gate)), so ids / weights are ``[T, k + 1]`` and there is one group more.
    ``pairs_per_record`` (1..16): an expert's pairs go into consecutive records of at most that many (``max_groups``
    is then ``T·slots``), for a grouped GEMV that takes two pairs per workgroup (``moe_gemv(group_max_pairs=2)``)."""
    torch = _torch()
    _bf16_2d(logits, "moe_route logits", aligned=False)
    t, e = logits.shape
    dev = logits.device
    sh = 1 if shared_expert > 0 else 0
    if sh and (shared_gate is None or not e <= shared_expert <= 512 or not 0 <= shared_gate < logits.stride(0)):
        raise ValueError("moe_route: the shared expert follows the routed ones and its gate column lies in the row")
    ks = top_k + sh
    if not 0 <= pairs_per_record <= GROUP_REC - 2:
        raise ValueError("moe_route: pairs_per_record in 0..16")
    max_groups = t * ks if pairs_per_record else min(e, t * top_k) + sh
    if out is not None:
        ids, w, g = out
        if (ids.dtype != torch.int32 or ids.numel() < t * ks or w.dtype != torch.float32 or w.numel() < t * ks
                or (groups and (g is None or g.dtype != torch.int32 or g.shape[0] < max_groups
                                or g.shape[1] != GROUP_REC))):
            raise ValueError("moe_route: out must be (int32 [T, k], float32 [T, k], int32 [max_groups, 18])")
        g = g if groups else None
    else:
        ids = torch.empty((t, ks), dtype=torch.int32, device=dev)
        w = torch.empty((t, ks), dtype=torch.float32, device=dev)
        g = torch.empty((max_groups, GROUP_REC), dtype=torch.int32, device=dev) if groups else None
    d = hip.MiMoeRouteDesc(t=t, n_experts=e, top_k=top_k, renorm=int(renorm), logits=hip.ptr(logits),
                           ld_logits=logits.stride(0), ids=hip.ptr(ids), weights=hip.ptr(w), groups=hip.ptr(g),
                           max_groups=max_groups if groups else 0, shared_expert=shared_expert,
                           shared_gate_col=shared_gate if sh else 0, pairs_per_record=pairs_per_record)
    hip.call("mi_moe_route", C.byref(d), hip.stream_handle(stream))
    return ids, w, g


def moe_gemv(w: PackedWeight, x, groups, *, tokens: int, top_k: int, x_per_slot: bool, epilogue=None, norm_w=None,
             eps: float = 1e-6, out=None, stream=None, shared_expert: int = 0, shared_epilogue=None, route=None,
             group_max_pairs: int = 0):
    """``moe_gemv`` (``ops/moe.py``; the grouped mode of ``gemv``): for every group record (expert e, its pairs
    p = t·k + j), ``out[p] = x_row · W_eᵀ`` with ``x_row = x[p]`` (``x_per_slot``) or ``x[p // k]``; ``w`` holds the
    experts back to back. ``out [T·k, n_out]`` bf16. ``shared_expert`` > 0: that expert's group (the shared expert
    stacked after the routed ones) takes ``shared_epilogue``. ``route`` (one token): ``dict(logits=…, ids=…,
    weights=…, top_k=k, renorm=True, gate_col=…)`` — the launch routes for itself from the token's router row
    (exactly ``moe_route``'s ids and weights), group g = slot g, and writes ids / weights and the group records into
    ``groups`` for the launches after it; ``top_k`` is then k (+1 with ``shared_expert``). ``group_max_pairs``: the
    records hold at most that many pairs (``moe_route(pairs_per_record=…)``; 0 = up to 16)."""
    torch = _torch()
    _bf16_2d(x, "moe_gemv x")
    if x.shape[1] != w.k:
        raise ValueError(f"moe_gemv: x has {x.shape[1]} columns, the experts take K={w.k}")
    if x.shape[0] < (tokens * top_k if x_per_slot else tokens):
        raise ValueError("moe_gemv: x has too few rows")
    if groups.dtype != torch.int32 or groups.dim() != 2 or groups.shape[1] != GROUP_REC:
        raise ValueError("moe_gemv: groups must be int32 [max_groups, 18] (moe_route)")
    if not 1 <= tokens <= 16:
        raise ValueError("moe_gemv: 1..16 tokens")
    n_out = w.n // 2 if epilogue in ("silu_mul", "silu_mul_rounded") else w.n
    if out is None:
        out = torch.empty((tokens * top_k, n_out), dtype=torch.bfloat16, device=x.device)
    _bf16_2d(out, "moe_gemv out", aligned=False)
    if norm_w is not None and (norm_w.dtype != torch.float32 or norm_w.numel() != w.k):
        raise ValueError("moe_gemv: norm_w must be float32 [K]")
    d = hip.MiGemvDesc(format=hip.MI_FMT[w.format], n=w.n, k=w.k, m=tokens, w=hip.ptr(w.data),
                       row_scale=hip.ptr(w.row_scale), x=hip.ptr(x), ldx=x.stride(0), y=hip.ptr(out),
                       ldy=out.stride(0), epilogue=hip.MI_EPI[epilogue], residual=0, ldr=0, norm_w=hip.ptr(norm_w),
                       eps=eps, groups=hip.ptr(groups), max_groups=groups.shape[0], top_k=top_k,
                       x_per_slot=int(x_per_slot), workspace=0, workspace_bytes=0, out_f32=0,
                       shared_expert=shared_expert, shared_epilogue=hip.MI_EPI[shared_epilogue],
                       group_max_pairs=group_max_pairs)
    if route is not None:
        lg = route["logits"]
        if lg.dtype != torch.bfloat16 or lg.dim() != 2 or lg.shape[0] != 1 or tokens != 1:
            raise ValueError("moe_gemv: routing in the launch takes one token's bf16 logits row [1, E]")
        d.route_logits, d.route_experts = hip.ptr(lg), lg.shape[1]
        d.route_top_k, d.route_renorm = route["top_k"], int(route.get("renorm", True))
        d.route_gate_col, d.route_ld = route.get("gate_col", 0), lg.stride(0)
        d.route_ids, d.route_weights = hip.ptr(route["ids"]), hip.ptr(route["weights"])
    hip.call("mi_gemv", C.byref(d), hip.stream_handle(stream))
    return out


def moe_combine(h, weights, *, top_k: int, shared=None, shared_gate=None, residual=None, out=None, stream=None,
                next_norm=None):
    """``moe_combine`` (``ops/moe.py``): ``out[t] = Σ_j w[t, j]·h[t·k + j] (+ bf16(σ(shared_gate[t]))·shared[t])
    (+ residual[t])``, FP32, one BF16 rounding. ``h [T·k, H]``, ``weights [T, k]`` float32. ``next_norm = (w [H]
    float32, x_next [T, H] bf16, eps)`` also writes the next RMSNorm of ``out`` (bit for bit :func:`norm_apply`)."""
    torch = _torch()
    _bf16_2d(h, "moe_combine h")
    t = weights.shape[0]
    hidden = h.shape[1]
    if weights.dtype != torch.float32 or tuple(weights.shape) != (t, top_k) or not weights.is_contiguous():
        raise ValueError("moe_combine: weights must be contiguous float32 [T, k]")
    if h.shape[0] < t * top_k:
        raise ValueError("moe_combine: h has too few rows")
    for name, a in (("shared", shared), ("residual", residual)):
        if a is not None:
            _bf16_2d(a, f"moe_combine {name}")
    if shared_gate is not None:
        _bf16_2d(shared_gate, "moe_combine shared_gate", aligned=False)
    if out is None:
        out = torch.empty((t, hidden), dtype=torch.bfloat16, device=h.device)
    _bf16_2d(out, "moe_combine out")
    d = hip.MiMoeCombineDesc(t=t, hidden=hidden, top_k=top_k, h=hip.ptr(h), ldh=h.stride(0), weights=hip.ptr(weights),
                             shared=hip.ptr(shared), ld_shared=shared.stride(0) if shared is not None else 0,
                             shared_gate=hip.ptr(shared_gate),
                             ld_gate=shared_gate.stride(0) if shared_gate is not None else 0,
                             residual=hip.ptr(residual), ldr=residual.stride(0) if residual is not None else 0,
                             out=hip.ptr(out), ldo=out.stride(0))
    if next_norm is not None:
        nw, nx, neps = next_norm
        if nw.dtype != torch.float32 or nw.numel() != hidden or not nw.is_contiguous():
            raise ValueError("moe_combine next_norm: w must be a contiguous float32 [H]")
        _bf16_2d(nx, "moe_combine next_norm x")
        if nx.shape[0] < t or nx.shape[1] < hidden:
            raise ValueError("moe_combine next_norm: x too small")
        d.next_norm_w, d.next_x, d.ld_next_x, d.next_eps = hip.ptr(nw), hip.ptr(nx), nx.stride(0), float(neps)
    hip.call("mi_moe_combine", C.byref(d), hip.stream_handle(stream))
    return out


def embed(table, tokens, *, t: Optional[int] = None, out=None, stream=None):
    """``embed`` (``ops/embed.py:1-7``): ``out[i] = table[tokens[i]]`` for ``i < t`` over a BF16 ``table
    [vocab, hidden]`` — or a BF16 ``PackedWeight`` (the pack's embedding slab, gathered from its T16 tiles);
    ``tokens`` is a device int32 vector (a view of the step state's ``pending_tokens`` in a step program); an id
    outside ``[0, vocab)`` reads row 0."""
    torch = _torch()
    t16 = isinstance(table, PackedWeight)
    if t16:
        if table.format != "bf16" or table.experts != 1:
            raise ValueError("embed: a packed table must be one BF16 slab")
        vocab, hidden, src = table.n, table.k, table.data
    else:
        _bf16_2d(table, "embed table")
        vocab, hidden = table.shape
        src = table
    t = tokens.numel() if t is None else t
    if tokens.dtype != torch.int32 or tokens.numel() < t or not 1 <= t <= 16:
        raise ValueError("embed: tokens must be a device int32 vector of 1..16 ids")
    if out is None:
        out = torch.empty((t, hidden), dtype=torch.bfloat16, device=src.device)
    _bf16_2d(out, "embed out")
    if out.shape[0] < t or out.shape[1] != hidden:
        raise ValueError("embed: out must be [t, hidden]")
    d = hip.MiEmbedDesc(t=t, vocab=vocab, hidden=hidden, tokens=hip.ptr(tokens), table=hip.ptr(src),
                        out=hip.ptr(out), ldo=out.stride(0), t16=int(t16))
    hip.call("mi_embed", C.byref(d), hip.stream_handle(stream))
    return out


def argmax(logits, *, out=None, stream=None):
    """``argmax`` (``ops/sample.py:1-9``): ``logits [T, V]`` float32 or bf16 → ``ids [T]`` int32; ties → the lowest
    index, NaN never wins, a row without a number gives -1."""
    torch = _torch()
    if logits.dim() != 2 or logits.stride(1) != 1 or logits.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("argmax: logits must be a row-major 2-D float32 or bfloat16 tensor")
    t, v = logits.shape
    if not 1 <= t <= 16:
        raise ValueError("argmax: 1..16 rows")
    if out is None:
        out = torch.empty(t, dtype=torch.int32, device=logits.device)
    if out.dtype != torch.int32 or out.numel() < t:
        raise ValueError("argmax: out must be int32 [t]")
    d = hip.MiArgmaxDesc(t=t, vocab=v, logits=hip.ptr(logits), ld=logits.stride(0),
                         f32=int(logits.dtype == torch.float32), ids=hip.ptr(out))
    hip.call("mi_argmax", C.byref(d), hip.stream_handle(stream))
    return out


def sample(logits, *, temperature: float = 1.0, top_k: int = 0, top_p: float = 0.0, min_p: float = 0.0,
           topp_in_topk: bool = False, seed: int = 0, step: int = 0, state=None, out=None, stream=None):
    """``sample`` (``ops/sample.py:1-10``): ``logits [T, V]`` bf16 → ``ids [T]`` int32 drawn from the warped softmax
    (top-k / top-p / min-p thresholds, temperature) by Gumbel-max with the reference's counter-based noise, so the
    draw for (seed, step, row) is reproducible. ``state``: a step state whose ``rng_lo/rng_hi`` and ``step`` give the
    seed and step on the device (a captured program). Temperature 0 is greedy: :func:`argmax`."""
    torch = _torch()
    _bf16_2d(logits, "sample logits", aligned=False)
    t, v = logits.shape
    if not 1 <= t <= 16:
        raise ValueError("sample: 1..16 rows")
    if temperature <= 0:
        return argmax(logits, out=out, stream=stream)
    if out is None:
        out = torch.empty(t, dtype=torch.int32, device=logits.device)
    if out.dtype != torch.int32 or out.numel() < t:
        raise ValueError("sample: out must be int32 [t]")
    if state is not None:
        _check_state(state, "sample")
    d = hip.MiSampleDesc(t=t, vocab=v, logits=hip.ptr(logits), ld=logits.stride(0), ids=hip.ptr(out),
                         temperature=temperature, top_p=top_p, min_p=min_p, top_k=top_k,
                         topp_in_topk=int(topp_in_topk), seed=seed & 0xFFFFFFFFFFFFFFFF, step=step,
                         state=hip.ptr(state))
    hip.call("mi_sample", C.byref(d), hip.stream_handle(stream))
    return out


def advance(state, tokens, ring, ring_cap: int, *, eos=(), ctx_cap: int = 0, host_ctl=None, stream=None):
    """``advance`` (``kernels/common/advance.metal:15-37``): close a step — publish the last row's token to the ring,
    make it the next step's pending token, move position and step, stop at EOS / ``stop_at`` / the context capacity.
    ``state``: the device step state (int32 tensor of 68 words); ``ring`` / ``host_ctl``: pinned host addresses."""
    _check_state(state, "advance")
    n_eos, eos_arr = _eos_list(eos)
    d = hip.MiAdvanceDesc(state=hip.ptr(state), tokens=hip.ptr(tokens), ring=hip.ptr(ring), ring_cap=ring_cap,
                          ctx_cap=ctx_cap, n_eos=n_eos, eos=eos_arr, host_ctl=hip.ptr(host_ctl))
    hip.call("mi_advance", C.byref(d), hip.stream_handle(stream))


def _eos_list(eos):
    eos = [int(e) for e in ([eos] if isinstance(eos, int) else eos) if e is not None and int(e) >= 0]
    if len(eos) > 8:
        raise ValueError("at most 8 EOS ids")
    return len(eos), (C.c_int32 * 8)(*eos)


def _check_state(state, name):
    torch = _torch()
    if state.dtype != torch.int32 or state.numel() * 4 < C.sizeof(hip.MiStepState) or not state.is_cuda:
        raise ValueError(f"{name}: state must be a device int32 tensor of the step-state size")


def verify_select(state, drafts, conf, *, gamma: int, threshold: float = 0.0, t_max: int = 8, mode: int = 0,
                  cost=None, conf_log=None, ctx_cap: int = 0, lm: bool = False, stream=None):
    """``verify_select`` (``ops/draft.py:13-15,27``; ``spec_ops.metal:108-146``): choose the verify length of the next
    step from the drafter's block (``drafts [γ]`` int32, ``conf [γ]`` float32 on the device) and set its pending
    tokens. ``mode`` 0 confident prefix (``threshold``), 1 cost-aware (``cost [16]``), 2 fixed L = ``threshold``;
    ``conf_log [log_cap, 16]`` float32 receives the block's confidences."""
    torch = _torch()
    _check_state(state, "verify_select")
    if not 0 <= gamma <= 15 or not 1 <= t_max <= 16 or mode not in (0, 1, 2):
        raise ValueError("verify_select: gamma 0..15, t_max 1..16, mode 0..2")
    if gamma and (drafts.dtype != torch.int32 or drafts.numel() < gamma or conf.dtype != torch.float32
                  or conf.numel() < gamma):
        raise ValueError("verify_select: drafts int32 [gamma], conf float32 [gamma]")
    c = list(cost) if cost is not None else [1.0] * 16
    if mode == 1 and (len(c) < min(gamma, t_max - 1) + 1 or any(v <= 0 for v in c[: gamma + 1])):
        raise ValueError("verify_select: cost needs a positive entry per length 0..gamma")
    log_cap = 0 if conf_log is None else conf_log.numel() // 16
    d = hip.MiVerifySelectDesc(state=hip.ptr(state), drafts=hip.ptr(drafts), conf=hip.ptr(conf), gamma=gamma,
                               t_max=t_max, mode=mode, threshold=threshold, cost=(C.c_float * 16)(*c[:16]),
                               conf_log=hip.ptr(conf_log), log_cap=log_cap, ctx_cap=ctx_cap, lm=int(lm))
    hip.call("mi_verify_select", C.byref(d), hip.stream_handle(stream))


def accept_scan(state, tokens, ring, ring_cap: int, *, eos=(), log=None, ctx_cap: int = 0, lm: bool = False,
                host_ctl=None, stream=None):
    """``accept_scan`` (``ops/draft.py:16-18,28``; ``spec_ops.metal:148-195``): the closing serial op of a
    speculative step — commit the accepted drafts and the bonus token to the ring, advance the state.
    ``tokens``: the target's argmax per row (device int32); ``ring`` / ``host_ctl``: pinned host addresses;
    ``log [log_cap]`` int32 receives ``(committed << 16) | (L << 8) | accepted`` per step."""
    _check_state(state, "accept_scan")
    n_eos, eos_arr = _eos_list(eos)
    d = hip.MiAcceptScanDesc(state=hip.ptr(state), tokens=hip.ptr(tokens), ring=hip.ptr(ring), ring_cap=ring_cap,
                             ctx_cap=ctx_cap, lm=int(lm), n_eos=n_eos, eos=eos_arr, log=hip.ptr(log),
                             log_cap=0 if log is None else log.numel(), host_ctl=hip.ptr(host_ctl))
    hip.call("mi_accept_scan", C.byref(d), hip.stream_handle(stream))
