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


@dataclass
class PackedWeight:
    """A T16 pack resident in HBM: ``data`` uint8 ``[experts·nbytes]``, NVFP4 ``row_scale`` float32
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


def _bf16_2d(t, name):
    torch = _torch()
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name}: expected a row-major 2-D bfloat16 tensor, got {t.dtype} {tuple(t.shape)}")
    if t.data_ptr() % 16 or t.stride(0) % 8:
        raise ValueError(f"{name}: needs 16-byte alignment and a row stride multiple of 8")


def gemv(w: PackedWeight, x, *, epilogue=None, residual=None, norm_w=None, eps: float = 1e-6, out=None,
         stream=None, workspace=None, out_f32: bool = False):
    """``gemv`` (``ops/gemv.py:1-12``): ``y = x·Wᵀ`` for ``x [M, K]`` bf16, M ≤ 16; ``epilogue`` None | "residual" |
    "silu_mul" (rows gate|up interleaved by 8, output N/2 columns) | "silu_mul_rounded"; ``norm_w`` = the (1 + w)
    float32 weight of a fused input RMSNorm; ``out_f32`` writes the unrounded FP32 result (``lm_head``)."""
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
    d = hip.MiGemvDesc(format=hip.MI_FMT[w.format], n=w.n, k=w.k, m=m, w=hip.ptr(w.data),
                       row_scale=hip.ptr(w.row_scale), x=hip.ptr(x), ldx=x.stride(0), y=hip.ptr(out),
                       ldy=out.stride(0), epilogue=hip.MI_EPI[epilogue],
                       residual=hip.ptr(residual) if epilogue == "residual" else 0,
                       ldr=residual.stride(0) if epilogue == "residual" else 0, norm_w=hip.ptr(norm_w), eps=eps,
                       groups=0, max_groups=0, top_k=0, x_per_slot=0,
                       workspace=hip.ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel(),
                       out_f32=int(out_f32))
    hip.call("mi_gemv", C.byref(d), hip.stream_handle(stream))
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
