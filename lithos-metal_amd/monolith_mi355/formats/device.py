"""Quantize and pack on the GPU (torch ops): the same arithmetic as the host quantizers and the T16 pack in
:mod:`monolith_mi355.formats` / :mod:`.pack`, for synthetic and load-time weights too large to quantize in numpy
quickly (a [17408, 5120] matrix: ~20 s in numpy, milliseconds here). Bit-identical to the host path (tested).

* NVFP4 (``formats/nvfp4.py:146-161``): ``s2 = f32(amax / (6·448))``; block scale = E4M3(RNE, saturating) of
  ``bmax / 6 / s2``; codes = E2M1(RNE) of ``w / (e4m3(scale) · s2)``.
"""

from __future__ import annotations

import torch

E4M3_MAX = 448.0


def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """float32 → E4M3 byte (uint8), nearest even, saturating at 448, NaN → 0x7F."""
    m = x.abs().double()
    sub = m < 2.0 ** -6
    code_sub = torch.round(m * 2.0 ** 9)                      # torch.round: half to even
    safe = torch.where(sub, torch.ones_like(m), m)
    e = torch.floor(torch.log2(safe))
    frac = torch.round((safe / torch.exp2(e) - 1.0) * 8.0)
    e = torch.where(frac == 8, e + 1, e)
    frac = torch.where(frac == 8, torch.zeros_like(frac), frac)
    code_norm = (e + 7) * 8 + frac
    code = torch.where(sub, code_sub, code_norm)
    code = torch.where(m > E4M3_MAX, torch.full_like(code, 0x7E), code).to(torch.int32)
    code = torch.where(torch.signbit(x), code | 0x80, code)
    code = torch.where(torch.isnan(x), torch.full_like(code, 0x7F), code)
    return code.to(torch.uint8)


def e4m3_decode(codes: torch.Tensor) -> torch.Tensor:
    c = codes.to(torch.int32)
    e, f = (c >> 3) & 0xF, c & 7
    ed, fd = e.double(), f.double()
    mag = torch.where(e == 0, fd * 2.0 ** -9, (1.0 + fd / 8.0) * torch.exp2(ed - 7))
    mag = torch.where((e == 15) & (f == 7), torch.full_like(mag, float("nan")), mag)
    return torch.where((c & 0x80) != 0, -mag, mag).float()


def e2m1_encode(x: torch.Tensor) -> torch.Tensor:
    m = torch.clamp(x.abs().double(), max=6.0)
    code = torch.where(m < 2, torch.round(m * 2), torch.where(m < 4, 4 + torch.round(m - 2), 6 + torch.round((m - 4) / 2)))
    code = code.to(torch.int32)
    return torch.where(torch.signbit(x), code | 8, code).to(torch.uint8)


def nvfp4_quantize(w: torch.Tensor):
    """``(codes uint8 [N, K/2] low nibble first, scales uint8 [N, K/16], s2 float)``."""
    w = w.float()
    n, k = w.shape
    if k % 16:
        raise ValueError("nvfp4: K must be a multiple of 16")
    amax = float(w.abs().max().item()) or 1.0
    s2 = float(torch.tensor(amax / (6.0 * E4M3_MAX), dtype=torch.float32).item())
    blocks = w.reshape(n, k // 16, 16)
    bmax = blocks.abs().amax(dim=-1)
    s2t = torch.tensor(s2, dtype=torch.float32, device=w.device)
    val = torch.where(bmax > 0, bmax / torch.tensor(6.0, device=w.device) / s2t, torch.zeros_like(bmax))
    sc = e4m3_encode(val)
    denom = e4m3_decode(sc)[..., None] * s2t
    scaled = torch.where(denom > 0, blocks / torch.where(denom > 0, denom, torch.ones_like(denom)), torch.zeros_like(blocks))
    codes = e2m1_encode(scaled.reshape(n, k))
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    return packed, sc, s2


def pack_nvfp4(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """The T16 NVFP4 layout (see :mod:`.pack`) of ``codes [N, K/2]``, ``scales [N, K/16]`` → uint8 [bytes]."""
    from .pack import nvfp4_groups
    n, kh = codes.shape
    k = kh * 2
    nt, c = -(-n // 16), k // 128
    rows = nt * 16
    if rows != n:
        codes = torch.cat([codes, codes.new_zeros(rows - n, kh)])
        scales = torch.cat([scales, scales.new_zeros(rows - n, k // 16)])
    cw = codes.reshape(nt, 16, c, 4, 16).permute(0, 2, 3, 1, 4).reshape(nt, c, 1024)
    sw = scales.reshape(nt, 16, c, 4, 2).permute(0, 2, 3, 1, 4).reshape(nt, c, 64, 2)
    parts = []
    for c0, g, _, sb in nvfp4_groups(c)[0]:
        parts.append(cw[:, c0: c0 + g].reshape(nt, g * 1024))
        piece = sw.new_zeros(nt, 64, sb // 64)
        piece[:, :, : 2 * g] = sw[:, c0: c0 + g].permute(0, 2, 1, 3).reshape(nt, 64, 2 * g)
        parts.append(piece.reshape(nt, sb))
    return torch.cat(parts, dim=-1).reshape(-1).contiguous()


def interleave_rows(gate: torch.Tensor, up: torch.Tensor, chunk: int = 8) -> torch.Tensor:
    """``[gate; up]`` rows reordered ``chunk`` gate rows then ``chunk`` up rows (``packs/transforms.py:16-24``)."""
    n = gate.shape[0]
    return torch.stack([gate.reshape(n // chunk, chunk, -1), up.reshape(n // chunk, chunk, -1)], dim=1).reshape(2 * n, -1)


def pack_bf16(w: torch.Tensor) -> torch.Tensor:
    """The T16 BF16 layout (see :mod:`.pack`) of ``w [N, K]`` bfloat16 (K a multiple of 32) → uint8 [bytes]."""
    n, k = w.shape
    if k % 32:
        raise ValueError("pack_bf16: K must be a multiple of 32")
    nt = -(-n // 16)
    if nt * 16 != n:
        w = torch.cat([w, w.new_zeros(nt * 16 - n, k)])
    u = w.contiguous().view(torch.int16).reshape(nt, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4)
    return u.contiguous().view(torch.uint8).reshape(-1)
