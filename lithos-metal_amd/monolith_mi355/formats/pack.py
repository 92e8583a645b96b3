"""The T16 weight pack streamed by the gfx950 GEMV kernels — this backend's counterpart of the reference's
block-lane-major pack (``monolith/formats/blm.py:56-266``), laid out for wave64 MFMA operands instead of 32-lane
stripes.

A matrix ``[N, K]`` is cut into 16-row tiles (the last one zero-padded) and 128-column chunks (32 for BF16). Each
(tile, chunk) is one unit, tile-major then chunk, so one wave walking a tile's K reads a contiguous stream:

* NVFP4: the chunks of a tile come in groups of 8 (the last group holds the rest): the group's 1 KiB code blocks,
  then one scale block. In the code block of chunk ``c``, bytes ``[16·l, 16·l+16)`` for lane ``l`` (row
  ``r = l % 16``, k-group ``g = l // 16``) hold the 32 codes of row ``r`` at columns ``128·c + 32·g + [0, 32)`` —
  the checkpoint's own bytes, low nibble first. The scale block gives lane ``l`` a piece of 16 bytes (8 bytes when
  the group has at most 4 chunks) whose bytes ``2·i, 2·i + 1`` are the two E4M3 block scales of chunk ``i`` of the
  group for that lane's 32 columns — one 16-byte load per lane brings the scales of 8 chunks.
* INT4 affine (1152 B): lane ``l``'s dword ``s`` (``s = 0..3``) holds the 8 codes of row ``r`` at columns
  ``128·c + 32·s + 8·g + [0, 8)``; bytes ``[1024 + 8·r, +8)`` the BF16 (scale, bias) pairs of groups ``2c`` and
  ``2c + 1`` of row ``r`` (scale in the low half, as the reference's pairs, ``formats/int4_affine.py:460``).
* BF16 (1024 B): lane ``l``'s 16 bytes are the 8 values of row ``r`` at columns ``32·c + 8·g + [0, 8)``.
* FP8 E4M3 (1024 B, 64-column chunks): lane ``l``'s 16 bytes are the codes of row ``r`` at columns
  ``64·c + 16·g + [0, 16)``; the FP32 tensor scale is the per-row table, as for NVFP4.

The byte count per weight is the format's own (0.5625 B for NVFP4 and INT4) except for the scale block of a short
last NVFP4 group (K not a multiple of 1024 columns), padded to 8 or 16 bytes per lane.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

from . import DequantSpec
from .fp import bf16_to_f32, f32_to_bf16

UNIT_Q = 1152
UNIT_B = 1024
FORMAT_IDS = {"nvfp4": 1, "int4_affine": 2, "bf16": 3, "fp8_e4m3": 4}


def chunk_cols(fmt: str) -> int:
    return {"bf16": 32, "fp8_e4m3": 64}.get(fmt, 128)


def unit_bytes(fmt: str) -> int:
    return UNIT_B if fmt in ("bf16", "fp8_e4m3") else UNIT_Q


def nvfp4_groups(chunks: int):
    """``[(first chunk, chunks in the group, byte offset in the tile, scale-block bytes), …]`` and the tile bytes."""
    out, off = [], 0
    for c0 in range(0, chunks, 8):
        g = min(8, chunks - c0)
        sb = 1024 if g > 4 else 512
        out.append((c0, g, off, sb))
        off += g * 1024 + sb
    return out, off


def pack_bytes(fmt: str, n: int, k: int) -> int:
    if fmt == "nvfp4":
        return -(-n // 16) * nvfp4_groups(k // 128)[1]
    return -(-n // 16) * (k // chunk_cols(fmt)) * unit_bytes(fmt)


@dataclass
class PackInfo:
    format: str
    n: int
    k: int
    n_tiles: int
    chunks: int
    nbytes: int
    row_scale: Optional[np.ndarray] = None     # NVFP4 / FP8: per-row tensor scale [n_tiles·16] float32


def _pad_rows(a: np.ndarray, rows: int) -> np.ndarray:
    if a.shape[0] == rows:
        return np.ascontiguousarray(a)
    out = np.zeros((rows,) + a.shape[1:], a.dtype)
    out[: a.shape[0]] = a
    return out


def pack(spec: DequantSpec, row_scale: Optional[np.ndarray] = None) -> Tuple[np.ndarray, PackInfo]:
    """``(bytes as uint8 array, PackInfo)`` of the T16 layout. ``row_scale`` overrides the NVFP4 / FP8 per-row tensor
    scale (stacked slabs whose parts carry different tensor scales)."""
    fmt = spec.format
    n, k = spec.shape
    kc = chunk_cols(fmt)
    if k % kc:
        raise ValueError(f"T16 pack: {fmt} needs K % {kc} == 0 (K={k})")
    nt, c = -(-n // 16), k // kc
    rows = nt * 16
    if fmt == "nvfp4":
        w = _pad_rows(np.asarray(spec.tensors["weight"], np.uint8), rows)            # [rows, K/2]
        sc = _pad_rows(np.asarray(spec.tensors["weight_scale"], np.uint8), rows)     # [rows, K/16]
        codes = w.reshape(nt, 16, c, 4, 16).transpose(0, 2, 3, 1, 4).reshape(nt, c, 1024)
        scales = sc.reshape(nt, 16, c, 4, 2).transpose(0, 2, 3, 1, 4).reshape(nt, c, 64, 2)      # [nt, c, lane, 2]
        parts = []
        for c0, g, _, sb in nvfp4_groups(c)[0]:
            parts.append(codes[:, c0: c0 + g].reshape(nt, g * 1024))
            piece = np.zeros((nt, 64, sb // 64), np.uint8)
            piece[:, :, : 2 * g] = scales[:, c0: c0 + g].transpose(0, 2, 1, 3).reshape(nt, 64, 2 * g)
            parts.append(piece.reshape(nt, sb))
        data = np.concatenate(parts, axis=-1)
        if row_scale is None:
            row_scale = np.full(n, spec.params["weight_scale_2"], np.float32)
        rs = np.zeros(rows, np.float32)
        rs[:n] = np.asarray(row_scale, np.float32)
        info = PackInfo(fmt, n, k, nt, c, data.size, rs)
    elif fmt == "int4_affine":
        w = _pad_rows(np.asarray(spec.tensors["weight"], np.uint8), rows)            # [rows, K/2]
        codes = w.reshape(nt, 16, c, 4, 4, 4).transpose(0, 2, 4, 1, 3, 5).reshape(nt, c, 1024)   # (s, g) → (g, r, s)
        sc = f32_to_bf16(_pad_rows(np.asarray(spec.tensors["scales"], np.float32), rows))       # [rows, K/64]
        bi = f32_to_bf16(_pad_rows(np.asarray(spec.tensors["biases"], np.float32), rows))
        pairs = np.stack([sc, bi], axis=-1).reshape(nt, 16, c, 2, 2).transpose(0, 2, 1, 3, 4)   # [nt, c, r, grp, 2]
        data = np.concatenate([codes, np.ascontiguousarray(pairs).view(np.uint8).reshape(nt, c, 128)], axis=-1)
        info = PackInfo(fmt, n, k, nt, c, data.size)
    elif fmt == "bf16":
        w = _pad_rows(np.asarray(spec.tensors["weight"], np.uint16), rows)           # [rows, K]
        data = np.ascontiguousarray(w.reshape(nt, 16, c, 4, 8).transpose(0, 2, 3, 1, 4)).reshape(nt, c, 512).view(np.uint8)
        info = PackInfo(fmt, n, k, nt, c, data.size)
    elif fmt == "fp8_e4m3":
        w = _pad_rows(np.asarray(spec.tensors["weight"], np.uint8), rows)            # [rows, K]
        data = np.ascontiguousarray(w.reshape(nt, 16, c, 4, 16).transpose(0, 2, 3, 1, 4)).reshape(nt, c, 1024)
        if row_scale is None:
            row_scale = np.full(n, spec.params["weight_scale"], np.float32)
        rs = np.zeros(rows, np.float32)
        rs[:n] = np.asarray(row_scale, np.float32)
        info = PackInfo(fmt, n, k, nt, c, data.size, rs)
    else:
        raise ValueError(f"T16 pack: unknown format {fmt!r}")
    return np.ascontiguousarray(data).reshape(-1), info


def unpack(data: np.ndarray, info: PackInfo) -> DequantSpec:
    """Inverse of :func:`pack` (round-trip tests)."""
    nt, c, n, k = info.n_tiles, info.chunks, info.n, info.k
    d = np.asarray(data, np.uint8)
    if info.format == "nvfp4":
        groups, tile = nvfp4_groups(c)
        d = d.reshape(nt, tile)
        codes = np.empty((nt, c, 1024), np.uint8)
        scales = np.empty((nt, c, 64, 2), np.uint8)
        for c0, g, off, sb in groups:
            codes[:, c0: c0 + g] = d[:, off: off + g * 1024].reshape(nt, g, 1024)
            piece = d[:, off + g * 1024: off + g * 1024 + sb].reshape(nt, 64, sb // 64)[:, :, : 2 * g]
            scales[:, c0: c0 + g] = piece.reshape(nt, 64, g, 2).transpose(0, 2, 1, 3)
        w = codes.reshape(nt, c, 4, 16, 16).transpose(0, 3, 1, 2, 4).reshape(nt * 16, k // 2)
        sc = scales.reshape(nt, c, 4, 16, 2).transpose(0, 3, 1, 2, 4).reshape(nt * 16, k // 16)
        rs = info.row_scale[:n] if info.row_scale is not None else np.ones(n, np.float32)
        s2 = float(rs[0]) if n else 1.0
        return DequantSpec("nvfp4", (n, k), {"weight": w[:n], "weight_scale": sc[:n]}, {"weight_scale_2": s2})
    if info.format == "int4_affine":
        d = d.reshape(nt, c, UNIT_Q)
        w = d[..., :1024].reshape(nt, c, 4, 16, 4, 4).transpose(0, 3, 1, 4, 2, 5).reshape(nt * 16, k // 2)
        pairs = np.ascontiguousarray(d[..., 1024:]).view(np.uint16).reshape(nt, c, 16, 2, 2).transpose(0, 2, 1, 3, 4)
        pairs = pairs.reshape(nt * 16, k // 64, 2)
        return DequantSpec("int4_affine", (n, k), {"weight": w[:n], "scales": bf16_to_f32(pairs[:n, :, 0]),
                                                   "biases": bf16_to_f32(pairs[:n, :, 1])}, {"group": 64})
    if info.format == "fp8_e4m3":
        w = d.reshape(nt, c, 4, 16, 16).transpose(0, 3, 1, 2, 4).reshape(nt * 16, k)
        s = float(info.row_scale[0]) if info.row_scale is not None and n else 1.0
        return DequantSpec("fp8_e4m3", (n, k), {"weight": w[:n]}, {"weight_scale": s})
    d = d.reshape(nt, c, UNIT_B).view(np.uint16).reshape(nt, c, 4, 16, 8)
    w = d.transpose(0, 3, 1, 2, 4).reshape(nt * 16, k)
    return DequantSpec("bf16", (n, k), {"weight": w[:n]})
