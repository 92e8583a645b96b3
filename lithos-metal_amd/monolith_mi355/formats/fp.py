"""Host-side float-code helpers the packers need (numpy): BF16 rounding and nibble packing.

Conventions follow the reference's storage formats (``monolith/formats/fp.py``): BF16 is the top half of an IEEE
float32 rounded to nearest even; E2M1 / INT4 codes sit two per byte, low nibble first.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16(x) -> np.ndarray:
    xf = np.asarray(x, dtype=np.float32)
    u = xf.view(np.uint32).astype(np.uint64)
    out = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(np.isnan(xf), (u >> 16) | 0x40, out).astype(np.uint16)


def bf16_to_f32(u16) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16_values(x) -> np.ndarray:
    """float32 array rounded to BF16-representable values."""
    return bf16_to_f32(f32_to_bf16(x))


def nibbles_to_bytes(codes) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def bytes_to_nibbles(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8)
    out = np.empty(b.shape[:-1] + (2 * b.shape[-1],), np.uint8)
    out[..., 0::2] = b & 0xF
    out[..., 1::2] = b >> 4
    return out
