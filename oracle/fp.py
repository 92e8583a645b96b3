"""Exact float-code tables and conversions (numpy), restating ``monolith/formats/fp.py``.

* E4M3 (OCP ``float8_e4m3fn``): bias 7, no infinities, ``0x7F``/``0xFF`` NaN, max finite 448
  (``formats/fp.py:18-29``). Encoding rounds to nearest, ties to the even code, saturates above 448 to ``0x7E``
  (or raises), NaN → ``0x7F`` (``formats/fp.py:40-61``).
* E2M1 (NVFP4 codes): magnitudes ``0 .5 1 1.5 2 3 4 6`` plus a sign bit; two codes per byte, low nibble first
  (``formats/fp.py:65-102``). Encoding: nearest, ties to the even code, saturating at 6 (``formats/fp.py:77-86``).
* BF16: the top half of an IEEE float32, rounded to nearest even; NaN keeps its payload with the quiet bit
  (``formats/fp.py:106-117``).
"""

from __future__ import annotations

import numpy as np


def _build_e4m3() -> np.ndarray:
    """Value of every E4M3 byte (``formats/fp.py:18-26``)."""
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * 2.0 ** -9            # subnormal: m · 2^(1-7) / 8
        else:
            out[code] = sign * (8 + man) * 2.0 ** (exp - 10)
    return out


E4M3_TABLE = _build_e4m3()
E4M3_MAX = 448.0
E2M1_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                       -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
E2M1_MAX = 6.0

_E4M3_FINITE_POS = np.array([c for c in range(0x7F)], dtype=np.uint8)       # 0x00..0x7E, ascending in value
_E4M3_FINITE_VAL = E4M3_TABLE[_E4M3_FINITE_POS].astype(np.float64)
_E2M1_POS_VAL = E2M1_TABLE[:8].astype(np.float64)


def _nearest_even(mag: np.ndarray, values: np.ndarray) -> np.ndarray:
    """Index of the nearest entry of the ascending ``values`` to each ``mag``; an exact tie takes the even index
    (the code of the even mantissa: codes and indices coincide for the positive halves of both tables)."""
    hi = np.clip(np.searchsorted(values, mag, side="left"), 0, len(values) - 1)
    lo = np.clip(hi - 1, 0, len(values) - 1)
    d_lo = mag - values[lo]
    d_hi = values[hi] - mag
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    return np.where(take_hi, hi, lo)


def e4m3_to_f32(codes) -> np.ndarray:
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3(x, *, saturate: bool = True) -> np.ndarray:
    """Round to nearest even E4M3 (``formats/fp.py:40-61``)."""
    x = np.asarray(x, dtype=np.float32)
    mag = np.abs(x).astype(np.float64)
    over = mag > E4M3_MAX
    if over.any() and not saturate:
        raise ValueError("f32_to_e4m3: magnitude above 448")
    code = _E4M3_FINITE_POS[_nearest_even(np.minimum(mag, E4M3_MAX), _E4M3_FINITE_VAL)].astype(np.uint8)
    code = np.where(np.signbit(x), code | np.uint8(0x80), code).astype(np.uint8)
    return np.where(np.isnan(x), np.uint8(0x7F), code).astype(np.uint8)


def e2m1_to_f32(codes) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8)
    if c.size and int(c.max()) > 15:
        raise ValueError("e2m1_to_f32: codes must be 4-bit")
    return E2M1_TABLE[c]


def f32_to_e2m1(x) -> np.ndarray:
    """Round to nearest even E2M1, saturating at 6 (``formats/fp.py:77-86``)."""
    x = np.asarray(x, dtype=np.float32)
    mag = np.minimum(np.abs(x).astype(np.float64), E2M1_MAX)
    code = _nearest_even(mag, _E2M1_POS_VAL).astype(np.uint8)
    return np.where(np.signbit(x), code | np.uint8(8), code).astype(np.uint8)


def unpack_nibbles(packed) -> np.ndarray:
    """``[..., K/2]`` bytes → ``[..., K]`` codes, low nibble first (``formats/fp.py:89-95``)."""
    p = np.asarray(packed, dtype=np.uint8)
    return np.stack([p & 0xF, p >> 4], axis=-1).reshape(p.shape[:-1] + (2 * p.shape[-1],))


def pack_nibbles(codes) -> np.ndarray:
    """Inverse of :func:`unpack_nibbles` (``formats/fp.py:98-102``)."""
    c = np.asarray(codes, dtype=np.uint8)
    if c.shape[-1] % 2:
        raise ValueError("pack_nibbles: last dimension must be even")
    pairs = c.reshape(c.shape[:-1] + (c.shape[-1] // 2, 2))
    return (pairs[..., 0] | (pairs[..., 1] << 4)).astype(np.uint8)


def bf16_to_f32(u16) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    """Round to nearest even; NaN keeps its payload with the quiet bit set (``formats/fp.py:111-117``)."""
    xf = np.asarray(x, dtype=np.float32)
    u = xf.view(np.uint32).astype(np.uint64)
    rne = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(np.isnan(xf), (u >> 16) | 0x40, rne).astype(np.uint16)


def rbf(x) -> np.ndarray:
    """Round float32 values to BF16 and widen back (the ``.to(bfloat16)`` of the torch oracles)."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, dtype=np.float32)))


def f16_round(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
