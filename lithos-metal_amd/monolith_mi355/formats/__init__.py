"""Weight formats of the gfx950 backend: the reference's ``Format`` plugin contract (``monolith/formats/base.py:169-217``)
for the three formats the decode layer streams, with the T16 pack instead of the 32-lane BLM pack.

``unpack`` groups checkpoint tensors (ModelOpt NVFP4 ``weight/weight_scale/weight_scale_2``, MLX NVFP4
``weight(U32)/scales``, MLX affine ``weight(U32)/scales/biases``, BF16 ``weight``) into a :class:`DequantSpec`;
``quantize`` implements the reference quantizers (``formats/nvfp4.py:146-161``, ``formats/int4_affine.py:93-119``);
``pack`` writes the T16 layout the HIP kernels stream (:mod:`.pack`).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Mapping, Tuple

import numpy as np

from .fp import bf16_to_f32, bytes_to_nibbles, f32_to_bf16, nibbles_to_bytes, to_bf16_values

E4M3_MAX = 448.0
E2M1_MAX = 6.0


@dataclass
class DequantSpec:
    """Checkpoint tensors of one matrix by role, its logical ``[N, K]`` shape and format constants
    (``monolith/formats/base.py:154-166``)."""

    format: str
    shape: Tuple[int, int]
    tensors: Dict[str, Any] = field(default_factory=dict)
    params: Dict[str, Any] = field(default_factory=dict)


# ---- code conversions (arithmetic, not tables) ------------------------------------------------------------------------
def e4m3_encode(x) -> np.ndarray:
    """Float → E4M3 byte, round to nearest even, saturating at 448 (0x7E), NaN → 0x7F."""
    x = np.asarray(x, dtype=np.float32)
    m = np.abs(x).astype(np.float64)
    code = np.zeros(x.shape, np.int64)
    sub = m < 2.0 ** -6
    code = np.where(sub, np.rint(m * 2.0 ** 9), code)
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(sub, 1.0, m)))
        frac = np.rint((np.where(sub, 1.0, m) / 2.0 ** e - 1.0) * 8.0)
    e = np.where(frac == 8, e + 1, e)
    frac = np.where(frac == 8, 0, frac)
    normal = ((e + 7).astype(np.int64) << 3) | frac.astype(np.int64)
    code = np.where(sub, code, normal)
    code = np.where(m > E4M3_MAX, 0x7E, code).astype(np.uint8)
    code = np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)
    return np.where(np.isnan(x), 0x7F, code).astype(np.uint8)


def e4m3_decode(codes) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e, f = (c >> 3) & 0xF, c & 7
    mag = np.where(e == 0, f * 2.0 ** -9, (1.0 + f / 8.0) * 2.0 ** (e - 7))
    mag = np.where((e == 15) & (f == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def e2m1_encode(x) -> np.ndarray:
    """Float (pre-scaled into [-6, 6]) → E2M1 code, round to nearest even code, saturating at 6."""
    x = np.asarray(x, dtype=np.float32)
    m = np.minimum(np.abs(x).astype(np.float64), E2M1_MAX)
    code = np.where(m < 2, np.rint(m * 2), np.where(m < 4, 4 + np.rint(m - 2), 6 + np.rint((m - 4) / 2)))
    code = code.astype(np.uint8)
    return np.where(np.signbit(x), code | 8, code).astype(np.uint8)


_E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def e2m1_decode(codes) -> np.ndarray:
    return _E2M1[np.asarray(codes, dtype=np.uint8)]


# ---- formats -------------------------------------------------------------------------------------------------------------
class NVFP4:
    name = "nvfp4"
    block = 16
    bytes_per_weight = 0.5 + 1.0 / 16

    def unpack(self, tensors: Mapping[str, Any], *, shape: Tuple[int, int]) -> DequantSpec:
        """ModelOpt (``weight`` U8, ``weight_scale`` E4M3, ``weight_scale_2``) or MLX (``weight`` U32, ``scales`` U8,
        no tensor scale) — ``formats/nvfp4.py:122-137``."""
        n, k = shape
        if "weight_scale_2" in tensors:
            w = np.asarray(tensors["weight"], np.uint8)
            sc = np.asarray(tensors["weight_scale"], np.uint8)
            s2 = float(np.asarray(tensors["weight_scale_2"], np.float32).reshape(()))
        elif "scales" in tensors:
            w32 = np.ascontiguousarray(np.asarray(tensors["weight"], np.uint32))
            w = w32.view(np.uint8).reshape(w32.shape[0], -1)
            sc = np.asarray(tensors["scales"], np.uint8)
            s2 = 1.0
        else:
            raise ValueError("nvfp4: expected weight_scale + weight_scale_2 (ModelOpt) or scales (MLX)")
        if k % 16 or w.shape != (n, k // 2) or sc.shape != (n, k // 16):
            raise ValueError(f"nvfp4: weight {w.shape}, scales {sc.shape} do not match shape {shape}")
        return DequantSpec("nvfp4", (n, k), {"weight": w, "weight_scale": sc}, {"weight_scale_2": s2})

    def quantize(self, w) -> DequantSpec:
        w = np.asarray(w, dtype=np.float32)
        n, k = w.shape
        if k % 16:
            raise ValueError("nvfp4: K must be a multiple of 16")
        amax = float(np.abs(w).max()) or 1.0
        s2 = np.float32(amax / (E2M1_MAX * E4M3_MAX))
        blocks = w.reshape(n, k // 16, 16)
        bmax = np.abs(blocks).max(axis=-1)
        sc = e4m3_encode(np.where(bmax > 0, bmax / E2M1_MAX / s2, 0.0))
        d = e4m3_decode(sc)[..., None] * s2
        scaled = np.divide(blocks, d, out=np.zeros_like(blocks), where=d > 0)
        codes = e2m1_encode(scaled.reshape(n, k))
        return DequantSpec("nvfp4", (n, k), {"weight": nibbles_to_bytes(codes), "weight_scale": sc},
                           {"weight_scale_2": float(s2)})

    def dequantize(self, spec: DequantSpec) -> np.ndarray:
        n, k = spec.shape
        v = e2m1_decode(bytes_to_nibbles(spec.tensors["weight"])).reshape(n, k // 16, 16)
        s = e4m3_decode(spec.tensors["weight_scale"]).reshape(n, k // 16, 1)
        return ((v * s) * np.float32(spec.params["weight_scale_2"])).reshape(n, k).astype(np.float32)


def _round_away(x):
    x = np.asarray(x, dtype=np.float32)
    t = np.trunc(x)
    return np.where(np.abs(x - t) == np.float32(0.5), t + np.sign(x), np.rint(x)).astype(np.float32)


class INT4Affine:
    name = "int4_affine"
    group = 64
    bytes_per_weight = 0.5 + 4.0 / 64

    def unpack(self, tensors: Mapping[str, Any], *, shape: Tuple[int, int]) -> DequantSpec:
        """MLX ``weight`` U32 ``[N, K/8]`` + ``scales``/``biases`` (BF16 bit patterns or floats)
        (``formats/int4_affine.py:73-83``). The kernels decode BF16 pairs: F16 pairs are refused here."""
        n, k = shape
        w = np.asarray(tensors["weight"])
        if w.dtype != np.uint32 or w.shape != (n, k // 8):
            raise ValueError(f"int4_affine: weight {w.shape} {w.dtype} does not match shape {shape}")

        def f32(a):
            a = np.asarray(a)
            if a.dtype == np.float16:
                raise ValueError("int4_affine: F16 (scale, bias) pairs are not supported by the gfx950 kernels")
            return bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)

        sc, bi = f32(tensors["scales"]), f32(tensors["biases"])
        if sc.shape != (n, k // 64) or bi.shape != sc.shape:
            raise ValueError(f"int4_affine: scales {sc.shape} do not match groups of 64 for shape {shape}")
        if not (np.array_equal(to_bf16_values(sc), sc) and np.array_equal(to_bf16_values(bi), bi)):
            raise ValueError("int4_affine: scales / biases are not BF16-representable")
        return DequantSpec("int4_affine", (n, k), {"weight": np.ascontiguousarray(w.view(np.uint8).reshape(n, k // 2)),
                                                   "scales": sc, "biases": bi}, {"group": 64})

    def quantize(self, w) -> DequantSpec:
        w = np.asarray(w, dtype=np.float32)
        n, k = w.shape
        g = self.group
        if k % g:
            raise ValueError(f"int4_affine: K must be a multiple of {g}")
        b = w.reshape(n, k // g, g)
        w_min = b.min(axis=-1)
        w_max = np.maximum(b.max(axis=-1), np.float32(0))
        s0 = np.maximum((w_max - w_min) / np.float32(15), np.float32(1e-7)).astype(np.float32)
        use_min = np.abs(w_min) > np.abs(w_max)
        s0 = np.where(use_min, s0, -s0).astype(np.float32)
        edge = np.where(use_min, w_min, w_max).astype(np.float32)
        q0 = _round_away(edge / s0)
        z = q0 == 0
        scale = np.where(z, s0, edge / np.where(z, np.float32(1), q0)).astype(np.float32)
        bias = np.where(z, np.float32(0), edge).astype(np.float32)
        codes = np.clip(_round_away((b - bias[..., None]) / scale[..., None]), 0, 15).astype(np.uint8).reshape(n, k)
        return DequantSpec("int4_affine", (n, k), {"weight": nibbles_to_bytes(codes), "scales": to_bf16_values(scale),
                                                   "biases": to_bf16_values(bias)}, {"group": 64})

    def dequantize(self, spec: DequantSpec) -> np.ndarray:
        n, k = spec.shape
        c = bytes_to_nibbles(spec.tensors["weight"]).astype(np.float32).reshape(n, k // 64, 64)
        return (c * spec.tensors["scales"][..., None] + spec.tensors["biases"][..., None]).reshape(n, k).astype(np.float32)


class BF16:
    name = "bf16"
    bytes_per_weight = 2.0

    def unpack(self, tensors: Mapping[str, Any], *, shape: Tuple[int, int]) -> DequantSpec:
        w = np.asarray(tensors["weight"])
        w = w if w.dtype == np.uint16 else f32_to_bf16(w)
        if w.shape != tuple(shape):
            raise ValueError(f"bf16: weight {w.shape} does not match {shape}")
        return DequantSpec("bf16", tuple(shape), {"weight": w})

    def quantize(self, w) -> DequantSpec:
        w = np.asarray(w, np.float32)
        return DequantSpec("bf16", w.shape, {"weight": f32_to_bf16(w)})

    def dequantize(self, spec: DequantSpec) -> np.ndarray:
        return bf16_to_f32(spec.tensors["weight"])


class FP8E4M3:
    """FP8 E4M3 codes with one FP32 tensor scale (ModelOpt ``FP8``: ``weight`` F8_E4M3 ``[N, K]``, ``weight_scale``
    F32 ``[]``; ``input_scale`` ignored) — ``formats/fp8_e4m3.py:1-79``."""
    name = "fp8_e4m3"
    bytes_per_weight = 1.0

    def unpack(self, tensors: Mapping[str, Any], *, shape: Tuple[int, int]) -> DequantSpec:
        n, k = shape
        w = np.asarray(tensors["weight"])
        w = w.view(np.uint8) if w.dtype.itemsize == 1 else w.astype(np.uint8)
        s = float(np.asarray(tensors["weight_scale"], np.float32).reshape(()))
        if w.shape != (n, k):
            raise ValueError(f"fp8_e4m3: weight {w.shape} does not match shape {shape}")
        return DequantSpec("fp8_e4m3", (n, k), {"weight": w}, {"weight_scale": s})

    def quantize(self, w) -> DequantSpec:
        w = np.asarray(w, dtype=np.float32)
        amax = float(np.abs(w).max()) or 1.0
        s = np.float32(amax / E4M3_MAX)
        return DequantSpec("fp8_e4m3", w.shape, {"weight": e4m3_encode(w / s)}, {"weight_scale": float(s)})

    def dequantize(self, spec: DequantSpec) -> np.ndarray:
        return (e4m3_decode(spec.tensors["weight"]) * np.float32(spec.params["weight_scale"])).astype(np.float32)


FORMATS = {"nvfp4": NVFP4(), "int4_affine": INT4Affine(), "bf16": BF16(), "fp8_e4m3": FP8E4M3()}

__all__ = ["DequantSpec", "FORMATS", "NVFP4", "INT4Affine", "BF16", "FP8E4M3", "e4m3_encode", "e4m3_decode", "e2m1_encode",
           "e2m1_decode", "f32_to_bf16", "bf16_to_f32", "to_bf16_values"]
