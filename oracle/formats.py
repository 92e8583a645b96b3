"""NVFP4 and affine-INT4 weight formats: exact dequantization (the numerics reference) and the quantizers.

A quantized matrix is a plain dict of checkpoint-shaped arrays, in the reference's ``DequantSpec.tensors`` roles:

* ``nvfp4``: ``weight`` U8 ``[N, K/2]`` (E2M1 codes, low nibble first), ``weight_scale`` U8 ``[N, K/16]`` (E4M3),
  ``weight_scale_2`` float (the FP32 tensor scale) — ``formats/nvfp4.py:122-161``;
* ``int4_affine``: ``weight`` U8 ``[N, K/2]`` (unsigned codes, low nibble first), ``scales`` / ``biases`` F32
  ``[N, K/64]`` holding BF16-valued numbers — ``formats/int4_affine.py:73-119``;
* ``fp8_e4m3``: ``weight`` U8 ``[N, K]`` (E4M3 codes), ``weight_scale`` float (the FP32 tensor scale) —
  ``formats/fp8_e4m3.py:62-79``.
"""

from __future__ import annotations

import numpy as np

from .fp import (E2M1_MAX, E4M3_MAX, bf16_to_f32, e2m1_to_f32, e4m3_to_f32, f32_to_bf16, f32_to_e2m1, f32_to_e4m3,
                 pack_nibbles, unpack_nibbles)

NVFP4_BLOCK = 16
INT4_GROUP = 64


# ---- NVFP4 ---------------------------------------------------------------------------------------------------------
def nvfp4_dequantize(m: dict) -> np.ndarray:
    """``w = e2m1(code) · e4m3(block scale) · weight_scale_2`` in float32, evaluated as numpy does in
    ``formats/nvfp4.py:139-144``: ``(value · scale)`` (exact) then ``· s2`` (one rounding)."""
    codes = unpack_nibbles(m["weight"])
    n, k = codes.shape
    vals = e2m1_to_f32(codes).reshape(n, k // NVFP4_BLOCK, NVFP4_BLOCK)
    sc = e4m3_to_f32(m["weight_scale"]).reshape(n, k // NVFP4_BLOCK, 1)
    return ((vals * sc) * np.float32(m["weight_scale_2"])).reshape(n, k).astype(np.float32)


def nvfp4_quantize(w: np.ndarray) -> dict:
    """The reference quantizer (``formats/nvfp4.py:146-161``): ``s2 = amax / (6·448)``; per block of 16 the E4M3
    scale of ``bmax / 6 / s2``; codes = E2M1 of ``w / (scale · s2)`` (zero where the block scale is zero)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % NVFP4_BLOCK:
        raise ValueError("nvfp4: K must be a multiple of 16")
    amax = float(np.abs(w).max()) or 1.0
    s2 = np.float32(amax / (E2M1_MAX * E4M3_MAX))
    blocks = w.reshape(n, k // NVFP4_BLOCK, NVFP4_BLOCK)
    bmax = np.abs(blocks).max(axis=-1)
    sc = f32_to_e4m3(np.where(bmax > 0, bmax / E2M1_MAX / s2, 0.0))
    denom = e4m3_to_f32(sc)[..., None] * s2
    scaled = np.divide(blocks, denom, out=np.zeros_like(blocks), where=denom > 0)
    codes = f32_to_e2m1(scaled.reshape(n, k))
    return {"format": "nvfp4", "weight": pack_nibbles(codes), "weight_scale": sc, "weight_scale_2": float(s2)}


def nvfp4_random(n: int, k: int, rng: np.random.Generator, s2: float = 0.02 / (E2M1_MAX * E4M3_MAX) * 64) -> dict:
    """Random codes drawn directly in the format (``monolith/bench.py:17-23``): any nibble, E4M3 block scales in
    ``[2^-3, 2^2)``."""
    return {"format": "nvfp4", "weight": rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8),
            "weight_scale": rng.integers(0x20, 0x48, size=(n, k // NVFP4_BLOCK), dtype=np.uint8),
            "weight_scale_2": float(np.float32(s2))}


# ---- affine INT4 ---------------------------------------------------------------------------------------------------
def int4_dequantize(m: dict) -> np.ndarray:
    """``w = code · scale + bias`` per group in float32, two numpy roundings (``formats/int4_affine.py:85-91``);
    the product is exact (BF16 scale × 4-bit code), so this equals one fused rounding."""
    codes = unpack_nibbles(m["weight"]).astype(np.float32)
    n, k = codes.shape
    g = k // m["scales"].shape[1]
    sc = np.asarray(m["scales"], np.float32).reshape(n, k // g, 1)
    bi = np.asarray(m["biases"], np.float32).reshape(n, k // g, 1)
    return (codes.reshape(n, k // g, g) * sc + bi).reshape(n, k).astype(np.float32)


def round_half_away(x: np.ndarray) -> np.ndarray:
    """Round to nearest, halves away from zero (Metal's / MLX's ``round``; ``formats/int4_affine.py:189-194``)."""
    x = np.asarray(x, dtype=np.float32)
    t = np.trunc(x)
    frac_half = np.abs(x - t) == np.float32(0.5)
    return np.where(frac_half, t + np.sign(x), np.rint(x)).astype(np.float32)


def int4_quantize(w: np.ndarray, group: int = INT4_GROUP) -> dict:
    """MLX's affine rule in float32 (``formats/int4_affine.py:93-119``): per group the edge of larger magnitude lands
    on an integer code; ``scale = edge / q0`` (``scale0`` and a zero bias when ``q0 == 0``), ``bias = edge``;
    codes ``= clip(round_away((w - bias) / scale), 0, 15)``; scale and bias rounded to BF16."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group:
        raise ValueError(f"int4_affine: K must be a multiple of the group ({group})")
    blocks = w.reshape(n, k // group, group)
    lo = blocks.min(axis=-1)
    hi = np.maximum(blocks.max(axis=-1), np.float32(0))
    scale0 = np.maximum((hi - lo) / np.float32(15), np.float32(1e-7)).astype(np.float32)
    neg_edge = np.abs(lo) > np.abs(hi)
    scale0 = np.where(neg_edge, scale0, -scale0).astype(np.float32)
    edge = np.where(neg_edge, lo, hi).astype(np.float32)
    q0 = round_half_away(edge / scale0)
    zero = q0 == 0
    scale = np.where(zero, scale0, edge / np.where(zero, np.float32(1), q0)).astype(np.float32)
    bias = np.where(zero, np.float32(0), edge).astype(np.float32)
    codes = np.clip(round_half_away((blocks - bias[..., None]) / scale[..., None]), 0, 15).astype(np.uint8)
    return {"format": "int4_affine", "weight": pack_nibbles(codes.reshape(n, k)),
            "scales": bf16_to_f32(f32_to_bf16(scale)), "biases": bf16_to_f32(f32_to_bf16(bias))}


def int4_random(n: int, k: int, rng: np.random.Generator) -> dict:
    """Random codes and BF16 pairs drawn directly (``monolith/bench.py:34-38``)."""
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = (rng.uniform(0.5, 2.0, size=(n, k // INT4_GROUP)) * 0.02 / 7.5).astype(np.float32)
    biases = (-7.5 * scales * rng.uniform(0.8, 1.2, size=scales.shape)).astype(np.float32)
    return {"format": "int4_affine", "weight": codes, "scales": bf16_to_f32(f32_to_bf16(scales)),
            "biases": bf16_to_f32(f32_to_bf16(biases))}


# ---- FP8 E4M3 with a tensor scale ----------------------------------------------------------------------------------
def fp8_dequantize(m: dict) -> np.ndarray:
    """``w = e4m3(code) · weight_scale`` in float32, one rounding (``formats/fp8_e4m3.py:69-70``)."""
    return (e4m3_to_f32(m["weight"]) * np.float32(m["weight_scale"])).astype(np.float32)


def fp8_quantize(w: np.ndarray) -> dict:
    """The reference quantizer (``formats/fp8_e4m3.py:72-76``): ``s = amax / 448``, codes = E4M3 of ``w / s``."""
    w = np.asarray(w, dtype=np.float32)
    amax = float(np.abs(w).max()) or 1.0
    s = np.float32(amax / E4M3_MAX)
    return {"format": "fp8_e4m3", "weight": f32_to_e4m3(w / s), "weight_scale": float(s)}


def fp8_random(n: int, k: int, rng: np.random.Generator, s: float = 0.02 / E4M3_MAX * 8) -> dict:
    """Random finite codes (every code but the NaNs 0x7F / 0xFF) and a tensor scale."""
    codes = rng.integers(0, 254, size=(n, k), dtype=np.uint8)
    codes = np.where(codes >= 0x7F, codes + 1, codes).astype(np.uint8)          # skip 0x7F; 0xFF is never drawn
    return {"format": "fp8_e4m3", "weight": codes, "weight_scale": float(np.float32(s))}


def dequantize(m: dict) -> np.ndarray:
    return {"nvfp4": nvfp4_dequantize, "fp8_e4m3": fp8_dequantize}.get(m["format"], int4_dequantize)(m)


def quantize(fmt: str, w: np.ndarray) -> dict:
    return {"nvfp4": nvfp4_quantize, "fp8_e4m3": fp8_quantize}.get(fmt, int4_quantize)(w)


def stack_rows(mats) -> dict:
    """Row-stack matrices of one format (a ``q|k|v`` or ``gate|up`` slab). NVFP4 parts may carry different tensor
    scales: the stacked dict gets a per-row ``row_scale`` (the reference's row-scale table, ``monolith/bench.py:46-54``)
    and ``weight_scale_2 = 1``."""
    fmt = mats[0]["format"]
    out = {"format": fmt, "weight": np.concatenate([m["weight"] for m in mats], axis=0)}
    if fmt == "nvfp4":
        out["weight_scale"] = np.concatenate([m["weight_scale"] for m in mats], axis=0)
        out["row_scale"] = np.concatenate([np.full(m["weight"].shape[0], m["weight_scale_2"], np.float32) for m in mats])
        out["weight_scale_2"] = 1.0
    elif fmt == "fp8_e4m3":
        out["row_scale"] = np.concatenate([np.full(m["weight"].shape[0], m["weight_scale"], np.float32) for m in mats])
        out["weight_scale"] = 1.0
    else:
        out["scales"] = np.concatenate([m["scales"] for m in mats], axis=0)
        out["biases"] = np.concatenate([m["biases"] for m in mats], axis=0)
    return out


def dequantize_rows(m: dict) -> np.ndarray:
    """Dequantize, applying a per-row tensor-scale table when present (exactly ``w · s2`` per row)."""
    if m["format"] == "nvfp4" and "row_scale" in m:
        base = dict(m, weight_scale_2=1.0)
        return (nvfp4_dequantize(base) * m["row_scale"][:, None].astype(np.float32)).astype(np.float32)
    if m["format"] == "fp8_e4m3" and "row_scale" in m:
        return (e4m3_to_f32(m["weight"]) * m["row_scale"][:, None].astype(np.float32)).astype(np.float32)
    return dequantize(m)


def permute_rows(m: dict, perm: np.ndarray) -> dict:
    out = dict(m)
    for key in ("weight", "weight_scale", "scales", "biases", "row_scale"):
        if key in m and np.ndim(m[key]) > 0:                  # per-row arrays; a tensor scale stays as it is
            out[key] = np.ascontiguousarray(np.asarray(m[key])[perm])
    return out
