"""Conversions between the oracle's quantized-matrix dicts and the product's DequantSpec, and BF16 tensors."""

from __future__ import annotations

import numpy as np

from monolith_mi355.formats import DequantSpec
from oracle.fp import bf16_to_f32, f32_to_bf16


def spec_of(m: dict) -> DequantSpec:
    """The product's DequantSpec for an oracle quantized-matrix dict."""
    n = m["weight"].shape[0]
    if m["format"] == "nvfp4":
        k = m["weight"].shape[1] * 2
        return DequantSpec("nvfp4", (n, k), {"weight": m["weight"], "weight_scale": m["weight_scale"]},
                           {"weight_scale_2": m["weight_scale_2"]})
    if m["format"] == "int4_affine":
        k = m["weight"].shape[1] * 2
        return DequantSpec("int4_affine", (n, k), {"weight": m["weight"], "scales": m["scales"], "biases": m["biases"]},
                           {"group": 64})
    if m["format"] == "fp8_e4m3":
        return DequantSpec("fp8_e4m3", m["weight"].shape, {"weight": m["weight"]}, {"weight_scale": m["weight_scale"]})
    return DequantSpec("bf16", m["weight"].shape, {"weight": m["weight"]})


def to_dev_bf16(torch, a, device="cuda"):
    """float32 numpy (BF16-valued or not) → device bfloat16 tensor (RNE)."""
    u = f32_to_bf16(np.asarray(a, np.float32)).astype(np.int16)
    return torch.from_numpy(u).view(torch.bfloat16).to(device)


def from_dev_bf16(t) -> np.ndarray:
    return bf16_to_f32(t.detach().cpu().view(__import__("torch").int16).numpy().astype(np.uint16))
