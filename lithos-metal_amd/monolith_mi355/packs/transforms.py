"""Pack-time row orders and small parameter maps (``packs/transforms.py:16-78`` of the reference): row orders are
index arrays ``perm[new] = old``; the maps turn stored parameters into what the kernels take."""

from __future__ import annotations

import numpy as np

from ..formats.fp import bf16_to_f32, f32_to_bf16


def interleave_chunks(n_a: int, n_b: int, chunk: int) -> np.ndarray:
    """``A`` (rows ``0..n_a``) and ``B`` (the next ``n_b``) in alternating runs of ``chunk`` rows — the gate|up slab
    order that lets one 16-row tile hold 8 gate rows and their 8 up rows."""
    if n_a != n_b or n_a % chunk:
        raise ValueError(f"interleave_chunks: need n_a == n_b, a multiple of chunk ({n_a}, {n_b}, {chunk})")
    runs = np.arange(n_a).reshape(-1, chunk)
    return np.concatenate([runs, runs + n_a], axis=1).reshape(-1)


def rope_head_perm(head_dim: int, rotary_dim: int) -> np.ndarray:
    """One head's dims reordered so the rotary pairs ``(i, i + rotary/2)`` become ``(i, i + head_dim/2)``; the other
    dims fill the remaining places in order."""
    if rotary_dim % 2 or head_dim % 2 or rotary_dim > head_dim:
        raise ValueError("rope_head_perm: rotary_dim and head_dim even, rotary_dim <= head_dim")
    half, mid = rotary_dim // 2, head_dim // 2
    rest = np.arange(rotary_dim, head_dim)
    perm = np.concatenate([np.arange(half), rest[: mid - half], np.arange(half, rotary_dim), rest[mid - half:]])
    return perm.astype(np.int64)


def bf16_round_f32(w: np.ndarray, *, dtype_in: str = "BF16") -> np.ndarray:
    """The BF16 value a BF16 reference model holds, as float32 (F32 inputs rounded to BF16 first)."""
    if dtype_in == "BF16":
        return bf16_to_f32(np.asarray(w, np.uint16))
    return bf16_to_f32(f32_to_bf16(np.asarray(w, np.float32)))


def one_plus(w: np.ndarray, *, dtype_in: str = "BF16") -> np.ndarray:
    """``(1 + w)`` in float32: the RMSNorm weight the GEMV's fused norm takes."""
    return (np.float32(1.0) + bf16_round_f32(w, dtype_in=dtype_in)).astype(np.float32)


def neg_exp(w: np.ndarray, *, dtype_in: str = "BF16") -> np.ndarray:
    """``−exp(A_log)`` in float32: the Gated DeltaNet decay coefficient."""
    return (-np.exp(bf16_round_f32(w, dtype_in=dtype_in))).astype(np.float32)
