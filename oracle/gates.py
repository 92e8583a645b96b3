"""The numerics gates of the reference (``monolith/bench.py:57-101``), restated.

* :meth:`OracleCheck.ok` — leaf GEMV ops: max error ≤ 2 BF16 ULP at the output RMS and max relative error < 1e-4.
* :meth:`OracleCheck.ok_rounded` — outputs after rounding chains: every element within 2 ULP of its own magnitude
  (floored at the RMS) and max relative error < 1e-2.
* :func:`within_tolerance` — the build's stated bar for BF16 outputs: ``|y − ref| ≤ 1e-3 +
  1e-2·|ref|`` element-wise.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .fp import f32_to_bf16


def bf16_ulp_of(magnitude: float) -> float:
    """BF16 spacing at ``magnitude`` (8 significand bits)."""
    return float(2.0 ** (np.floor(np.log2(max(magnitude, 1e-30))) - 7))


def bf16_ulp_diff(a, b) -> np.ndarray:
    """|a − b| in BF16 code steps after rounding both to BF16 (sign-magnitude codes mapped to a monotone line)."""
    def key(x):
        u = f32_to_bf16(np.asarray(x, dtype=np.float32)).astype(np.int64)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), u + 0x8000)
    return np.abs(key(a) - key(b))


@dataclass
class OracleCheck:
    max_ulp_at_rms: float
    max_ulp_elementwise: int
    max_rel_err: float
    max_ulp_at_scale: float = 0.0
    tol_violations: int = 0          # elements outside |y − ref| ≤ 1e-3 + 1e-2·|ref|
    n: int = 0

    @property
    def within(self) -> bool:
        """Every element within the stated tolerance (``within_tolerance``)."""
        return self.tol_violations == 0

    def ok(self) -> bool:
        return self.max_ulp_at_rms <= 2.0 and self.max_rel_err < 1e-4

    def ok_rounded(self) -> bool:
        return self.max_ulp_at_scale <= 2.0 and self.max_rel_err < 1e-2


def check_against_oracle(y, y_ref) -> OracleCheck:
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    err = np.abs(y - y_ref)
    rms = float(np.sqrt(np.mean(y_ref ** 2)))
    denom = max(float(np.abs(y_ref).max()), 1e-30)
    mags = np.maximum(np.abs(y_ref), rms)
    ulps = 2.0 ** (np.floor(np.log2(np.maximum(mags, 1e-30))) - 7)
    return OracleCheck(float(err.max() / bf16_ulp_of(rms)), int(bf16_ulp_diff(y, y_ref).max()),
                       float(err.max() / denom), float((err / ulps).max()),
                       int(np.count_nonzero(~(err <= 1e-3 + 1e-2 * np.abs(y_ref)))), int(err.size))


def tolerance_violations(y, y_ref, rtol: float = 1e-2, atol: float = 1e-3) -> int:
    """How many elements miss ``|y − ref| ≤ atol + rtol·|ref|`` (NaN counts as a miss)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return int(np.count_nonzero(~(np.abs(y - y_ref) <= atol + rtol * np.abs(y_ref))))


def within_tolerance(y, y_ref, rtol: float = 1e-2, atol: float = 1e-3) -> bool:
    """The north-star bar for BF16 outputs with FP32 accumulation: every element within 1e-2 relative / 1e-3
    absolute of the oracle."""
    return tolerance_violations(y, y_ref, rtol, atol) == 0
