"""The tolerance contract for every parity check (mdlc/testing/tolerances.py:46-54).

Tiers are keyed by what makes two correct computations differ:

  BITWISE           data movement, integer and quantized codes: any
                    difference is a bug.
  FP32_SAME_ORDER   the same fp32 math in the same order (elementwise chains,
                    folded Conv+BN); also the per-tensor bar the MI355X
                    backend is held to for every tensor (rtol 1e-4, atol 1e-5).
  FP32_REDUCTION    one reduction (GEMM, conv, pooling, mean) accumulated in a
                    different order than NumPy.
  FP32_NETWORK      a whole network against another backend.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Tol:
    rtol: float
    atol: float


BITWISE = Tol(rtol=0.0, atol=0.0)
FP32_SAME_ORDER = Tol(rtol=1e-4, atol=1e-5)
FP32_REDUCTION = Tol(rtol=1e-4, atol=1e-4)
FP32_NETWORK = Tol(rtol=1e-3, atol=1e-4)

# The bar for every device tensor in this backend (fp32): rtol 1e-4 / atol 1e-5.
DEVICE_TENSOR = FP32_SAME_ORDER
