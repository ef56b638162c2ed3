"""Parity tooling: tolerance tiers and array comparison."""

from mdlc_amd.testing.harness import CheckResult, compare_arrays, tolerance_ratio
from mdlc_amd.testing.tolerances import BITWISE, DEVICE_TENSOR, FP32_NETWORK, FP32_REDUCTION, FP32_SAME_ORDER

__all__ = ["CheckResult", "compare_arrays", "tolerance_ratio", "BITWISE", "DEVICE_TENSOR",
           "FP32_NETWORK", "FP32_REDUCTION", "FP32_SAME_ORDER"]
