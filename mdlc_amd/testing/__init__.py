"""Parity tooling: tolerance tiers and array comparison."""

from mdlc_amd.testing.harness import (CheckResult, Float64Check, check_against_float64,
                                      compare_arrays, graph_checks, pass_checker, tolerance_ratio)
from mdlc_amd.testing.tolerances import BITWISE, DEVICE_TENSOR, FP32_NETWORK, FP32_REDUCTION, FP32_SAME_ORDER

__all__ = ["CheckResult", "Float64Check", "check_against_float64", "compare_arrays", "graph_checks",
           "pass_checker", "tolerance_ratio", "BITWISE", "DEVICE_TENSOR", "FP32_NETWORK",
           "FP32_REDUCTION", "FP32_SAME_ORDER"]
