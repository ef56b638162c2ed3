"""Schedule autotuning for the gfx950 MFMA kernels."""

from mdlc_amd.autotuner.tuner import (
    AutotuneCache, Tuner, analytical_cost, tune_gemm, tune_problem, tuned_schedules,
)

__all__ = ["AutotuneCache", "Tuner", "analytical_cost", "tune_gemm", "tune_problem",
           "tuned_schedules"]
