"""Code generation: MFMA schedules and the gfx950 HIP backend."""

from mdlc_amd.codegen.schedule import DEFAULT_GEMM, MfmaSchedule, gemm_search_space

__all__ = ["DEFAULT_GEMM", "MfmaSchedule", "gemm_search_space"]
