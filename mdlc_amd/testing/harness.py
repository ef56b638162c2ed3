"""Array comparison with diagnostics and the vacuous-pass guard
(mdlc/testing/harness.py:50-81).

A comparison whose golden values sit at the scale of ``atol`` passes no
matter what was computed, so it is reported as a failure (VACUOUS) instead.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from mdlc_amd.testing.tolerances import FP32_NETWORK


@dataclass
class CheckResult:
    name: str
    ok: bool
    max_abs: float
    max_rel: float
    detail: str = ""

    def __str__(self) -> str:
        flag = "OK  " if self.ok else "FAIL"
        return (f"[{flag}] {self.name:24s} max_abs={self.max_abs:.3e} "
                f"max_rel={self.max_rel:.3e} {self.detail}")


def compare_arrays(name: str, got, want, *, rtol: float = FP32_NETWORK.rtol,
                   atol: float = FP32_NETWORK.atol) -> CheckResult:
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    if g.shape != w.shape:
        return CheckResult(name, False, float("inf"), float("inf"),
                           f"shape mismatch got{g.shape} want{w.shape}")
    if g.size == 0:
        return CheckResult(name, True, 0.0, 0.0)
    diff = np.abs(g - w)
    max_abs = float(diff.max())
    max_rel = float((diff / (np.abs(w) + atol)).max())
    ok = bool(np.allclose(g, w, rtol=rtol, atol=atol))
    detail = ""
    if not ok:
        # the worst element relative to its own tolerance
        worst = np.unravel_index(int((diff - rtol * np.abs(w)).argmax()), diff.shape)
        detail = f"worst@{worst}: got={g[worst]:.6g} want={w[worst]:.6g}"
    mag = float(np.abs(w).max())
    if ok and atol > 0 and mag < 100 * atol:
        return CheckResult(name, False, max_abs, max_rel,
                           f"VACUOUS: golden magnitude {mag:.3e} < 100*atol={100 * atol:.0e}; "
                           "comparison has no power")
    return CheckResult(name, ok, max_abs, max_rel, detail)


def tolerance_ratio(got, want, *, rtol: float, atol: float) -> float:
    """max |got-want| / (atol + rtol*|want|): <= 1 means within tolerance."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    if g.size == 0:
        return 0.0
    return float((np.abs(g - w) / (atol + rtol * np.abs(w))).max())
