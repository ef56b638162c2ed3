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


@dataclass
class Float64Check:
    """A float32 result and the float32 reference, each measured against the
    float64 evaluation of the same inputs (``tolerance_ratio`` at one tier)."""
    name: str
    device: float          # ratio of the device's result to the float64 values
    reference: float       # ratio of the float32 reference's result to them
    bound: float           # the largest device ratio that passes
    ok: bool

    def __str__(self) -> str:
        flag = "OK  " if self.ok else "FAIL"
        return (f"[{flag}] {self.name:24s} device/f64={self.device:.3f} "
                f"f32-reference/f64={self.reference:.3f} bound={self.bound:.3f}")


def check_against_float64(name: str, got, want32, want64, *, rtol: float, atol: float,
                          factor: float = 2.0) -> Float64Check:
    """Hold ``got`` to the tier (ratio <= 1 against the float64 values)
    wherever the float32 reference meets it there; where the float32
    reference itself misses the tier (large magnitudes that cancel, as in a
    network whose activations reach the hundreds), hold the device to within
    ``factor`` of the reference's own error instead. A float32 kernel that
    is as accurate as the float32 reference passes either way; one with a
    dropped term or a wrong operand misses by orders of magnitude."""
    r_dev = tolerance_ratio(got, want64, rtol=rtol, atol=atol)
    r_ref = tolerance_ratio(want32, want64, rtol=rtol, atol=atol)
    bound = 1.0 if r_ref <= 1.0 else factor * r_ref
    return Float64Check(name, r_dev, r_ref, bound, bool(r_dev <= bound))


def graph_checks(evaluate, graph, feeds: dict, golden: dict, *, rtol: float = FP32_NETWORK.rtol,
                 atol: float = FP32_NETWORK.atol) -> list:
    """``evaluate(graph, feeds)`` (a host executor of IR graphs) compared
    with ``golden`` on every graph output: one ``CheckResult`` each (the
    role of mdlc/testing/harness.py:102-125)."""
    got = evaluate(graph, feeds)
    out = []
    for name in graph.outputs:
        if name not in golden:
            out.append(CheckResult(name, False, float("inf"), float("inf"), "no golden value"))
        else:
            out.append(compare_arrays(name, got[name], golden[name], rtol=rtol, atol=atol))
    return out


def pass_checker(evaluate, feeds: dict, golden: dict, *, rtol: float = FP32_NETWORK.rtol,
                 atol: float = FP32_NETWORK.atol):
    """A ``verify(graph, pass_name)`` hook for the pass manager: after every
    pass that changed the graph, evaluate it on ``feeds`` and raise
    ``AssertionError`` naming the pass if an output left the tolerance of
    ``golden`` (the role of mdlc/testing/harness.py:128-149)."""
    def verify(graph, pass_name: str) -> None:
        bad = [r for r in graph_checks(evaluate, graph, feeds, golden, rtol=rtol, atol=atol)
               if not r.ok]
        if bad:
            raise AssertionError(f"pass {pass_name!r} changed the outputs:\n"
                                 + "\n".join(str(r) for r in bad))
    return verify

