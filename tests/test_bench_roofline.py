"""bench.py's roofline record on the CPU (no device): which kernel it names,
the per-launch work it divides, and where a launch's duration comes from —
the dispatch events of a multi-launch plan, the timed region of a plan whose
step is one launch."""

from __future__ import annotations

import importlib.util
import os

import pytest

from mdlc_amd.codegen.hip.plan import Launch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _launch(name, kind="conv", **meta):
    return Launch(kind, name, [], [], (1, 1, 1), (256, 1, 1), meta)


def test_one_launch_step_takes_the_timed_region(bench):
    ops = 2 * 4096 ** 3
    prof = [(_launch("qgemm_x", kind="qgemm", ops=ops, bytes=3 * 4096 ** 2), 0.0813)]
    roof, _ = bench.roofline(prof, verbose=False, step_ms=0.0726)
    assert roof["kernel"] == "qgemm_x" and roof["unit"] == "TOP/s"
    assert roof["avg_launch_ms"] == 0.0726 and roof["dispatch_event_ms"] == 0.0813
    assert roof["achieved"] == pytest.approx(ops / 0.0726e-3 / 1e12)
    assert roof["frac"] == pytest.approx(roof["achieved"] / 5000.0)
    roof, _ = bench.roofline(prof, verbose=False)                 # no timed region given
    assert roof["avg_launch_ms"] == 0.0813 and "dispatch_event_ms" not in roof


def test_multi_launch_plans_keep_their_dispatch_events(bench):
    f = 4.0e9
    prof = [(_launch("conv_a", flops=f, bytes=1e7), 0.050), (_launch("conv_b", flops=f / 4, bytes=1e7), 0.010),
            (_launch("conv_a", flops=f, bytes=1e7), 0.046)]
    roof, per = bench.roofline(prof, verbose=False, step_ms=0.2)
    assert roof["kernel"] == "conv_a" and roof["launches_per_step"] == 2
    assert roof["avg_launch_ms"] == pytest.approx(0.048) and "dispatch_event_ms" not in roof
    assert roof["achieved"] == pytest.approx(f / 0.048e-3 / 1e12)
    assert roof["share_of_step"] == pytest.approx(0.096 / 0.106)
