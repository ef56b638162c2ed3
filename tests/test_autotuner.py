"""Autotuner: schedule-space validity, cost-model ranking, cache round trip
(reference tests/test_autotuner.py:9-42, re-parameterised for MFMA)."""

from __future__ import annotations

import os

import pytest

from mdlc_amd.autotuner import AutotuneCache, Tuner, analytical_cost, tune_gemm
from mdlc_amd.autotuner.tuner import TUNED_PATH, candidates, conv_schedule_ok, problem_key
from mdlc_amd.codegen.schedule import (
    DEFAULT_GEMM, MfmaSchedule, default_schedule, gemm_search_space, split_slices,
)


def test_schedule_validity_and_pruning():
    space = list(gemm_search_space((1, 2, 4)))
    assert space
    for s in space:
        assert s.is_valid()
        assert s.lds_bytes() <= 160 * 1024
        assert 64 <= s.threads_per_block() <= 1024
        wm, wn = s.wave_tile()
        assert wm % s.MS == 0 and wn % s.MS == 0
    assert not MfmaSchedule(32, 32, 8, 1, 1, 16).is_valid()       # BK too shallow for 16x16x4
    assert not MfmaSchedule(64, 48, 16, 2, 2, 32).is_valid()      # wave tile not MFMA multiple


def test_split_slices_cover_k_without_empty_slices():
    for K in (33, 147, 576, 4608):
        for sk in (1, 2, 3, 4, 8):
            s = MfmaSchedule(64, 64, 16, 2, 2, 32, True, sk)
            n, chunk = split_slices(K, s)
            assert chunk % s.BK == 0 or n == 1
            assert (n - 1) * chunk < K <= n * chunk


def test_cost_model_prefers_no_quant_waste_on_small_gemm():
    perfect = MfmaSchedule(64, 64, 16, 2, 2, 32)
    oversized = MfmaSchedule(256, 256, 16, 2, 4, 32)
    assert analytical_cost(perfect, 64, 64, 64) < analytical_cost(oversized, 64, 64, 64)


def test_cost_model_prefers_split_k_for_deep_small_grids():
    base = MfmaSchedule(64, 64, 16, 2, 2, 32)
    assert analytical_cost(base.with_split(8), 512, 49, 4608) < analytical_cost(base, 512, 49, 4608)


def test_default_schedule_fills_the_chip():
    for M, N, K in [(64, 100352, 576), (512, 1568, 4608), (256, 6272, 2304)]:
        s = default_schedule(M, N, K)
        n, _ = split_slices(K, s)
        assert s.is_valid()
        assert -(-M // s.BM) * -(-N // s.BN) * n >= 256


def test_tune_gemm_returns_valid_best():
    res = tune_gemm(512, 512, 512, budget=16)
    assert res.best.is_valid() and res.n_evaluated >= 16
    metrics = [m for _, m in res.ranking]
    assert metrics == sorted(metrics)
    assert not res.measured


def test_candidates_include_default_and_are_valid():
    c = candidates(256, 6272, 2304, budget=8)
    assert default_schedule(256, 6272, 2304) in c
    assert all(s.is_valid() for s in c)


def test_cache_roundtrip(tmp_path):
    path = os.path.join(tmp_path, "cache.json")
    c = AutotuneCache(path)
    s = MfmaSchedule(64, 64, 16, 2, 2, 32, False, 2)
    c.put(128, 256, 64, s, 1.23, measured=False)
    c.save()
    assert AutotuneCache(path).get(128, 256, 64) == s


def test_tuner_caches_per_shape(tmp_path):
    cache = AutotuneCache(os.path.join(tmp_path, "c.json"))
    tuner = Tuner(cache=cache, budget=8)
    s1 = tuner.schedule_for(None, (256, 256, 256))
    s2 = tuner.schedule_for(None, (256, 256, 256))
    assert s1 == s2 and cache.get(256, 256, 256) is not None


def test_shipped_tuned_schedules_are_valid():
    """The measured gfx950 schedules shipped with the backend parse and are
    valid for their kernel (fp32 GEMM, implicit-GEMM conv gather, or int8),
    and cover every conv/GEMM problem of the benchmarked models."""
    from mdlc_amd.codegen.schedule import qsched_valid
    from mdlc_amd.tools.tune import model_problems

    cache = AutotuneCache(TUNED_PATH)
    assert cache.entries
    for key, e in cache.entries.items():
        s = MfmaSchedule(**e["sched"])
        if key.startswith("i8:"):
            assert qsched_valid(s), key
        elif key.startswith("conv:") and key.endswith(":implicit"):
            # the tiled gather kernels, or the wave-split kernel on whole taps
            cin = int(key.split(":")[3].split("x")[0])
            assert conv_schedule_ok(s, {"C": cin}), key
        else:
            assert s.is_valid(), key
        assert e["measured"]
    for model, batch in (("resnet18", 32), ("resnet18", 1), ("mobilenetv2", 32),
                         ("mobilenetv2", 1), ("repvit_int8", 32)):
        for p in model_problems(model, batch, "implicit"):
            assert problem_key(p) in cache.entries, (model, batch, problem_key(p))
    assert DEFAULT_GEMM.is_valid() and DEFAULT_GEMM.conv_valid()


@pytest.mark.gpu
def test_measured_tuning_picks_a_correct_schedule(hip_ctx):
    """The measured tuner on one small convolution: every candidate is timed
    on the device and checked against the default schedule's output, and
    the chosen schedule's module matches the oracle."""
    from gpu_util import assert_close, device_run
    from mdlc_amd.autotuner.tuner import _problem_graph, tune_problem

    problem = {"kind": "conv", "mode": "implicit", "M": 32, "N": 2 * 14 * 14, "K": 16 * 9,
               "batch": 2, "bias": False, "act": None, "C": 16, "H": 14, "W": 14, "KH": 3, "KW": 3,
               "SH": 1, "SW": 1, "DH": 1, "DW": 1, "PT": 1, "PB": 1, "PL": 1, "PR": 1, "OH": 14, "OW": 14}
    res = tune_problem(problem, budget=4, ctx=hip_ctx)
    assert res.measured and res.n_evaluated >= 4 and res.rejected == []
    assert all(ms > 0 for _, ms in res.ranking)
    assert conv_schedule_ok(res.best, problem)
    g, feeds = _problem_graph(problem)
    _, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=lambda n, mnk: res.best,
                              small_conv=False)
    assert_close("y", got["y"], want["y"])
