"""Autotuner over MFMA schedules (macro tile, wave grid, MFMA shape, LDS
double buffering, split-K).

Same roles as the reference tuner (mdlc/autotuner/tuner.py:31-174): an
analytical cost model ranks candidates without a device; on a device each
candidate is compiled and timed with HIP events; the best schedule per
problem is kept in a JSON cache (same entry format: ``{"sched": {...},
"metric": ..., "measured": ...}``). Two differences:

* Candidates are chosen model-first: the whole valid space is ranked by the
  cost model and the best ``budget`` are measured, plus a seeded random few
  and the default, instead of a blind random sample.
* Convolutions are tuned as the implicit-GEMM kernel they lower to, keyed by
  their full problem (window, batch, channels), not only by (M, N, K).
"""

from __future__ import annotations

import json
import os
import random
from dataclasses import dataclass, field
from typing import Optional

from mdlc_amd.codegen.schedule import (
    CUS, DEFAULT_GEMM, MfmaSchedule, default_qdw_schedule, default_qschedule, default_schedule,
    gemm_search_space, qdw_search_space, qdw_valid, qgemm_search_space, qsched_valid, split_slices,
    unsplit_if_one_slice, wsplit_conv_search_space,
    wsplit_search_space,
)

LDS_PER_CU = 160 * 1024
MFMA_FLOPS_PER_CU_CLK = 256          # fp32 MFMA, dense
CLOCK_GHZ = 2.4
HBM_GBS = 8000.0
LAUNCH_US = 2.0
L2_CU_GBS = 150.0                    # one CU's L2 -> L1 read rate (64 B/clk)
LDS_B_PER_CLK = 64.0                 # LDS bytes per clock a CU sustains (128-bit accesses)
SPLITS = (1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32)


def analytical_cost(sched: MfmaSchedule, M: int, N: int, K: int) -> float:
    """Estimated microseconds (lower is better) for one GEMM with this schedule.

    * Occupancy: workgroups resident per CU, limited by LDS, by 8 waves per
      SIMD, and by the accumulator registers; the grid runs in rounds of
      (CUs x resident) workgroups — tile quantization shows up as a partial
      last round.
    * Compute per round: the tile's MFMA flops at the per-CU rate, derated
      when fewer than 2 waves per SIMD are resident (no one to hide latency).
    * LDS: the tile writes plus every wave's fragment reads per K step, at
      the rate a CU sustains; partly overlapped with the MFMAs.
    * Memory: A re-read once per column tile and B once per row tile, at
      HBM bandwidth, overlapped with compute.
    * Split-K adds the workspace round trip and a second launch.
    * The wave-split kernel (``WK`` > 1) is one launch whose tiles each
      stream (BM + BN) x K operands through one CU: costed by that per-CU
      traffic at the L2-to-CU rate, against its MFMA time.
    """
    if sched.WK > 1:
        tiles = -(-M // sched.BM) * -(-N // sched.BN)
        per_cu = -(-tiles // CUS)
        load = per_cu * (sched.BM + sched.BN) * K * 4.0 / (L2_CU_GBS * 1e3)
        mfma = per_cu * 2.0 * sched.BM * sched.BN * K / (MFMA_FLOPS_PER_CU_CLK * CLOCK_GHZ * 1e3) / 0.5
        return max(load, mfma) + LAUNCH_US
    slices, chunk = split_slices(K, sched)
    tiles = -(-M // sched.BM) * -(-N // sched.BN)
    wgs = tiles * slices
    waves = sched.WGM * sched.WGN
    by_lds = max(1, LDS_PER_CU // sched.lds_bytes())
    vgprs = 64 + sched.acc_regs() + 32
    by_regs = max(1, (512 // vgprs) * 4 // waves)
    resident = max(1, min(by_lds, by_regs, 32 // waves))
    rounds = -(-wgs // (CUS * resident))
    per_cu = min(resident, -(-wgs // CUS))
    waves_per_simd = per_cu * waves / 4.0
    eff = min(1.0, 0.35 + 0.3 * waves_per_simd)
    kp = -(-chunk // sched.BK) * sched.BK
    wg_flops = 2.0 * sched.BM * sched.BN * kp
    round_us = wg_flops * per_cu / (MFMA_FLOPS_PER_CU_CLK * CLOCK_GHZ * 1e3) / eff
    compute = rounds * round_us
    # LDS: each K step writes the A and B tiles once and every wave reads
    # its WM rows of A and WN columns of B; at the ~64 B/clk a CU sustains
    # for 128-bit reads this rivals the MFMA time for small wave tiles
    wm, wn = sched.wave_tile()
    lds_step = 4.0 * sched.BK * ((sched.BM + sched.BN) + waves * (wm + wn))
    lds = rounds * per_cu * lds_step * (kp // sched.BK) / (LDS_B_PER_CLK * CLOCK_GHZ * 1e3)
    traffic = 4.0 * (-(-N // sched.BN) * M * K + -(-M // sched.BM) * K * N)
    memory = traffic / (HBM_GBS * 1e3)
    t = max(compute, lds, memory) + 0.3 * min(compute, lds) + LAUNCH_US
    if slices > 1:
        t += 4.0 * (slices + 1) * M * N / (HBM_GBS * 1e3) + LAUNCH_US
    return t


INT8_OPS_PER_CU_CLK = 8192          # v_mfma_i32_32x32x32_i8, dense


def analytical_qcost(sched: MfmaSchedule, M: int, N: int, K: int) -> float:
    """Estimated microseconds for one int8 GEMM: the fp32 model's occupancy
    and tile-quantization terms at the int8 MFMA rate, with K padded to BK
    and one byte per operand element."""
    tiles = -(-M // sched.BM) * -(-N // sched.BN)
    waves = sched.WGM * sched.WGN
    by_lds = max(1, LDS_PER_CU // (2 * (sched.BM + sched.BN) * (sched.BK + 16)))
    vgprs = 64 + sched.acc_regs() + 32
    by_regs = max(1, (512 // vgprs) * 4 // waves)
    resident = max(1, min(by_lds, by_regs, 32 // waves))
    rounds = -(-tiles // (CUS * resident))
    per_cu = min(resident, -(-tiles // CUS))
    eff = min(1.0, 0.35 + 0.3 * per_cu * waves / 4.0)
    kp = -(-K // sched.BK) * sched.BK
    round_us = 2.0 * sched.BM * sched.BN * kp * per_cu / (INT8_OPS_PER_CU_CLK * CLOCK_GHZ * 1e3) / eff
    traffic = -(-N // sched.BN) * M * K + -(-M // sched.BM) * K * N + M * N
    return max(rounds * round_us, traffic / (HBM_GBS * 1e3)) + LAUNCH_US


def is_int8(problem: dict) -> bool:
    return problem.get("kind") in ("qconv", "qgemm", "qdw")


def problem_key(problem: dict) -> str:
    M, N, K = problem["M"], problem["N"], problem["K"]
    if problem.get("kind") == "qconv":
        return (f"i8:qconv:{M}x{N}x{K}:{problem['KH']}x{problem['KW']}s{problem['SH']}"
                f":{problem['C']}x{problem['H']}x{problem['W']}")
    if problem.get("kind") == "qgemm":
        return f"i8:qgemm:{M}x{N}x{K}"
    if problem.get("kind") == "qdw":
        return (f"i8:qdw:{M}x{N}:{problem['KH']}x{problem['KW']}s{problem['SH']}"
                f":{problem['C']}x{problem['H']}x{problem['W']}")
    if problem.get("kind") == "conv":
        return (f"conv:{M}x{N}x{K}:{problem['KH']}x{problem['KW']}s{problem['SH']}"
                f":{problem['C']}x{problem['H']}x{problem['W']}:{problem.get('mode', 'implicit')}")
    return f"{M}x{N}x{K}"


@dataclass
class TuneResult:
    key: str
    best: MfmaSchedule
    best_metric: float
    measured: bool
    n_evaluated: int
    ranking: list = field(default_factory=list)
    rejected: list = field(default_factory=list)   # "schedule: reason" per dropped candidate


class AutotuneCache:
    """Best schedule per problem, persisted as JSON."""

    def __init__(self, path: Optional[str] = None) -> None:
        self.path = path
        self.entries: dict = {}
        if path and os.path.exists(path):
            with open(path) as f:
                self.entries = json.load(f)

    @staticmethod
    def key(M, N, K) -> str:
        return f"{M}x{N}x{K}"

    def get_key(self, key: str) -> Optional[MfmaSchedule]:
        e = self.entries.get(key)
        return None if not e else MfmaSchedule(**e["sched"])

    def get(self, M, N, K) -> Optional[MfmaSchedule]:
        return self.get_key(self.key(M, N, K))

    def put_key(self, key: str, sched: MfmaSchedule, metric: float, measured: bool) -> None:
        self.entries[key] = {"sched": sched.as_dict(), "metric": metric, "measured": measured}

    def put(self, M, N, K, sched: MfmaSchedule, metric: float, measured: bool) -> None:
        self.put_key(self.key(M, N, K), sched, metric, measured)

    def save(self, path: Optional[str] = None) -> None:
        path = path or self.path
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(self.entries, f, indent=1, sort_keys=True)


def conv_schedule_ok(sched: MfmaSchedule, problem: dict) -> bool:
    """A schedule the implicit-GEMM conv lowering accepts for this problem:
    the tiled gather kernels', or a wave-split form when the K steps hold
    whole taps (Cin % 16 == 0, one group)."""
    if sched.WK > 1:
        return sched.is_valid() and problem.get("C", 1) % 16 == 0 and problem.get("group", 1) == 1
    return sched.conv_valid()


def is_implicit_conv(problem: dict) -> bool:
    """True for convolutions lowered to the implicit-GEMM gather kernels,
    whose schedules must also satisfy ``MfmaSchedule.conv_valid``."""
    return problem.get("kind") == "conv" and problem.get("mode", "implicit") == "implicit"


def candidates(M: int, N: int, K: int, *, budget: int = 24, seed: int = 0, extra_random: int = 4,
               conv: bool = False, stream_k: int = 4, unroll: int = 4) -> list:
    """The ``budget`` best schedules by the cost model, a seeded random few
    more, the shape-aware default (``conv``: implicit-GEMM convolution
    schedules only), the stream-K form of the ``stream_k`` best unsplit
    ones whose tile count is above the CU count and not a multiple of it,
    and the K loop unrolled by two of the ``unroll`` best double-buffered
    ones (the cost model does not see the unroll, so it is measured)."""
    space = list(gemm_search_space(SPLITS))
    space = [s for s in space if split_slices(K, s)[0] == s.SK or s.SK == 1]
    if conv:
        space = [s for s in space if s.conv_valid()]
    ranked = sorted(space, key=lambda s: analytical_cost(s, M, N, K))
    pick = ranked[:budget]
    rest = ranked[budget:]
    rng = random.Random(seed)
    pick += rng.sample(rest, min(extra_random, len(rest)))
    d = default_schedule(M, N, K)
    if d not in pick:
        pick.append(d)
    # the model's best form of every large-wave-tile layout (wave tile of at
    # least 32 x 64: fewer LDS bytes per flop), so that those are measured
    # even where the model ranks small tiles first
    seen = {(s.BM, s.BN, s.WGM, s.WGN, s.MS) for s in pick}
    for s in ranked:
        wm, wn = s.wave_tile()
        key = (s.BM, s.BN, s.WGM, s.WGN, s.MS)
        if wm * wn >= 2048 and s.BK >= 16 and key not in seen and len(seen) < budget + 24:
            seen.add(key)
            pick.append(s)
    uneven = [s for s in pick if s.SK == 1 and _tiles(s, M, N) > CUS and _tiles(s, M, N) % CUS]
    pick += [s.with_stream_k() for s in uneven[:stream_k]]
    pick += [s.with_unroll(2) for s in [s for s in pick if s.DB and s.UN == 1][:unroll]]
    if not conv:                      # dense GEMMs: every wave-split form is measured too
        pick += list(wsplit_search_space())
    return unique_forms(pick, K)


def _tiles(s: MfmaSchedule, M: int, N: int) -> int:
    return -(-M // s.BM) * -(-N // s.BN)


def qcandidates(M: int, N: int, K: int, *, budget: int = 24, seed: int = 0,
                extra_random: int = 4) -> list:
    """int8 counterpart of ``candidates`` over ``qgemm_search_space``."""
    space = list(qgemm_search_space())
    ranked = sorted(space, key=lambda s: analytical_qcost(s, M, N, K))
    pick = ranked[:budget]
    rest = ranked[budget:]
    rng = random.Random(seed)
    pick += rng.sample(rest, min(extra_random, len(rest)))
    d = default_qschedule(M, N, K)
    if d not in pick:
        pick.append(d)
    return pick


def problem_candidates(problem: dict, *, budget: int = 24, seed: int = 0) -> list:
    M, N, K = problem["M"], problem["N"], problem["K"]
    if problem.get("kind") == "qdw":          # the small space is measured whole
        return list(qdw_search_space())
    if is_int8(problem):
        return qcandidates(M, N, K, budget=budget, seed=seed)
    cands = candidates(M, N, K, budget=budget, seed=seed, conv=is_implicit_conv(problem))
    if is_implicit_conv(problem) and problem.get("C", 1) % 16 == 0 and problem.get("group", 1) == 1:
        cands += list(wsplit_conv_search_space())      # tap-major gathers on the wave-split kernel
    return unique_forms(cands, K)


def unique_forms(cands: list, K: int) -> list:
    """The candidates as the lowering will build them (a split that leaves
    one slice of K is no split), each form once, in first-seen order."""
    seen, out = set(), []
    for s in cands:
        s = unsplit_if_one_slice(s, K)
        if s not in seen:
            seen.add(s)
            out.append(s)
    return out


def _problem_graph(problem: dict, sched_seed: int = 0):
    """A one-group graph (and feeds) that lowers to exactly this problem."""
    import numpy as np

    from mdlc_amd.tools.graph_builder import GraphBuilder

    rng = np.random.default_rng(sched_seed)
    b = GraphBuilder("tune")
    if problem["kind"] in ("qconv", "qdw"):
        n, c, h, w = problem["batch"], problem["C"], problem["H"], problem["W"]
        oc, kh, kw = problem["N"], problem["KH"], problem["KW"]
        group = c if problem["kind"] == "qdw" else 1
        b.input("x", (n, c, h, w))
        b.node("QuantizeLinear", ["x"], "xq", inv_scale=20.0)
        b.const("w", rng.integers(-127, 128, (oc, c // group, kh, kw)).astype(np.int8))
        b.const("b", rng.integers(-1000, 1000, oc).astype(np.int32))
        b.const("m", rng.uniform(1e-4, 1e-3, oc).astype(np.float32))
        attrs = dict(kernel_shape=[kh, kw], strides=[problem["SH"], problem["SW"]],
                     dilations=[problem["DH"], problem["DW"]], group=group,
                     pads=[problem["PT"], problem["PL"], problem["PB"], problem["PR"]])
        if problem.get("relu"):
            attrs["activation"] = "Relu"
        b.node("QConv", ["xq", "w", "b", "m"], "y", **attrs)
        b.output("y")
        return b.graph(), {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}
    if problem["kind"] == "qgemm":
        M, N, K = problem["M"], problem["N"], problem["K"]
        b.input("xq", (M, K), dtype="int8")
        b.const("w", rng.integers(-127, 128, (N, K)).astype(np.int8))
        b.const("b", rng.integers(-1000, 1000, N).astype(np.int32))
        b.const("m", rng.uniform(2e-6, 1e-5, N).astype(np.float32))
        b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1,
               out_dtype="float32" if problem.get("out_f32") else "int8")
        b.output("y")
        return b.graph(), {"xq": rng.integers(-127, 128, (M, K)).astype(np.int8)}
    if problem["kind"] == "conv":
        n, c, h, w = problem["batch"], problem["C"], problem["H"], problem["W"]
        oc, kh, kw = problem["M"], problem["KH"], problem["KW"]
        b.input("x", (n, c, h, w))
        b.const("w", (rng.standard_normal((oc, c, kh, kw)) / np.sqrt(c * kh * kw)).astype(np.float32))
        ins = ["x", "w"]
        if problem.get("bias"):
            b.const("b", rng.standard_normal(oc).astype(np.float32))
            ins.append("b")
        out = "y" if not problem.get("act") else "pre"
        b.node("Conv", ins, out, kernel_shape=[kh, kw], strides=[problem["SH"], problem["SW"]],
               dilations=[problem["DH"], problem["DW"]],
               pads=[problem["PT"], problem["PL"], problem["PB"], problem["PR"]])
        if problem.get("act"):
            b.node(problem["act"], [out], "y")
        b.output("y")
        feeds = {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}
    else:
        M, N, K = problem["M"], problem["N"], problem["K"]
        b.input("A", (M, K))
        b.const("B", rng.standard_normal((K, N)).astype(np.float32))
        b.node("Gemm", ["A", "B"], "y")
        b.output("y")
        feeds = {"A": rng.standard_normal((M, K)).astype(np.float32)}
    return b.graph(), feeds


def _compile_for(problem: dict, sched: Optional[MfmaSchedule]):
    """Compile the problem's graph with ``sched`` for every GEMM-shaped
    launch (``None``: the lowering's own shape-aware default)."""
    from mdlc_amd.compiler import compile_graph

    g, feeds = _problem_graph(problem)
    fn = None if sched is None else (lambda node, mnk: sched)
    # the GEMM schedule is what is measured: convs stay on the implicit GEMM
    c = compile_graph(g, feeds=feeds, schedule_fn=fn, conv_mode=problem.get("mode", "implicit"),
                      winograd=False)
    return c, feeds


def precompile(problem: dict, sched: MfmaSchedule) -> None:
    """Compile the candidate's module into the code-object cache (no device)."""
    from mdlc_amd.codegen.hip.hiprtc_runtime import compile_code_object

    c, _ = _compile_for(problem, sched)
    compile_code_object(c.module.sources())


def measure(problem: dict, sched: Optional[MfmaSchedule], ctx, *, iters: int = 20,
            warmup: int = 3, with_output: bool = False):
    """Device time (ms) of one run of the problem's launches with ``sched``;
    with ``with_output`` also the problem's output ``y`` after the runs."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor

    c, feeds = _compile_for(problem, sched)
    ex = HipExecutor(c.module, ctx)
    try:
        ex._upload_feeds(feeds)
        ms = ex.plan.time_ms(warmup, iters)
        return (ms, ex.read("y")) if with_output else ms
    finally:
        ex.close()


# A measured candidate is accepted only if its output agrees with the
# default schedule's on the same feed: bit-exact for int8 (the integer
# result does not depend on the schedule), and for fp32 within rtol 1e-4
# plus an absolute 1e-5 of the output's RMS magnitude (split-K and tile
# shape change the summation order, so outputs near zero differ by a few
# ulps of the typical term, not of themselves; a wrong tile is off by the
# whole magnitude).
AGREE_RTOL, AGREE_ATOL = 1e-4, 1e-5


def outputs_agree(got, want) -> bool:
    import numpy as np

    got, want = np.asarray(got), np.asarray(want)
    if got.shape != want.shape:
        return False
    if np.issubdtype(want.dtype, np.integer):
        return bool(np.array_equal(got, want))
    w = want.astype(np.float64)
    scale = float(np.sqrt(np.mean(w * w))) if w.size else 0.0
    return bool(np.all(np.abs(got.astype(np.float64) - w) <= AGREE_ATOL * max(scale, 1.0)
                       + AGREE_RTOL * np.abs(w)))


class TuneError(RuntimeError):
    pass


def tune_problem(problem: dict, *, budget: int = 24, ctx=None, seed: int = 0) -> TuneResult:
    """Best schedule for ``problem``: by the cost model, or (``ctx`` given)
    by device time among candidates whose output matches the default
    schedule's. Raises ``TuneError`` when no candidate survives."""
    M, N, K = problem["M"], problem["N"], problem["K"]
    cands = problem_candidates(problem, budget=budget, seed=seed)
    model = analytical_qcost if is_int8(problem) else analytical_cost
    scored, rejected = [], []
    want = measure(problem, None, ctx, iters=1, warmup=0, with_output=True)[1] if ctx else None
    for s in cands:
        if ctx is None:
            scored.append((s, model(s, M, N, K)))
            continue
        try:
            metric, got = measure(problem, s, ctx, with_output=True)
        except Exception as exc:  # a candidate the lowering or hipRTC rejects
            rejected.append(f"{s.key_full()}: {type(exc).__name__}: {exc}".splitlines()[0])
            continue
        if not outputs_agree(got, want):
            rejected.append(f"{s.key_full()}: output differs from the default schedule's")
            continue
        scored.append((s, metric))
    if not scored:
        raise TuneError(f"no candidate schedule for {problem_key(problem)} could be measured "
                        f"({len(cands)} tried): " + "; ".join(rejected[:4]))
    scored.sort(key=lambda t: t[1])
    best, best_metric = scored[0]
    return TuneResult(problem_key(problem), best, best_metric, ctx is not None, len(scored),
                      [(s.key_full(), m) for s, m in scored], rejected)


def tune_gemm(M: int, N: int, K: int, *, budget: int = 24, ctx=None, seed: int = 0) -> TuneResult:
    """Tune a plain GEMM (activation A, constant B) of shape (M, N, K)."""
    return tune_problem({"kind": "gemm", "M": M, "N": N, "K": K}, budget=budget, ctx=ctx, seed=seed)


class Tuner:
    """A cache-backed schedule source usable as the codegen's ``schedule_fn``.

    A cache hit is returned as is; a miss is tuned (measured when ``ctx`` is
    given, else by the cost model) and recorded.
    """

    def __init__(self, cache: Optional[AutotuneCache] = None, ctx=None, budget: int = 24,
                 tune_misses: bool = True) -> None:
        self.cache = cache or AutotuneCache()
        self.ctx = ctx
        self.budget = budget
        self.tune_misses = tune_misses

    def schedule_problem(self, problem: dict) -> MfmaSchedule:
        key = problem_key(problem)
        hit = self.cache.get_key(key)
        if problem.get("kind") == "qdw":
            if hit is not None and qdw_valid(hit):
                return hit
            if not self.tune_misses:
                return default_qdw_schedule(problem["M"])
        elif is_int8(problem):
            if hit is not None and qsched_valid(hit):
                return hit
            if not self.tune_misses:
                return default_qschedule(problem["M"], problem["N"], problem["K"])
        elif hit is not None and (conv_schedule_ok(hit, problem) if is_implicit_conv(problem)
                                  else hit.is_valid()):
            return hit
        if not self.tune_misses:
            return default_schedule(problem["M"], problem["N"], problem["K"])
        res = tune_problem(problem, budget=self.budget, ctx=self.ctx)
        self.cache.put_key(key, res.best, res.best_metric, res.measured)
        return res.best

    def schedule_for(self, node, mnk) -> MfmaSchedule:
        M, N, K = mnk
        return self.schedule_problem({"kind": "gemm", "M": M, "N": N, "K": K})

    def __call__(self, node, mnk) -> MfmaSchedule:
        return self.schedule_for(node, mnk)


TUNED_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned_gfx950.json")


def tuned_schedules() -> Tuner:
    """The shipped measured schedules for gfx950 (cache misses fall back to
    the shape-aware default without tuning)."""
    return Tuner(AutotuneCache(TUNED_PATH if os.path.exists(TUNED_PATH) else None),
                 tune_misses=False)


__all__ = ["AutotuneCache", "Tuner", "TuneResult", "analytical_cost", "candidates",
           "is_implicit_conv", "is_int8", "measure", "problem_candidates", "qcandidates",
           "analytical_qcost",
           "outputs_agree", "precompile", "problem_key", "TuneError", "tune_gemm", "tune_problem", "tuned_schedules",
           "DEFAULT_GEMM"]
