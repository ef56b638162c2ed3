"""Every launch's packed arguments against its kernel's declaration, and a
host-side replay of the GEMM/conv epilogue stores (CPU only).

The regression this pins: a schedule whose split-K factor leaves one slice
of K (MobileNetV2 batch 1's 96x12544x16 conv with SK = 8, one 16-deep step)
was compiled as the split-K form, which has no bias parameter, but launched
as the unsplit form with its bias. hipModuleLaunchKernel copies arguments by
the kernel's declaration, so every argument after the bias shifted by one:
the kernel stored through the bias pointer with the low half of the output
address as its row count, tens of megabytes past a 384-byte tensor. That is
the GPU memory fault seen with these schedules; the fixture holds them.
"""

from __future__ import annotations

import json
import os

import pytest

from mdlc_amd.autotuner.tuner import AutotuneCache, Tuner, TUNED_PATH, problem_candidates
from mdlc_amd.codegen.hip.abi import LaunchAbiError, check_launch, declared_kinds
from mdlc_amd.codegen.hip.hip_executor import launch_args
from mdlc_amd.codegen.hip.hiprtc_runtime import Arg
from mdlc_amd.codegen.schedule import MfmaSchedule, split_slices, unsplit_if_one_slice
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
from mdlc_amd.tools.build_models import build as build_small
from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8
from mdlc_amd.tools.build_resnet18 import build_resnet18
from mdlc_amd.tools.micro_gemm import build_micro_gemm

from launch_replay import modelled, operand_overlaps, out_of_bounds

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "mobilenetv2_b1_wsplit_schedules.json")


def _abi_errors(module) -> list:
    declared = declared_kinds("\n".join(module.kernels.values()))
    bad = []
    for l in module.plan:
        try:
            check_launch(l.kernel_name, declared, [a.kind for a in launch_args(l, lambda e: Arg.ptr(0))])
        except LaunchAbiError as e:
            bad.append(str(e))
    return bad


def _fixture_tuner() -> Tuner:
    cache = AutotuneCache(TUNED_PATH)
    with open(FIXTURE) as f:
        cache.entries.update(json.load(f))
    return Tuner(cache, tune_misses=False)


CASES = {
    "resnet18_b1": lambda: compile_graph(build_resnet18(batch=1), batch=1),
    "resnet18_b32": lambda: compile_graph(build_resnet18(batch=32), batch=32),
    "resnet18_b32_direct": lambda: compile_graph(build_resnet18(batch=32), batch=32, winograd=False),
    "resnet18_b2_im2col": lambda: compile_graph(build_resnet18(batch=2), batch=2, conv_mode="im2col"),
    "resnet18_b1_reference_groups": lambda: compile_graph(build_resnet18(batch=1), batch=1,
                                                          fuse_residual=False),
    "mobilenetv2_b1": lambda: compile_graph(build_mobilenetv2(batch=1), batch=1),
    "mobilenetv2_b32": lambda: compile_graph(build_mobilenetv2(batch=32), batch=32),
    "mobilenetv2_b1_fault_schedules": lambda: compile_graph(build_mobilenetv2(batch=1), batch=1,
                                                            schedule_fn=_fixture_tuner()),
    "repvit_int8_b1": lambda: compile_graph(build_repvit_int8(batch=1), batch=1),
    "repvit_int8_b32": lambda: compile_graph(build_repvit_int8(batch=32), batch=32),
    "micro_49x512x4608": lambda: compile_graph(build_micro_gemm(49, 512, 4608)[0]),
    "micro_1x1000x512": lambda: compile_graph(build_micro_gemm(1, 1000, 512)[0]),
    "small_models": None,
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_every_launch_matches_its_kernel(case):
    mods = ([compile_graph(build_small(n)).module for n in ("conv_bn_relu", "residual_block", "mlp")]
            if CASES[case] is None else [CASES[case]().module])
    for m in mods:
        assert _abi_errors(m) == []
        assert out_of_bounds(m) == []
        assert operand_overlaps(m) == []


def test_fault_schedules_compile_to_the_unsplit_form():
    """The fixture's SK = 8 schedule on K = 16 is one slice: its conv is now
    the unsplit wave-split kernel with bias and activation in its epilogue,
    and the replay models every wave-split launch of the plan."""
    c = compile_graph(build_mobilenetv2(batch=1), batch=1, schedule_fn=_fixture_tuner())
    ws = [l for l in c.module.plan if l.kind == "conv_ws"]
    assert len(ws) >= 15
    hit = [l for l in ws if (l.meta["M"], l.meta["N"], l.meta["K"]) == (96, 12544, 16)]
    assert len(hit) == 1 and hit[0].grid[1] == 1 and len(hit[0].inputs) == 3
    kinds = declared_kinds(c.module.kernels[hit[0].kernel_name])[hit[0].kernel_name]
    assert kinds == "pppp" + "i" * 11
    assert modelled(c.module) >= len(ws)


def test_the_checks_catch_the_original_fault(monkeypatch):
    """With the lowering's one-slice normalization taken out (planted on the
    CPU), the fixture's plan has exactly the mismatched launch, and the
    replay finds its stores outside every tensor."""
    import mdlc_amd.codegen.hip.emit as emit_mod

    monkeypatch.setattr(emit_mod, "unsplit_if_one_slice", lambda s, K: s)
    c = compile_graph(build_mobilenetv2(batch=1), batch=1, schedule_fn=_fixture_tuner())
    errs = _abi_errors(c.module)
    assert len(errs) == 1 and "ppp" in errs[0]
    oob = out_of_bounds(c.module)
    assert len(oob) == 1 and "conv_WS4_BM32_BN32" in oob[0]


def test_planted_declaration_mismatch_is_refused():
    """A kernel whose declaration loses a parameter (planted in the CPU copy
    of the module) fails the check before any device call."""
    c = compile_graph(build_small("residual_block"))
    l = next(l for l in c.module.plan if "int lda, " in c.module.kernels[l.kernel_name])
    src = c.module.kernels[l.kernel_name]
    c.module.kernels[l.kernel_name] = src.replace("int lda, ", "", 1)
    errs = _abi_errors(c.module)
    assert len(errs) == 1 and l.kernel_name in errs[0]
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor

    class NoDevice:                               # never reached: the check comes first
        def __getattr__(self, name):
            raise AssertionError("device touched before the argument check")

    with pytest.raises(LaunchAbiError):
        HipExecutor(c.module, NoDevice())


def test_one_slice_split_is_no_split():
    s = MfmaSchedule.wsplit(32, 32, 4, 1, False, 8)
    assert split_slices(16, s)[0] == 1 and unsplit_if_one_slice(s, 16).SK == 1
    assert unsplit_if_one_slice(s, 4608).SK == 8
    t = MfmaSchedule(64, 64, 32, 2, 2, 32, True, 4)
    assert unsplit_if_one_slice(t, 32).SK == 1 and unsplit_if_one_slice(t, 128).SK == 4


@pytest.mark.parametrize("shape", [(96, 12544, 16, 16, 112), (160, 49, 960, 960, 7),
                                   (24, 3136, 96, 96, 56), (64, 196, 384, 384, 14)],
                         ids=["K16", "K960", "K96", "K384"])
def test_every_tuner_candidate_launches_consistently(shape):
    """Every schedule the measured tuner would try on MobileNetV2 batch-1
    1x1 conv shapes (tiled, wave-split, split-K forms) lowers to launches
    that match their kernels and store inside their outputs."""
    from mdlc_amd.autotuner.tuner import _compile_for

    M, N, K, C, H = shape
    problem = {"kind": "conv", "mode": "implicit", "M": M, "N": N, "K": K, "batch": 1, "bias": True,
               "act": "Relu", "group": 1, "C": C, "H": H, "W": H, "KH": 1, "KW": 1, "SH": 1, "SW": 1,
               "DH": 1, "DW": 1, "PT": 0, "PB": 0, "PL": 0, "PR": 0, "OH": H, "OW": H}
    cands = problem_candidates(problem)
    assert len(cands) == len(set(cands))
    assert all(split_slices(K, s)[0] > 1 for s in cands if s.SK > 1)
    for s in cands:
        c, _ = _compile_for(problem, s)
        assert _abi_errors(c.module) == [], s
        assert out_of_bounds(c.module) == [], s
