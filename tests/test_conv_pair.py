"""Two independent implicit-GEMM convolutions in one launch, on the CPU:
where the lowering pairs them (ResNet-18's stride-2 conv and its 1x1
downsample at batch 32, whose 196-workgroup grid leaves 60 CUs idle), where
it must not (a second conv that reads the first's output, a first conv whose
grid fills the chip, split-K or different workgroup sizes), and the kernel
it generates: both bodies unchanged but for the block index, both parameter
lists in the ABI."""

from __future__ import annotations

import numpy as np
import pytest

import mdlc_amd.codegen.schedule as S
from mdlc_amd.codegen.hip.abi import declared_kinds
from mdlc_amd.codegen.hip.hip_executor import launch_args
from mdlc_amd.codegen.hip.hiprtc_runtime import Arg
from mdlc_amd.codegen.schedule import MfmaSchedule
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.build_resnet18 import build_resnet18, make_input
from mdlc_amd.tools.graph_builder import GraphBuilder


def test_resnet18_b32_pairs_the_stage2_downsample():
    c = compile_graph(build_resnet18(batch=32), feeds={"input": make_input(32)})
    pairs = [l for l in c.module.plan if l.kind == "conv_pair"]
    assert len(pairs) == 1 and len(c.module.plan) == 29
    (p,) = pairs
    a, b = p.meta["first"], p.meta["second"]
    assert a.meta["node"].outputs == ["/layer2.0.relu/Relu_output_0"]
    assert b.outputs == ["/layer2.0.downsample.1/BatchNormalization_output_0"]
    assert p.grid == (S.CUS, 1, 1) and p.meta["g0"] == a.grid[0] == 196 and p.meta["nb"] == b.grid[0]
    assert p.inputs == a.inputs + b.inputs and p.outputs == a.outputs + b.outputs
    assert p.meta["flops"] == a.meta["flops"] + b.meta["flops"]
    src = c.module.kernels[p.kernel_name]
    assert src.count("(g, (int)blockIdx.x);") == 1 and src.count("(g, t);") == 1
    # the ABI: both launches' arguments, then g0 and nb
    decl = declared_kinds(c.module.sources())[p.kernel_name]
    kinds = "".join(x.kind for x in launch_args(p, lambda e: Arg.ptr(0)))
    assert kinds == decl and len(kinds) == 2 * 15 + 2
    off = compile_graph(build_resnet18(batch=32), feeds={"input": make_input(32)}, pair_convs=False)
    assert len(off.module.plan) == 30 and "conv_pair" not in {l.kind for l in off.module.plan}
    assert [l.kernel_name for l in off.module.plan[5:7]] == [a.kernel_name, b.kernel_name]


def _two_convs(second_reads_first=False, oc2=16):
    rng = np.random.default_rng(7)
    b = GraphBuilder("two")
    b.input("x", (2, 16, 12, 12))
    b.const("w1", rng.standard_normal((32, 16, 3, 3)).astype(np.float32))
    b.const("w2", rng.standard_normal((oc2, 32 if second_reads_first else 16, 1, 1)).astype(np.float32))
    b.node("Conv", ["x", "w1"], "y1", kernel_shape=[3, 3], strides=[1, 1], pads=[1, 1, 1, 1])
    b.node("Conv", ["y1" if second_reads_first else "x", "w2"], "y2", kernel_shape=[1, 1],
           strides=[1, 1], pads=[0, 0, 0, 0])
    b.output("y1")
    b.output("y2")
    return b.graph(), {"x": rng.standard_normal((2, 16, 12, 12)).astype(np.float32)}


class _Tiled:
    """A tiled schedule for every conv (no wave-split, no Winograd)."""
    def __init__(self, sched):
        self.s = sched

    def schedule_problem(self, p):
        return self.s

    def __call__(self, node, mnk):
        return self.s


TILED = MfmaSchedule(32, 32, 16, 2, 2, 16, True, 1)


def test_independent_convs_pair_and_dependent_ones_do_not():
    g, feeds = _two_convs()
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(TILED), winograd=False)
    assert [l.kind for l in c.module.plan] == ["conv_pair"]
    g, feeds = _two_convs(second_reads_first=True)
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(TILED), winograd=False)
    assert [l.kind for l in c.module.plan] == ["conv", "conv"]
    g, feeds = _two_convs()
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(TILED), winograd=False, pair_convs=False)
    assert [l.kind for l in c.module.plan] == ["conv", "conv"]


def test_no_pair_without_idle_cus_or_with_split_k(monkeypatch):
    g, feeds = _two_convs()
    monkeypatch.setattr(S, "CUS", 8)          # the first grid (10 tiles) fills the chip
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(TILED), winograd=False)
    assert "conv_pair" not in [l.kind for l in c.module.plan]
    monkeypatch.setattr(S, "CUS", 256)
    split = MfmaSchedule(32, 32, 16, 2, 2, 16, True, 2)
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(split), winograd=False)
    assert "conv_pair" not in [l.kind for l in c.module.plan]


@pytest.mark.parametrize("oc2", [512, 2048])
def test_second_conv_must_fit_the_first_ones_shadow(oc2, monkeypatch):
    """The second conv's work per idle CU may not exceed the first's per
    workgroup: with 48 CUs the first (9 workgroups, 2.65 MFLOP) leaves 39
    idle, which a 512-channel second conv (4.7 MFLOP) fits and a 2048-channel
    one (18.9 MFLOP) does not."""
    monkeypatch.setattr(S, "CUS", 48)
    g, feeds = _two_convs(oc2=oc2)
    c = compile_graph(g, feeds=feeds, schedule_fn=_Tiled(TILED), winograd=False)
    assert ("conv_pair" in [l.kind for l in c.module.plan]) == (oc2 == 512)


def test_no_pair_across_workgroup_sizes():
    """A 256-thread first conv and a 512-thread second conv stay two launches."""
    wide = MfmaSchedule(64, 32, 16, 4, 2, 16, True, 1)

    class PerK(_Tiled):
        def schedule_problem(self, p):
            return TILED if p["K"] == 144 else wide

    g, feeds = _two_convs()
    c = compile_graph(g, feeds=feeds, schedule_fn=PerK(TILED), winograd=False)
    assert [l.block[0] for l in c.module.plan] == [256, 512]
    assert [l.kind for l in c.module.plan] == ["conv", "conv"]
