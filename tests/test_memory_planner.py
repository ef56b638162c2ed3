"""Memory planner: live ranges never overlap inside a buffer, offsets are
aligned and disjoint (reference tests/test_memory_planner.py:11-62)."""

from __future__ import annotations

from conftest import build_graph
from mdlc_amd.passes import default_pipeline
from mdlc_amd.passes.shape_inference import infer_shapes
from mdlc_amd.runtime import plan_memory
from mdlc_amd.runtime.memory_planner import ARENA_ALIGN
from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
from mdlc_amd.tools.build_resnet18 import build_resnet18


def no_live_overlap(graph, plan):
    order = graph.topo_sort()
    never = len(order) + 1
    birth, death = {}, {}
    for k, n in enumerate(order):
        for o in n.outputs:
            if o in plan.assignment:
                birth[o] = k
        for e in n.real_inputs():
            if e in plan.assignment:
                death[e] = k
    for o in graph.outputs:
        if o in plan.assignment:
            death[o] = never
    by_buf: dict = {}
    for t, b in plan.assignment.items():
        by_buf.setdefault(b, []).append(t)
    for b, ts in by_buf.items():
        iv = sorted((birth.get(t, 0), death.get(t, never)) for t in ts)
        for (s1, e1), (s2, e2) in zip(iv, iv[1:]):
            assert e1 <= s2, f"buffer {b}: live ranges overlap {(s1, e1)} {(s2, e2)}"


def arena_is_consistent(graph, plan):
    spans = sorted((plan.offsets[b.id], plan.offsets[b.id] + b.size) for b in plan.buffers)
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert all(o % ARENA_ALIGN == 0 for o in plan.offsets.values())
    for t, b in plan.assignment.items():
        assert graph.info(t).nbytes() <= plan.buffers[b].size


def test_plan_reuses_and_is_safe():
    g, feeds = build_graph("residual_block", c=8, h=16, w=16)
    g = default_pipeline().run(g)
    infer_shapes(g, feeds)
    p = plan_memory(g)
    assert p.planned_activation_bytes <= p.naive_activation_bytes
    assert len(p.buffers) >= 1
    no_live_overlap(g, p)
    arena_is_consistent(g, p)


def test_plan_saves_memory_on_deep_graphs():
    for build in (build_resnet18, build_mobilenetv2):
        g = default_pipeline().run(build(batch=1, calibrate=False))
        infer_shapes(g)
        p = plan_memory(g)
        assert p.planned_activation_bytes < 0.6 * p.naive_activation_bytes
        no_live_overlap(g, p)
        arena_is_consistent(g, p)
