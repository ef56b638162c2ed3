"""Memory planner: a simulated arena shows that no tensor is overwritten
while it is still needed, and the buffers are aligned and disjoint.

The planner's assignment is the reference's (mdlc/runtime/memory_planner.py
:66-146); the check here is this build's own. Instead of comparing live
intervals it replays the plan in the planner's order on an array of 4-byte
words the size of the arena: a node first verifies that every pooled input
still carries its own stamp over its whole range, then stamps its outputs
over theirs, and then verifies the inputs again (a kernel reads its inputs
while it writes its outputs, so an output may not share a word with them).
At the end every graph output must still carry its stamp.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import build_graph
from mdlc_amd.passes import default_pipeline
from mdlc_amd.passes.shape_inference import infer_shapes
from mdlc_amd.runtime import plan_memory
from mdlc_amd.runtime.memory_planner import ARENA_ALIGN
from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
from mdlc_amd.tools.build_resnet18 import build_resnet18


def simulate_arena(graph, plan) -> list:
    """Replay ``plan`` on a stamped arena; returns the violations found."""
    words = np.zeros(plan.arena_bytes // 4 + 1, dtype=np.int32)
    ids = {t: i + 1 for i, t in enumerate(sorted(plan.assignment))}
    bad = []

    def span(t):
        start = plan.offset_of(t) // 4
        return start, start + -(-graph.info(t).nbytes() // 4)

    def intact(t, when):
        a, b = span(t)
        if not (words[a:b] == ids[t]).all():
            others = sorted({int(v) for v in words[a:b]} - {ids[t]})
            names = [n for n, i in ids.items() if i in others]
            bad.append(f"{t!r} overwritten {when} (by {names or 'nothing: never written'})")

    for node in graph.topo_sort():
        pooled_in = [e for e in node.real_inputs() if e in plan.assignment]
        for e in pooled_in:
            intact(e, f"before {node.name or node.op_type} reads it")
        for o in node.outputs:
            if o in plan.assignment:
                a, b = span(o)
                words[a:b] = ids[o]
        for e in pooled_in:
            intact(e, f"while {node.name or node.op_type} writes its outputs")
    for o in graph.outputs:
        if o in plan.assignment:
            intact(o, "before the graph returns it")
    return bad


def buffer_violations(graph, plan) -> list:
    bad = []
    spans = sorted((plan.offsets[b.id], plan.offsets[b.id] + b.size, b.id) for b in plan.buffers)
    for (a0, a1, i), (b0, _, j) in zip(spans, spans[1:]):
        if a1 > b0:
            bad.append(f"buffers {i} and {j} overlap")
    bad += [f"buffer {b} at {o} is not {ARENA_ALIGN}-byte aligned"
            for b, o in plan.offsets.items() if o % ARENA_ALIGN]
    bad += [f"{t!r} ({graph.info(t).nbytes()} B) exceeds buffer {b} ({plan.buffers[b].size} B)"
            for t, b in plan.assignment.items() if graph.info(t).nbytes() > plan.buffers[b].size]
    if spans and spans[-1][1] > plan.arena_bytes:
        bad.append("a buffer ends past the arena")
    return bad


def _planned(build):
    g = default_pipeline().run(build)
    infer_shapes(g)
    return g, plan_memory(g)


def test_small_residual_model_reuses_safely():
    g, feeds = build_graph("residual_block", c=8, h=16, w=16)
    g = default_pipeline().run(g)
    infer_shapes(g, feeds)
    p = plan_memory(g)
    assert p.planned_activation_bytes <= p.naive_activation_bytes and len(p.buffers) >= 1
    assert simulate_arena(g, p) == []
    assert buffer_violations(g, p) == []


@pytest.mark.parametrize("net", ["resnet18", "mobilenetv2"])
def test_deep_graphs_save_memory_safely(net):
    build = {"resnet18": build_resnet18, "mobilenetv2": build_mobilenetv2}[net]
    g, p = _planned(build(batch=1))
    assert p.planned_activation_bytes < 0.6 * p.naive_activation_bytes
    assert simulate_arena(g, p) == []
    assert buffer_violations(g, p) == []


def test_resnet18_known_answer():
    """13.119 MiB of activations naively, 4.594 MiB planned in 3 buffers at
    batch 1 (the reference's published figure)."""
    g, p = _planned(build_resnet18(batch=1))
    mib = 2 ** 20
    assert round(p.naive_activation_bytes / mib, 3) == 13.119
    assert round(p.planned_activation_bytes / mib, 3) == 4.594
    assert len(p.buffers) == 3


def test_simulation_catches_planted_reuse():
    """Two planted slips in the plan (on the CPU): a tensor moved into the
    buffer of one that is still live, and a node's output placed over its
    own input. The simulation reports both; the interval bookkeeping of the
    buffers alone would not see the second."""
    g, p = _planned(build_resnet18(batch=1))
    order = g.topo_sort()
    # slip 1: a tensor that is read again later (the first residual input)
    # shares its buffer with an output born before that read
    pos = {n.name or id(n): i for i, n in enumerate(order)}
    last = {}
    for i, n in enumerate(order):
        for e in n.real_inputs():
            last[e] = i
    t, born = next((n.outputs[0], i) for i, n in enumerate(order)
                   if n.outputs[0] in p.assignment and last.get(n.outputs[0], i) > i + 2)
    mid = next(n for n in order[born + 1:last[t]] if n.outputs[0] in p.assignment)
    assert pos[mid.name or id(mid)] < last[t]
    saved = dict(p.assignment)
    p.assignment[mid.outputs[0]] = p.assignment[t]
    assert any(v.startswith(repr(t)) and "before" in v for v in simulate_arena(g, p))
    p.assignment.clear()
    p.assignment.update(saved)
    assert simulate_arena(g, p) == []
    # slip 2: a node's output in the same buffer as its pooled input
    n = next(n for n in order if any(e in p.assignment for e in n.real_inputs())
             and n.outputs[0] in p.assignment)
    e = next(e for e in n.real_inputs() if e in p.assignment)
    p.assignment[n.outputs[0]] = p.assignment[e]
    assert any("while" in v and repr(e) in v for v in simulate_arena(g, p))
