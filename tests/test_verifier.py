"""Structural verifier catches broken graphs; every pass keeps the invariants
and is idempotent (reference tests/test_verifier.py:29-110)."""

from __future__ import annotations

import pytest

from conftest import build_graph
from mdlc_amd.ir import Graph, GraphVerifyError, Node, verify_graph
from mdlc_amd.passes import (
    ConstantFolding, DeadCodeElimination, FuseActivation, FuseConvBN, FuseElementwise, default_pipeline,
)

ALL_PASSES = [ConstantFolding, FuseConvBN, DeadCodeElimination, FuseActivation, FuseElementwise]


def _structure(g: Graph):
    return [(n.op_type, tuple(n.inputs), tuple(n.outputs)) for n in g.topo_sort()]


def test_verifier_accepts_valid_graph(model_case):
    name, kw = model_case
    g, _ = build_graph(name, **kw)
    verify_graph(g)


def _bad(outputs):
    g = Graph("bad")
    g.inputs = ["x"]
    g.outputs = outputs
    return g


def test_verifier_rejects_undefined_input():
    g = _bad(["y"])
    g.add_node(Node("Relu", ["nonexistent"], ["y"]))
    with pytest.raises(GraphVerifyError, match="undefined"):
        verify_graph(g)


def test_verifier_rejects_duplicate_producer():
    g = _bad(["y"])
    g.add_node(Node("Relu", ["x"], ["y"]))
    g.add_node(Node("Sigmoid", ["x"], ["y"]))
    with pytest.raises(GraphVerifyError, match="two producers"):
        verify_graph(g)


def test_verifier_rejects_cycle():
    g = _bad(["y"])
    g.add_node(Node("Add", ["x", "b"], ["a"]))
    g.add_node(Node("Add", ["a", "x"], ["b"]))
    g.add_node(Node("Relu", ["a"], ["y"]))
    with pytest.raises(GraphVerifyError):
        verify_graph(g)


def test_verifier_rejects_orphan_node():
    g = _bad(["y"])
    g.add_node(Node("Relu", ["x"], ["y"]))
    g.add_node(Node("Sigmoid", ["x"], ["dead"]))
    with pytest.raises(GraphVerifyError, match="orphan"):
        verify_graph(g)


def test_verifier_rejects_missing_output():
    g = _bad(["y", "never_made"])
    g.add_node(Node("Relu", ["x"], ["y"]))
    with pytest.raises(GraphVerifyError, match="not produced"):
        verify_graph(g)


def test_verifier_rejects_shadowing_and_bad_initializer_shape():
    import numpy as np

    g = _bad(["y"])
    g.add_node(Node("Relu", ["x"], ["x"]))
    with pytest.raises(GraphVerifyError, match="shadows"):
        verify_graph(g)
    g = _bad(["y"])
    g.set_initializer("w", np.zeros((2, 3), np.float32))
    g.value_info["w"].shape = (3, 2)
    g.add_node(Node("Add", ["x", "w"], ["y"]))
    with pytest.raises(GraphVerifyError, match="initializer"):
        verify_graph(g)


@pytest.mark.parametrize("pass_cls", ALL_PASSES)
def test_pass_keeps_invariants_and_is_idempotent(pass_cls, model_case):
    name, kw = model_case
    g, _ = build_graph(name, **kw)
    for cls in ALL_PASSES:
        p = cls()
        p.run(g)
        verify_graph(g, context=p.name)
        if cls is pass_cls:
            break
    snap = _structure(g)
    again = pass_cls().run(g)
    verify_graph(g, context=f"{pass_cls.__name__} (2nd run)")
    assert _structure(g) == snap, f"{pass_cls.__name__} is not idempotent"
    assert not again, f"{pass_cls.__name__} reported changes on a converged graph"


def test_full_pipeline_output_verifies(model_case):
    name, kw = model_case
    g, _ = build_graph(name, **kw)
    verify_graph(default_pipeline().run(g), context="full pipeline")
