"""Compiler driver: IR graph (or ONNX model) -> optimized, lowered HIP module.

Same pipeline as mdlc/compiler.py:64-95 — import, passes (optionally
verified after every change), static shapes, memory plan, codegen — with two
differences: ONNX files are read by this package's own protobuf reader
(``mdlc_amd.frontend``; the ``onnx`` package is not needed) and an IR
``Graph`` is accepted directly, and numerical pass verification is injected
by the caller (``verify``) instead of running a CPU executor inside the
compiler. Structural verification always runs.
"""

from __future__ import annotations

import os

from dataclasses import dataclass, field
from typing import Callable, Optional

from mdlc_amd.codegen.hip.emit import HipModule, emit_hip_module
from mdlc_amd.ir import Graph, verify_graph
from mdlc_amd.passes import default_pipeline
from mdlc_amd.passes.base import PassManager
from mdlc_amd.passes.fold_flatten import FoldPoolFlatten
from mdlc_amd.passes.fuse_quant_epilogue import FuseInputQuantize, FuseQuantEpilogue
from mdlc_amd.passes.fuse_quant_mlp import FuseQuantMixer, FuseQuantMlp
from mdlc_amd.passes.fuse_conv_pool import FuseConvMaxPool
from mdlc_amd.passes.fuse_residual import FuseResidualEpilogue
from mdlc_amd.passes.shape_inference import infer_shapes, make_dummy_feeds
from mdlc_amd.runtime.memory_planner import MemoryPlan, plan_memory


@dataclass
class Compiled:
    original: Graph
    graph: Graph
    module: HipModule
    mem_plan: MemoryPlan
    passes: PassManager
    feeds: dict
    checks: list = field(default_factory=list)
    golden: Optional[dict] = None          # outputs of the original graph on ``feeds``
    evaluate: Optional[Callable] = None     # the host evaluator they came from

    def verify(self, evaluate: Optional[Callable] = None, *, rtol: Optional[float] = None,
               atol: Optional[float] = None) -> list:
        """The optimized graph's outputs on ``feeds`` against the original
        graph's (mdlc/compiler.py:43-46), both computed by ``evaluate(graph,
        feeds)`` — the evaluator given to ``compile_onnx(verify_passes=...)``
        unless another is passed here. Returns one ``CheckResult`` per
        output and keeps them in ``checks`` for the report."""
        from mdlc_amd.testing import FP32_NETWORK, graph_checks

        evaluate = evaluate or self.evaluate
        if evaluate is None:
            raise ValueError("Compiled.verify needs a host evaluator of IR graphs, "
                             "evaluate(graph, feeds) -> outputs (this package has no CPU executor)")
        golden = self.golden if self.golden is not None and evaluate is self.evaluate \
            else evaluate(self.original, self.feeds)
        self.checks = graph_checks(evaluate, self.graph, self.feeds, golden,
                                   rtol=FP32_NETWORK.rtol if rtol is None else rtol,
                                   atol=FP32_NETWORK.atol if atol is None else atol)
        return self.checks

    def report(self) -> str:
        n_fused = sum(1 for n in self.graph.nodes if n.is_fused)
        lines = ["== mdlc_amd compile report ==", self.original.summary(), "-> optimized:",
                 self.graph.summary(), f"  fused groups: {n_fused}", self.passes.report(),
                 self.module.report(), self.mem_plan.report()]
        if self.checks:
            ok = all(c.ok for c in self.checks)
            lines.append(f"correctness vs golden: {'PASS' if ok else 'FAIL'}")
            lines += [f"  {c}" for c in self.checks]
        return "\n".join(lines)


def _structural_verifier(extra: Optional[Callable]) -> Callable:
    def verify(graph: Graph, pass_name: str) -> None:
        verify_graph(graph, context=pass_name)
        if extra is not None:
            extra(graph, pass_name)
    return verify


def compile_graph(graph: Graph, *, batch: int = 1, feeds: Optional[dict] = None,
                  schedule_fn=None, verify: Optional[Callable] = None,
                  conv_mode: str = "implicit", fuse_int8_epilogues: bool = True,
                  int8_depthwise: str = "mfma", fuse_residual: bool = True,
                  fuse_int8_mlp=True, small_conv: bool = True, winograd="auto",
                  fuse_pool: bool = True, pair_convs: bool = True) -> Compiled:
    """Optimize, plan and lower ``graph``. The reference pipeline runs first,
    unchanged. Then backend epilogue folds: ``fuse_int8_epilogues`` folds a
    QLut or QAdd into the QConv that feeds it; ``fuse_residual`` folds a
    float residual add (and the pointwise ops after it) into the conv that
    feeds it; ``fuse_int8_mlp`` (with the int8 folds) turns a 1x1 QConv +
    lookup followed by a 1x1 QConv + residual add of the first's input into
    one ``QMlp`` node where that pays ("always": wherever the kernel tiles),
    and folds the depthwise token mixer that feeds it into the same node; the
    int8 folds also let a small first conv quantize its own float input.
    With ``fuse_residual`` a global average pool also writes the flattened
    output of a Flatten that follows it. ``int8_depthwise`` picks the int8 depthwise kernel
    ("mfma" or "vector"). ``small_conv`` runs convs with at most four input
    channels (stems) on the direct small-channel kernel in implicit mode. ``winograd``
    runs 3x3 stride-1 convs as Winograd F(2x2, 3x3) in implicit mode: "auto" where its
    grid fills at least half the CUs, True always, False never (the implicit GEMM).
    ``fuse_pool`` (with ``small_conv`` in implicit mode) folds a 3x3 stride-2 max pool
    into the small-channel conv that feeds it where every CU gets a band of its rows.
    ``pair_convs`` runs two adjacent independent implicit-GEMM convs as one launch
    where the first leaves CUs idle (ResNet's stride-2 conv and its downsample)."""
    original = graph.clone()
    if feeds is None:
        feeds = make_dummy_feeds(graph, batch=batch)
    pm = default_pipeline(verify=_structural_verifier(verify))
    quant = fuse_int8_epilogues and any(n.op_type == "QConv" for n in graph.nodes)
    if quant:
        pm.add(FuseQuantEpilogue())
    graph = pm.run(graph)
    infer_shapes(graph, feeds)
    post = ([FuseResidualEpilogue()] if fuse_residual else []) + \
        ([FuseQuantMlp(always=fuse_int8_mlp == "always"), FuseQuantMixer()]
         if quant and fuse_int8_mlp else []) + \
        ([FuseInputQuantize()] if quant else []) + ([FoldPoolFlatten()] if fuse_residual else []) + \
        ([FuseConvMaxPool()] if fuse_pool and small_conv and conv_mode == "implicit" else [])
    if post:
        PassManager(post, verify=_structural_verifier(verify), history=pm.history).run(graph)
    mem_plan = plan_memory(graph)
    module = emit_hip_module(graph, schedule_fn, conv_mode=conv_mode, int8_depthwise=int8_depthwise,
                             small_conv=small_conv, winograd=winograd, pair_convs=pair_convs)
    return Compiled(original, graph, module, mem_plan, pm, feeds)


def compile_onnx(source, *, verify_passes=False, **kw) -> Compiled:
    """Compile an ONNX model (mdlc/compiler.py:64-95): a path to an ``.onnx``
    file, its bytes, a decoded ``ModelProto`` of ``mdlc_amd.frontend``, or an
    IR ``Graph``. The model is imported by this package's own protobuf reader
    (the ``onnx`` package is not needed) and then compiled by
    ``compile_graph``, which takes the remaining keywords (``batch``,
    ``feeds``, ``schedule_fn``, backend options). Structural verification runs
    after every pass.

    ``verify_passes`` adds the reference's numerical check: given a host
    evaluator of IR graphs, ``evaluate(graph, feeds) -> {output: array}``
    (for instance the NumPy oracle's ``run_reference``), the original graph's
    outputs on the feeds become the golden values, every pass that changes
    the graph is re-evaluated against them at the network tolerance
    (raising ``AssertionError`` naming the pass), and ``Compiled.verify()``
    checks the optimized graph. This package ships no CPU executor, so
    ``True`` raises instead of checking nothing."""
    from mdlc_amd.frontend import import_onnx, import_onnx_model
    from mdlc_amd.frontend.onnx_proto import ModelProto

    if isinstance(source, Graph):
        graph = source
    elif isinstance(source, (str, os.PathLike)):
        graph = import_onnx(source)
    elif isinstance(source, (bytes, bytearray, memoryview, ModelProto)):
        graph = import_onnx_model(source)
    else:
        raise TypeError(f"compile_onnx takes a path, model bytes, a ModelProto or a Graph, "
                        f"not {type(source).__name__}")
    if verify_passes is True:
        raise TypeError("verify_passes=True needs the host evaluator that computes the golden "
                        "outputs: pass verify_passes=evaluate, a function (graph, feeds) -> "
                        "{output: array} such as the NumPy oracle's run_reference")
    if not verify_passes:
        return compile_graph(graph, **kw)
    from mdlc_amd.testing import pass_checker

    evaluate = verify_passes
    feeds = kw.pop("feeds", None)
    if feeds is None:
        feeds = make_dummy_feeds(graph, batch=kw.get("batch", 1))
    golden = evaluate(graph.clone(), feeds)
    c = compile_graph(graph, feeds=feeds, verify=pass_checker(evaluate, feeds, golden), **kw)
    c.golden, c.evaluate = golden, evaluate
    return c
