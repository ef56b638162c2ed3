"""Fold an int8 channel-mixer MLP — two 1x1 QConvs with a table lookup
between them and a residual add after — into one ``QMlp`` node.

The reference has no quantized path, so this pass has no counterpart there;
it extends what ``FuseQuantEpilogue`` does for one conv to the pair. After
that fold a RepViT-style channel mixer reads

    h = QConv(x, W1, b1, m1, T)        epilogue "lut"   (1x1, C -> E)
    y = QConv(h, W2, b2, m2, x)        epilogue "add"   (1x1, E -> C, residual x)

and becomes ``y = QMlp(x, W1, b1, m1, T, W2, b2, m2)`` with attributes
``activation1`` / ``activation2`` (the convs' fused activations, if any),
``res_mult`` / ``acc_mult`` (the add's multipliers) and ``hidden`` (the name
``h`` had). Its value is defined as that composition, so every remaining
tensor keeps its value bit for bit; the device kernel keeps ``h`` on chip.

The fold fires only when both convs are plain 1x1 (stride 1, no padding,
group 1) with constant weights, bias, multipliers and table; ``h`` has no
other consumer and is not a graph output; the second conv's residual is the
first conv's input; and the device kernel has a tiling for the channel
counts (both multiples of 16, K small enough for its register budget). Run
after shape inference, it also leaves the pair alone when the weights are
large next to the rows they serve (see ``MAX_WEIGHT_BYTES_PER_ROW``).
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.codegen.schedule import qmlp_layout
from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass


def _pointwise_qconv(graph: Graph, n: Node) -> bool:
    a = n.attrs
    if n.op_type != "QConv" or int(a.get("group", 1)) != 1 or len(n.inputs) < 5:
        return False
    if list(a.get("kernel_shape", [1, 1])) != [1, 1] or list(a.get("strides", [1, 1])) != [1, 1]:
        return False
    if any(int(p) for p in a.get("pads", [0, 0, 0, 0])):
        return False
    return all(graph.is_constant(e) for e in n.inputs[1:4])


# Each workgroup of the fused kernel streams both weight matrices for its
# rows; past this many weight bytes per row of x (2*C*E / M) the two
# separately tiled launches are faster (measured on MI355X at RepViT's batch
# 32 shapes: 23.5 B/row fused wins 7.8 vs 14.0 us, 376 B/row loses 20 vs 13.8).
MAX_WEIGHT_BYTES_PER_ROW = 64


class FuseQuantMlp(Pass):
    """``always``: fold every matching pair whatever its weight size."""
    name = "fuse_quant_mlp"

    def __init__(self, always: bool = False) -> None:
        self.always = always

    def run(self, graph: Graph) -> bool:
        changed = False
        for first in list(graph.nodes):
            if not _pointwise_qconv(graph, first) or first.attrs.get("epilogue") != "lut":
                continue
            if not graph.is_constant(first.inputs[4]):
                continue
            x, h = first.inputs[0], first.outputs[0]
            if h in graph.outputs or graph.use_count().get(h, 0) != 1:
                continue
            (second,) = graph.consumers()[h]
            if (not _pointwise_qconv(graph, second) or second.attrs.get("epilogue") != "add"
                    or second.inputs[0] != h or second.inputs[4] != x):
                continue
            w1 = graph.initializers[first.inputs[1]]
            w2 = graph.initializers[second.inputs[1]]
            if w2.shape[0] != w1.shape[1] or w2.shape[1] != w1.shape[0]:
                continue
            C, E = w1.shape[1], w1.shape[0]
            info = graph.info(x)
            M = int(np.prod(info.shape)) // C if info is not None and info.shape else None
            if not self.always and M is not None and 2 * C * E > MAX_WEIGHT_BYTES_PER_ROW * M:
                continue
            if qmlp_layout(C, E, M or 1) is None:                    # no kernel tiling
                continue
            attrs = {"activation1": first.attrs.get("activation"),
                     "activation2": second.attrs.get("activation"),
                     "res_mult": float(second.attrs["res_mult"]),
                     "acc_mult": float(second.attrs["acc_mult"]), "hidden": h}
            ins = list(first.inputs[:5]) + list(second.inputs[1:4])
            fused = Node("QMlp", ins, list(second.outputs), attrs,
                         (first.name or "QConv") + "+mlp",
                         list(first.fused_from or ["QConv"]) + list(second.fused_from or ["QConv"]))
            graph.nodes[graph.nodes.index(first)] = fused
            graph.remove_nodes([second])
            changed = True
        return changed


__all__ = ["FuseQuantMlp"]
