"""Fold a 3x3 stride-2 max pool into the small-channel conv that feeds it (a
network's stem), so one launch writes the pooled output and the conv's
output never reaches memory.

The reference keeps ``MaxPool`` a host op of its own (mdlc/runtime/
ops.py:109-125, -inf padding) after the stem's ``FusedConvAct``. This
backend pass runs after the reference pipeline and shape inference and
rewrites

    y = FusedConvAct(x, w, b)         (or Conv / FusedConvBNAct)
    z = MaxPool(y)                    3x3, stride 2, padding 1

into the conv node with output ``z`` and ``attrs["maxpool"]`` holding the
pool's window (``kernel_shape``, ``strides``, ``pads``) and
``attrs["pool_from"]`` the name ``y`` had. The values are the pool of the
conv's output, element for element: the fused kernel takes the maximum of
the raw sums and then adds the bias and applies the activation, which for a
non-decreasing activation (none, Relu, Relu6, Clip) and rounded float32
addition gives the same float32 as pooling the activated outputs.

The fold fires only when ``y`` has no other consumer and is not a graph
output, the conv has no folded residual, one group and no dilation, the
activation is non-decreasing, the pool has no ``Indices`` output, no
dilation and floor rounding, and ``conv_pool_band`` finds a band for the
shapes (few input channels, enough images to give every CU a band).
"""

from __future__ import annotations

from mdlc_amd.codegen.schedule import conv_pool_band
from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass
from mdlc_amd.passes.shape_inference import conv_geometry, resolve_pads

CONVS = ("Conv", "FusedConvAct", "FusedConvBNAct")
MONOTONE = (None, "Identity", "Relu", "Relu6", "Clip")


class FuseConvMaxPool(Pass):
    name = "fuse_conv_maxpool"

    @staticmethod
    def _pool_window(graph: Graph, pool: Node, shape) -> dict | None:
        a = pool.attrs
        if len(pool.outputs) > 1 and pool.outputs[1]:
            return None
        if list(a.get("kernel_shape", [])) != [3, 3] or list(a.get("strides", [1, 1])) != [2, 2]:
            return None
        if list(a.get("dilations", [1, 1])) != [1, 1] or int(a.get("ceil_mode", 0)):
            return None
        (pt, pb), (pl, pr) = resolve_pads(a.get("auto_pad", "NOTSET"), a.get("pads"),
                                          tuple(shape[2:]), (3, 3), (2, 2), (1, 1))
        if (pt, pb, pl, pr) != (1, 1, 1, 1):
            return None
        return {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]}

    def run(self, graph: Graph) -> bool:
        changed = False
        prod = graph.producers()
        for pool in list(graph.nodes):
            if pool.op_type != "MaxPool":
                continue
            y = pool.inputs[0]
            conv = prod.get(y)
            if conv is None or conv.op_type not in CONVS or conv.attrs.get("maxpool"):
                continue
            if y in graph.outputs or graph.use_count().get(y, 0) != 1:
                continue
            a = conv.attrs
            if a.get("residual_subgraph") or a.get("activation") not in MONOTONE:
                continue
            xi, wi = graph.info(conv.inputs[0]), graph.info(conv.inputs[1])
            if xi is None or wi is None or len(xi.shape) != 4 or len(wi.shape) != 4:
                continue
            geo = conv_geometry(conv, xi.shape, wi.shape)
            if geo["group"] != 1:
                continue
            win = self._pool_window(graph, pool, (geo["N"], geo["OC"], geo["OH"], geo["OW"]))
            if win is None or conv_pool_band(geo["C"], geo["KH"], geo["KW"], geo["SH"], geo["SW"],
                                             geo["DH"], geo["DW"], geo["N"], geo["OH"],
                                             geo["OW"]) is None:
                continue
            fused = Node(conv.op_type, list(conv.inputs), [pool.outputs[0]],
                         dict(a, maxpool=win, pool_from=y),
                         (conv.name or conv.op_type) + "+MaxPool",
                         list(conv.fused_from or [conv.op_type]) + ["MaxPool"])
            graph.nodes[graph.nodes.index(conv)] = fused
            graph.remove_nodes([pool])
            prod = graph.producers()
            changed = True
        return changed


__all__ = ["FuseConvMaxPool"]
