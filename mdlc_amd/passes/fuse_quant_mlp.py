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
both large next to the rows they serve and large outright (see
``MAX_WEIGHT_BYTES_PER_ROW`` and ``MAX_FUSED_WEIGHT_BYTES``).
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
# rows. The fold fires where those weights are small next to the rows they
# serve (at most MAX_WEIGHT_BYTES_PER_ROW bytes per row of x, 2*C*E / M) or
# small outright (at most MAX_FUSED_WEIGHT_BYTES): measured on MI355X at
# RepViT's shapes, 23.5 B/row (stage 3, batch 32) fused wins 7.8 vs 14.0 us;
# 376 B/row with 590 KB of weights (stage 4, batch 32) loses 20 vs 13.8 us;
# stage 3 at batch 1 (147 KB, 752 B/row) wins 8.1-8.5 us against ~15 us for
# the depthwise conv and the two convs, while stage 4 there (590 KB) loses
# 25-28 us against ~15.
MAX_WEIGHT_BYTES_PER_ROW = 64
MAX_FUSED_WEIGHT_BYTES = 256 * 1024


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
            if (not self.always and M is not None and 2 * C * E > MAX_WEIGHT_BYTES_PER_ROW * M
                    and 2 * C * E > MAX_FUSED_WEIGHT_BYTES):
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


class FuseQuantMixer(Pass):
    """Fold a block's depthwise token mixer into the ``QMlp`` that consumes
    it: ``x = QConv(z, Wd, bd, md)`` (depthwise, KxK odd, stride 1, same-size
    padding, no epilogue) feeding only ``y = QMlp(x, ...)`` becomes
    ``y = QMlp(z, Wd, bd, md, ...)`` with ``attrs["mixer"]`` holding the
    conv's window (``kernel_shape``, ``pads``, ``activation``) and
    ``attrs["mixed"]`` the name ``x`` had. The value is the composition, so it
    is bit-identical; the device kernel computes ``x`` in its prologue and
    keeps it on chip (it is also the residual). Runs after shape inference."""
    name = "fuse_quant_mixer"

    def run(self, graph: Graph) -> bool:
        changed = False
        prod = graph.producers()
        for q in list(graph.nodes):
            if q.op_type != "QMlp" or q.attrs.get("mixer"):
                continue
            x = q.inputs[0]
            d = prod.get(x)
            if d is None or d.op_type != "QConv" or d.attrs.get("epilogue"):
                continue
            if x in graph.outputs or graph.use_count().get(x, 0) != 1:
                continue
            if not all(graph.is_constant(e) for e in d.inputs[1:4]):
                continue
            zi, xi = graph.info(d.inputs[0]), graph.info(x)
            if zi is None or xi is None or tuple(zi.shape) != tuple(xi.shape) or len(zi.shape) != 4:
                continue
            C = zi.shape[1]
            w = graph.initializers[d.inputs[1]]
            a = d.attrs
            kh, kw = (list(a.get("kernel_shape") or w.shape[2:]) + [1, 1])[:2]
            pads = [int(p) for p in a.get("pads", [0, 0, 0, 0])]
            if (int(a.get("group", 1)) != C or w.shape[:2] != (C, 1) or kh % 2 == 0 or kw % 2 == 0
                    or list(a.get("strides", [1, 1])) != [1, 1]
                    or any(int(v) != 1 for v in a.get("dilations", [1, 1]))
                    or pads != [kh // 2, kw // 2, kh // 2, kw // 2]):
                continue
            E = graph.initializers[q.inputs[1]].shape[0]
            M = zi.shape[0] * zi.shape[2] * zi.shape[3]
            if qmlp_layout(C, E, M or 1, mixer_taps=int(kh) * int(kw)) is None:
                continue                 # the mixer's weights leave no tiling room in LDS
            mixer = {"kernel_shape": [int(kh), int(kw)], "pads": pads, "activation": a.get("activation")}
            fused = Node("QMlp", list(d.inputs[:4]) + list(q.inputs[1:]), list(q.outputs),
                         dict(q.attrs, mixer=mixer, mixed=x), (d.name or "QConv") + "+" + (q.name or "mlp"),
                         list(d.fused_from or ["QConv"]) + list(q.fused_from or ["QMlp"]))
            graph.nodes[graph.nodes.index(d)] = fused
            graph.remove_nodes([q])
            changed = True
        return changed


__all__ = ["FuseQuantMlp", "FuseQuantMixer"]
