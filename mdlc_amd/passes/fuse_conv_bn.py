"""Fold an inference BatchNormalization into the Conv that feeds it.

BN is a per-channel affine map y = x*s + t with s = gamma/sqrt(var+eps) and
t = beta - mean*s, so the conv's weights become w*s (per output channel) and
its bias b*s + t. The arithmetic is done in float32 in the same operation
order as mdlc/passes/fuse_conv_bn.py:53-68 so the folded constants are the
same bits. Legal only when the conv output feeds this BN alone, is not a
graph output, and every parameter is a constant.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph
from mdlc_amd.passes.base import Pass


class FuseConvBN(Pass):
    name = "fuse_conv_bn"

    def run(self, graph: Graph) -> bool:
        changed = False
        prod = graph.producers()
        uses = graph.use_count()
        taken = set(graph.value_info) | set(graph.initializers)

        def fresh(base: str) -> str:
            name, k = base, 1
            while name in taken:
                name, k = f"{base}_{k}", k + 1
            taken.add(name)
            return name

        for bn in list(graph.nodes):
            if bn.op_type != "BatchNormalization":
                continue
            conv = prod.get(bn.inputs[0])
            if conv is None or conv.op_type != "Conv":
                continue
            y = conv.outputs[0]
            if uses.get(y, 0) != 1 or y in graph.outputs:
                continue
            w_name = conv.inputs[1]
            params = bn.inputs[1:5]
            if not graph.is_constant(w_name) or not all(graph.is_constant(p) for p in params):
                continue

            eps = bn.attr("epsilon", 1e-5)
            f32 = lambda e: graph.initializers[e].astype(np.float32)  # noqa: E731
            w = f32(w_name)
            gamma, beta, mean, var = (f32(p) for p in params)
            scale = gamma / np.sqrt(var + eps)
            oc = w.shape[0]
            w_fold = w * scale.reshape((oc,) + (1,) * (w.ndim - 1))
            has_bias = len(conv.inputs) > 2 and conv.inputs[2]
            b_conv = f32(conv.inputs[2]) if has_bias else np.zeros(oc, dtype=np.float32)
            b_fold = b_conv * scale + (beta - mean * scale)

            wn = fresh(w_name + "_bnfold")
            bname = fresh((conv.name or "conv") + "_bias_bnfold")
            graph.set_initializer(wn, w_fold)
            graph.set_initializer(bname, b_fold)
            conv.inputs = [conv.inputs[0], wn, bname]
            conv.outputs = [bn.outputs[0]]
            graph.remove_nodes([bn])
            changed = True
        return changed
