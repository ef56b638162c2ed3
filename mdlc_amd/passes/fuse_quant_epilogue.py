"""Fold an int8 table lookup or residual add into the QConv that feeds it.

The reference has no quantized path, so this pass has no counterpart there;
it plays the role ``FuseActivation`` plays for float graphs
(mdlc/passes/fuse_activation.py:17-94): work that would be a separate
memory-bound launch runs in the producing GEMM's epilogue instead.

* ``QConv -> QLut(table)``: the conv's requantized codes index the table
  in the epilogue. The fused QConv gets the table as a fifth input and
  ``epilogue="lut"``.
* ``QConv -> QAdd(r, .)`` (either operand order): the epilogue requantizes
  the conv output exactly as before and adds the residual ``r`` with the
  add's multipliers. The fused QConv gets ``r`` as a fifth input,
  ``epilogue="add"``, ``res_mult`` (the multiplier of ``r``) and
  ``acc_mult`` (the multiplier of the conv's codes).

Either rewrite fires only when the conv output has no other consumer and is
not a graph output, the conv is not grouped, and (for the add) ``r`` does
not depend on the conv. The fused semantics are the composition of the
unfused ops, so every remaining tensor keeps its value bit for bit.
"""

from __future__ import annotations

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass


def _descendants(graph: Graph, start: str) -> set:
    cons = graph.consumers()
    seen, stack = set(), [start]
    while stack:
        e = stack.pop()
        for n in cons.get(e, []):
            for o in n.outputs:
                if o and o not in seen:
                    seen.add(o)
                    stack.append(o)
    return seen


class FuseQuantEpilogue(Pass):
    name = "fuse_quant_epilogue"

    def run(self, graph: Graph) -> bool:
        changed = False
        for conv in list(graph.nodes):
            if conv.op_type != "QConv" or conv.attrs.get("epilogue") or int(conv.attrs.get("group", 1)) != 1:
                continue
            y = conv.outputs[0]
            if y in graph.outputs or graph.use_count().get(y, 0) != 1:
                continue
            (nxt,) = graph.consumers()[y]
            attrs = dict(conv.attrs)
            if nxt.op_type == "QLut" and graph.is_constant(nxt.inputs[1]):
                extra = nxt.inputs[1]
                attrs["epilogue"] = "lut"
            elif nxt.op_type == "QAdd" and nxt.inputs[0] != nxt.inputs[1]:
                side = 0 if nxt.inputs[0] == y else 1
                r = nxt.inputs[1 - side]
                if r in _descendants(graph, y):
                    continue
                mults = (nxt.attrs["ma"], nxt.attrs["mb"])
                extra = r
                attrs.update(epilogue="add", res_mult=float(mults[1 - side]),
                             acc_mult=float(mults[side]))
            else:
                continue
            fused = Node("QConv", list(conv.inputs[:4]) + [extra], list(nxt.outputs), attrs,
                         (conv.name or "QConv") + "+" + nxt.op_type,
                         list(conv.fused_from or ["QConv"]) + [nxt.op_type])
            graph.nodes[graph.nodes.index(conv)] = fused
            graph.remove_nodes([nxt])
            changed = True
        return changed


# With this few input channels the channels-last byte gather of the int8
# conv kernels is at its least efficient; wider inputs keep the quantize
# launch and the GEMM conv.
MAX_FIRST_CIN = 4


class FuseInputQuantize(Pass):
    """Fold ``xq = QuantizeLinear(x)`` into the one QConv that reads it when
    that conv is small enough to quantize its own window (the first layer of
    an int8 network: float32 NCHW input with at most ``MAX_FIRST_CIN``
    channels, C*KH*KW <= 64, ungrouped, no dilation, at most 64 output
    channels and a multiple of 4, no epilogue or a lookup). The
    conv then takes ``x`` itself and ``attrs["quantize_input"]`` = the
    quantizer's ``inv_scale``; its value is the composition, bit for bit.
    Runs after shape inference."""
    name = "fuse_input_quantize"

    def run(self, graph: Graph) -> bool:
        changed = False
        for qn in list(graph.nodes):
            if qn.op_type != "QuantizeLinear":
                continue
            x, xq = qn.inputs[0], qn.outputs[0]
            xi = graph.info(x)
            if xi is None or len(xi.shape) != 4 or xi.dtype != "float32":
                continue
            if xq in graph.outputs or graph.use_count().get(xq, 0) != 1:
                continue
            (conv,) = graph.consumers()[xq]
            a = conv.attrs
            if conv.op_type != "QConv" or conv.inputs[0] != xq or a.get("epilogue") not in (None, "lut"):
                continue
            w = graph.initializers.get(conv.inputs[1])
            if w is None or int(a.get("group", 1)) != 1 or w.shape[0] % 4 or w.shape[0] > 64 \
                    or w.shape[1] > MAX_FIRST_CIN or w[0].size > 64:
                continue
            if any(int(d) != 1 for d in a.get("dilations", [1, 1])):
                continue
            attrs = dict(a, quantize_input=float(qn.attrs["inv_scale"]))
            fused = Node("QConv", [x] + list(conv.inputs[1:]), list(conv.outputs), attrs,
                         "QuantizeLinear+" + (conv.name or "QConv"),
                         ["QuantizeLinear"] + list(conv.fused_from or ["QConv"]))
            graph.nodes[graph.nodes.index(conv)] = fused
            graph.remove_nodes([qn])
            changed = True
        return changed


__all__ = ["FuseQuantEpilogue", "FuseInputQuantize"]
