"""NumPy reference executor — oracle restatement of mdlc/runtime/reference.py.

Test infrastructure only (see ``oracle/__init__.py``). Executes an
``mdlc_amd.ir.Graph`` node by node in a dependency order of its own (any
valid order gives the same values) and returns the graph outputs, or every
edge value with ``return_all=True`` — the per-tensor oracle.
"""

from __future__ import annotations

import numpy as np

from oracle import ops, quant


def act(name, x, attrs):
    """reference.py:19-38 — the activation table shared by fused and bare ops."""
    if not name or name == "Identity":
        return x
    if name == "Relu":
        return ops.relu(x)
    if name == "Clip":
        return ops.clip(x, attrs.get("clip_min"), attrs.get("clip_max"))
    if name == "Relu6":
        return ops.clip(x, 0.0, 6.0)
    if name == "Sigmoid":
        return ops.sigmoid(x)
    if name == "Tanh":
        return ops.tanh(x)
    if name == "LeakyRelu":
        return ops.leaky_relu(x, attrs.get("alpha", 0.01))
    if name == "HardSigmoid":
        return ops.hard_sigmoid(x, attrs.get("alpha", 0.2), attrs.get("beta", 0.5))
    if name == "HardSwish":
        return ops.hard_swish(x)
    raise NotImplementedError(f"activation {name!r} not implemented")


def _conv_kw(a):
    return dict(strides=a.get("strides", [1, 1]), pads=a.get("pads"),
                dilations=a.get("dilations", [1, 1]), group=a.get("group", 1),
                auto_pad=a.get("auto_pad", "NOTSET"))


def _gemm_kw(a):
    return dict(alpha=a.get("alpha", 1.0), beta=a.get("beta", 1.0),
                transA=a.get("transA", 0), transB=a.get("transB", 0))


class ReferenceExecutor:
    def __init__(self, graph) -> None:
        self.graph = graph

    def _order(self):
        g = self.graph
        ready = set(g.inputs) | set(g.initializers)
        todo = list(g.nodes)
        out = []
        while todo:
            rest = []
            for n in todo:
                if all(e in ready for e in n.inputs if e):
                    out.append(n)
                    ready.update(o for o in n.outputs if o)
                else:
                    rest.append(n)
            if len(rest) == len(todo):
                raise ValueError("graph has a cycle or dangling dependency")
            todo = rest
        return out

    def run(self, feeds, *, return_all=False):
        """reference.py:47-70."""
        env = {k: np.asarray(v) for k, v in self.graph.initializers.items()}
        env.update({k: np.asarray(v) for k, v in feeds.items()})
        for node in self._order():
            for name, val in zip(node.outputs, self.exec_node(node, env)):
                if name:
                    env[name] = val
        return env if return_all else {o: env[o] for o in self.graph.outputs}

    def exec_node(self, node, env):
        """reference.py:80-184 plus the build-defined quantized ops."""
        op = node.op_type
        a = node.attrs
        ins = [env[e] if e else None for e in node.inputs]
        opt = lambda i: ins[i] if len(ins) > i else None  # noqa: E731

        if op in ("Conv", "FusedConvAct", "FusedConvBNAct") and a.get("residual_subgraph"):
            # backend residual fusion: the folded FusedElementwise group runs on
            # the conv's output exactly as it did unfused
            local = dict(env)
            local[a["residual_from"]] = act(a.get("activation"),
                                            ops.conv(ins[0], ins[1], opt(2), **_conv_kw(a)), a)
            for sn in a["residual_subgraph"]:
                for name, val in zip(sn.outputs, self.exec_node(sn, local)):
                    if name:
                        local[name] = val
            return [local[node.outputs[0]]]
        if op in ("Conv", "FusedConvAct", "FusedConvBNAct") and a.get("maxpool"):
            # backend pool fold: the conv (and its activation), then the max
            # pool the reference ran as its own host op (ops.py:109-125)
            mp = a["maxpool"]
            y = act(a.get("activation"), ops.conv(ins[0], ins[1], opt(2), **_conv_kw(a)), a)
            return [ops.maxpool(y, kernel=mp["kernel_shape"], strides=mp["strides"], pads=mp["pads"],
                                dilations=[1, 1], auto_pad="NOTSET", ceil_mode=0)]
        if op in ("FusedConvAct", "FusedConvBNAct"):
            return [act(a.get("activation"), ops.conv(ins[0], ins[1], opt(2), **_conv_kw(a)), a)]
        if op == "FusedGemmAct":
            return [act(a.get("activation"), ops.gemm(ins[0], ins[1], opt(2), **_gemm_kw(a)), a)]
        if op == "FusedElementwise":
            local = dict(env)
            for sn in a["subgraph"]:
                for name, val in zip(sn.outputs, self.exec_node(sn, local)):
                    if name:
                        local[name] = val
            return [local[o] for o in node.outputs]

        if op == "Conv":
            return [ops.conv(ins[0], ins[1], opt(2), **_conv_kw(a))]
        if op == "Gemm":
            return [ops.gemm(ins[0], ins[1], opt(2), **_gemm_kw(a))]
        if op == "MatMul":
            return [ops.matmul(ins[0], ins[1])]
        if op == "BatchNormalization":
            return [ops.batchnorm(*ins[:5], epsilon=a.get("epsilon", 1e-5))]
        if op == "MaxPool":
            return [ops.maxpool(ins[0], kernel=a["kernel_shape"], strides=a.get("strides", [1, 1]),
                                pads=a.get("pads"), dilations=a.get("dilations", [1, 1]),
                                auto_pad=a.get("auto_pad", "NOTSET"),
                                ceil_mode=a.get("ceil_mode", 0))]
        if op == "AveragePool":
            return [ops.averagepool(ins[0], kernel=a["kernel_shape"],
                                    strides=a.get("strides", [1, 1]), pads=a.get("pads"),
                                    auto_pad=a.get("auto_pad", "NOTSET"),
                                    count_include_pad=a.get("count_include_pad", 0),
                                    ceil_mode=a.get("ceil_mode", 0))]
        if op == "GlobalAveragePool":
            y = ops.global_average_pool(ins[0])
            return [y.reshape(y.shape[:2]) if a.get("flatten") else y]
        if op in ("Relu", "Sigmoid", "Tanh", "HardSwish"):
            return [act(op, ins[0], a)]
        if op == "Clip":
            lo = opt(1) if opt(1) is not None else a.get("min")
            hi = opt(2) if opt(2) is not None else a.get("max")
            lo = None if lo is None else float(np.asarray(lo).item())
            hi = None if hi is None else float(np.asarray(hi).item())
            return [ops.clip(ins[0], lo, hi)]
        if op == "LeakyRelu":
            return [ops.leaky_relu(ins[0], a.get("alpha", 0.01))]
        if op == "HardSigmoid":
            return [ops.hard_sigmoid(ins[0], a.get("alpha", 0.2), a.get("beta", 0.5))]
        if op == "Softmax":
            return [ops.softmax(ins[0], a.get("axis", -1))]
        if op == "Add":
            return [ins[0] + ins[1]]
        if op == "Sub":
            return [ins[0] - ins[1]]
        if op == "Mul":
            return [ins[0] * ins[1]]
        if op == "Div":
            return [ins[0] / ins[1]]
        if op == "Flatten":
            return [ops.flatten(ins[0], a.get("axis", 1))]
        if op == "Reshape":
            return [ops.reshape(ins[0], ins[1])]
        if op == "Transpose":
            return [np.transpose(ins[0], a.get("perm"))]
        if op == "Concat":
            return [np.concatenate([x for x in ins if x is not None], axis=a.get("axis", 0))]
        if op in ("Squeeze", "Unsqueeze"):
            axes = opt(1) if opt(1) is not None else a.get("axes")
            if op == "Squeeze":
                if axes is None:
                    return [np.squeeze(ins[0])]
                return [np.squeeze(ins[0], axis=tuple(int(v) for v in np.asarray(axes).ravel()))]
            x = ins[0]
            for ax in sorted(int(v) for v in np.asarray(axes).ravel()):
                x = np.expand_dims(x, ax)
            return [x]
        if op == "Pad":
            pads = opt(1) if opt(1) is not None else a.get("pads")
            val = opt(2) if opt(2) is not None else a.get("value", 0.0)
            return [ops.pad(ins[0], pads, float(np.asarray(val).item()), a.get("mode", "constant"))]
        if op == "Constant":
            return [a["value"]]
        if op == "Identity":
            return [ins[0]]
        if op == "Shape":
            return [np.array(ins[0].shape, dtype=np.int64)]

        # ---- build-defined INT8 ops (oracle/quant.py) ----
        if op == "QuantizeLinear":
            return [quant.quantize(ins[0], a["inv_scale"])]
        if op == "DequantizeLinear":
            return [quant.dequantize(ins[0], a["scale"])]
        if op == "QConv":
            if a.get("quantize_input") is not None:      # a folded QuantizeLinear
                ins = [quant.quantize(ins[0], a["quantize_input"])] + list(ins[1:])
            acc = quant.conv_acc(ins[0], ins[1], opt(2), strides=a.get("strides", [1, 1]),
                                 pads=a.get("pads"), dilations=a.get("dilations", [1, 1]),
                                 group=a.get("group", 1))
            lo = 0 if a.get("activation") == "Relu" else quant.QMIN
            q = quant.requant(acc, ins[3].reshape(1, -1, 1, 1), lo)
            # fused epilogues: the composition of the unfused QLut / QAdd
            if a.get("epilogue") == "lut":
                return [quant.lut(q, ins[4])]
            if a.get("epilogue") == "add":
                return [quant.qadd(ins[4], q, a["res_mult"], a["acc_mult"])]
            return [q]
        if op == "QMlp":
            # the composition it folds: [a depthwise stride-1 QConv token
            # mixer,] QConv 1x1 + lookup, then QConv 1x1 + residual add of the
            # first 1x1 conv's input
            if a.get("mixer"):
                mx = a["mixer"]
                lod = 0 if mx.get("activation") == "Relu" else quant.QMIN
                xm = quant.requant(quant.conv_acc(ins[0], ins[1], ins[2], strides=[1, 1], pads=mx["pads"],
                                                  dilations=[1, 1], group=ins[0].shape[1]),
                                   ins[3].reshape(1, -1, 1, 1), lod)
                ins = [xm] + list(ins[4:])
            one = dict(strides=[1, 1], pads=[0, 0, 0, 0], dilations=[1, 1], group=1)
            lo1 = 0 if a.get("activation1") == "Relu" else quant.QMIN
            lo2 = 0 if a.get("activation2") == "Relu" else quant.QMIN
            h = quant.lut(quant.requant(quant.conv_acc(ins[0], ins[1], ins[2], **one),
                                        ins[3].reshape(1, -1, 1, 1), lo1), ins[4])
            q = quant.requant(quant.conv_acc(h, ins[5], ins[6], **one), ins[7].reshape(1, -1, 1, 1), lo2)
            return [quant.qadd(ins[0], q, a["res_mult"], a["acc_mult"])]
        if op == "QGemm":
            acc = quant.gemm_acc(ins[0], ins[1], opt(2))
            if a.get("out_dtype", "int8") == "int32":
                return [acc]
            if a.get("out_dtype", "int8") == "float32":
                return [acc.astype(np.float32) * ins[3].astype(np.float32)[None, :]]
            lo = 0 if a.get("activation") == "Relu" else quant.QMIN
            return [quant.requant(acc, ins[3][None, :], lo)]
        if op == "QAdd":
            return [quant.qadd(ins[0], ins[1], a["ma"], a["mb"])]
        if op == "QLut":
            return [quant.lut(ins[0], ins[1])]
        if op == "QGlobalAveragePool":
            y = quant.global_avg_pool(ins[0], a["mult"])
            return [y.reshape(y.shape[:2]) if a.get("flatten") else y]

        raise NotImplementedError(f"reference executor: op {op!r} not implemented")


def run_reference(graph, feeds, **kw):
    return ReferenceExecutor(graph).run(feeds, **kw)


def run_groups_float64(graph, env32):
    """Every node of ``graph`` re-run in float64 on the float32 values of its
    inputs in ``env32`` (the float32 oracle's ``return_all`` environment,
    constants included; float32 inputs and constants are widened exactly).
    The result is each group's exact answer to the rounding of float64 for
    the same inputs the device's isolated run receives, so the float32
    oracle's own rounding error can be measured beside the device's. The ops
    of runtime/ops.py keep their inputs' dtype (NumPy promotes nothing to
    float32), so the same restatement runs in float64."""
    ex = ReferenceExecutor(graph)
    env64 = {k: (np.asarray(v, np.float64) if np.asarray(v).dtype == np.float32 else v)
             for k, v in env32.items()}
    out = {}
    for node in graph.nodes:
        for name, val in zip(node.outputs, ex.exec_node(node, env64)):
            if name:
                out[name] = val
    return out

