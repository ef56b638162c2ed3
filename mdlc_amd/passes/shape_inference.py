"""Static shape inference by per-op rules.

The reference infers shapes by running its NumPy executor once on dummy
feeds (mdlc/passes/shape_inference.py:36-50). Here every op has a shape rule,
so compiling a batch-32 graph costs no CPU forward pass; the rules are
checked against the NumPy executor's actual shapes in the test suite.
``make_dummy_feeds`` keeps the reference's seeded feed recipe
(shape_inference.py:19-33): seed 0, standard normal for floats, {0,1} for
integers, symbolic dims bound to ``batch``.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

from mdlc_amd.ir import DType, Graph, Node, TensorInfo


def make_dummy_feeds(graph: Graph, batch: int = 1, seed: int = 0) -> dict:
    rng = np.random.default_rng(seed)
    feeds = {}
    for name in graph.runtime_inputs:
        info = graph.info(name)
        if info is None or not info.shape:
            raise ValueError(f"input {name!r} has no shape; cannot fabricate")
        shape = [int(d) if isinstance(d, (int, np.integer)) and d >= 0 else batch
                 for d in info.shape]
        dt = DType.to_numpy(info.dtype)
        if np.issubdtype(dt, np.integer):
            feeds[name] = rng.integers(0, 2, size=shape).astype(dt)
        else:
            feeds[name] = rng.standard_normal(shape).astype(dt)
    return feeds


# ----- window geometry ----------------------------------------------------

def resolve_pads(auto_pad: str, pads, in_hw, k_hw, s_hw, d_hw):
    """((top, bottom), (left, right)) padding, honouring ONNX ``auto_pad``
    (same rule as mdlc/runtime/ops.py:15-32)."""
    if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        res = []
        for i, k, s, d in zip(in_hw, k_hw, s_hw, d_hw):
            o = -(-i // s)
            total = max(0, (o - 1) * s + (k - 1) * d + 1 - i)
            small, big = total // 2, total - total // 2
            res.append((small, big) if auto_pad == "SAME_UPPER" else (big, small))
        return tuple(res)
    if pads is None:
        return (0, 0), (0, 0)
    return (int(pads[0]), int(pads[2])), (int(pads[1]), int(pads[3]))


def window_out(size: int, lo: int, hi: int, k: int, s: int, d: int, ceil_mode: int = 0) -> int:
    span = size + lo + hi - (d * (k - 1) + 1)
    return (-(-span // s) if ceil_mode else span // s) + 1


def conv_geometry(node: Node, x_shape, w_shape) -> dict:
    """Every integer a conv kernel needs, from attrs and operand shapes."""
    n, c, h, w = (int(v) for v in x_shape)
    oc, icg, kh, kw = (int(v) for v in w_shape)
    a = node.attrs
    sh, sw = (int(v) for v in a.get("strides", [1, 1]))
    dh, dw = (int(v) for v in a.get("dilations", [1, 1]))
    (pt, pb), (pl, pr) = resolve_pads(a.get("auto_pad", "NOTSET"), a.get("pads"),
                                      (h, w), (kh, kw), (sh, sw), (dh, dw))
    oh = window_out(h, pt, pb, kh, sh, dh)
    ow = window_out(w, pl, pr, kw, sw, dw)
    return dict(N=n, C=c, H=h, W=w, OC=oc, ICG=icg, KH=kh, KW=kw, SH=sh, SW=sw,
                DH=dh, DW=dw, PT=pt, PB=pb, PL=pl, PR=pr, OH=oh, OW=ow,
                group=int(a.get("group", 1)))


# ----- per-op rules -----------------------------------------------------------

def _broadcast(*shapes):
    return tuple(np.broadcast_shapes(*[tuple(s) for s in shapes]))


def _pool_shape(node: Node, xs, ceil_key=True, dil=True):
    a = node.attrs
    kh, kw = a["kernel_shape"]
    sh, sw = a.get("strides", [1, 1])
    dh, dw = a.get("dilations", [1, 1]) if dil else (1, 1)
    (pt, pb), (pl, pr) = resolve_pads(a.get("auto_pad", "NOTSET"), a.get("pads"),
                                      xs[2:], (kh, kw), (sh, sw), (dh, dw))
    cm = a.get("ceil_mode", 0) if ceil_key else 0
    return (xs[0], xs[1], window_out(xs[2], pt, pb, kh, sh, dh, cm),
            window_out(xs[3], pl, pr, kw, sw, dw, cm))


def node_output_infos(node: Node, shape_of, dtype_of, const_of) -> list:
    """[(shape, dtype)] per output of ``node``. ``shape_of``/``dtype_of`` map
    an edge name to its shape/dtype; ``const_of`` returns a constant's array
    or None."""
    op = node.op_type
    a = node.attrs
    ins = node.inputs
    s0 = shape_of(ins[0]) if ins and ins[0] else None
    d0 = dtype_of(ins[0]) if ins and ins[0] else DType.FLOAT32

    if op in ("Conv", "FusedConvAct", "FusedConvBNAct", "QConv"):
        g = conv_geometry(node, s0, shape_of(ins[1]))
        dt = DType.INT8 if op == "QConv" else d0
        if a.get("maxpool"):             # a folded max pool: the pooled output
            return [(_pool_shape(Node("MaxPool", [], [], dict(a["maxpool"])),
                                 (g["N"], g["OC"], g["OH"], g["OW"])), dt)]
        return [((g["N"], g["OC"], g["OH"], g["OW"]), dt)]
    if op == "QMlp":                 # [token mixer,] two 1x1 QConvs C -> E -> C, residual
        return [((s0[0], shape_of(ins[-3])[0]) + tuple(s0[2:]), DType.INT8)]
    if op in ("Gemm", "FusedGemmAct", "QGemm"):
        sa, sb = shape_of(ins[0]), shape_of(ins[1])
        m = sa[1] if a.get("transA", 0) else sa[0]
        nn = sb[0] if a.get("transB", 0) else sb[1]
        if op == "QGemm":
            od = a.get("out_dtype", "int8")
            return [((m, nn), {"float32": DType.FLOAT32, "int32": DType.INT32}.get(od, DType.INT8))]
        return [((m, nn), d0)]
    if op == "MatMul":
        sa, sb = shape_of(ins[0]), shape_of(ins[1])
        return [(np.matmul(np.empty(sa, np.float32), np.empty(sb, np.float32)).shape, d0)]
    if op in ("MaxPool",):
        return [(_pool_shape(node, s0), d0)]
    if op == "AveragePool":
        return [(_pool_shape(node, s0, dil=False), d0)]
    if op in ("GlobalAveragePool", "QGlobalAveragePool"):
        if a.get("flatten"):                 # a folded Flatten(axis=1)
            return [(tuple(s0[:2]), d0)]
        return [(tuple(s0[:2]) + (1,) * (len(s0) - 2), d0)]
    if op in ("BatchNormalization", "Relu", "Sigmoid", "Tanh", "HardSwish", "HardSigmoid",
              "LeakyRelu", "Clip", "Softmax", "Identity", "QLut"):
        return [(tuple(s0), d0)]
    if op in ("Add", "Sub", "Mul", "Div"):
        return [(_broadcast(s0, shape_of(ins[1])), d0)]
    if op == "QAdd":
        return [(_broadcast(s0, shape_of(ins[1])), DType.INT8)]
    if op == "QuantizeLinear":
        return [(tuple(s0), DType.INT8)]
    if op == "DequantizeLinear":
        return [(tuple(s0), DType.FLOAT32)]
    if op == "Flatten":
        ax = int(a.get("axis", 1))
        ax = ax + len(s0) if ax < 0 else ax
        lead = int(np.prod(s0[:ax])) if ax > 0 else 1
        return [((lead, int(np.prod(s0[ax:]))), d0)]
    if op == "Reshape":
        tgt = const_of(ins[1])
        if tgt is None:
            raise ValueError(f"Reshape {node.name!r}: target shape is not constant")
        tgt = [int(v) for v in np.asarray(tgt).ravel()]
        tgt = [s0[i] if v == 0 else v for i, v in enumerate(tgt)]
        return [(np.empty(s0, np.int8).reshape(tgt).shape, d0)]
    if op == "Transpose":
        perm = a.get("perm") or list(range(len(s0)))[::-1]
        return [(tuple(s0[p] for p in perm), d0)]
    if op == "Concat":
        parts = [shape_of(e) for e in ins if e]
        ax = int(a.get("axis", 0))
        ax = ax + len(parts[0]) if ax < 0 else ax
        out = list(parts[0])
        out[ax] = sum(p[ax] for p in parts)
        return [(tuple(out), d0)]
    if op in ("Squeeze", "Unsqueeze"):
        axes = const_of(ins[1]) if len(ins) > 1 and ins[1] else a.get("axes")
        x = np.empty(s0, np.int8)
        if op == "Squeeze":
            x = np.squeeze(x) if axes is None else np.squeeze(
                x, axis=tuple(int(v) for v in np.asarray(axes).ravel()))
        else:
            for ax in sorted(int(v) for v in np.asarray(axes).ravel()):
                x = np.expand_dims(x, ax)
        return [(x.shape, d0)]
    if op == "Pad":
        pads = const_of(ins[1]) if len(ins) > 1 and ins[1] else a.get("pads")
        pads = [int(v) for v in np.asarray(pads).ravel()]
        half = len(pads) // 2
        return [(tuple(s0[i] + pads[i] + pads[i + half] for i in range(half)), d0)]
    if op == "Shape":
        return [((len(s0),), DType.INT64)]
    if op == "Constant":
        v = np.asarray(a["value"])
        return [(v.shape, DType.from_numpy(v.dtype))]
    if op == "FusedElementwise":
        local_shape, local_dt = {}, {}
        sub_shape = lambda e: local_shape[e] if e in local_shape else shape_of(e)  # noqa: E731
        sub_dt = lambda e: local_dt[e] if e in local_dt else dtype_of(e)  # noqa: E731
        for sn in a["subgraph"]:
            for o, (shp, dt) in zip(sn.outputs, node_output_infos(sn, sub_shape, sub_dt, const_of)):
                local_shape[o], local_dt[o] = tuple(shp), dt
        return [(local_shape[o], local_dt[o]) for o in node.outputs]
    raise NotImplementedError(f"shape inference: no rule for {op!r}")


def infer_shapes(graph: Graph, feeds: Optional[dict] = None, *, batch: int = 1) -> Graph:
    """Fill ``graph.value_info`` with static shapes for every edge.

    Runtime input shapes come from ``feeds`` when given, else from the
    declared input shapes with symbolic dims bound to ``batch``.
    """
    shapes: dict = {}
    dtypes: dict = {}
    for name, arr in graph.initializers.items():
        shapes[name] = tuple(arr.shape)
        dtypes[name] = DType.from_numpy(arr.dtype)
    for name in graph.runtime_inputs:
        if feeds is not None and name in feeds:
            arr = np.asarray(feeds[name])
            shapes[name] = tuple(arr.shape)
            dtypes[name] = DType.from_numpy(arr.dtype)
        else:
            info = graph.info(name)
            shapes[name] = tuple(int(d) if isinstance(d, (int, np.integer)) and d >= 0 else batch
                                 for d in info.shape)
            dtypes[name] = info.dtype
    const_of = graph.initializers.get
    for node in graph.topo_sort():
        infos = node_output_infos(node, lambda e: shapes[e], lambda e: dtypes[e], const_of)
        for o, (shp, dt) in zip(node.outputs, infos):
            if o:
                shapes[o] = tuple(int(d) for d in shp)
                dtypes[o] = dt
    for name in shapes:
        graph.set_info(TensorInfo(name, dtypes[name], shapes[name]))
    return graph


# The reference's name for the same step; shapes come from rules here.
infer_shapes_by_execution = infer_shapes
