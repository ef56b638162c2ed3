"""Compile-time evaluation of nodes whose inputs are all constants.

Constant folding needs to compute a node's value when every input is an
initializer. The reference does this by calling its NumPy executor
(mdlc/passes/constant_folding.py:30-56). This module is the compiler's own
small evaluator for the shape/constant plumbing that exported graphs carry
(Constant, Identity, Shape, Reshape, Squeeze/Unsqueeze, Concat, Transpose,
Cast-free arithmetic on small constants). It never sees a runtime tensor:
anything it does not know raises ``NotImplementedError`` and the node is left
for the device.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Node


def _axes(node: Node, vals: list, idx: int):
    if len(vals) > idx and vals[idx] is not None:
        return [int(a) for a in np.asarray(vals[idx]).ravel()]
    a = node.attrs.get("axes")
    return None if a is None else [int(v) for v in a]


def evaluate(node: Node, vals: list) -> list:
    """Values of ``node``'s outputs given constant input arrays ``vals``
    (``None`` for omitted optional inputs)."""
    op = node.op_type
    a = node.attrs
    if op == "Constant":
        return [np.asarray(a["value"])]
    if op == "Identity":
        return [vals[0]]
    if op == "Shape":
        return [np.array(np.shape(vals[0]), dtype=np.int64)]
    if op in ("Add", "Sub", "Mul", "Div"):
        x, y = vals[0], vals[1]
        if op == "Add":
            return [x + y]
        if op == "Sub":
            return [x - y]
        if op == "Mul":
            return [x * y]
        return [x / y]
    if op == "Reshape":
        x = vals[0]
        tgt = [int(s) for s in np.asarray(vals[1]).ravel()]
        shape = [x.shape[i] if s == 0 else s for i, s in enumerate(tgt)]
        return [x.reshape(shape)]
    if op == "Flatten":
        x = vals[0]
        ax = int(a.get("axis", 1))
        ax = ax + x.ndim if ax < 0 else ax
        lead = int(np.prod(x.shape[:ax])) if ax > 0 else 1
        return [x.reshape(lead, -1)]
    if op == "Transpose":
        return [np.transpose(vals[0], a.get("perm"))]
    if op == "Concat":
        return [np.concatenate([v for v in vals if v is not None], axis=int(a.get("axis", 0)))]
    if op == "Squeeze":
        axes = _axes(node, vals, 1)
        return [np.squeeze(vals[0]) if axes is None else np.squeeze(vals[0], axis=tuple(axes))]
    if op == "Unsqueeze":
        x = vals[0]
        for ax in sorted(_axes(node, vals, 1)):
            x = np.expand_dims(x, ax)
        return [x]
    raise NotImplementedError(f"no compile-time evaluation for {op!r}")
