"""LSUV-style weight calibration for the synthetic benchmark models.

Follows the reference exporters' ``lsuv_calibrate`` (mdlc/tools/
export_utils.py:16-50): one forward pass over a seeded dummy input, in graph
order; after each Conv / Gemm its weight and bias are divided by the observed
output standard deviation (and the output with them), so every such layer
emits ~unit-std activations and downstream layers calibrate against already
calibrated inputs. Without it, random-init residual networks grow their
activations to |x| ~ 100-500 by the last stage, where an absolute tolerance
of 1e-5 is below float32 resolution and parity checks lose their meaning.

Runs once at model-build time on the CPU with torch (as the reference's
exporters do); it is not part of the compile or execution path.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph


def lsuv_calibrate(g: Graph, dummy: dict, *, target_std: float = 1.0, eps: float = 1e-8) -> Graph:
    import torch
    import torch.nn.functional as F

    from mdlc_amd.passes.shape_inference import resolve_pads

    env = {k: torch.from_numpy(np.asarray(v, np.float32)) for k, v in g.initializers.items()}
    env.update({k: torch.from_numpy(np.asarray(v, np.float32)) for k, v in dummy.items()})

    def rescale(node, y, wname, bname):
        std = float(y.std())
        if std < eps:
            return y
        s = std / target_std
        g.set_initializer(wname, (np.asarray(g.initializers[wname], np.float32) / np.float32(s)))
        env[wname] = torch.from_numpy(g.initializers[wname])
        if bname:
            g.set_initializer(bname, (np.asarray(g.initializers[bname], np.float32) / np.float32(s)))
            env[bname] = torch.from_numpy(g.initializers[bname])
        return y / s

    with torch.no_grad():
        for node in g.topo_sort():
            a = node.attrs
            ins = [env[e] if e else None for e in node.inputs]
            op = node.op_type
            if op == "Conv":
                x, w = ins[0], ins[1]
                b = ins[2] if len(ins) > 2 else None
                kh, kw = w.shape[2:]
                st = a.get("strides", [1, 1])
                dl = a.get("dilations", [1, 1])
                (pt, pb), (pl, pr) = resolve_pads(a.get("auto_pad", "NOTSET"), a.get("pads"),
                                                  x.shape[2:], (kh, kw), st, dl)
                y = F.conv2d(F.pad(x, (pl, pr, pt, pb)), w, b, stride=tuple(st), dilation=tuple(dl),
                             groups=a.get("group", 1))
                y = rescale(node, y, node.inputs[1], node.inputs[2] if len(node.inputs) > 2 else "")
            elif op == "Gemm":
                x, w = ins[0], ins[1]
                y = x @ (w.T if a.get("transB", 0) else w)
                if len(ins) > 2 and ins[2] is not None:
                    y = y + ins[2]
                y = rescale(node, y, node.inputs[1], node.inputs[2] if len(node.inputs) > 2 else "")
            elif op == "BatchNormalization":
                y = F.batch_norm(ins[0], ins[3], ins[4], ins[1], ins[2], training=False,
                                 eps=a.get("epsilon", 1e-5))
            elif op == "Relu":
                y = torch.relu(ins[0])
            elif op == "Clip":
                lo = float(ins[1]) if len(ins) > 1 and ins[1] is not None else None
                hi = float(ins[2]) if len(ins) > 2 and ins[2] is not None else None
                y = torch.clamp(ins[0], lo, hi)
            elif op == "Add":
                y = ins[0] + ins[1]
            elif op == "MaxPool":
                y = F.max_pool2d(F.pad(ins[0], (a["pads"][1], a["pads"][3], a["pads"][0], a["pads"][2]),
                                       value=-float("inf")),
                                 a["kernel_shape"], a.get("strides", [1, 1]))
            elif op == "GlobalAveragePool":
                y = ins[0].mean(dim=(2, 3), keepdim=True)
            elif op == "Flatten":
                y = ins[0].reshape(ins[0].shape[0], -1)
            elif op == "Identity":
                y = ins[0]
            elif op == "Constant":
                y = torch.as_tensor(np.asarray(a["value"], np.float32))
            else:
                raise NotImplementedError(f"calibration: op {op!r}")
            env[node.outputs[0]] = y
    return g
