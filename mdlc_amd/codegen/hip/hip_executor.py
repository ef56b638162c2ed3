"""Run a ``HipModule`` on one MI355X: one arena, one stream, one C++ plan.

Replaces the reference's ``GpuExecutor`` (mdlc/codegen/cuda/gpu_executor.py:
26-114). Differences that matter on the device:

* Memory is one ``hipMalloc`` arena laid out at construction: constants
  (weights and packed device layouts), runtime inputs, the planner's pooled
  activation buffers at their 256-byte-aligned offsets, and one scratch
  region shared by every column matrix (column matrices are used strictly in
  stream order, so they never overlap in time). Weights are uploaded once.
* The launch loop is the C++ plan runner of libmdlc_hip.so (optionally a
  captured hipGraph); Python only packs it once.
* No host fallbacks: every launch is a device kernel.

``run(feeds, timing=False)`` returns ``{"outputs": ..., "ms": ...}`` like the
reference. ``run_all`` returns every tensor the plan produces (launch by
launch, read back after each), and ``run_isolated`` runs each launch group on
externally supplied inputs, so a single group's error can be told apart from
drift accumulated along the chain.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from mdlc_amd.codegen.hip.abi import check_launch, declared_kinds
from mdlc_amd.codegen.hip.emit import HipModule, Launch
from mdlc_amd.codegen.hip.hiprtc_runtime import (STATIC_SCRATCH_BYTES, Arg, HipContext, HipError, Plan,
                                                 compile_code_object)
from mdlc_amd.ir import DType
from mdlc_amd.runtime.memory_planner import align_up, plan_memory


@dataclass
class ArenaLayout:
    """Byte offsets of every tensor in the executor's one allocation:
    constants (sorted by name), runtime inputs, the planner's pooled buffers,
    then one scratch region per class (or, with ``static_scratch``, offsets
    into the separate workspace in ``ws_offsets``)."""
    mem_plan: object
    offsets: dict = field(default_factory=dict)
    shapes: dict = field(default_factory=dict)
    dtypes: dict = field(default_factory=dict)
    ws_offsets: dict = field(default_factory=dict)
    ws_bytes: int = 0
    arena_bytes: int = 0
    constants: dict = field(default_factory=dict)

    def nbytes(self, name: str) -> int:
        return int(np.prod(self.shapes[name], dtype=np.int64)) * np.dtype(self.dtypes[name]).itemsize


def arena_layout(module: HipModule, *, static_scratch: bool = False) -> ArenaLayout:
    """The arena layout ``HipExecutor`` allocates for ``module`` (no device
    needed)."""
    g = module.graph
    lay = ArenaLayout(plan_memory(g))
    cur = 0
    const_vals: dict = {}
    for l in module.plan:
        for e in l.inputs:
            if e in module.device_constants:
                const_vals[e] = module.device_constants[e]
            elif g.is_constant(e):
                const_vals[e] = np.asarray(g.initializers[e])
    for name in sorted(const_vals):
        arr = np.ascontiguousarray(const_vals[name])
        lay.constants[name] = arr
        lay.offsets[name] = cur
        lay.shapes[name], lay.dtypes[name] = arr.shape, arr.dtype
        cur += align_up(arr.nbytes)
    for name in g.runtime_inputs:
        info = g.info(name)
        lay.offsets[name] = cur
        lay.shapes[name] = tuple(info.shape)
        lay.dtypes[name] = DType.to_numpy(info.dtype)
        cur += align_up(info.nbytes())
    act_base = cur
    for t, bid in lay.mem_plan.assignment.items():
        info = g.info(t)
        lay.offsets[t] = act_base + lay.mem_plan.offsets[bid]
        lay.shapes[t] = tuple(info.shape)
        lay.dtypes[t] = DType.to_numpy(info.dtype)
    cur = act_base + lay.mem_plan.arena_bytes
    regions: dict = {}
    for name, (r, ld) in module.scratch_shapes.items():
        cls = module.scratch_class.get(name, "cols")
        regions[cls] = max(regions.get(cls, 0), r * ld * 4)
    region_at: dict = {}
    ws = 0                                  # static mode: offsets within the workspace
    for cls in sorted(regions):
        if static_scratch:
            region_at[cls] = ws
            ws += align_up(regions[cls])
        else:
            region_at[cls] = cur
            cur += align_up(regions[cls])
    for name, (r, ld) in module.scratch_shapes.items():
        at = region_at[module.scratch_class.get(name, "cols")]
        if static_scratch:
            lay.ws_offsets[name] = at
        else:
            lay.offsets[name] = at
        lay.shapes[name], lay.dtypes[name] = (r, ld), np.dtype(np.float32)
    lay.ws_bytes = ws
    lay.arena_bytes = cur
    return lay


class HipExecutor:
    def __init__(self, module: HipModule, ctx: Optional[HipContext] = None, *,
                 use_graph: bool = False, use_cache: bool = True,
                 static_scratch: bool = False) -> None:
        """``static_scratch``: the scratch regions (split-K / stream-K
        workspace, column matrices) are not part of the arena; the plan runs
        through ``mdlc_plan_run_static`` on the library's per-GPU static
        scratch, so ``run`` allocates no device memory for them."""
        self.module = module
        self.static_scratch = static_scratch
        # every launch's arguments against its kernel's declaration, before
        # any device call
        self._declared = declared_kinds("\n".join(module.kernels.values()))
        for l in module.plan:
            check_launch(l.kernel_name, self._declared,
                         [a.kind for a in launch_args(l, lambda e: Arg.ptr(0))])
        self.ctx = ctx or HipContext()
        self.code = self.ctx.load_code(compile_code_object(module.sources(), arch=self.ctx.arch,
                                                           use_cache=use_cache))
        self.funcs = {name: self.code.func(name) for name in module.kernels}
        for l in module.plan:
            if l.kernel_name not in self.funcs:
                self.funcs[l.kernel_name] = self.code.func(l.kernel_name)

        # ---- arena layout ------------------------------------------------
        lay = arena_layout(module, static_scratch=static_scratch)
        self.mem_plan = lay.mem_plan
        self.offsets, self.shapes, self.dtypes = lay.offsets, lay.shapes, lay.dtypes
        self.ws_offsets, self.ws_bytes = lay.ws_offsets, lay.ws_bytes
        if static_scratch and self.ws_bytes > STATIC_SCRATCH_BYTES:
            raise HipError(f"the plan's workspace of {self.ws_bytes} bytes exceeds the static scratch "
                           f"of {STATIC_SCRATCH_BYTES} bytes; run it with the arena's workspace")
        self.arena_bytes = cur = lay.arena_bytes
        const_vals = lay.constants
        self.arena = self.ctx.malloc(max(cur, 256))
        self.base = int(self.arena.value)
        for name, arr in const_vals.items():
            self.ctx.htod(self.base + self.offsets[name], arr)

        self.launch_records = [self._record(l) for l in module.plan]
        self.plan = self._make_plan(self.launch_records)
        if use_graph:
            self.plan.use_graph(True)
        self._single: Optional[list] = None

    # ---- plan packing -----------------------------------------------------

    def ptr(self, name: str) -> int:
        if name not in self.offsets:
            raise HipError(f"tensor {name!r} has no arena slot")
        return self.base + self.offsets[name]

    def _make_plan(self, records: list) -> Plan:
        return Plan(records, (0, max(self.ws_bytes, 1)) if self.static_scratch else None)

    def _arg_ptr(self, e: str) -> Arg:
        if e in self.ws_offsets:
            return Arg.ws(self.ws_offsets[e])
        return Arg.ptr(self.ptr(e))

    def _record(self, l: Launch) -> tuple:
        args = launch_args(l, self._arg_ptr)
        check_launch(l.kernel_name, self._declared, [a.kind for a in args])
        return (self.funcs[l.kernel_name].value, l.grid, l.block, 0, args)

    # ---- execution ----------------------------------------------------------

    def _upload_feeds(self, feeds: dict) -> None:
        g = self.module.graph
        for name in g.runtime_inputs:
            if name not in feeds:
                raise HipError(f"missing feed {name!r}")
            arr = np.ascontiguousarray(feeds[name], dtype=self.dtypes[name])
            if tuple(arr.shape) != tuple(self.shapes[name]):
                raise HipError(f"feed {name!r} has shape {arr.shape}, compiled for {self.shapes[name]}")
            self.ctx.htod(self.ptr(name), arr)

    def _nhwc(self, name: str) -> bool:
        return (self.module.device_layout.get(name) == "NHWC" and len(self.shapes[name]) == 4)

    def read(self, name: str) -> np.ndarray:
        """A tensor's value in the IR's layout (channels-last device tensors
        are transposed back to NCHW)."""
        shp = tuple(self.shapes[name])
        if self._nhwc(name):
            n, c, h, w = shp
            dev = self.ctx.dtoh(self.ptr(name), (n, h, w, c), self.dtypes[name])
            return np.ascontiguousarray(dev.transpose(0, 3, 1, 2))
        return self.ctx.dtoh(self.ptr(name), shp, self.dtypes[name])

    def write(self, name: str, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtypes[name])
        if tuple(arr.shape) != tuple(self.shapes[name]):
            raise HipError(f"{name!r}: shape {arr.shape} != {self.shapes[name]}")
        if self._nhwc(name):
            arr = np.ascontiguousarray(arr.transpose(0, 2, 3, 1))
        self.ctx.htod(self.ptr(name), arr)

    def _run_plan(self, plan: Plan, iters: int = 1) -> None:
        if self.static_scratch:
            plan.run_static(iters)
        else:
            plan.run(iters)

    def run(self, feeds: dict, *, timing: bool = False, warmup: int = 3, iters: int = 10) -> dict:
        self._upload_feeds(feeds)
        self._run_plan(self.plan)
        self.ctx.synchronize()
        out = {"outputs": {o: self.read(o) for o in self.module.graph.outputs}}
        if timing:
            out["ms"] = (self.ctx.time_ms(lambda: self.plan.run_static(1), iters, warmup)
                         if self.static_scratch else self.plan.time_ms(warmup, iters))
        return out

    def _singles(self) -> list:
        if self._single is None:
            self._single = [self._make_plan([r]) for r in self.launch_records]
        return self._single

    def run_all(self, feeds: dict) -> dict:
        """Every tensor the plan writes (except scratch), read back right after
        the launch that produced it, so pooled buffers can be reused safely."""
        self._upload_feeds(feeds)
        env = {}
        for l, p in zip(self.module.plan, self._singles()):
            self._run_plan(p)
            self.ctx.synchronize()
            for o in l.outputs:
                if o not in self.module.scratch_shapes:
                    env[o] = self.read(o)
        return env

    def run_isolated(self, env: dict) -> dict:
        """Run each launch group on the tensors in ``env`` (e.g. the oracle's
        values of its inputs) and return what each group wrote."""
        got = {}
        groups: list = []                       # (the nodes a group computes, its launches)
        for i, l in enumerate(self.module.plan):
            node = l.meta.get("node")
            nodes = ([l.meta["first"].meta["node"], l.meta["second"].meta["node"]]
                     if l.kind == "conv_pair" else [node])
            if groups and groups[-1][0][-1] is node and l.kind != "conv_pair":
                groups[-1][1].append(i)
            else:
                groups.append((nodes, [i]))
        singles = self._singles()
        consts = set(self.module.device_constants) | set(self.module.graph.initializers)
        for nodes, idxs in groups:
            for node in nodes:
                for e in node.real_inputs():
                    if e in env and e not in consts:
                        self.write(e, env[e])
            for i in idxs:
                self._run_plan(singles[i])
            self.ctx.synchronize()
            for node in nodes:
                for o in node.outputs:
                    if o:
                        got[o] = self.read(o)
        return got

    def profile(self, iters: int = 25) -> list:
        """[(launch, ms)]: each launch's kernel time from start and stop
        events attached to its own dispatch, the median over ``iters`` runs
        of the plan."""
        return list(zip(self.module.plan, self.plan.profile(iters)))

    def close(self) -> None:
        if getattr(self, "arena", None) is not None:
            self.plan.close()
            for p in self._single or []:
                p.close()
            self.ctx.free(self.arena)
            self.arena = None
            self.code.close()


def run_on_gpu(module: HipModule, feeds: dict, *, timing: bool = False) -> dict:
    ex = HipExecutor(module)
    try:
        return ex.run(feeds, timing=timing)
    finally:
        ex.close()


def launch_args(l: Launch, arg_ptr) -> list:
    """The packed argument list of one launch, in its kernel's ABI order.
    ``arg_ptr(tensor)`` gives the ``Arg`` for a tensor's device address (a
    pointer, or an offset into the plan's workspace)."""
    m = l.meta
    P = arg_ptr
    I = Arg.i32  # noqa: E741
    k = l.kind
    if k == "gemm":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m["M"]), I(m["N"]), I(m["K"]), I(m["lda"]), I(m["ldb"]), I(m["ldc"]),
                 I(m["hw"]), I(m["ksplit"]), I(m["kchunk"])]
    elif k == "gemm_ws":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m["M"]), I(m["N"]), I(m["K"]), I(m["lda"]), I(m["ldb"]), I(m["ldc"]),
                 I(m["kchunk"])]
    elif k == "conv_ws":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("M", "N", "K", "lda", "Cin", "H", "W", "OH", "OW", "ldc",
                                   "kchunk")]
    elif k == "conv_pair":
        args = launch_args(m["first"], arg_ptr) + launch_args(m["second"], arg_ptr)
        args += [I(m["g0"]), I(m["nb"])]
    elif k == "conv":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m["M"]), I(m["N"]), I(m["K"]), I(m["lda"]), I(m["Cin"]), I(m["H"]),
                 I(m["W"]), I(m["OH"]), I(m["OW"]), I(m["ksplit"]), I(m["kchunk"])]
    elif k == "gconv":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("M", "N", "K", "lda", "Cin", "H", "W", "OH", "OW", "ksplit",
                                   "kchunk", "ximg", "cimg")]
    elif k == "wino":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("N", "C", "H", "W", "OC", "OH", "OW", "TH", "TW", "CP", "OCP",
                                   "PT", "PL", "nchunk")]
    elif k == "conv_smallc":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("batch", "H", "W", "OC", "OH", "OW")]
    elif k == "conv_pool":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("batch", "H", "W", "OC", "OH")]
    elif k == "streamk_fixup":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("M", "N", "K", "full", "ldc", "hw")]
    elif k == "splitk_reduce":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m["S"]), I(m["M"]), I(m["N"]), I(m["ldc"]), I(m["hw"])]
    elif k == "im2col":
        args = [P(l.inputs[0]), P(l.outputs[0])]
        args += [I(m[f]) for f in ("C", "H", "W", "KH", "KW", "OH", "OW", "SH", "SW",
                                   "PH", "PW", "DH", "DW", "batch", "ldc")]
    elif k == "dwconv":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("N", "C", "H", "W", "OC", "OH", "OW", "PT", "PL")]
    elif k == "elementwise":
        args = [P(e) for e in l.inputs] + [P(o) for o in l.outputs] + [I(m["N"])]
    elif k in ("maxpool", "avgpool"):
        args = [P(l.inputs[0]), P(l.outputs[0])]
        args += [I(m[f]) for f in ("planes", "H", "W", "OH", "OW", "KH", "KW", "SH", "SW",
                                   "PT", "PL", "DH", "DW")]
    elif k == "gap":
        args = [P(l.inputs[0]), P(l.outputs[0]), I(m["planes"]), I(m["HW"])]
    elif k == "softmax":
        args = [P(l.inputs[0]), P(l.outputs[0])]
        args += ([Arg.i64(m["outer"]), I(m["L"])] if m["rows"] else
                 [Arg.i64(m["outer"]), I(m["L"]), I(m["inner"])])
    elif k == "transpose":
        args = [P(l.inputs[0]), P(l.outputs[0]), Arg.i64(m["total"]), Arg.dims6(m["out_dims"]),
                Arg.dims6(m["src_strides"])]
    elif k == "pad":
        args = [P(l.inputs[0]), P(l.outputs[0]), Arg.i64(m["total"]), Arg.dims6(m["out_dims"]),
                Arg.dims6(m["in_dims"]), Arg.dims6(m["before"], fill=0), Arg.f32(m["value"])]
    elif k == "concat":
        args = [P(l.inputs[0]), P(l.outputs[0])] + [Arg.i64(m[f]) for f in
                                                     ("rows", "run", "dst_stride", "dst_off")]
    elif k == "copy":
        args = [P(l.inputs[0]), P(l.outputs[0]), Arg.i64(m["nbytes"])]
    elif k == "quantize":
        args = [P(l.inputs[0]), P(l.outputs[0]), I(m["N"]), I(m["C"]), I(m["HW"]),
                Arg.f32(m["inv_s"])]
    elif k == "qgemm":
        args = [P(e) for e in l.inputs[:4]] + [P(l.outputs[0])]
        args += [P(l.inputs[4]) if len(l.inputs) > 4 else Arg.ptr(0)]
        args += [I(m[f]) for f in ("M", "N", "K", "lda", "ldb", "ldc", "Cin", "H", "W", "OH", "OW")]
        args += [Arg.f32(m.get("res_mult", 0.0)), Arg.f32(m.get("acc_mult", 0.0))]
    elif k == "qconv_first":
        args = [P(l.inputs[0]), Arg.f32(m["inv_s"])] + [P(e) for e in l.inputs[1:4]]
        args += [P(l.inputs[4]) if len(l.inputs) > 4 else Arg.ptr(0), P(l.outputs[0])]
        args += [I(m[f]) for f in ("N", "H", "W", "OH", "OW")]
    elif k == "qmlp":
        args = [P(e) for e in l.inputs]
        if not m["mixer"]:                     # no token mixer: null Wd, bd, md
            args[1:1] = [Arg.ptr(0)] * 3
        args += [P(l.outputs[0]), I(m["M"]), I(m["H"]), I(m["W"]), Arg.f32(m["res_mult"]),
                 Arg.f32(m["acc_mult"])]
    elif k == "qdwconv":
        args = [P(e) for e in l.inputs] + [P(l.outputs[0])]
        args += [I(m[f]) for f in ("N", "C", "H", "W", "OH", "OW", "PT", "PL")]
    elif k == "qadd":
        args = [P(l.inputs[0]), P(l.inputs[1]), P(l.outputs[0]), Arg.i64(m["n"]),
                Arg.f32(m["ma"]), Arg.f32(m["mb"])]
    elif k == "qlut":
        args = [P(l.inputs[0]), P(l.inputs[1]), P(l.outputs[0]), Arg.i64(m["n"])]
    elif k == "qgap":
        args = [P(l.inputs[0]), P(l.outputs[0]), I(m["N"]), I(m["C"]), I(m["HW"]),
                Arg.f32(m["m"])]
    elif k == "dequantize":
        args = [P(l.inputs[0]), P(l.outputs[0]), Arg.i64(m["n"]), I(m["C"]), I(m["HW"]),
                Arg.f32(m["s"])]
    else:
        raise HipError(f"launch kind {k!r} has no device implementation")
    return args
