"""Lower an optimized IR graph to a HIP module: kernel sources + launch plan.

Walks the fused graph in topological order, picks an MFMA schedule per GEMM
through ``schedule_fn(node, (M, N, K))``, instantiates the gfx950 templates
(deduplicating identical instantiations) and records an ordered plan of
``Launch`` records with concrete grid/block and edge bindings in kernel
argument order. The plan contract and field names follow
mdlc/codegen/cuda/emit.py:38-95 (``Launch``, ``CudaModule``); the kinds are
extended because nothing runs on the host here:

  gemm        dense GEMM + epilogue (Gemm/MatMul, and conv after im2col)
  gemm_ws     dense GEMM with the K range split over the waves of a workgroup
              (small M x N, deep K: one launch, no split-K workspace)
  conv        implicit-GEMM convolution (no column buffer)
  wino        3x3 stride-1 convolution by Winograd F(2x2, 3x3), transforms fused
  gconv       grouped convolution: the implicit GEMM with one grid row per group
  conv_smallc direct convolution for few input channels (stems): input patch
              in LDS, weights in registers, matrix cores
  im2col      batched column matrix for the explicit conv path
  dwconv      direct depthwise convolution + epilogue
  splitk_reduce  sums split-K partial slices in order + epilogue
  streamk_fixup  finishes the stream-K remainder tiles (pieces in K order + epilogue)
  quantize, qgemm, qconv, qdwconv, qadd, qlut, qgap, dequantize, qmlp,
  qconv_first (INT8 path, int8 activations channels-last on the device)
  elementwise fused pointwise chain (also single pointwise ops)
  maxpool, avgpool, gap, copy (reshaping views: Flatten/Reshape/Identity/...)
  softmax, transpose, pad, concat (one launch per Concat operand)

Every op of the graph gets a device launch or lowering raises
``NotImplementedError``: there is no host fallback. Constant operands that
need a device layout (conv weights as [OC][K padded to 4], a transB weight as
[K][N padded to 4]) are packed here, at compile time, into
``HipModule.device_constants``.

Conv as GEMM uses the reference orientation (emit.py:187-209): M = OC,
N = P = batch*OH*OW, K = C*KH*KW, with the output scattered to NCHW in the
epilogue, which also fixes the reference's batch>1 bug (emit.py:187-188).
"""

from __future__ import annotations

from typing import Callable, Optional

import numpy as np

from mdlc_amd.codegen.hip import templates as T
from mdlc_amd.codegen.hip.emit_int8 import Int8LoweringMixin
from mdlc_amd.codegen.hip.plan import (LIBRARY_PARTS, QUANT_OPS, HipModule, Launch,  # noqa: F401
                                       library_parts, round4, round16)
from mdlc_amd.codegen import schedule as schedule_mod
from mdlc_amd.codegen.schedule import (WINO_BK, WINO_BM, WINO_BN, MfmaSchedule, conv_pool_band,
                                      default_schedule, smallc_fits, smallc_pairs, smallc_tile, split_slices,
                                      unsplit_if_one_slice, wino_fits,
                                      wino_patch, wino_pays, wino_slices)
from mdlc_amd.ir import DType, Graph, Node
from mdlc_amd.passes.fuse_elementwise import ELEMENTWISE
from mdlc_amd.passes.shape_inference import conv_geometry
from mdlc_amd.runtime.memory_planner import plan_memory

ScheduleFn = Callable[[Optional[Node], tuple], MfmaSchedule]

VIEW_OPS = {"Flatten", "Reshape", "Identity", "Squeeze", "Unsqueeze"}
REDUCE_VEC = 4        # outputs per thread of the split-K reduce where the layout allows (else 1)
STREAM_K_WGS = 256    # stream-K workgroups: one per CU
PAIR_MIN_IDLE = 32    # idle CUs a conv's grid must leave for a second conv to share its launch
SMALLC_WGS = 512      # workgroups stepping through the blocks of the small-channel conv


def _check_reduce_size(M: int, N: int) -> None:
    """The split-K reduce indexes one slice with 32-bit integers."""
    if M * N >= 2 ** 31:
        raise NotImplementedError(f"HIP codegen: split-K output of {M * N} elements (2^31 or more)")


def dw_rows_per_thread(oh: int) -> int:
    """Outputs per thread down a column in the depthwise kernel: 8 (fewer
    loads per output), 4 for planes of at most 7 rows, where 8 leaves too few
    threads to cover the memory latency (MobileNetV2's 7x7 layers: 7.9 -> 6.8 us;
    shorter strips were slower on every larger plane measured)."""
    return 4 if oh <= 7 else T.WINDOW_VH


class HipCodegen(Int8LoweringMixin):
    def __init__(self, schedule_fn: Optional[ScheduleFn] = None, *, conv_mode: str = "implicit",
                 int8_depthwise: str = "mfma", small_conv: bool = True,
                 winograd="auto", pair_convs: bool = True) -> None:
        """``int8_depthwise``: "mfma" runs 16-channel-aligned int8 depthwise
        convs as block-diagonal GEMMs on the matrix cores, "vector" keeps
        them on the per-pixel vector kernel. ``small_conv``: convs with few
        input channels take the direct kernel (implicit mode). ``winograd``:
        3x3 stride-1 convs run as Winograd F(2x2, 3x3) (implicit mode): True
        always, "auto" where its grid fills at least half the CUs
        (``wino_pays``), False never. ``pair_convs``: two adjacent independent
        implicit-GEMM convolutions run as one launch where the first leaves
        CUs idle (``_pair_convs``)."""
        if winograd not in (True, False, "auto"):
            raise ValueError(f"winograd must be True, False or 'auto', not {winograd!r}")
        if conv_mode not in ("implicit", "im2col"):
            raise ValueError(f"conv_mode must be 'implicit' or 'im2col', not {conv_mode!r}")
        if int8_depthwise not in ("mfma", "vector"):
            raise ValueError(f"int8_depthwise must be 'mfma' or 'vector', not {int8_depthwise!r}")
        self.int8_depthwise_mfma = int8_depthwise == "mfma"
        if schedule_fn is None:
            from mdlc_amd.autotuner.tuner import tuned_schedules

            schedule_fn = tuned_schedules()
        self.schedule_fn = schedule_fn
        self.conv_mode = conv_mode
        self.small_conv = small_conv
        self.winograd = winograd
        self.pair_convs = pair_convs
        self.kernels: dict = {}
        self.plan: list = []
        self.scratch: dict = {}
        self.scratch_class: dict = {}
        self.consts: dict = {}
        self.layout: dict = {}
        self._dedup: dict = {}

    # -- helpers ------------------------------------------------------------

    def _shape(self, g: Graph, name: str) -> tuple:
        info = g.info(name)
        if info is None or not info.is_static:
            raise ValueError(f"{name!r} lacks a static shape; run shape inference")
        return tuple(int(d) for d in info.shape)

    def _schedule(self, node: Node, mnk: tuple, problem: dict) -> MfmaSchedule:
        """Ask the schedule source; tuners that key on the whole problem (conv
        window, batch) expose ``schedule_problem``."""
        fn = getattr(self.schedule_fn, "schedule_problem", None)
        sched = fn(problem) if fn is not None else self.schedule_fn(node, mnk)
        if not sched.is_valid():
            raise ValueError(f"invalid schedule {sched} for {mnk}")
        return unsplit_if_one_slice(sched, mnk[2])

    def _kernel(self, sig: tuple, make) -> str:
        """Return the kernel for ``sig``, generating it once."""
        if sig not in self._dedup:
            name, src = make(len(self._dedup))
            self.kernels[name] = src
            self._dedup[sig] = name
        return self._dedup[sig]

    def _pack(self, name: str, array: np.ndarray) -> str:
        self.consts[name] = np.ascontiguousarray(array, dtype=np.float32)
        return name

    def _pack_rows(self, g: Graph, src: str, rows: int, cols: int, transpose: bool = False,
                   tag: str = "") -> tuple:
        """Constant as a row-major [rows][ld] float32 matrix, ld = cols rounded
        up to 4, zero padded. ``tag`` names a second layout of the same
        constant. Returns (device name, ld)."""
        arr = np.asarray(g.initializers[src], dtype=np.float32)
        mat = arr.T if transpose else arr.reshape(rows, cols) if arr.ndim != 2 else arr
        mat = np.asarray(mat).reshape(rows, cols)
        ld = round4(cols)
        if ld == cols:
            return self._pack(f"{src}__dev{tag}", mat), ld
        pad = np.zeros((rows, ld), dtype=np.float32)
        pad[:, :cols] = mat
        return self._pack(f"{src}__dev{tag}_ld{ld}", pad), ld

    @staticmethod
    def _act_sig(a: dict) -> tuple:
        return (a.get("activation"), a.get("clip_min"), a.get("clip_max"),
                a.get("alpha") if a.get("activation") in ("LeakyRelu", "HardSigmoid") else None,
                a.get("beta") if a.get("activation") == "HardSigmoid" else None)

    @staticmethod
    def _act_attrs(a: dict) -> dict:
        keep = {k: a[k] for k in ("clip_min", "clip_max") if k in a}
        if a.get("activation") in ("LeakyRelu", "HardSigmoid"):
            keep["alpha"] = a.get("alpha")
        if a.get("activation") == "HardSigmoid":
            keep["beta"] = a.get("beta")
        return keep

    # -- lowering -------------------------------------------------------------

    def lower(self, g: Graph) -> HipModule:
        self._graph = g
        for node in g.topo_sort():
            op = node.op_type
            if op in ("Conv", "FusedConvAct", "FusedConvBNAct"):
                self._lower_conv(g, node)
            elif op in ("Gemm", "FusedGemmAct", "MatMul"):
                self._lower_gemm(g, node)
            elif op == "FusedElementwise":
                self._lower_elementwise(g, node)
            elif op in ELEMENTWISE:
                solo = Node("FusedElementwise", node.real_inputs(), list(node.outputs),
                            {"subgraph": [node]}, node.name, [op])
                self._lower_elementwise(g, solo, origin=node)
            elif op in ("MaxPool", "AveragePool"):
                self._lower_pool(g, node)
            elif op == "GlobalAveragePool":
                self._lower_gap(g, node)
            elif op in VIEW_OPS:
                self._lower_view(g, node)
            elif op in ("Softmax", "Transpose", "Pad", "Concat"):
                getattr(self, "_lower_" + op.lower())(g, node)
            elif op in QUANT_OPS:
                getattr(self, "_lower_" + op.lower())(g, node)
            else:
                raise NotImplementedError(f"HIP codegen: no device lowering for {op!r}")
        if self.pair_convs:
            self._pair_convs(g)
        lib = library_parts({l.kind for l in self.plan})
        return HipModule(g, self.kernels, self.plan, self.scratch, self.consts, lib,
                         scratch_class=self.scratch_class, device_layout=dict(self.layout))

    def _pair_convs(self, g: Graph) -> None:
        """Run two adjacent implicit-GEMM convolutions as one launch where the
        first's grid leaves at least PAIR_MIN_IDLE CUs idle and the second
        reads nothing the first writes (ResNet's stride-2 conv and its 1x1
        downsample both read the block input): the first keeps its grid, the
        idle CUs take the second's tiles in turn (``conv_pair_kernel``). Both
        are one-slice launches of the same workgroup size, the second's work
        per idle CU is at most the first's per workgroup, and the memory plan
        gives no tensor of one a buffer that a tensor of the other uses, so
        running them at once changes no value (each tile is computed by the
        same code as before)."""
        mem = plan_memory(g)

        def bufs(names):
            return {mem.assignment[e] for e in names if e in mem.assignment}

        def one_slice_conv(l):
            return (l.kind == "conv" and not l.meta.get("partial") and not l.meta.get("stream_k")
                    and l.grid[1:] == (1, 1) and l.meta.get("ksplit", 1) == 1)

        cus = schedule_mod.CUS
        out, i = [], 0
        while i < len(self.plan):
            a = self.plan[i]
            b = self.plan[i + 1] if i + 1 < len(self.plan) else None
            ok = (b is not None and one_slice_conv(a) and one_slice_conv(b) and a.block == b.block
                  and cus - a.grid[0] >= PAIR_MIN_IDLE
                  and not set(b.inputs) & set(a.outputs) and not set(a.inputs) & set(b.outputs)
                  and not set(a.outputs) & set(b.outputs)
                  and not bufs(b.outputs) & bufs(a.inputs + a.outputs)
                  and not bufs(a.outputs) & bufs(b.inputs + b.outputs)
                  and b.meta.get("flops", 0) * a.grid[0] <= a.meta.get("flops", 0) * (cus - a.grid[0]))
            if not ok:
                out.append(a)
                i += 1
                continue
            kname = self._kernel(("conv_pair", a.kernel_name, b.kernel_name), lambda j: T.conv_pair_kernel(
                f"conv_pair_{j}", (a.kernel_name, self.kernels[a.kernel_name]),
                (b.kernel_name, self.kernels[b.kernel_name])))
            meta = {"first": a, "second": b, "g0": a.grid[0], "nb": b.grid[0], "node": a.meta["node"],
                    "flops": a.meta.get("flops", 0) + b.meta.get("flops", 0),
                    "bytes": a.meta.get("bytes", 0) + b.meta.get("bytes", 0)}
            out.append(Launch("conv_pair", kname, a.inputs + b.inputs, a.outputs + b.outputs,
                              (cus, 1, 1), a.block, meta))
            i += 2
        self.plan = out

    def _lower_conv(self, g: Graph, node: Node) -> None:
        x, w = node.inputs[0], node.inputs[1]
        has_bias = len(node.inputs) > 2 and bool(node.inputs[2])
        if not g.is_constant(w):
            raise NotImplementedError("HIP codegen: conv weights must be constants")
        geo = conv_geometry(node, self._shape(g, x), self._shape(g, w))
        y = node.outputs[0]
        a = node.attrs
        act = a.get("activation")
        if a.get("maxpool"):
            self._lower_conv_pool(g, node, geo, has_bias)
            return
        if geo["group"] != 1:
            if geo["ICG"] == 1 and geo["OC"] % geo["C"] == 0:
                self._lower_dwconv(g, node, geo, has_bias)
            else:
                self._lower_grouped_conv(g, node, geo, has_bias)
            return
        # the small-channel kernel reads its input and writes its output through
        # buffer resources of byte offsets below 2^31 - 16
        if self.conv_mode == "implicit" and self.small_conv and smallc_fits(geo["C"], geo["KH"], geo["KW"], geo["DH"],
                                                        geo["DW"]) \
                and 4 * geo["N"] * max(geo["C"] * geo["H"] * geo["W"],
                                       geo["OC"] * geo["OH"] * geo["OW"]) < 0x7ffffff0:
            self._lower_conv_smallc(g, node, geo, has_bias)
            return
        # the Winograd kernel reads its input, bias and residual through buffer
        # resources of byte offsets below 2^31 (offsets at 0x7ffffff0 read as zeros) and
        # divides tile indices and workgroup indices (at most one per channel-block,
        # tile-block and chunk) below 2^21 in float
        wino_tiles = geo["N"] * -(-geo["OH"] // 2) * -(-geo["OW"] // 2)
        if (self.conv_mode == "implicit" and self.winograd and wino_fits(geo)
                and geo["N"] * geo["C"] * geo["H"] * geo["W"] * 4 < 0x7ffffff0
                and geo["N"] * geo["OC"] * geo["OH"] * geo["OW"] * 4 < 0x7ffffff0
                and wino_tiles < 2 ** 21
                and -(-geo["OC"] // WINO_BM) * -(-wino_tiles // WINO_BN) * -(-geo["C"] // WINO_BK) < 2 ** 21
                and (self.winograd is True or wino_pays(
                    geo["OC"], geo["N"] * -(-geo["OH"] // 2) * -(-geo["OW"] // 2), geo["C"]))):
            self._lower_wino(g, node, geo, has_bias)
            return
        OC, K = geo["OC"], geo["C"] * geo["KH"] * geo["KW"]
        OH, OW, N = geo["OH"], geo["OW"], geo["N"]
        P = N * OH * OW
        problem = {"kind": "conv", "mode": self.conv_mode, "M": OC, "N": P, "K": K,
                   "batch": N, "bias": has_bias, "act": act,
                   **{k: geo[k] for k in ("C", "H", "W", "KH", "KW", "SH", "SW", "DH", "DW",
                                          "PT", "PB", "PL", "PR", "OH", "OW")}}
        sched = self._schedule(node, (OC, P, K), problem)
        if self.conv_mode == "implicit" and sched.WK > 1 and (geo["C"] % 16 or not sched.is_valid()):
            raise ValueError(f"wave-split schedule {sched.key_full()} needs Cin % 16 == 0")
        if self.conv_mode == "implicit" and sched.WK == 1 and not sched.conv_valid():
            raise ValueError(f"schedule {sched.key_full()} does not fit the convolution gather "
                             f"(threads per block must be a multiple of BN and BK of NT/BN)")
        tap_major = self.conv_mode == "implicit" and geo["C"] % sched.BK == 0
        if tap_major:
            # k ordered (kh, kw, c): weights [OC][KH][KW][C]
            warr = np.asarray(g.initializers[w], np.float32).transpose(0, 2, 3, 1).reshape(OC, K)
            wdev, lda = self._pack(f"{w}__dev_tap", warr), K
        else:
            wdev, lda = self._pack_rows(g, w, OC, K)
        bias = [node.inputs[2]] if has_bias else []
        meta = {"M": OC, "N": P, "K": K, "lda": lda, "with_bias": has_bias, "node": node,
                "weight_2d": (OC, K), "out_4d": (N, OC, OH, OW), "sched": sched,
                "flops": 2 * OC * P * K,
                # algorithmic HBM bytes: input, weights, bias and output once each
                "bytes": 4 * (N * geo["C"] * geo["H"] * geo["W"] + OC * K + P * OC
                              + (OC if has_bias else 0))}
        epi = dict(bias_mode="row", act=act, attrs=self._act_attrs(a), act_sig=self._act_sig(a),
                   alpha=1.0, beta=1.0, ldc=0, hw=OH * OW, **self._residual_epilogue(g, node))
        if epi["res_input"]:
            meta["bytes"] += 4 * P * OC
        if self.conv_mode == "implicit":
            win = (geo["KH"], geo["KW"], geo["SH"], geo["SW"], geo["DH"], geo["DW"], geo["PT"], geo["PL"])
            meta.update({"Cin": geo["C"], "H": geo["H"], "W": geo["W"], "OH": OH, "OW": OW,
                         "k_order": "tap" if tap_major else "channel"})
            if sched.WK > 1:
                self._emit_conv_ws(sched, wdev, x, bias, y, meta, epi, win)
                return
            self._emit_gemm("conv", sched, [wdev, x], bias, y, meta, epi, bmode=3 if tap_major else 2,
                            vec_a=lda % 4 == 0, win=win, out_nchw=True)
            return
        # explicit im2col + GEMM
        if "im2col" not in self._dedup:
            self._kernel("im2col", lambda i: T.im2col_kernel("im2col"))
        cols = y + "__cols"
        ldc = round4(P)
        self.scratch[cols] = (K, ldc)
        self.scratch_class[cols] = "cols"
        self.plan.append(Launch(
            "im2col", "im2col", [x], [cols], (-(-(ldc // 4) // 256), K, 1), (256, 1, 1),
            {"C": geo["C"], "H": geo["H"], "W": geo["W"], "KH": geo["KH"], "KW": geo["KW"],
             "OH": OH, "OW": OW, "SH": geo["SH"], "SW": geo["SW"], "PH": geo["PT"],
             "PW": geo["PL"], "DH": geo["DH"], "DW": geo["DW"], "batch": N, "ldc": ldc,
             "node": node, "bytes": 4 * (N * geo["C"] * geo["H"] * geo["W"] + K * ldc)}))
        meta.update({"ldb": ldc})
        self._emit_gemm("gemm", sched, [wdev, cols], bias, y, meta, epi, bmode=0, vec_a=True,
                        out_nchw=True)

    def _lower_grouped_conv(self, g: Graph, node: Node, geo: dict, has_bias: bool) -> None:
        """A grouped convolution (1 < group, more than one input channel per
        group) as one launch of the implicit-GEMM conv over all groups: the
        grid's y index is the group, whose GEMM is M = OC/group, N = batch *
        OH * OW, K = C/group * KH * KW over its own input channels and weight
        rows, scattered to its own output channels. The reference runs this
        op on the host (mdlc/codegen/cuda/emit.py:175-180, runtime/ops.py:69-78).
        Both conv modes use the gather (no per-group column matrices); the
        schedule runs without split-K or stream-K."""
        G, OC, C = geo["group"], geo["OC"], geo["C"]
        if OC % G or C % G:
            raise ValueError(f"group {G} does not divide channels {C} -> {OC}")
        ocg, icg = OC // G, geo["ICG"]
        KH, KW, OH, OW, N = geo["KH"], geo["KW"], geo["OH"], geo["OW"], geo["N"]
        K, P = icg * KH * KW, N * OH * OW
        x, w, y = node.inputs[0], node.inputs[1], node.outputs[0]
        a = node.attrs
        act = a.get("activation")
        problem = {"kind": "conv", "mode": "implicit", "M": ocg, "N": P, "K": K, "batch": N,
                   "bias": has_bias, "act": act, "group": G,
                   **{k: geo[k] for k in ("H", "W", "KH", "KW", "SH", "SW", "DH", "DW",
                                          "PT", "PB", "PL", "PR", "OH", "OW")}, "C": icg}
        sched = self._schedule(node, (ocg, P, K), problem)
        if sched.SK > 1 or sched.ST:
            sched = MfmaSchedule(sched.BM, sched.BN, sched.BK, sched.WGM, sched.WGN, sched.MS, sched.DB,
                                 1, False, sched.UN)
        if not sched.conv_valid():
            raise ValueError(f"schedule {sched.key_full()} does not fit the convolution gather")
        tap_major = icg % sched.BK == 0
        warr = np.asarray(g.initializers[w], np.float32)          # [OC][icg][KH][KW]
        if tap_major:
            wdev, lda = self._pack(f"{w}__dev_tap", warr.transpose(0, 2, 3, 1).reshape(OC, K)), K
        else:
            wdev, lda = self._pack_rows(g, w, OC, K)
        bias = [node.inputs[2]] if has_bias else []
        res = self._residual_epilogue(g, node)
        extra = [res["res_input"]] if res["res_input"] else []
        win = (KH, KW, geo["SH"], geo["SW"], geo["DH"], geo["DW"], geo["PT"], geo["PL"])
        bmode = 3 if tap_major else 2
        sig = ("gconv", sched, has_bias, self._act_sig(a), bmode, lda % 4 == 0, win, res["residual"])
        rtag = "_res" if extra else ""
        kname = self._kernel(sig, lambda i: T.gemm_kernel(
            f"gconv_{sched.key()}_{act or 'none'}{rtag}_{i}", sched, with_bias=has_bias,
            bias_mode="row", activation=act, attrs=self._act_attrs(a), bmode=bmode,
            out_nchw=True, vec_a=lda % 4 == 0, win=win, residual=res["residual"], grouped=True))
        tiles = -(-ocg // sched.BM) * -(-P // sched.BN)
        self.plan.append(Launch(
            "gconv", kname, [wdev, x] + bias + extra, [y], (tiles, G, 1),
            (sched.threads_per_block(), 1, 1),
            {"M": ocg, "N": P, "K": K, "lda": lda, "Cin": icg, "H": geo["H"], "W": geo["W"],
             "OH": OH, "OW": OW, "ksplit": 1, "kchunk": K, "ximg": C * geo["H"] * geo["W"],
             "cimg": OC * OH * OW, "group": G, "with_bias": has_bias, "node": node,
             "sched": sched, "k_order": "tap" if tap_major else "channel",
             "flops": 2 * OC * P * K,
             "bytes": 4 * (N * C * geo["H"] * geo["W"] + OC * K + P * OC * (1 + len(extra))
                           + (OC if has_bias else 0))}))

    def _lower_wino(self, g: Graph, node: Node, geo: dict, has_bias: bool) -> None:
        """3x3 stride-1 conv as Winograd F(2x2, 3x3): the filters are
        transformed here (``wino_filter_transform``), the input and output
        transforms run inside the kernel. Grids too small for the chip split
        the channel sum over ``wino_slices`` slices, added by the split-K
        reduce, which then applies bias, activation and residual."""
        N, C, H, W = geo["N"], geo["C"], geo["H"], geo["W"]
        OC, OH, OW = geo["OC"], geo["OH"], geo["OW"]
        TH, TW = -(-OH // 2), -(-OW // 2)
        tiles = N * TH * TW
        chunks = -(-C // WINO_BK)
        nchunk = -(-chunks // wino_slices(OC, tiles, C))
        slices = -(-chunks // nchunk)              # no empty slice
        CP, OCP = slices * nchunk * WINO_BK, -(-OC // WINO_BM) * WINO_BM
        w, x, y = node.inputs[1], node.inputs[0], node.outputs[0]
        u = wino_pack_filters(wino_filter_transform(np.asarray(g.initializers[w])), OCP, CP)
        udev = self._pack(f"{w}__dev_wino", u)
        a = node.attrs
        act = a.get("activation")
        epi = dict(act_sig=self._act_sig(a), attrs=self._act_attrs(a), **self._residual_epilogue(g, node))
        residual, res = epi["residual"], epi["res_input"]
        bias = [node.inputs[2]] if has_bias else []
        extra = [res] if res else []
        P = N * OH * OW
        split = slices > 1
        grid = (-(-OC // WINO_BM) * -(-tiles // WINO_BN), slices, 1)
        meta = {"N": N, "C": C, "H": H, "W": W, "OC": OC, "OH": OH, "OW": OW, "TH": TH, "TW": TW,
                "CP": CP, "OCP": OCP, "PT": geo["PT"], "PL": geo["PL"], "nchunk": nchunk,
                "node": node, "ksplit": slices, "out_4d": (N, OC, OH, OW),
                # the multiply-adds this algorithm performs (16 per tile, channel
                # pair), and those of the direct convolution it replaces
                "flops": 2 * 16 * OC * C * tiles, "direct_flops": 2 * 9 * OC * C * P,
                "bytes": 4 * (N * C * H * W + 16 * OC * C + OC * P)}
        rtag = "_res" if residual and not split else ""
        ploads = -(-wino_patch(N, H, W, geo["PT"], OH, OW) // 64)
        meta["ploads"] = ploads
        full = OH % 2 == 0 and OW % 2 == 0
        sig = ("wino", split, ploads, full, bool(bias) and not split,
               None if split else epi["act_sig"], None if split else residual)
        kname = self._kernel(sig, lambda i: T.wino_kernel(
            f"conv_wino{'_SK' if split else ''}_P{ploads}_{'none' if split else act or 'none'}{rtag}_{i}",
            split=split, ploads=ploads, full=full, with_bias=bool(bias), activation=act,
            attrs=epi["attrs"], residual=residual))
        if not split:
            if res:
                meta["bytes"] += 4 * OC * P
            if bias:
                meta["bytes"] += 4 * OC
            self.plan.append(Launch("wino", kname, [udev, x] + bias + extra, [y], grid, (512, 1, 1),
                                    meta))
            return
        ws = y + "__splitk"
        self.scratch[ws] = (slices * OC, P)
        self.scratch_class[ws] = "splitk"
        meta["bytes"] += 4 * (slices - 1) * OC * P
        self.plan.append(Launch("wino", kname, [udev, x], [ws], grid, (512, 1, 1),
                                dict(meta, partial=True)))
        vec = REDUCE_VEC if P % 4 == 0 and (OH * OW) % 4 == 0 else 1
        _check_reduce_size(OC, P)
        rsig = ("splitk_reduce", bool(bias), "row", epi["act_sig"], 1.0, 1.0, residual, vec, slices,
                OH * OW)
        rname = self._kernel(rsig, lambda i: T.splitk_reduce_kernel(
            f"splitk_reduce{'4' if vec == 4 else ''}_{act or 'none'}_row{'_res' if residual else ''}_{i}",
            with_bias=bool(bias), bias_mode="row", activation=act, attrs=epi["attrs"],
            residual=residual, vec=vec, slices=slices, hw=OH * OW))
        self.plan.append(Launch(
            "splitk_reduce", rname, [ws] + bias + extra, [y], (-(-(OC * P) // (256 * vec)), 1, 1),
            (256, 1, 1),
            {"S": slices, "M": OC, "N": P, "ldc": 0, "hw": OH * OW, "node": node,
             "bytes": 4 * (slices + 1 + len(extra)) * OC * P}))

    def _lower_conv_pool(self, g: Graph, node: Node, geo: dict, has_bias: bool) -> None:
        """A small-channel conv carrying the 3x3 stride-2 max pool that
        followed it (``attrs["maxpool"]``, folded by ``FuseConvMaxPool``): one
        launch writes the pooled output. The weights are packed here as
        [16-channel block][4-deep k step][lane], lane 16 lk + li holding
        w[16 block + li][4 step + lk] in (c, kh, kw) order, zeros past K and
        past OC."""
        mp = node.attrs["maxpool"]
        if (list(mp["kernel_shape"]) != [3, 3] or list(mp["strides"]) != [2, 2]
                or list(mp["pads"]) != [1, 1, 1, 1]):
            raise NotImplementedError(f"HIP codegen: fused max pool {mp} (only 3x3, stride 2, pad 1)")
        if self.conv_mode != "implicit" or not self.small_conv or geo["group"] != 1:
            raise NotImplementedError("HIP codegen: a conv with a folded max pool needs the implicit "
                                      "small-channel lowering")
        C, KH, KW, SH, SW = geo["C"], geo["KH"], geo["KW"], geo["SH"], geo["SW"]
        OC, OH, OW, N, H, W = geo["OC"], geo["OH"], geo["OW"], geo["N"], geo["H"], geo["W"]
        R = conv_pool_band(C, KH, KW, SH, SW, geo["DH"], geo["DW"], N, OH, OW)
        if R is None:
            raise NotImplementedError(f"HIP codegen: no fused conv + pool band for {geo}")
        PH, PW = OH // 2, OW // 2
        if 4 * N * max(C * H * W, OC * PH * PW) >= 0x7ffffff0:
            raise NotImplementedError("HIP codegen: fused conv + pool tensors of 2^31 bytes or more")
        x, w, y = node.inputs[0], node.inputs[1], node.outputs[0]
        K = C * KH * KW
        ns = -(-K // 4)
        groups = -(-OC // 64)
        wpad = np.zeros((groups * 64, ns * 4), np.float32)
        wpad[:OC, :K] = np.asarray(g.initializers[w], np.float32).reshape(OC, K)
        packed = wpad.reshape(groups * 4, 16, ns, 4).transpose(0, 2, 3, 1).reshape(groups * 4, ns, 64)
        wdev = self._pack(f"{w}__dev_convpool", packed)
        bias = [node.inputs[2]] if has_bias else []
        a = node.attrs
        act = a.get("activation")
        if act not in (None, "Identity", "Relu", "Relu6", "Clip"):
            raise NotImplementedError(f"HIP codegen: max pool after {act!r} (not non-decreasing)")
        win = (C, KH, KW, SH, SW, geo["PT"], geo["PL"])
        sig = ("conv_pool", win, R, OW // 16, has_bias, self._act_sig(a))
        kname = self._kernel(sig, lambda i: T.conv_pool_kernel(
            f"conv_pool_{KH}x{KW}s{SH}_{act or 'none'}_R{R}_{i}", win, R, OW // 16,
            with_bias=has_bias, activation=act, attrs=self._act_attrs(a)))
        P = N * OH * OW
        self.plan.append(Launch(
            "conv_pool", kname, [x, wdev] + bias, [y], (N * (PH // R), groups, 1), (256, 1, 1),
            {"M": OC, "N": P, "K": K, "batch": N, "H": H, "W": W, "OC": OC, "OH": OH, "OW": OW,
             "band": R, "node": node, "flops": 2 * OC * P * K,
             "bytes": 4 * (N * C * H * W + OC * K + N * OC * PH * PW + (OC if has_bias else 0))}))

    def _lower_conv_smallc(self, g: Graph, node: Node, geo: dict, has_bias: bool) -> None:
        """A conv with few input channels (a network's stem): the direct
        matrix-core kernel, input patch in LDS and weights in registers. The
        weights are packed here as [channel block][pair i][lane], lane =
        (k % 2) * 32 + oc % 32, k = 2i + k % 2 in (c, kh, kw) order (a zero
        weight pads an odd K)."""
        C, KH, KW = geo["C"], geo["KH"], geo["KW"]
        OC, OH, OW, N = geo["OC"], geo["OH"], geo["OW"], geo["N"]
        x, w, y = node.inputs[0], node.inputs[1], node.outputs[0]
        a = node.attrs
        TR, TC, OCW = smallc_tile(N, OC, OH, OW)
        npair = smallc_pairs(C, KH, KW)
        nblk = -(-OC // (32 * OCW)) * OCW
        wpad = np.zeros((nblk * 32, 2 * npair), np.float32)
        wpad[:OC, :C * KH * KW] = np.asarray(g.initializers[w], np.float32).reshape(OC, -1)
        packed = wpad.reshape(nblk, 32, npair, 2).transpose(0, 2, 3, 1).reshape(nblk, npair, 64)
        wdev = self._pack(f"{w}__dev_smallc", packed)
        bias = [node.inputs[2]] if has_bias else []
        res = self._residual_epilogue(g, node)
        extra = [res["res_input"]] if res["res_input"] else []
        win = (C, KH, KW, geo["SH"], geo["SW"], geo["PT"], geo["PL"])
        act = a.get("activation")
        sig = ("conv_smallc", win, (TR, TC, OCW), has_bias, self._act_sig(a), res["residual"])
        kname = self._kernel(sig, lambda i: T.conv_smallc_kernel(
            f"conv_smallc_{KH}x{KW}s{geo['SH']}_{act or 'none'}{'_res' if extra else ''}_{i}", win,
            (TR, TC, OCW), with_bias=has_bias, activation=act, attrs=self._act_attrs(a),
            residual=res["residual"]))
        P, K = N * OH * OW, C * KH * KW
        grid = (min(N * -(-OH // TR) * -(-OW // TC), SMALLC_WGS), nblk // OCW, 1)
        self.plan.append(Launch(
            "conv_smallc", kname, [x, wdev] + bias + extra, [y], grid, (256, 1, 1),
            {"M": OC, "N": P, "K": K, "batch": N, "H": geo["H"], "W": geo["W"], "OC": OC,
             "OH": OH, "OW": OW,
             "tile": (TR, TC, OCW), "node": node, "flops": 2 * OC * P * K,
             "bytes": 4 * (N * C * geo["H"] * geo["W"] + OC * K + P * OC * (1 + len(extra))
                           + (OC if has_bias else 0))}))

    def _residual_epilogue(self, g: Graph, node: Node) -> dict:
        """``residual`` (the epilogue's post() body) and ``res_input`` for a
        conv carrying a folded residual group, else both None."""
        sub = node.attrs.get("residual_subgraph")
        if not sub:
            return {"residual": None, "res_input": None}
        r = node.inputs[3]
        y = node.attrs["residual_from"]
        consts = {}
        for n in sub:
            for e in n.real_inputs():
                if e not in (y, r) and g.is_constant(e):
                    consts[e] = float(np.asarray(g.initializers[e], np.float32).reshape(()))
        return {"residual": T.residual_post_body(sub, y, r, consts), "res_input": r}

    def _emit_gemm(self, kind: str, sched: MfmaSchedule, operands: list, bias: list, out: str,
                   meta: dict, epi: dict, *, bmode: int, vec_a: bool, out_nchw: bool,
                   win: Optional[tuple] = None) -> None:
        """Append the GEMM launch (and, with split-K, its reduce launch)."""
        M, N, K = meta["M"], meta["N"], meta["K"]
        # the kernel reads A, dense B and the conv gather's input through
        # buffer resources of byte offsets below 2^31 - 16
        nbytes = [4 * M * meta["lda"]]
        if bmode <= 1:
            nbytes.append(4 * K * max(meta.get("ldb", 0), N))
        elif bmode == 3:
            nbytes.append(4 * N // (meta["OH"] * meta["OW"]) * meta["Cin"] * meta["H"] * meta["W"])
        if max(nbytes) >= 0x7ffffff0:
            raise NotImplementedError(f"GEMM operands of {max(nbytes)} bytes exceed the kernel's "
                                      "2 GiB buffer range")
        slices, chunk = split_slices(K, sched)
        tiles = -(-M // sched.BM) * -(-N // sched.BN)
        block = (sched.threads_per_block(), 1, 1)
        act = epi["act"]
        tag = "conv" if kind == "conv" else "gemm"
        residual, res = epi.get("residual"), epi.get("res_input")
        extra = [res] if res else []
        rtag = "_res" if residual else ""
        sig = (kind, sched, bool(bias), epi["bias_mode"], epi["act_sig"], bmode, out_nchw, vec_a,
               epi["alpha"], epi["beta"], win, residual)
        meta = dict(meta, ksplit=slices, kchunk=chunk, ldc=epi["ldc"], hw=epi["hw"])
        meta.setdefault("ldb", 0)
        if sched.WK > 1:
            if kind != "gemm" or bmode > 1 or out_nchw or residual:
                raise ValueError(f"schedule {sched.key()} is for dense GEMMs only")
            b_kn = bool(meta.get("b_kn"))
            va = vec_a and K % 16 == 0 and meta["lda"] % 4 == 0 and (not b_kn or meta["ldb"] % 4 == 0)
            if slices == 1:
                wsig = ("gemm_ws", sched, bool(bias), epi["bias_mode"], epi["act_sig"], epi["alpha"],
                        epi["beta"], va, b_kn)
                kname = self._kernel(wsig, lambda i: T.gemm_wsplit_kernel(
                    f"gemm_{sched.key()}_{act or 'none'}_{epi['bias_mode']}_{i}", sched,
                    with_bias=bool(bias), bias_mode=epi["bias_mode"], activation=act,
                    attrs=epi["attrs"], alpha=epi["alpha"], beta=epi["beta"], vec_a=va, b_kn=b_kn))
                self.plan.append(Launch("gemm_ws", kname, operands + bias, [out], (tiles, 1, 1),
                                        block, meta))
                return
            # K also split over workgroups: raw slices to the workspace (ldc = N), then the reduce
            ws = out + "__splitk"
            self.scratch[ws] = (slices * M, N)
            self.scratch_class[ws] = "splitk"
            wsig = ("gemm_ws", sched, va, b_kn, "partial")
            kname = self._kernel(wsig, lambda i: T.gemm_wsplit_kernel(
                f"gemm_{sched.key()}_SK{slices}_{i}", sched, with_bias=False,
                bias_mode=epi["bias_mode"], activation=None, attrs={}, vec_a=va, b_kn=b_kn))
            extra_bytes = 4 * (M * N + (M if epi["bias_mode"] == "row" else N) * len(bias))
            self.plan.append(Launch("gemm_ws", kname, list(operands), [ws], (tiles, slices, 1), block,
                                    dict(meta, partial=True, ldc=N,
                                         bytes=meta["bytes"] - extra_bytes + 4 * slices * M * N)))
            self._emit_reduce(ws, bias, [], out, M, N, slices, epi, meta, act, "", None)
            return
        if sched.ST and tiles % STREAM_K_WGS:
            self._emit_stream_k(kind, sched, operands, bias, out, meta, epi, bmode=bmode,
                                vec_a=vec_a, out_nchw=out_nchw, win=win, tiles=tiles)
            return
        if slices == 1:
            kname = self._kernel(sig, lambda i: T.gemm_kernel(
                f"{tag}_{sched.key()}_{act or 'none'}_{epi['bias_mode']}{rtag}_{i}", sched,
                with_bias=bool(bias), bias_mode=epi["bias_mode"], activation=act,
                attrs=epi["attrs"], alpha=epi["alpha"], beta=epi["beta"], bmode=bmode,
                out_nchw=out_nchw, vec_a=vec_a, win=win, residual=residual))
            self.plan.append(Launch(kind, kname, operands + bias + extra, [out], (tiles, 1, 1), block,
                                    meta))
            return
        ws = out + "__splitk"
        self.scratch[ws] = (slices * M, N)
        self.scratch_class[ws] = "splitk"
        sig = (kind, sched, bmode, vec_a, win, "partial")
        kname = self._kernel(sig, lambda i: T.gemm_kernel(
            f"{tag}_{sched.key()}_SK_{i}", sched, with_bias=False, bmode=bmode, vec_a=vec_a,
            win=win))
        # the partial kernel reads the operands and writes every slice's sums;
        # bias, residual and the output belong to the reduce launch
        extra_bytes = 4 * (M * N * (1 + len(extra)) + (M if epi["bias_mode"] == "row" else N) * len(bias))
        self.plan.append(Launch(kind, kname, list(operands), [ws], (tiles * slices, 1, 1), block,
                                dict(meta, partial=True,
                                     bytes=meta["bytes"] - extra_bytes + 4 * slices * M * N)))
        self._emit_reduce(ws, bias, extra, out, M, N, slices, epi, meta, act, rtag, residual)

    def _emit_conv_ws(self, sched, wdev, x, bias, y, meta, epi, win) -> None:
        """A tap-major implicit-GEMM convolution on the wave-split kernel: one
        launch with the epilogue, or (``sched.SK > 1``) K also split over
        workgroups into the split-K workspace plus the ordered reduce."""
        M, N, K = meta["M"], meta["N"], meta["K"]
        batch = meta["out_4d"][0]
        if max(4 * batch * meta["Cin"] * meta["H"] * meta["W"], 4 * M * K, 4 * M * N) >= 0x7ffffff0:
            raise NotImplementedError("HIP codegen: conv operands exceed the wave-split kernel's "
                                      "2 GiB buffer range")
        slices, chunk = split_slices(K, sched)
        tiles = -(-M // sched.BM) * -(-N // sched.BN)
        block = (sched.threads_per_block(), 1, 1)
        act = epi["act"]
        residual, res = epi.get("residual"), epi.get("res_input")
        extra = [res] if res else []
        meta = dict(meta, ksplit=slices, kchunk=chunk, ldc=0, hw=epi["hw"])
        if slices == 1:
            sig = ("conv_ws", sched, win, bool(bias), epi["act_sig"], residual)
            kname = self._kernel(sig, lambda i: T.conv_wsplit_kernel(
                f"conv_{sched.key()}_{act or 'none'}{'_res' if residual else ''}_{i}", sched, win,
                with_bias=bool(bias), activation=act, attrs=epi["attrs"], residual=residual))
            self.plan.append(Launch("conv_ws", kname, [wdev, x] + bias + extra, [y], (tiles, 1, 1),
                                    block, meta))
            return
        ws = y + "__splitk"
        self.scratch[ws] = (slices * M, N)
        self.scratch_class[ws] = "splitk"
        sig = ("conv_ws", sched, win, "partial")
        kname = self._kernel(sig, lambda i: T.conv_wsplit_kernel(
            f"conv_{sched.key()}_SK{slices}_{i}", sched, win, with_bias=False, activation=None,
            attrs={}))
        extra_bytes = 4 * (M * N * (1 + len(extra)) + M * len(bias))
        self.plan.append(Launch("conv_ws", kname, [wdev, x], [ws], (tiles, slices, 1), block,
                                dict(meta, partial=True, ldc=N,
                                     bytes=meta["bytes"] - extra_bytes + 4 * slices * M * N)))
        self._emit_reduce(ws, bias, extra, y, M, N, slices, epi, meta, act,
                          "_res" if residual else "", residual)

    def _emit_reduce(self, ws, bias, extra, out, M, N, slices, epi, meta, act, rtag, residual) -> None:
        """The split-K reduce launch: adds the ``slices`` partial sums in ws in
        slice order and applies bias, activation and residual."""
        # four contiguous, 16-byte aligned outputs per thread when the layout allows
        vec = REDUCE_VEC if N % 4 == 0 and (epi["hw"] % 4 == 0 if epi["hw"] else epi["ldc"] % 4 == 0) \
            else 1
        _check_reduce_size(M, N)
        rsig = ("splitk_reduce", bool(bias), epi["bias_mode"], epi["act_sig"], epi["alpha"], epi["beta"],
                residual, vec, slices, epi["hw"])
        rname = self._kernel(rsig, lambda i: T.splitk_reduce_kernel(
            f"splitk_reduce{'4' if vec == 4 else ''}_{act or 'none'}_{epi['bias_mode']}{rtag}_{i}",
            with_bias=bool(bias), bias_mode=epi["bias_mode"], activation=act, attrs=epi["attrs"],
            alpha=epi["alpha"], beta=epi["beta"], residual=residual, vec=vec, slices=slices,
            hw=epi["hw"]))
        self.plan.append(Launch(
            "splitk_reduce", rname, [ws] + bias + extra, [out], (-(-(M * N) // (256 * vec)), 1, 1),
            (256, 1, 1),
            {"S": slices, "M": M, "N": N, "ldc": epi["ldc"], "hw": epi["hw"],
             "node": meta["node"], "bytes": 4 * (slices + 1 + len(extra)) * M * N}))

    def _emit_stream_k(self, kind, sched, operands, bias, out, meta, epi, *, bmode, vec_a, out_nchw,
                       win, tiles) -> None:
        """Stream-K: the first ``full`` tiles (a multiple of the CU count) one
        per workgroup, the remaining ones cut into equal K-step ranges over
        STREAM_K_WGS more workgroups, whose pieces the fix-up launch adds."""
        M, N, K = meta["M"], meta["N"], meta["K"]
        full = tiles - tiles % STREAM_K_WGS
        act = epi["act"]
        tag = "conv" if kind == "conv" else "gemm"
        residual, res = epi.get("residual"), epi.get("res_input")
        extra = [res] if res else []
        rtag = "_res" if residual else ""
        ws = out + "__streamk"
        self.scratch[ws] = (2 * STREAM_K_WGS * sched.BM, sched.BN)
        self.scratch_class[ws] = "splitk"
        sig = (kind, sched, bool(bias), epi["bias_mode"], epi["act_sig"], bmode, out_nchw, vec_a,
               epi["alpha"], epi["beta"], win, residual, "streamk")
        kname = self._kernel(sig, lambda i: T.gemm_kernel(
            f"{tag}_{sched.key()}_ST_{act or 'none'}_{epi['bias_mode']}{rtag}_{i}", sched,
            with_bias=bool(bias), bias_mode=epi["bias_mode"], activation=act,
            attrs=epi["attrs"], alpha=epi["alpha"], beta=epi["beta"], bmode=bmode,
            out_nchw=out_nchw, vec_a=vec_a, win=win, residual=residual, stream_k=STREAM_K_WGS))
        self.plan.append(Launch(kind, kname, operands + bias + extra + [ws], [out],
                                (full + STREAM_K_WGS, 1, 1), (sched.threads_per_block(), 1, 1),
                                dict(meta, ksplit=full, kchunk=K, stream_k=True)))
        fsig = ("streamk_fixup", sched.BM, sched.BN, sched.BK, bool(bias), epi["bias_mode"],
                epi["act_sig"], epi["alpha"], epi["beta"], residual)
        fname = self._kernel(fsig, lambda i: T.streamk_fixup_kernel(
            f"streamk_fixup_{act or 'none'}_{epi['bias_mode']}{rtag}_{i}", sched, STREAM_K_WGS,
            with_bias=bool(bias), bias_mode=epi["bias_mode"], activation=act, attrs=epi["attrs"],
            alpha=epi["alpha"], beta=epi["beta"], residual=residual))
        rest = tiles - full
        self.plan.append(Launch(
            "streamk_fixup", fname, [ws] + bias + extra, [out],
            (rest * (sched.BM * sched.BN // 1024), 1, 1), (256, 1, 1),
            {"M": M, "N": N, "K": K, "full": full, "ldc": epi["ldc"], "hw": epi["hw"],
             "node": meta["node"],
             "bytes": 4 * rest * sched.BM * sched.BN * (2 + len(extra))}))

    def _lower_dwconv(self, g: Graph, node: Node, geo: dict, has_bias: bool) -> None:
        a = node.attrs
        act = a.get("activation")
        win = (geo["KH"], geo["KW"], geo["SH"], geo["SW"], geo["DH"], geo["DW"])
        vh = dw_rows_per_thread(geo["OH"])
        sig = ("dwconv", win, has_bias, self._act_sig(a), vh)
        kname = self._kernel(sig, lambda i: T.dwconv_kernel(
            f"dwconv_{'x'.join(str(v) for v in win)}_{act or 'none'}_v{vh}_{i}", win,
            with_bias=has_bias, activation=act, attrs=self._act_attrs(a), vh=vh))
        w = node.inputs[1]
        wdev = self._pack(f"{w}__dev", np.asarray(g.initializers[w], np.float32).reshape(geo["OC"], -1))
        total = geo["N"] * geo["OC"] * geo["OH"] * geo["OW"]
        threads = geo["N"] * geo["OC"] * -(-geo["OH"] // vh) * geo["OW"]
        if max(threads, geo["H"] * geo["W"]) >= 2 ** 31:
            raise NotImplementedError("HIP codegen: depthwise conv too large for 32-bit indices")
        ins = [node.inputs[0], wdev] + ([node.inputs[2]] if has_bias else [])
        self.plan.append(Launch(
            "dwconv", kname, ins, [node.outputs[0]], (-(-threads // 256), 1, 1), (256, 1, 1),
            {**{k: geo[k] for k in ("N", "C", "H", "W", "OC", "OH", "OW", "PT", "PL")},
             "with_bias": has_bias, "node": node,
             "flops": 2 * total * geo["KH"] * geo["KW"],
             "bytes": 4 * (geo["N"] * geo["C"] * geo["H"] * geo["W"] + total
                           + geo["OC"] * geo["KH"] * geo["KW"] + (geo["OC"] if has_bias else 0))}))

    def _lower_gemm(self, g: Graph, node: Node) -> None:
        a = node.attrs
        A, B = node.inputs[0], node.inputs[1]
        has_bias = node.op_type != "MatMul" and len(node.inputs) > 2 and bool(node.inputs[2])
        ta, tb = int(a.get("transA", 0)), int(a.get("transB", 0))
        sa, sb = self._shape(g, A), self._shape(g, B)
        if len(sa) != 2 or len(sb) != 2:
            raise NotImplementedError("HIP codegen: only 2-D Gemm/MatMul operands are supported")
        M, K = (sa[1], sa[0]) if ta else sa
        N = sb[0] if tb else sb[1]
        alpha = float(a.get("alpha", 1.0)) if node.op_type != "MatMul" else 1.0
        beta = float(a.get("beta", 1.0)) if node.op_type != "MatMul" else 1.0
        if g.is_constant(A):
            adev, lda = self._pack_rows(g, A, M, K, transpose=bool(ta))
            vec_a = True
        elif ta:
            raise NotImplementedError("HIP codegen: transA on a runtime operand is unsupported")
        else:
            adev, lda = A, K
            vec_a = K % 4 == 0
        act = a.get("activation")
        problem = {"kind": "gemm", "M": M, "N": N, "K": K, "bias": has_bias, "act": act,
                   "vec_a": vec_a, "bmode": 0 if g.is_constant(B) or N % 4 == 0 else 1}
        sched = self._schedule(node, (M, N, K), problem)
        b_kn = sched.WK > 1 and sched.BT and g.is_constant(B)
        if b_kn:
            # the wave-split kernel reads constant weights K-contiguous per column
            bdev, ldb = self._pack_rows(g, B, N, K, transpose=not tb, tag="_kn")
            bmode = 0
        elif g.is_constant(B):
            bdev, ldb = self._pack_rows(g, B, K, N, transpose=bool(tb))
            bmode = 0
        elif tb:
            raise NotImplementedError("HIP codegen: transB on a runtime operand is unsupported")
        else:
            bdev, ldb = B, N
            bmode = 0 if N % 4 == 0 else 1
        bias_ins = []
        if has_bias:
            c = node.inputs[2]
            if not g.is_constant(c):
                raise NotImplementedError("HIP codegen: Gemm C must be a constant")
            carr = np.asarray(g.initializers[c], np.float32)
            if carr.size == N:
                bias_ins = [self._pack(f"{c}__col", carr.reshape(N))]
            elif carr.size == 1:
                bias_ins = [self._pack(f"{c}__col{N}", np.full(N, carr.reshape(()), np.float32))]
            else:
                raise NotImplementedError(f"HIP codegen: Gemm C of shape {carr.shape} unsupported")
        meta = {"M": M, "N": N, "K": K, "lda": lda, "ldb": ldb, "transA": ta, "transB": tb,
                "b_kn": b_kn,
                "alpha": alpha, "beta": beta, "with_bias": has_bias, "node": node,
                "sched": sched, "flops": 2 * M * N * K,
                "bytes": 4 * (M * K + K * N + M * N + (N if has_bias else 0))}
        epi = dict(bias_mode="col", act=act, attrs=self._act_attrs(a), act_sig=self._act_sig(a),
                   alpha=alpha, beta=beta, ldc=N, hw=0)
        self._emit_gemm("gemm", sched, [adev, bdev], bias_ins, node.outputs[0], meta, epi,
                        bmode=bmode, vec_a=vec_a, out_nchw=False)

    def _lower_elementwise(self, g: Graph, node: Node, origin: Optional[Node] = None) -> None:
        out_n = int(np.prod(self._shape(g, node.outputs[0])))
        consts: dict = {}
        sub = node.attrs["subgraph"]
        internal = {o for n in sub for o in n.outputs if o}
        for n in sub:
            for e in n.real_inputs():
                if e in internal:
                    continue
                if g.is_constant(e):
                    arr = g.initializers[e]
                    if arr.size != 1:
                        raise NotImplementedError(
                            f"HIP codegen: elementwise constant {e!r} of shape {arr.shape} "
                            "is not a scalar")
                    consts[e] = float(np.asarray(arr, np.float32).reshape(()))
                elif int(np.prod(self._shape(g, e))) != out_n:
                    raise NotImplementedError(
                        f"HIP codegen: broadcasting elementwise input {e!r} unsupported")
        for o in node.outputs:
            if int(np.prod(self._shape(g, o))) != out_n:
                raise NotImplementedError("HIP codegen: elementwise outputs differ in size")
        sig = ("ew",) + T.elementwise_signature(node, consts)
        holder = {}

        def make(i):
            name, src, ext = T.elementwise_kernel(f"fused_ew_{i}", node, scalar_consts=consts)
            holder["ext"] = ext
            return name, src

        kname = self._kernel(sig, make)
        internal_ext = [e for n in sub for e in n.real_inputs()
                        if e not in internal and e not in consts]
        ext = []
        for e in internal_ext:
            if e not in ext:
                ext.append(e)
        threads = out_n // 4 + out_n % 4
        nin = len(ext)
        self.plan.append(Launch(
            "elementwise", kname, ext, list(node.outputs), (max(1, -(-threads // 256)), 1, 1),
            (256, 1, 1), {"N": out_n, "node": origin or node, "scalar_consts": consts,
                          "bytes": 4 * out_n * (nin + len(node.outputs))}))

    def _lower_pool(self, g: Graph, node: Node) -> None:
        """MaxPool (-inf padding, ops.py:109-125) or AveragePool (zero
        padding, divisor KH*KW with count_include_pad, else the taps inside
        the input, ops.py:128-146) on the sliding-window kernel."""
        from mdlc_amd.passes.shape_inference import resolve_pads

        xs = self._shape(g, node.inputs[0])
        ys = self._shape(g, node.outputs[0])
        a = node.attrs
        avg = node.op_type == "AveragePool"
        kh, kw = a["kernel_shape"]
        sh, sw = a.get("strides", [1, 1])
        dh, dw = (1, 1) if avg else a.get("dilations", [1, 1])
        (pt, _), (pl, _) = resolve_pads(a.get("auto_pad", "NOTSET"), a.get("pads"), xs[2:],
                                        (kh, kw), (sh, sw), (dh, dw))
        win = (kh, kw, sh, sw, dh, dw)
        tag = "x".join(str(v) for v in win)
        if avg:
            cip = bool(a.get("count_include_pad", 0))
            kname = self._kernel(("avgpool", win, cip), lambda i: T.avgpool_kernel(
                f"avgpool_{tag}_{'cip' if cip else 'valid'}_{i}", win, cip))
        else:
            kname = self._kernel(("maxpool", win), lambda i: T.maxpool_kernel(f"maxpool_{tag}_{i}", win))
        total = int(np.prod(ys))
        threads = xs[0] * xs[1] * -(-ys[2] // T.WINDOW_VH) * ys[3]
        if max(threads, xs[2] * xs[3]) >= 2 ** 31:
            raise NotImplementedError("HIP codegen: pooling too large for 32-bit indices")
        self.plan.append(Launch(
            "avgpool" if avg else "maxpool", kname, [node.inputs[0]], [node.outputs[0]],
            (-(-threads // 256), 1, 1),
            (256, 1, 1), {"planes": xs[0] * xs[1], "H": xs[2], "W": xs[3], "OH": ys[2],
                          "OW": ys[3], "KH": kh, "KW": kw, "SH": sh, "SW": sw, "PT": pt, "PL": pl,
                          "DH": dh, "DW": dw, "node": node,
                          "bytes": 4 * (int(np.prod(xs)) + total)}))

    def _lower_gap(self, g: Graph, node: Node) -> None:
        xs = self._shape(g, node.inputs[0])
        planes = xs[0] * xs[1]
        hw = int(np.prod(xs[2:]))
        self._kernel("gap", lambda i: T.gap_kernel("global_avg_pool"))
        self.plan.append(Launch(
            "gap", "global_avg_pool", [node.inputs[0]], [node.outputs[0]],
            (-(-planes // 4), 1, 1), (256, 1, 1),
            {"planes": planes, "HW": hw, "node": node, "bytes": 4 * (planes * hw + planes)}))

    def _lower_view(self, g: Graph, node: Node) -> None:
        src = node.inputs[0]
        if self.layout.get(src) == "NHWC":
            shp = self._shape(g, src)
            if len(shp) == 4 and shp[2] * shp[3] != 1 and shp[1] != 1:
                raise NotImplementedError(
                    f"HIP codegen: {node.op_type} of a channels-last int8 tensor {shp}")
        info = g.info(node.outputs[0])
        nbytes = int(info.nbytes())
        self._kernel("copy", lambda i: T.copy_kernel("copy_bytes"))
        threads = nbytes // 16 + nbytes % 16
        self.plan.append(Launch(
            "copy", "copy_bytes", [src], [node.outputs[0]], (max(1, -(-threads // 256)), 1, 1),
            (256, 1, 1), {"nbytes": nbytes, "node": node, "bytes": 2 * nbytes}))

    # -- ops the reference ran on the host (emit.py:32-35) ------------------

    def _float_operand(self, g: Graph, node: Node, e: str) -> tuple:
        if self.layout.get(e) == "NHWC" or g.info(e).dtype != DType.FLOAT32:
            raise NotImplementedError(
                f"HIP codegen: {node.op_type} on {e!r} needs a float32 NCHW tensor")
        return self._shape(g, e)

    def _lower_softmax(self, g: Graph, node: Node) -> None:
        """Softmax over ``axis`` (default -1, as the reference executor
        reads it, reference.py:172-173): the tensor as [outer][L][inner]."""
        xs = self._float_operand(g, node, node.inputs[0])
        ax = int(node.attrs.get("axis", -1))
        ax = ax + len(xs) if ax < 0 else ax
        outer = int(np.prod(xs[:ax])) if ax else 1
        L, inner = xs[ax], int(np.prod(xs[ax + 1:])) if ax + 1 < len(xs) else 1
        rows = inner == 1
        kname = self._kernel(("softmax", rows), lambda i: T.softmax_kernel(
            "softmax_rows_f32" if rows else "softmax_cols_f32", rows))
        grid = (-(-outer // 4),) if rows else (-(-(outer * inner) // 256),)
        total = outer * L * inner
        self.plan.append(Launch(
            "softmax", kname, [node.inputs[0]], [node.outputs[0]], grid + (1, 1), (256, 1, 1),
            {"outer": outer, "L": L, "inner": inner, "rows": rows, "node": node,
             "bytes": 8 * total}))

    def _lower_transpose(self, g: Graph, node: Node) -> None:
        xs = self._float_operand(g, node, node.inputs[0])
        perm = node.attrs.get("perm") or list(range(len(xs)))[::-1]
        if len(xs) > 6:
            raise NotImplementedError("HIP codegen: Transpose of more than six dimensions")
        strides = [int(np.prod(xs[d + 1:])) for d in range(len(xs))]
        od = [xs[p] for p in perm]
        total = int(np.prod(xs))
        self._kernel("transpose", lambda i: T.transpose_kernel("transpose_f32"))
        self.plan.append(Launch(
            "transpose", "transpose_f32", [node.inputs[0]], [node.outputs[0]],
            (max(1, -(-total // 256)), 1, 1), (256, 1, 1),
            {"total": total, "out_dims": od, "src_strides": [strides[p] for p in perm],
             "node": node, "bytes": 8 * total}))

    def _lower_pad(self, g: Graph, node: Node) -> None:
        """Pad with ``pads`` / ``value`` from inputs 1 / 2 or the attributes
        (reference.py Pad dispatch, ops.py:249-255)."""
        xs = self._float_operand(g, node, node.inputs[0])
        ins, a = node.inputs, node.attrs
        def operand(i, attr, default):
            if len(ins) > i and ins[i]:
                if not g.is_constant(ins[i]):
                    raise NotImplementedError(f"HIP codegen: Pad {attr} must be constant")
                return g.initializers[ins[i]]
            return a.get(attr, default)
        pads = [int(v) for v in np.asarray(operand(1, "pads", None)).ravel()]
        value = float(np.asarray(operand(2, "value", 0.0), np.float32).reshape(()))
        mode = a.get("mode", "constant")
        if isinstance(mode, bytes):
            mode = mode.decode()
        if mode not in T.PAD_MODES:
            raise NotImplementedError(f"HIP codegen: Pad mode {mode!r}")
        half = len(pads) // 2
        before, after = pads[:half], pads[half:]
        if len(xs) > 6 or half != len(xs) or min(pads) < 0:
            raise NotImplementedError(f"HIP codegen: Pad {pads} of a {len(xs)}-d tensor")
        if mode == "reflect" and any(p >= n for p, n in zip(before + after, xs + xs)):
            raise NotImplementedError("HIP codegen: reflect Pad wider than its axis")
        if mode == "edge" and any(n == 0 for n in xs):
            raise NotImplementedError("HIP codegen: edge Pad of an empty axis")
        od = [n + b + e for n, b, e in zip(xs, before, after)]
        total = int(np.prod(od))
        kname = self._kernel(("pad", mode), lambda i: T.pad_kernel(f"pad_{mode}_f32", mode))
        self.plan.append(Launch(
            "pad", kname, [ins[0]], [node.outputs[0]], (max(1, -(-total // 256)), 1, 1),
            (256, 1, 1),
            {"total": total, "out_dims": od, "in_dims": list(xs), "before": before,
             "value": value, "node": node, "bytes": 4 * (int(np.prod(xs)) + total)}))

    def _lower_concat(self, g: Graph, node: Node) -> None:
        """One launch per operand, each writing its slab of the output."""
        parts = [e for e in node.inputs if e]
        shapes = [self._float_operand(g, node, e) for e in parts]
        ax = int(node.attrs.get("axis", 0))
        ax = ax + len(shapes[0]) if ax < 0 else ax
        outer = int(np.prod(shapes[0][:ax])) if ax else 1
        inner = int(np.prod(shapes[0][ax + 1:])) if ax + 1 < len(shapes[0]) else 1
        total_ax = sum(s[ax] for s in shapes)
        self._kernel("concat", lambda i: T.concat_kernel("concat_part_f32"))
        off = 0
        for e, s in zip(parts, shapes):
            run = s[ax] * inner
            n = outer * run
            self.plan.append(Launch(
                "concat", "concat_part_f32", [e], [node.outputs[0]],
                (max(1, -(-n // 256)), 1, 1), (256, 1, 1),
                {"rows": outer, "run": run, "dst_stride": total_ax * inner, "dst_off": off * inner,
                 "node": node, "bytes": 8 * n}))
            off += s[ax]


_WINO_G = np.array([[1.0, 0.0, 0.0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0.0, 0.0, 1.0]])


def wino_filter_transform(w: np.ndarray) -> np.ndarray:
    """[OC][C][3][3] filters -> U[16][OC][C] float32, U[4a + b] = (G g G^T)[a][b],
    computed in float64 and rounded once."""
    w = np.asarray(w, np.float64)
    u = np.einsum("ai,ocij,bj->aboc", _WINO_G, w, _WINO_G)
    return u.reshape(16, w.shape[0], w.shape[1]).astype(np.float32)


def wino_pack_filters(u: np.ndarray, OCP: int, CP: int) -> np.ndarray:
    """U[16][OC][C] -> the Winograd kernel's LDS images (zero padded): one
    contiguous 32 KB block per (64-channel output block, 8-channel chunk),
    laid out as the kernel's A operands are read,
    [OCP/64][CP/8][h 2][blk 4][j 2][lane 64][slot 2][4]: lane l = 16 lk + li
    of a wave of half h holds U[xi][oc][k] for oc = 16 blk + li,
    k = lk + 4 j and the eight positions xi = 8 h + 4 q + e of rows 2h, 2h + 1
    as two 16-byte quartets; quartet q sits in slot q ^ sw(l),
    sw(l) = ((l >> 2) ^ (l >> 3)) & 1, so that the 16-byte reads of any 8 or
    16 consecutive lanes hit distinct banks."""
    full = np.zeros((16, OCP, CP), np.float32)
    full[:, :u.shape[1], :u.shape[2]] = u
    # axes: h, q, e, ocb, blk, li, chunk, j, lk
    v = full.reshape(2, 2, 4, OCP // 64, 4, 16, CP // 8, 2, 4)
    img = v.transpose(3, 6, 0, 4, 7, 8, 5, 1, 2).reshape(OCP // 64, CP // 8, 2, 4, 2, 64, 2, 4)
    lanes = np.arange(64)
    sw = ((lanes >> 2) ^ (lanes >> 3)) & 1
    slot_of = np.arange(2)[None, :] ^ sw[:, None]           # [lane][slot] -> quartet held
    img = img[:, :, :, :, :, lanes[:, None], slot_of, :]
    return np.ascontiguousarray(img)


def emit_hip_module(graph: Graph, schedule_fn: Optional[ScheduleFn] = None, *,
                    conv_mode: str = "implicit", int8_depthwise: str = "mfma",
                    small_conv: bool = True, winograd="auto", pair_convs: bool = True) -> HipModule:
    return HipCodegen(schedule_fn, conv_mode=conv_mode, int8_depthwise=int8_depthwise,
                      small_conv=small_conv, winograd=winograd, pair_convs=pair_convs).lower(graph)
