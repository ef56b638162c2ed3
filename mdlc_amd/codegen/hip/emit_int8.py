"""INT8 lowering for the HIP codegen (a mixin of ``HipCodegen``).

The quantized ops (semantics in the oracle's ``quant`` module and the
model builder) lower to the int8 kernels of ``kernels/int8.hip``. int8
activations are channels-last (NHWC) on the device — recorded in
``HipModule.device_layout`` — so both MFMA operands are contiguous along K:
a 1x1 conv is a plain GEMM over the NHWC input, a kxk conv gathers one
filter tap's channels per 16-byte load, and conv weights are packed with k
ordered (kh, kw, c).
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.codegen.hip import templates as T
from mdlc_amd.codegen.hip.plan import Launch, round16
from mdlc_amd.codegen.schedule import (
    LDS_LIMIT, default_qdw_schedule, default_qschedule, qdw_valid, qmlp_latency_form, qmlp_layout,
    qconv_first_band, qconv_first_grid, qmlp_lds_bytes, qsched_valid,
)
from mdlc_amd.passes.shape_inference import conv_geometry


def wdev_bytes(nob: int, ns: int) -> int:
    """Bytes of the first int8 conv's packed MFMA weight fragments."""
    return nob * ns * 64 * 16


class Int8LoweringMixin:

    def _pack_raw(self, name, array):
        self.consts[name] = np.ascontiguousarray(array)
        return name

    def _qsched(self, node, mnk, problem):
        fn = getattr(self.schedule_fn, "schedule_problem", None)
        sched = fn(problem) if fn is not None else self.schedule_fn(node, mnk)
        if sched is None or not qsched_valid(sched):
            sched = default_qschedule(*mnk)
        return sched

    def _check_dtype(self, g, name, want):
        info = g.info(name)
        if info is None or info.dtype != want:
            raise ValueError(f"{name!r} is {None if info is None else info.dtype}, the kernel "
                             f"writes {want}; rerun shape inference")

    def _emit_qgemm(self, node, sched, a_in, b_dev, bias, mult, out, meta, *, amode, out_f32, lo, win,
                    gv=16, epi=0, aux=None, depthwise=False, out_i32=False):
        """One int8 GEMM launch. The kernel reads bias and mult four columns
        at a time, so both are packed zero padded to a multiple of 16; its
        buffer loads take 32-bit offsets, so every operand stays under 2 GiB."""
        M, N, K = meta["M"], meta["N"], meta["K"]
        g = self._graph
        self._check_dtype(g, a_in, "int8")
        self._check_dtype(g, out, "float32" if out_f32 else ("int32" if out_i32 else "int8"))
        if meta["ldb"] % sched.BK or meta["ldb"] < K:
            raise ValueError(f"int8 weights must be padded to a multiple of BK={sched.BK}")
        a_bytes = (M * meta["lda"] if amode == 0 else
                   (M // (meta["OH"] * meta["OW"])) * meta["H"] * meta["W"] * meta["Cin"])
        if max(a_bytes, N * meta["ldb"], M * meta["ldc"]) >= 2 ** 31 - 2 ** 20:
            raise NotImplementedError("HIP codegen: int8 GEMM operand of 2 GiB or more")
        for name in (bias, mult):
            if not g.is_constant(name):
                raise NotImplementedError("HIP codegen: int8 bias and multipliers must be constants")
        n16 = round16(N)
        bpad = np.zeros(n16, np.int32)
        bpad[:N] = np.asarray(g.initializers[bias], np.int32).ravel()
        mpad = np.zeros(n16, np.float32)
        mpad[:N] = np.asarray(g.initializers[mult], np.float32).ravel()
        bias_dev = self._pack_raw(f"{bias}__dev{n16}", bpad)
        mult_dev = self._pack_raw(f"{mult}__dev{n16}", mpad)
        cin = sched.BN if depthwise else (meta["Cin"] if amode else 0)
        sig = ("qgemm", sched, amode, gv, cin, out_f32, lo, win, epi, depthwise, out_i32)
        tag = "qdwmfma" if depthwise else ("qconv" if amode else "qgemm")
        etag = ("", "_lut", "_add")[epi]
        kname = self._kernel(sig, lambda i: T.qgemm_kernel(
            f"{tag}_{sched.key()}_a{amode}{'' if not amode else f'g{gv}'}_"
            f"{'f32' if out_f32 else ('i32' if out_i32 else 'i8')}{etag}_{i}", sched, amode=amode,
            out_f32=out_f32, lo=lo, win=win, gv=gv, cin=cin, epi=epi, depthwise=depthwise,
            out_i32=out_i32))
        tiles = -(-M // sched.BM) * -(-N // sched.BN)
        ins = [a_in, b_dev, bias_dev, mult_dev] + ([aux] if aux else [])
        # algorithmic HBM bytes: activation, weights, bias/mult, output, residual
        a_read = a_bytes if amode else M * K
        w_read = N * (K // sched.BN if depthwise else K)
        ops = meta.get("depthwise_ops", 2 * M * N * K)
        nbytes = (a_read + w_read + 8 * N + M * N * (4 if out_f32 or out_i32 else 1)
                  + (M * N if epi == 2 else 0))
        self.plan.append(Launch("qgemm", kname, ins, [out], (tiles, 1, 1),
                                (sched.threads_per_block(), 1, 1),
                                dict(meta, node=node, sched=sched, ops=ops, bytes=nbytes,
                                     epilogue=epi)))

    def _lower_quantizelinear(self, g, node):
        """float32 -> int8 codes; a 4-D NCHW input becomes channels-last."""
        x, y = node.inputs[0], node.outputs[0]
        shp = self._shape(g, x)
        if len(shp) == 4:
            n, c, hw = shp[0], shp[1], shp[2] * shp[3]
            self.layout[y] = "NHWC"
        else:
            n, c, hw = 1, 1, int(np.prod(shp))
        self._kernel("quantize", lambda i: T.quantize_kernel("quantize_nchw_nhwc"))
        total = n * c * hw
        self.plan.append(Launch("quantize", "quantize_nchw_nhwc", [x], [y], (-(-total // 256), 1, 1),
                                (256, 1, 1), {"N": n, "C": c, "HW": hw,
                                              "inv_s": float(node.attrs["inv_scale"]), "node": node,
                                              "bytes": 5 * total}))

    def _lower_qconv_first(self, g, node):
        """A QConv that quantizes its own float32 NCHW input (at most four
        channels): one workgroup per band of output rows quantizes the band's
        input into LDS once and forms the outputs on 16x16x64 int8 MFMAs."""
        x, w, b, m = node.inputs[:4]
        geo = conv_geometry(node, self._shape(g, x), self._shape(g, w))
        OC, C, KH, KW = geo["OC"], geo["C"], geo["KH"], geo["KW"]
        band = None
        if geo["group"] == 1 and geo["DH"] == 1 and geo["DW"] == 1:
            band = qconv_first_band(C, KH, KW, geo["SH"], geo["SW"], geo["N"], geo["OH"], geo["OW"], OC)
        if band is None:
            raise NotImplementedError("HIP codegen: fused input quantization needs a small "
                                      "ungrouped conv (C <= 4, KH*KW <= 32, OC <= 64 and % 4 == 0, "
                                      "no dilation, a band of output rows within the LDS)")
        self._check_dtype(g, x, "float32")
        y = node.outputs[0]
        self.layout[y] = "NHWC"
        # row operand fragments: [block][step][lane 16 lk + li][word j] = the C
        # weight bytes of output channel 16 block + li at tap 16 step + 4 lk + j
        T_, nob, ns = KH * KW, -(-OC // 16), -(-KH * KW // 16)
        wq = np.asarray(g.initializers[w], np.int8).reshape(OC, C, T_).transpose(0, 2, 1)
        wb = np.zeros((16 * nob, 16 * ns, 4), np.int8)
        wb[:OC, :T_, :C] = wq
        words = wb.view(np.int32).reshape(nob, 16, ns, 4, 4)            # [ob][li][s][lk][j]
        wdev = self._pack_raw(f"{w}__dev_qfirst", np.ascontiguousarray(words.transpose(0, 2, 3, 1, 4)))
        epi, tab = 0, None
        kind = node.attrs.get("epilogue")
        if kind == "lut":
            epi, tab = 1, node.inputs[4]
            if not g.is_constant(tab) or np.asarray(g.initializers[tab]).size != 256:
                raise NotImplementedError("HIP codegen: a fused lookup needs a constant 256-entry table")
        elif kind:
            raise NotImplementedError(f"HIP codegen: epilogue {kind!r} on a conv that quantizes its input")
        lo = 0 if node.attrs.get("activation") == "Relu" else -127
        win = (KH, KW, geo["SH"], geo["SW"], geo["PT"], geo["PL"])
        dims = (geo["H"], geo["W"], geo["OH"], geo["OW"])
        kname = self._kernel(("qconv_first", C, win, OC, lo, epi, dims, band), lambda i: T.qconv_first_kernel(
            f"qconv_first_c{C}_{'x'.join(map(str, win))}_oc{OC}_R{band}{'_lut' if epi else ''}_{i}", C, win,
            OC, dims, band, lo=lo, epi=epi))
        P = geo["N"] * geo["OH"] * geo["OW"]
        if P * OC >= 2 ** 31 or 4 * C * geo["H"] * geo["W"] >= 2 ** 31:
            raise NotImplementedError("HIP codegen: int8 conv tensors of 2 GiB or more")
        ins = [x, wdev, self._padded_vector(g, b, OC, np.int32), self._padded_vector(g, m, OC, np.float32)]
        grid = (min(geo["N"] * -(-geo["OH"] // band), qconv_first_grid()), 1, 1)
        self.plan.append(Launch(
            "qconv_first", kname, ins + ([tab] if tab else []), [y], grid, (256, 1, 1),
            {**{k: geo[k] for k in ("N", "H", "W", "OH", "OW")}, "inv_s": float(node.attrs["quantize_input"]),
             "node": node, "band": band, "ops": 2 * P * OC * C * KH * KW,
             "bytes": 4 * geo["N"] * C * geo["H"] * geo["W"] + P * OC + wdev_bytes(nob, ns) + OC * 8}))

    def _lower_qconv(self, g, node):
        if node.attrs.get("quantize_input") is not None:
            self._lower_qconv_first(g, node)
            return
        x, w, b, m = node.inputs[:4]
        if self.layout.get(x) != "NHWC":
            raise NotImplementedError("HIP codegen: QConv input must come from the int8 path")
        geo = conv_geometry(node, self._shape(g, x), self._shape(g, w))
        lo = 0 if node.attrs.get("activation") == "Relu" else -127
        y = node.outputs[0]
        self.layout[y] = "NHWC"
        warr = np.asarray(g.initializers[w], np.int8)
        if geo["group"] != 1:
            if node.attrs.get("epilogue"):
                raise NotImplementedError("HIP codegen: fused epilogue on a grouped int8 conv")
            if geo["ICG"] != 1 or geo["OC"] != geo["C"]:
                raise NotImplementedError("HIP codegen: int8 grouped conv (only depthwise)")
            C = geo["C"]
            if C % 16 == 0 and self.int8_depthwise_mfma:
                self._lower_qdw_mfma(g, node, geo, warr, lo)
                return
            win = (geo["KH"], geo["KW"], geo["SH"], geo["SW"], geo["DH"], geo["DW"])
            cv = 16 if C % 16 == 0 else 1
            kname = self._kernel(("qdw", win, cv, lo), lambda i: T.qdwconv_kernel(
                f"qdwconv_{'x'.join(map(str, win))}_c{cv}_{i}", win, cv=cv, lo=lo))
            wdev = self._pack_raw(f"{w}__dev_khkwc", warr.reshape(C, geo["KH"], geo["KW"])
                                  .transpose(1, 2, 0).copy())
            total = geo["N"] * geo["OH"] * geo["OW"] * (C // cv)
            self.plan.append(Launch(
                "qdwconv", kname, [x, wdev, b, m], [y], (-(-total // 256), 1, 1), (256, 1, 1),
                {**{k: geo[k] for k in ("N", "C", "H", "W", "OH", "OW", "PT", "PL")}, "node": node,
                 "ops": 2 * geo["N"] * C * geo["OH"] * geo["OW"] * geo["KH"] * geo["KW"]}))
            return
        OC, C, KH, KW = geo["OC"], geo["C"], geo["KH"], geo["KW"]
        K = C * KH * KW
        P = geo["N"] * geo["OH"] * geo["OW"]
        pointwise = (KH == KW == 1 and geo["SH"] == geo["SW"] == 1 and
                     geo["PT"] == geo["PL"] == geo["PB"] == geo["PR"] == 0)
        # gather width: the widest of 16/8/4/2/1 bytes that divides Cin
        gv = next(v for v in (16, 8, 4, 2, 1) if C % v == 0)
        amode = 0 if pointwise and gv == 16 else 1
        problem = {"kind": "qconv", "M": P, "N": OC, "K": K, "amode": amode, "gv": gv,
                   "batch": geo["N"], "relu": lo == 0,
                   **{k: geo[k] for k in ("C", "H", "W", "KH", "KW", "SH", "SW", "DH", "DW",
                                          "PT", "PB", "PL", "PR", "OH", "OW")}}
        sched = self._qsched(node, (P, OC, K), problem)
        ldb = -(-K // sched.BK) * sched.BK
        wt = np.zeros((OC, ldb), np.int8)
        wt[:, :K] = warr.transpose(0, 2, 3, 1).reshape(OC, K)        # k = (kh, kw, c)
        wdev = self._pack_raw(f"{w}__dev_tap{ldb}", wt)
        win = (KH, KW, geo["SH"], geo["SW"], geo["DH"], geo["DW"], geo["PT"], geo["PL"])
        meta = {"M": P, "N": OC, "K": K, "lda": C, "ldb": ldb, "ldc": OC, "Cin": C,
                "H": geo["H"], "W": geo["W"], "OH": geo["OH"], "OW": geo["OW"]}
        epi, aux = 0, None
        kind = node.attrs.get("epilogue")
        if kind == "lut":
            epi, aux = 1, node.inputs[4]
            if not g.is_constant(aux) or np.asarray(g.initializers[aux]).size != 256:
                raise NotImplementedError("HIP codegen: a fused lookup needs a constant 256-entry table")
        elif kind == "add":
            epi, aux = 2, node.inputs[4]
            if self.layout.get(aux) != "NHWC" or self._shape(g, aux) != self._shape(g, y):
                raise NotImplementedError("HIP codegen: a fused residual must match the conv output")
            meta.update(res_mult=float(node.attrs["res_mult"]), acc_mult=float(node.attrs["acc_mult"]))
        elif kind:
            raise NotImplementedError(f"HIP codegen: QConv epilogue {kind!r}")
        self._emit_qgemm(node, sched, x, wdev, b, m, y, meta, amode=amode, out_f32=False, lo=lo,
                         win=None if amode == 0 else win, gv=gv, epi=epi, aux=aux)

    def _lower_qdw_mfma(self, g, node, geo, warr, lo):
        """Depthwise int8 conv (C % 16 == 0) on the matrix cores: 16-channel
        blocks, k = (tap, channel within the block), block-diagonal weights."""
        x, _, b, m = node.inputs[:4]
        y = node.outputs[0]
        C, KH, KW = geo["C"], geo["KH"], geo["KW"]
        P = geo["N"] * geo["OH"] * geo["OW"]
        problem = {"kind": "qdw", "M": P, "N": C, "K": KH * KW * 16, "batch": geo["N"],
                   "relu": lo == 0,
                   **{k: geo[k] for k in ("C", "H", "W", "KH", "KW", "SH", "SW", "DH", "DW",
                                          "PT", "PB", "PL", "PR", "OH", "OW")}}
        fn = getattr(self.schedule_fn, "schedule_problem", None)
        sched = fn(problem) if fn is not None else self.schedule_fn(node, (P, C, problem["K"]))
        if sched is None or not qdw_valid(sched):
            sched = default_qdw_schedule(P)
        K = KH * KW * sched.BN
        ldb = -(-K // sched.BK) * sched.BK
        wt = np.zeros((C, ldb), np.int8)
        n = np.arange(C)
        taps = warr.reshape(C, KH * KW)
        for t in range(KH * KW):
            wt[n, t * sched.BN + n % sched.BN] = taps[:, t]
        wdev = self._pack_raw(f"{node.inputs[1]}__dev_blockdiag{ldb}", wt)
        win = (KH, KW, geo["SH"], geo["SW"], geo["DH"], geo["DW"], geo["PT"], geo["PL"])
        meta = {"M": P, "N": C, "K": K, "lda": C, "ldb": ldb, "ldc": C, "Cin": C,
                "H": geo["H"], "W": geo["W"], "OH": geo["OH"], "OW": geo["OW"],
                "depthwise_ops": 2 * P * C * KH * KW}
        self._emit_qgemm(node, sched, x, wdev, b, m, y, meta, amode=1, out_f32=False, lo=lo, win=win,
                         gv=16, depthwise=True)

    def _padded_vector(self, g, name, n, dtype):
        """A constant per-channel vector packed zero padded to a multiple of 16."""
        n16 = round16(n)
        out = np.zeros(n16, dtype)
        out[:n] = np.asarray(g.initializers[name], dtype).ravel()
        return self._pack_raw(f"{name}__dev{n16}", out)

    def _lower_qmlp(self, g, node):
        """The fused channel mixer: h = T[q1(x W1^T + b1)], y = qadd(x, q2(h W2^T + b2)),
        both GEMMs over the NHWC rows of x in one launch (``qmlp_i8``); with a
        token mixer, x = qdw(z) is computed in the same launch."""
        mixer = node.attrs.get("mixer")
        x, w1, b1, m1, tab, w2, b2, m2 = [node.inputs[0]] + list(node.inputs[4 if mixer else 1:])
        if self.layout.get(x) != "NHWC":
            raise NotImplementedError("HIP codegen: QMlp input must come from the int8 path")
        n, C, H, W = self._shape(g, x)
        M = n * H * W
        W1 = np.asarray(g.initializers[w1], np.int8)
        W2 = np.asarray(g.initializers[w2], np.int8)
        E = W1.shape[0]
        if W1.reshape(E, -1).shape[1] != C or W2.reshape(W2.shape[0], -1).shape != (C, E):
            raise ValueError("QMlp weights do not match the input's channels")
        if np.asarray(g.initializers[tab]).size != 256:
            raise NotImplementedError("HIP codegen: QMlp needs a constant 256-entry table")
        taps = int(np.prod(mixer["kernel_shape"])) if mixer else 0
        lay = self._qmlp_layout(node, C, E, M, taps)
        if lay is None:
            raise NotImplementedError(f"HIP codegen: no fused MLP tiling for C={C}, E={E}")
        if M * C >= 2 ** 31 - 2 ** 20:
            raise NotImplementedError("HIP codegen: int8 MLP operand of 2 GiB or more")
        self._check_dtype(g, x, "int8")
        y = node.outputs[0]
        self._check_dtype(g, y, "int8")
        self.layout[y] = "NHWC"
        CP, EP = -(-C // 64) * 64, -(-E // 64) * 64
        w1p = np.zeros((E, CP), np.int8)
        w1p[:, :C] = W1.reshape(E, C)
        w2p = np.zeros((C, EP), np.int8)
        w2p[:, :E] = W2.reshape(C, E)
        ins = [x, self._pack_raw(f"{w1}__dev_mlp{CP}", w1p), self._padded_vector(g, b1, E, np.int32),
               self._padded_vector(g, m1, E, np.float32), tab,
               self._pack_raw(f"{w2}__dev_mlp{EP}", w2p), self._padded_vector(g, b2, C, np.int32),
               self._padded_vector(g, m2, C, np.float32)]
        lo1 = 0 if node.attrs.get("activation1") == "Relu" else -127
        lo2 = 0 if node.attrs.get("activation2") == "Relu" else -127
        mix, ops, wbytes = None, 4 * M * C * E, 0
        if mixer:
            wd, bd, md = node.inputs[1:4]
            kh, kw = mixer["kernel_shape"]
            wdarr = np.asarray(g.initializers[wd], np.int8)
            if wdarr.shape != (C, 1, kh, kw) or C % 16:
                raise NotImplementedError("HIP codegen: QMlp token mixer must be depthwise over C % 16 == 0")
            # the image size is compiled in (the pixel decomposition divides by it)
            mix = (kh, kw, mixer["pads"][0], mixer["pads"][1],
                   0 if mixer.get("activation") == "Relu" else -127, H, W)
            # block-diagonal [C][KD]: k = (tap, channel within its 16-channel block)
            taps = kh * kw
            kd = -(-taps * 16 // 64) * 64
            wbd = np.zeros((C, kd), np.int8)
            ch = np.arange(C)
            for t in range(taps):
                wbd[ch, t * 16 + ch % 16] = wdarr.reshape(C, taps)[:, t]
            ins[1:1] = [self._pack_raw(f"{wd}__dev_blockdiag{kd}", wbd),
                        self._padded_vector(g, bd, C, np.int32), self._padded_vector(g, md, C, np.float32)]
            ops += 2 * M * C * kh * kw
            wbytes = C * (kh * kw + 8)
        mixb, ew2, wregs = qmlp_latency_form(C, E, M, lay, mix)
        kname = self._kernel(("qmlp", C, E, lay, lo1, lo2, mix, mixb, ew2, wregs), lambda i: T.qmlp_kernel(
            f"qmlp_c{C}_e{E}_{lay.key()}{'_dw%dx%d' % mix[:2] if mix else ''}"
            f"{'_b%d' % mixb if mixb != 3 else ''}{'_w2' if ew2 else ''}{'_wr' if wregs else ''}_{i}",
            C, E, lay, lo1=lo1, lo2=lo2, mixer=mix, mix_batch=mixb, early_w2=ew2, mixer_regs=wregs))
        self.plan.append(Launch(
            "qmlp", kname, ins, [y], (-(-M // lay.BM), 1, 1), (256, 1, 1),
            {"M": M, "C": C, "E": E, "H": H, "W": W, "layout": lay, "node": node, "mixer": bool(mix),
             "res_mult": float(node.attrs["res_mult"]), "acc_mult": float(node.attrs["acc_mult"]),
             "ops": ops,
             # algorithmic HBM bytes: x (or z) once, y once, the weights, bias and mult
             "bytes": 2 * M * C + 2 * C * E + 8 * (C + E) + 256 + wbytes}))

    def _qmlp_layout(self, node, C, E, M, taps):
        """The schedule source's tiling when it gives one that fits LDS with
        the node's token mixer, else the default for these sizes."""
        fn = getattr(self.schedule_fn, "qmlp_layout", None)
        lay = fn(C, E, M) if fn is not None else None
        if lay is not None and qmlp_lds_bytes(C, E, lay.BM, taps) <= LDS_LIMIT:
            return lay
        return qmlp_layout(C, E, M, mixer_taps=taps)

    def _lower_qgemm(self, g, node):
        x, w, b, m = node.inputs[:4]
        if not node.attrs.get("transB", 0):
            raise NotImplementedError("HIP codegen: QGemm expects the weight as [N][K] (transB=1)")
        M, K = self._shape(g, x)
        N = self._shape(g, w)[0]
        out_dtype = node.attrs.get("out_dtype", "int8")
        out_f32, out_i32 = out_dtype == "float32", out_dtype == "int32"
        lo = 0 if node.attrs.get("activation") == "Relu" else -127
        if K % 16:
            raise NotImplementedError("HIP codegen: QGemm needs K % 16 == 0")
        sched = self._qsched(node, (M, N, K), {"kind": "qgemm", "M": M, "N": N, "K": K,
                                               "out_f32": out_f32})
        ldb = -(-K // sched.BK) * sched.BK
        wt = np.zeros((N, ldb), np.int8)
        wt[:, :K] = np.asarray(g.initializers[w], np.int8)
        wdev = self._pack_raw(f"{w}__dev{ldb}", wt)
        meta = {"M": M, "N": N, "K": K, "lda": K, "ldb": ldb, "ldc": N, "Cin": 0, "H": 0, "W": 0,
                "OH": 0, "OW": 0}
        self._emit_qgemm(node, sched, x, wdev, b, m, node.outputs[0], meta, amode=0,
                         out_f32=out_f32, lo=lo, win=None, out_i32=out_i32)

    def _lower_qadd(self, g, node):
        a, b = node.inputs[:2]
        if self._shape(g, a) != self._shape(g, b):
            raise NotImplementedError("HIP codegen: QAdd operands must have equal shapes")
        if self.layout.get(a) != self.layout.get(b):
            raise NotImplementedError("HIP codegen: QAdd operands in different layouts")
        y = node.outputs[0]
        if a in self.layout:
            self.layout[y] = self.layout[a]
        n = int(np.prod(self._shape(g, a)))
        self._kernel("qadd", lambda i: T.qadd_kernel("qadd"))
        threads = n // 16 + n % 16
        self.plan.append(Launch("qadd", "qadd", [a, b], [y], (max(1, -(-threads // 256)), 1, 1),
                                (256, 1, 1), {"n": n, "ma": float(node.attrs["ma"]),
                                              "mb": float(node.attrs["mb"]), "node": node,
                                              "bytes": 3 * n}))

    def _lower_qlut(self, g, node):
        x, t = node.inputs[:2]
        if np.asarray(g.initializers[t]).size != 256:
            raise NotImplementedError("HIP codegen: QLut needs a 256-entry table")
        y = node.outputs[0]
        if x in self.layout:
            self.layout[y] = self.layout[x]
        n = int(np.prod(self._shape(g, x)))
        self._kernel("qlut", lambda i: T.qlut_kernel("qlut"))
        threads = n // 16 + n % 16
        self.plan.append(Launch("qlut", "qlut", [x, t], [y], (max(1, -(-threads // 256)), 1, 1),
                                (256, 1, 1), {"n": n, "node": node, "bytes": 2 * n}))

    def _lower_qglobalaveragepool(self, g, node):
        x = node.inputs[0]
        n, c, h, w = self._shape(g, x)
        if self.layout.get(x) != "NHWC":
            raise NotImplementedError("HIP codegen: QGlobalAveragePool expects the int8 path")
        per_image = c % 4 == 0 and c <= 1024
        kname = "qgap_wg" if per_image else "qgap"
        self._kernel(kname, lambda i: T.qgap_kernel(kname, per_image))
        self.layout[node.outputs[0]] = "NHWC"
        # per image, blocks of 64 channels where they divide C (16 channel
        # quads x 16 pixel lanes a workgroup), else all of C
        cblocks = c // 64 if per_image and c % 64 == 0 else 1
        grid = (n, cblocks, 1) if per_image else (-(-(n * c) // 256), 1, 1)
        self.plan.append(Launch("qgap", kname, [x], [node.outputs[0]], grid,
                                (256, 1, 1), {"N": n, "C": c, "HW": h * w,
                                              "m": float(node.attrs["mult"]), "node": node,
                                              "bytes": n * c * (h * w + 1)}))

    def _lower_dequantizelinear(self, g, node):
        x = node.inputs[0]
        shp = self._shape(g, x)
        n = int(np.prod(shp))
        nhwc = self.layout.get(x) == "NHWC" and len(shp) == 4
        C, HW = (shp[1], shp[2] * shp[3]) if nhwc else (1, 1)
        self._kernel("dequant", lambda i: T.dequantize_kernel("dequantize"))
        self.plan.append(Launch("dequantize", "dequantize", [x], [node.outputs[0]],
                                (-(-n // 256), 1, 1), (256, 1, 1),
                                {"n": n, "C": C, "HW": HW, "s": float(node.attrs["scale"]),
                                 "node": node, "bytes": 5 * n}))
