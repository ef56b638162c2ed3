"""HIP kernel generators for gfx950.

Each fused-group kind has a hand-written HIP template under ``kernels/``
(C++ templates in namespace ``mdlc``); this module writes the small
``extern "C"`` wrappers that instantiate them for one group — tile schedule,
epilogue (bias + activation baked in as code), convolution window, vector
paths — plus the string-generated body of elementwise chains. Together they
replace the CUDA string templates of mdlc/codegen/cuda/templates.py:
``activation_expr`` (:24-51), ``gemm_kernel`` (:56-160), ``im2col_kernel``
(:165-201) and ``elementwise_kernel`` (:209-269).

Floating-point constants are emitted as exact hexadecimal literals so the
kernel uses the same float32 bits as the NumPy oracle.
"""

from __future__ import annotations

import os
import re
from typing import Optional

from mdlc_amd.codegen.schedule import MfmaSchedule
from mdlc_amd.ir import Node

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")


def library_source(part: str) -> str:
    with open(os.path.join(KERNEL_DIR, part + ".hip")) as f:
        return f.read()


def flit(x: float) -> str:
    """An exact float32 literal for ``x`` (``x`` is first rounded to float32)."""
    import numpy as np

    v = float(np.float32(x))
    if v != v:
        return "__builtin_nanf(\"\")"
    if v in (float("inf"), float("-inf")):
        return "__builtin_inff()" if v > 0 else "(-__builtin_inff())"
    return f"{v.hex()}f"


# ----- activation epilogue ------------------------------------------------

def activation_expr(activation: Optional[str], var: str, attrs: dict) -> str:
    """A HIP expression applying ``activation`` to float ``var``, with the
    NumPy float32 semantics of the oracle (mdlc/runtime/ops.py:155-185)."""
    v = var
    if not activation or activation == "Identity":
        return v
    if activation == "Relu":
        return f"fmaxf({v}, 0.0f)"
    if activation == "Relu6":
        return f"fminf(fmaxf({v}, 0.0f), 6.0f)"
    if activation == "Clip":
        lo, hi = attrs.get("clip_min"), attrs.get("clip_max")
        e = v if lo is None else f"fmaxf({v}, {flit(lo)})"
        return e if hi is None else f"fminf({e}, {flit(hi)})"
    if activation == "Sigmoid":
        return f"(1.0f / (1.0f + expf(-({v}))))"
    if activation == "Tanh":
        return f"tanhf({v})"
    if activation == "LeakyRelu":
        a = flit(attrs.get("alpha", 0.01))
        return f"(({v}) >= 0.0f ? ({v}) : {a} * ({v}))"
    if activation == "HardSigmoid":
        a, b = flit(attrs.get("alpha", 0.2)), flit(attrs.get("beta", 0.5))
        return f"fminf(fmaxf({a} * ({v}) + {b}, 0.0f), 1.0f)"
    if activation == "HardSwish":
        return f"(({v}) * fminf(fmaxf(({v}) / 6.0f + 0.5f, 0.0f), 1.0f))"
    raise NotImplementedError(f"no HIP epilogue for activation {activation!r}")


BIAS_CODE = {None: 0, "none": 0, "row": 1, "col": 2}


def epilogue_struct(name: str, *, bias_mode: Optional[str], activation: Optional[str],
                    attrs: dict, alpha: float = 1.0, beta: float = 1.0,
                    residual: Optional[str] = None) -> str:
    """``struct name { bias; residual; apply(acc, b); post(v, r) }``:
    alpha*acc (+ beta*b), then the activation — the order of
    mdlc/runtime/ops.py:84-92 followed by the act — and, for a folded
    residual group, ``post`` (the group's code on the conv value and the
    residual element; see ``residual_post_body``)."""
    code = BIAS_CODE[bias_mode]
    lines = ["float v = acc;"]
    if float(alpha) != 1.0:
        lines.append(f"v = {flit(alpha)} * v;")
    if code:
        lines.append("v = v + b;" if float(beta) == 1.0 else f"v = v + {flit(beta)} * b;")
    lines.append(f"return {activation_expr(activation, 'v', attrs)};")
    body = " ".join(lines)
    post = residual or "return v;"
    return (f"struct {name} {{\n  static constexpr int bias = {code};\n"
            f"  static constexpr bool residual = {'true' if residual else 'false'};\n"
            f"  __device__ __forceinline__ static float apply(float acc, float b) {{ {body} }}\n"
            f"  __device__ __forceinline__ static float post(float v, float r) {{ {post} }}\n}};\n")


def residual_post_body(sub: list, y: str, r: str, consts: dict) -> str:
    """The body of ``post(v, r)`` for a folded residual group: ``sub`` is the
    group's members (an Add of the conv output ``y`` and the residual ``r``,
    then single-input pointwise ops), evaluated one float32 operation per
    member exactly as the elementwise kernel would, with ``y`` read as ``v``
    and ``r`` as ``r``."""
    names = {y: "v", r: "r"}
    lines = []

    def ref(e: str) -> str:
        return flit(consts[e]) if e in consts else _cname(e, names)

    for n in sub:
        out = _cname(n.outputs[0], names)
        lines.append(f"float {out} = {_member_expr(n, ref, consts)};")
    lines.append(f"return {names[sub[-1].outputs[0]]};")
    return " ".join(lines)


# ----- GEMM / conv ----------------------------------------------------------

def gemm_kernel(name: str, sched: MfmaSchedule, *, with_bias: bool, bias_mode: str = "col",
                activation: Optional[str] = None, attrs: Optional[dict] = None,
                alpha: float = 1.0, beta: float = 1.0, bmode: int = 0, out_nchw: bool = False,
                vec_a: bool = True, win: Optional[tuple] = None,
                residual: Optional[str] = None, stream_k: int = 0,
                grouped: bool = False) -> tuple:
    """(name, source) of one GEMM instantiation.

    Kernel ABI (the reference's gemm ABI plus trailing layout arguments):
      dense  (bmode 0/1): (A, B, [bias], [res], C, int M, int N, int K, int lda, int ldb,
                           int ldc, int hw, int ksplit, int kchunk)
      conv   (bmode 2/3): (W, x, [bias], [res], y, int M, int N, int K, int lda,
                           int Cin, int H, int W, int OH, int OW, int ksplit, int kchunk)
    ``hw`` > 0 selects the NCHW output scatter for conv-as-GEMM; ``res`` is a
    folded residual read at each output's own position (``residual`` is the
    body of the epilogue's ``post``). With ``sched.SK > 1`` the kernel writes
    raw partial sums of each K slice to its C argument (the split-K
    workspace) and takes no bias or residual; the epilogue then lives in
    ``splitk_reduce_kernel``. With ``stream_k`` = SKW > 0 a workspace pointer
    ``ws`` precedes the output, ``ksplit`` is the number of tiles done whole
    and the last SKW workgroups compute the remaining tiles in pieces
    (``streamk_fixup_kernel`` finishes them). ``grouped`` (conv only): one
    launch runs every group of a grouped convolution, blockIdx.y selecting
    the group's weights, input channels, bias, residual and output channels;
    two trailing arguments give the whole input and output image strides.
    """
    attrs = attrs or {}
    s = sched
    split = s.SK > 1
    if split:
        with_bias = False
        residual = None
    epi = f"{name}_epi"
    src = [epilogue_struct(epi, bias_mode=bias_mode if with_bias else None,
                           activation=None if split else activation, attrs=attrs,
                           alpha=1.0 if split else alpha, beta=beta, residual=residual)]
    winty = "mdlc::NoWin" if win is None else "mdlc::ConvWin<%d, %d, %d, %d, %d, %d, %d, %d>" % tuple(win)
    bias_arg = ("const float* __restrict__ bias, " if with_bias else "") + \
        ("const float* __restrict__ res, " if residual else "")
    bias_val = ("bias" if with_bias else "nullptr") + (", res" if residual else ", nullptr")
    out = 2 if split else (1 if out_nchw else 0)
    tmpl = (f"mdlc::gemm_f32_mfma<{s.BM}, {s.BN}, {s.BK}, {s.WGM}, {s.WGN}, {s.MS}, "
            f"{'true' if s.DB else 'false'}, {'true' if vec_a else 'false'}, {bmode}, "
            f"{out}, {epi}, {winty}, {int(stream_k)}, {s.UN}>")
    nt = s.threads_per_block()
    ws_arg = "float* __restrict__ ws, " if stream_k else ""
    ws_val = "ws" if stream_k else "nullptr"
    if grouped and (split or stream_k or bmode < 2):
        raise ValueError("a grouped convolution runs the implicit gather without split-K or stream-K")
    if bmode >= 2:
        # grouped: blockIdx.y is the group; M, Cin and the weights are one
        # group's, ximg / cimg the whole images' strides
        shift = ""
        if grouped:
            shift = ("  const size_t grp = blockIdx.y;\n"
                     "  A += grp * M * lda; x += grp * Cin * H * W; y += grp * M * OH * OW;\n"
                     + ("  bias += grp * M;\n" if with_bias else "")
                     + ("  res += grp * M * OH * OW;\n" if residual else ""))
        strides = ", int ximg, int cimg" if grouped else ""
        img = "ximg, cimg" if grouped else "Cin * H * W, M * OH * OW"
        src.append(
            f'extern "C" __global__ __launch_bounds__({nt}) void {name}(\n'
            f"    const float* __restrict__ A, const float* __restrict__ x, {bias_arg}{ws_arg}"
            f"float* __restrict__ y,\n    int M, int N, int K, int lda, int Cin, int H, int W, "
            f"int OH, int OW, int ksplit, int kchunk{strides}) {{\n{shift}"
            f"  mdlc::GemmArgs g{{A, x, {bias_val}, y, M, N, K, lda, 0, 0, OH * OW, Cin, H, W, OH, OW, "
            f"ksplit, kchunk, {ws_val}, {img}}};\n"
            f"  {tmpl}(g);\n}}\n")
    else:
        src.append(
            f'extern "C" __global__ __launch_bounds__({nt}) void {name}(\n'
            f"    const float* __restrict__ A, const float* __restrict__ B, {bias_arg}{ws_arg}"
            f"float* __restrict__ C,\n    int M, int N, int K, int lda, int ldb, int ldc, int hw, "
            f"int ksplit, int kchunk) {{\n"
            f"  mdlc::GemmArgs g{{A, B, {bias_val}, C, M, N, K, lda, ldb, ldc, hw, 0, 0, 0, 0, 0, "
            f"ksplit, kchunk, {ws_val}, 0, M * hw}};\n"
            f"  {tmpl}(g);\n}}\n")
    return name, "\n".join(src)


def gemm_wsplit_kernel(name: str, sched: MfmaSchedule, *, with_bias: bool, bias_mode: str,
                       activation: Optional[str], attrs: dict, alpha: float = 1.0,
                       beta: float = 1.0, vec_a: bool, b_kn: bool) -> tuple:
    """The wave-split GEMM (``sched.WK`` waves share the K range of one
    tile). ABI: (A, B, [bias], C, int M, int N, int K, int lda, int ldb,
    int ldc, int kchunk); one workgroup of 64 * WK threads per BM x BN tile,
    m fastest. ``b_kn``: B is stored [N][ldb] (K contiguous per output
    column). With ``sched.SK > 1`` grid y is the K slice (``kchunk`` values
    of K each) and C the split-K workspace: raw partial sums, no bias or
    epilogue (``splitk_reduce_kernel`` finishes)."""
    s = sched
    split = s.SK > 1
    if split:
        with_bias, activation, alpha = False, None, 1.0
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode=bias_mode if with_bias else None, activation=activation,
                          attrs=attrs, alpha=alpha, beta=beta)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    return name, src + (
        f'extern "C" __global__ __launch_bounds__({s.threads_per_block()}) void {name}(\n'
        f"    const float* __restrict__ A, const float* __restrict__ B, {bias_arg}"
        "float* __restrict__ C, int M, int N,\n    int K, int lda, int ldb, int ldc, int kchunk) {\n"
        f"  mdlc::gemm_f32_wsplit<{s.BM // 16}, {s.BN // 16}, {s.WK}, {s.UN}, "
        f"{'true' if vec_a else 'false'}, {'true' if b_kn else 'false'}, {epi}, "
        f"{'true' if split else 'false'}>(A, B, "
        f"{'bias' if with_bias else 'nullptr'}, C, "
        "M, N, K, lda, ldb, ldc, kchunk);\n}\n")


def conv_wsplit_kernel(name: str, sched: MfmaSchedule, win: tuple, *, with_bias: bool,
                       activation: Optional[str], attrs: dict,
                       residual: Optional[str] = None) -> tuple:
    """The wave-split kernel on an implicit-GEMM convolution (K ordered
    (kh, kw, c), Cin % 16 == 0): ABI (W, x, [bias], [res], y, int M, int N,
    int K, int lda, int Cin, int H, int W, int OH, int OW, int ldc,
    int kchunk); grid x the BM x BN tiles (M = output channels, N = batch x
    output pixels), y the K slices. Without a split the epilogue (bias,
    activation, folded residual) writes NCHW output; with ``sched.SK > 1`` y
    is the split-K workspace (row-major, ``ldc`` = N) and
    ``splitk_reduce_kernel`` finishes."""
    s = sched
    split = s.SK > 1
    if split:
        with_bias, activation, residual = False, None, None
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode="row" if with_bias else None, activation=activation,
                          attrs=attrs, residual=residual)
    winty = "mdlc::ConvWin<%d, %d, %d, %d, %d, %d, %d, %d>" % tuple(win)
    bias_arg = ("const float* __restrict__ bias, " if with_bias else "") + \
        ("const float* __restrict__ res, " if residual else "")
    return name, src + (
        f'extern "C" __global__ __launch_bounds__({s.threads_per_block()}) void {name}(\n'
        f"    const float* __restrict__ A, const float* __restrict__ B, {bias_arg}"
        "float* __restrict__ C, int M, int N,\n    int K, int lda, int Cin, int H, int W, int OH, "
        "int OW, int ldc, int kchunk) {\n"
        f"  mdlc::gemm_f32_wsplit<{s.BM // 16}, {s.BN // 16}, {s.WK}, {s.UN}, true, false, {epi}, "
        f"{'true' if split else 'false'}, {winty}, true>(A, B, "
        f"{'bias' if with_bias else 'nullptr'}, C, M, N, K, lda, 0, ldc, kchunk, "
        f"{'res' if residual else 'nullptr'}, Cin, H, W, OH, OW);\n}}\n")


_CONV_KERNEL = re.compile(r'extern "C" __global__ __launch_bounds__\((\d+)\) void (\w+)\(\n(.*?)\) \{\n'
                          r"(.*?)\n\}\n?$", re.S)


def conv_pair_kernel(name: str, first: tuple, second: tuple) -> tuple:
    """One launch of two independent implicit-GEMM convolutions (``first`` and
    ``second`` are (kernel name, source) as ``gemm_kernel`` made them, one
    K slice, no stream-K): workgroups below ``g0`` run the first's grid,
    the others take the second's tiles in turn (t = b - g0, then every
    gridDim.x - g0), so the second runs on the CUs the first leaves idle.
    Each body is its kernel's own, parameters renamed with a suffix; the
    first's workgroup keeps its block index, the second's takes t in its
    place. The two kernels' epilogue structs come from their own sources.
    ABI: (first's arguments, second's arguments, int g0, int nb)."""
    parts = []
    for suf, (kname, src) in (("_a", first), ("_b", second)):
        m = _CONV_KERNEL.search(src)
        if m is None or m.group(2) != kname:
            raise ValueError(f"{kname}: not a kernel of the implicit-GEMM conv form")
        params = [p.strip() for p in m.group(3).replace("\n", " ").split(",")]
        body = m.group(4)
        if body.count("(g);") != 1 or "ws" in [p.split()[-1] for p in params]:
            raise ValueError(f"{kname}: not a one-slice conv kernel")
        names = [p.split()[-1] for p in params]
        decl = [p[: len(p) - len(n)] + n + suf for p, n in zip(params, names)]
        for n in sorted(names, key=len, reverse=True):
            body = re.sub(r"\b" + re.escape(n) + r"\b", n + suf, body)
        parts.append((int(m.group(1)), decl, body))
    (nta, da, ba), (ntb, db, bb) = parts
    if nta != ntb:
        raise ValueError("paired convolutions must use the same workgroup size")
    ba = ba.replace("(g);", "(g, (int)blockIdx.x);")
    bb = bb.replace("(g);", "(g, t);")
    return name, (
        f'extern "C" __global__ __launch_bounds__({nta}) void {name}(\n    '
        + ", ".join(da + db) + ", int g0, int nb) {\n"
        "  if ((int)blockIdx.x < g0) {\n" + ba + "\n  } else {\n"
        "    for (int t = (int)blockIdx.x - g0; t < nb; t += (int)gridDim.x - g0) {\n" + bb
        + "\n    }\n  }\n}\n")


def splitk_reduce_kernel(name: str, *, with_bias: bool, bias_mode: str,
                         activation: Optional[str], attrs: dict, alpha: float = 1.0,
                         beta: float = 1.0, residual: Optional[str] = None, vec: int = 1,
                         slices: int, hw: int) -> tuple:
    """Split-K epilogue, ``vec`` (1 or 4) outputs per thread, for ``slices``
    slices and NCHW planes of ``hw`` pixels (0: row-major), both compiled in.
    ABI: (ws, [bias], [res], C, int S, int M, int N, int ldc, int hw); the S
    and hw arguments repeat the compiled values."""
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode=bias_mode if with_bias else None, activation=activation,
                          attrs=attrs, alpha=alpha, beta=beta, residual=residual)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    res_arg = "const float* __restrict__ res, " if residual else ""
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        f"    const float* __restrict__ ws, {bias_arg}{res_arg}float* __restrict__ C, int S, int M,\n"
        "    int N, int ldc, int hw) {\n"
        f"  mdlc::splitk_reduce_f32<{epi}, {int(vec)}, {int(slices)}, {int(hw)}>(ws, "
        f"{'bias' if with_bias else 'nullptr'}, {'res' if residual else 'nullptr'}, C, M, N, ldc);\n}}\n")


def streamk_fixup_kernel(name: str, sched: MfmaSchedule, skw: int, *, with_bias: bool,
                         bias_mode: str, activation: Optional[str], attrs: dict,
                         alpha: float = 1.0, beta: float = 1.0,
                         residual: Optional[str] = None) -> tuple:
    """Stream-K fix-up: sums the pieces of each remainder tile and applies
    the epilogue. ABI: (ws, [bias], [res], C, int M, int N, int K, int full,
    int ldc, int hw); BM * BN / 1024 workgroups of 256 threads per
    remainder tile, four elements per thread."""
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode=bias_mode if with_bias else None, activation=activation,
                          attrs=attrs, alpha=alpha, beta=beta, residual=residual)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    res_arg = "const float* __restrict__ res, " if residual else ""
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        f"    const float* __restrict__ ws, {bias_arg}{res_arg}float* __restrict__ C, int M, int N,\n"
        "    int K, int full, int ldc, int hw) {\n"
        f"  mdlc::streamk_fixup_f32<{epi}, {sched.BM}, {sched.BN}, {sched.BK}, {int(skw)}>(ws, "
        f"{'bias' if with_bias else 'nullptr'}, {'res' if residual else 'nullptr'}, C, M, N, K, full, "
        "ldc, hw);\n}\n")


def conv_smallc_kernel(name: str, win: tuple, tile: tuple, *, with_bias: bool,
                       activation: Optional[str], attrs: dict,
                       residual: Optional[str] = None) -> tuple:
    """Direct convolution for few input channels on the matrix cores.
    ``win`` = (C, KH, KW, SH, SW, PT, PL), ``tile`` = (TR, TC, OCW): a
    workgroup computes 32 * OCW channels of a TR x TC output block.
    ABI: (x, wp, [bias], [res], y, int N, int H, int W, int OC, int OH,
    int OW) with ``wp`` the weights packed [channel block][pair][lane]; grid
    x steps through the TR x TC blocks, y covers the channel groups."""
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode="row" if with_bias else None, activation=activation,
                          attrs=attrs, residual=residual)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    res_arg = "const float* __restrict__ res, " if residual else ""
    targs = ", ".join(str(int(v)) for v in tuple(win) + tuple(tile))
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        f"    const float* __restrict__ x, const float* __restrict__ wp, {bias_arg}{res_arg}"
        "float* __restrict__ y,\n    int N, int H, int W, int OC, int OH, int OW) {\n"
        f"  mdlc::conv_smallc_f32<{epi}, {targs}>(x, wp, {'bias' if with_bias else 'nullptr'}, "
        f"{'res' if residual else 'nullptr'}, y, N, H, W, OC, OH, OW);\n}}\n")


def conv_pool_kernel(name: str, win: tuple, band: int, nbx: int, *, with_bias: bool,
                     activation: Optional[str], attrs: dict) -> tuple:
    """Small-channel convolution fused with the 3x3 stride-2 max pool that
    follows it (the activation must be non-decreasing: none, Relu, Relu6,
    Clip). ``win`` = (C, KH, KW, SH, SW, PT, PL); a workgroup computes
    ``band`` pooled rows of one image for 64 output channels, the conv
    output being ``nbx`` column blocks of 16 wide.
    ABI: (x, wp, [bias], y, int N, int H, int W, int OC, int OH) with ``wp``
    the weights packed [16-channel block][4-deep k step][lane]; grid x =
    images x bands, y = 64-channel groups; 256 threads."""
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode="row" if with_bias else None, activation=activation,
                          attrs=attrs)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    targs = ", ".join(str(int(v)) for v in tuple(win) + (band, nbx))
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        f"    const float* __restrict__ x, const float* __restrict__ wp, {bias_arg}"
        "float* __restrict__ y,\n    int N, int H, int W, int OC, int OH) {\n"
        f"  mdlc::conv_pool_f32<{epi}, {targs}>(x, wp, {'bias' if with_bias else 'nullptr'}, "
        "y, N, H, W, OC, OH);\n}\n")


def wino_kernel(name: str, *, split: bool, ploads: int, full: bool, with_bias: bool,
                activation: Optional[str], attrs: dict, residual: Optional[str] = None) -> tuple:
    """3x3 stride-1 convolution by Winograd F(2x2, 3x3) on the matrix cores.
    ABI: (U, x, [bias], [res], y, int N, int C, int H, int W, int OC, int OH,
    int OW, int TH, int TW, int CP, int OCP, int PT, int PL, int nchunk) with
    U the packed transformed filters; 512 threads, grid x = output
    channel blocks of 64 x tile blocks of 64 (tiles fastest), grid y = the
    channel slices. ``split``: y is the split-K workspace and the kernel
    takes no bias or residual (``splitk_reduce_kernel`` finishes).
    ``ploads``: input patch loads per lane and channel (``wino_patch``).
    ``full``: OH and OW are even (every 2x2 tile lies inside the output)."""
    if split:
        with_bias, residual, activation = False, None, None
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode="row" if with_bias else None, activation=activation,
                          attrs=attrs, residual=residual)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    res_arg = "const float* __restrict__ res, " if residual else ""
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(512) void {name}(\n'
        f"    const float* __restrict__ U, const float* __restrict__ x, {bias_arg}{res_arg}"
        "float* __restrict__ y,\n    int N, int C, int H, int W, int OC, int OH, int OW, int TH, "
        "int TW, int CP, int OCP,\n    int PT, int PL, int nchunk) {\n"
        f"  mdlc::WinoArgs g{{U, x, {'bias' if with_bias else 'nullptr'}, "
        f"{'res' if residual else 'nullptr'}, y, N, C, H, W, OC, OH, OW, TH, TW, CP, OCP, PT, PL, "
        "nchunk};\n"
        f"  mdlc::conv_wino_f32<{'true' if split else 'false'}, {int(ploads)}, "
        f"{'true' if full else 'false'}, {epi}>(g);\n}}\n")


def im2col_kernel(name: str = "im2col") -> tuple:
    """ABI: the reference's (x, cols, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW,
    DH, DW) plus trailing (N, ldc) for the batched column matrix."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ cols, int C, int H, int W,\n"
        "    int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int DH, int DW,\n"
        "    int N, int ldc) {\n"
        "  mdlc::im2col_f32(x, cols, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW, DH, DW, N, ldc);\n}\n")


WINDOW_VH = 8          # outputs per thread down a column in the window kernels


def maxpool_kernel(name: str, win: tuple, vh: int = WINDOW_VH) -> tuple:
    """Max pool for the window ``win`` = (KH, KW, SH, SW, DH, DW), ``vh``
    outputs per thread down a column. ABI: (x, y, planes, H, W, OH, OW, KH,
    KW, SH, SW, PT, PL, DH, DW) — the window arguments repeat the compile-time
    ones; one thread per (plane, column, strip of ``vh`` rows)."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, int planes, int H, int W,\n"
        "    int OH, int OW, int KH, int KW, int SH, int SW, int PT, int PL, int DH, int DW) {\n"
        f"  mdlc::window_column_f32<{', '.join(str(v) for v in win)}, {vh}, mdlc::MaxOp>("
        "x, nullptr, nullptr, y, planes, 1, H, W, 1, OH, OW, PT, PL);\n}\n")


def avgpool_kernel(name: str, win: tuple, include_pad: bool, vh: int = WINDOW_VH) -> tuple:
    """Average pool for ``win`` = (KH, KW, SH, SW, 1, 1): the window sum in
    float32, (kh, kw) order, divided by KH*KW (``include_pad``) or by the
    number of taps inside the input. Same ABI and grid as ``maxpool_kernel``."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, int planes, int H, int W,\n"
        "    int OH, int OW, int KH, int KW, int SH, int SW, int PT, int PL, int DH, int DW) {\n"
        f"  mdlc::window_column_f32<{', '.join(str(v) for v in win)}, {vh}, "
        f"mdlc::AvgOp<{'true' if include_pad else 'false'}>>("
        "x, nullptr, nullptr, y, planes, 1, H, W, 1, OH, OW, PT, PL);\n}\n")


def softmax_kernel(name: str, rows: bool) -> tuple:
    """Softmax over one axis. ``rows`` (the axis is innermost): ABI (x, y,
    long long rows, int L), one 64-lane wave per row, four rows per 256-thread
    workgroup; otherwise ABI (x, y, long long outer, int L, int inner), one
    thread per (outer, inner) column."""
    if rows:
        return name, (
            f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
            "    const float* __restrict__ x, float* __restrict__ y, long long rows, int L) {\n"
            "  mdlc::softmax_rows_f32(x, y, rows, L);\n}\n")
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, long long outer, int L, int inner) {\n"
        "  mdlc::softmax_cols_f32(x, y, outer, L, inner);\n}\n")


def transpose_kernel(name: str = "transpose_f32") -> tuple:
    """ABI (x, y, long long total, Dims6 out_dims, Dims6 src_strides)."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, long long total, mdlc::Dims6 od,\n"
        "    mdlc::Dims6 ss) {\n  mdlc::transpose_f32(x, y, total, od, ss);\n}\n")


PAD_MODES = {"constant": 0, "edge": 1, "reflect": 2}


def pad_kernel(name: str, mode: str) -> tuple:
    """ABI (x, y, long long total, Dims6 out_dims, Dims6 in_dims, Dims6
    pads_before, float value)."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, long long total, mdlc::Dims6 od,\n"
        "    mdlc::Dims6 id, mdlc::Dims6 before, float value) {\n"
        f"  mdlc::pad_f32<{PAD_MODES[mode]}>(x, y, total, od, id, before, value);\n}}\n")


def concat_kernel(name: str = "concat_part_f32") -> tuple:
    """One Concat operand. ABI (x, y, long long rows, long long run, long
    long dst_stride, long long dst_off)."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, long long rows, long long run,\n"
        "    long long dst_stride, long long dst_off) {\n"
        "  mdlc::concat_part_f32(x, y, rows, run, dst_stride, dst_off);\n}\n")


def gap_kernel(name: str = "global_avg_pool") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float* __restrict__ y, int planes, int HW) {\n"
        "  mdlc::gap_f32(x, y, planes, HW);\n}\n")


def copy_kernel(name: str = "copy_bytes") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const void* __restrict__ src, void* __restrict__ dst, long long nbytes) {\n"
        "  mdlc::copy_bytes((const unsigned char*)src, (unsigned char*)dst, nbytes);\n}\n")


def dwconv_kernel(name: str, win: tuple, *, with_bias: bool, activation: Optional[str],
                  attrs: dict, vh: int = WINDOW_VH) -> tuple:
    """Depthwise conv with epilogue, ``vh`` outputs per thread down a
    column. ``win`` = (KH, KW, SH, SW, DH, DW).
    ABI: (x, w, [bias], y, N, C, H, W, OC, OH, OW, PT, PL); one thread per
    (plane, column, strip of ``vh`` rows)."""
    epi = f"{name}_epi"
    src = epilogue_struct(epi, bias_mode="row" if with_bias else None,
                          activation=activation, attrs=attrs)
    bias_arg = "const float* __restrict__ bias, " if with_bias else ""
    return name, src + (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        f"    const float* __restrict__ x, const float* __restrict__ w, {bias_arg}"
        "float* __restrict__ y,\n    int N, int C, int H, int W, int OC, int OH, int OW, int PT, int PL) {\n"
        f"  mdlc::window_column_f32<{', '.join(str(v) for v in win)}, {vh}, mdlc::DwOp<{epi}>>("
        f"x, w, {'bias' if with_bias else 'nullptr'}, y, N * OC, C, H, W, OC, OH, OW, PT, PL);\n}}\n")


# ----- fused elementwise ----------------------------------------------------

_BINARY = {"Add": "+", "Sub": "-", "Mul": "*", "Div": "/"}


def _cname(edge: str, table: dict) -> str:
    if edge not in table:
        table[edge] = f"t{len(table)}"
    return table[edge]


def _member_expr(n: Node, ref, consts: dict) -> str:
    """One pointwise group member as a float expression of its inputs."""
    if n.op_type in _BINARY:
        return f"{ref(n.inputs[0])} {_BINARY[n.op_type]} {ref(n.inputs[1])}"
    if n.op_type == "Clip":
        attrs = dict(n.attrs)
        lo = consts.get(n.inputs[1]) if len(n.inputs) > 1 and n.inputs[1] else n.attrs.get("min")
        hi = consts.get(n.inputs[2]) if len(n.inputs) > 2 and n.inputs[2] else n.attrs.get("max")
        attrs["clip_min"], attrs["clip_max"] = lo, hi
        return activation_expr("Clip", ref(n.inputs[0]), attrs)
    return activation_expr(n.op_type, ref(n.inputs[0]), n.attrs)


def elementwise_kernel(name: str, node: Node, *, scalar_consts: Optional[dict] = None) -> tuple:
    """String-generate a fused pointwise kernel from a ``FusedElementwise``
    (or a single pointwise node wrapped as a one-member group).

    External non-constant inputs become pointer arguments in first-use order,
    each member op one line of register arithmetic, and each group output one
    store. Each thread handles 4 consecutive elements with 128-bit loads and
    stores; the last N % 4 elements are handled one per thread.
    ABI: (in_0, ..., in_k, out_0, ..., out_m, int N). Returns
    ``(name, source, ordered_external_inputs)``.
    """
    consts = scalar_consts or {}
    sub = node.attrs["subgraph"]
    internal = {o for n in sub for o in n.outputs if o}
    ext: list = []
    for n in sub:
        for e in n.real_inputs():
            if e not in internal and e not in consts and e not in ext:
                ext.append(e)
    names: dict = {}

    def ref(e: str) -> str:
        return flit(consts[e]) if e in consts else _cname(e, names)

    body = []
    for n in sub:
        out = _cname(n.outputs[0], names)
        body.append(f"float {out} = {_member_expr(n, ref, consts)};")
    in_vars = [_cname(e, names) for e in ext]
    out_vars = [_cname(o, names) for o in node.outputs]
    params = [f"const float* __restrict__ p_{v}" for v in in_vars] + \
             [f"float* __restrict__ q_{v}" for v in out_vars] + ["int N"]

    def lane(idx: str, comp: str = "") -> str:
        loads = [f"float {v} = p_{v}[{idx}];" if not comp else f"float {v} = l_{v}.{comp};"
                 for v in in_vars]
        return " ".join(loads + body)

    quad = []
    for v in in_vars:
        quad.append(f"    const float4 l_{v} = mdlc::ld4(p_{v} + 4 * (long long)i);")
    comps = "xyzw"
    for o in out_vars:
        quad.append(f"    float4 s_{o};")
    for c in comps:
        stores = " ".join(f"s_{o}.{c} = {o};" for o in out_vars)
        quad.append(f"    {{ {lane('', c)} {stores} }}")
    for o in out_vars:
        quad.append(f"    mdlc::st4(q_{o} + 4 * (long long)i, s_{o});")
    tail_store = " ".join(f"q_{o}[j] = {o};" for o in out_vars)
    src = (
        f'extern "C" __global__ __launch_bounds__(256) void {name}({", ".join(params)}) {{\n'
        "  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n"
        "  const long long nq = N >> 2;\n"
        "  if (i < nq) {\n" + "\n".join(quad) + "\n"
        "  } else {\n"
        "    const long long j = nq * 4 + (i - nq);\n"
        f"    if (j < N) {{ {lane('j')} {tail_store} }}\n"
        "  }\n}\n")
    return name, src, ext


def elementwise_signature(node: Node, scalar_consts: dict) -> tuple:
    """Structural identity of an elementwise group: two groups with the same
    signature compile to the same kernel body, so one kernel serves both."""
    sub = node.attrs["subgraph"]
    internal = {o for n in sub for o in n.outputs if o}
    table: dict = {}

    def tag(e: str):
        if e in scalar_consts:
            return ("c", float(scalar_consts[e]))
        if e not in table:
            table[e] = len(table)
        return ("v", table[e], e in internal)

    ops = []
    for n in sub:
        extra = tuple(sorted((k, v) for k, v in n.attrs.items() if isinstance(v, (int, float, str))))
        ops.append((n.op_type, tuple(tag(e) for e in n.inputs if e), tag(n.outputs[0]), extra))
    return tuple(ops), tuple(tag(o) for o in node.outputs)


# ----- INT8 quantized path ----------------------------------------------------

def qgemm_kernel(name: str, sched: MfmaSchedule, *, amode: int, out_f32: bool, lo: int,
                 win: Optional[tuple] = None, gv: int = 16, cin: int = 0, epi: int = 0,
                 depthwise: bool = False, out_i32: bool = False) -> tuple:
    """int8 MFMA GEMM / implicit conv with the requant (or dequant) epilogue.
    ``amode`` 0 = dense A, 1 = NHWC gather of ``gv`` bytes over ``cin``
    channels; ``epi`` 1 = fused table lookup, 2 = fused residual add;
    ``depthwise``: block-diagonal depthwise conv (``cin`` = BN channels per
    block, the tensor's channel count passed as Cin). ``out_i32``: the raw
    int32 accumulators plus bias, no requantization.
    ABI: (A, B, bias, mult, C, aux, int M, int N, int K, int lda, int ldb,
    int ldc, int Cin, int H, int W, int OH, int OW, float res_mult,
    float acc_mult)."""
    s = sched
    winty = "mdlc::NoWin" if win is None else "mdlc::ConvWin<%d, %d, %d, %d, %d, %d, %d, %d>" % tuple(win)
    nt = s.threads_per_block()
    tmpl = (f"mdlc::qgemm_i8_mfma<{s.BM}, {s.BN}, {s.BK}, {s.WGM}, {s.WGN}, {s.MS}, "
            f"{'true' if s.DB else 'false'}, {amode}, "
            f"{gv}, {cin}, {1 if out_f32 else (2 if out_i32 else 0)}, {int(lo)}, {epi}, "
            f"{1 if depthwise else 0}, {winty}, "
            f"{'true' if s.UN == 2 else 'false'}>")
    return name, (
        f'extern "C" __global__ __launch_bounds__({nt}) void {name}(\n'
        "    const signed char* __restrict__ A, const signed char* __restrict__ B,\n"
        "    const int* __restrict__ bias, const float* __restrict__ mult, void* __restrict__ C,\n"
        "    const signed char* __restrict__ aux,\n"
        "    int M, int N, int K, int lda, int ldb, int ldc, int Cin, int H, int W, int OH, int OW,\n"
        "    float res_mult, float acc_mult) {\n"
        "  mdlc::QGemmArgs g{A, B, bias, mult, C, aux, M, N, K, lda, ldb, ldc, Cin, H, W, OH, OW,\n"
        "                    res_mult, acc_mult};\n"
        f"  {tmpl}(g);\n}}\n")


def qmlp_kernel(name: str, C: int, E: int, layout, *, lo1: int, lo2: int,
                mixer: Optional[tuple] = None, mix_batch: int = 3, early_w2: bool = False,
                mixer_regs: bool = False) -> tuple:
    """Fused int8 channel mixer (two 1x1 QConvs, lookup, residual add) over
    channels-last rows; ``layout`` is a ``QMlpLayout``; ``mixer`` = (KH, KW,
    PT, PL, LOD, H, W) adds the depthwise stride-1 token mixer that computes
    X from the kernel's input (an H x W image, compiled in); ``mix_batch`` tiles of it per load batch;
    ``early_w2`` fetches both GEMMs' weight fragments at the start;
    ``mixer_regs`` keeps the mixer's weights in registers instead of LDS.
    ABI: (X or Z, Wd, bd, md, W1, b1, m1, table, W2, b2, m2, Y, int M,
    int H, int W, float res_mult, float acc_mult)."""
    mix = (1,) + tuple(int(v) for v in mixer[:5]) if mixer else (0, 1, 1, 0, 0, -127)
    image = tuple(int(v) for v in mixer[5:7]) if mixer else (1, 1)
    args = (C, E, layout.BM) + tuple(layout.g1) + tuple(layout.g2) + (int(lo1), int(lo2)) + mix + \
        (int(mix_batch), "true" if early_w2 else "false", 1 if (mixer and mixer_regs) else 0) + image
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ X, const signed char* __restrict__ Wd,\n"
        "    const int* __restrict__ bd, const float* __restrict__ md,\n"
        "    const signed char* __restrict__ W1, const int* __restrict__ b1,\n"
        "    const float* __restrict__ m1, const signed char* __restrict__ table,\n"
        "    const signed char* __restrict__ W2, const int* __restrict__ b2,\n"
        "    const float* __restrict__ m2, signed char* __restrict__ Y,\n"
        "    int M, int H, int W, float res_mult, float acc_mult) {\n"
        "  mdlc::QMlpArgs g{X, Wd, bd, md, W1, b1, m1, table, W2, b2, m2, Y, M, H, W, res_mult,\n"
        "                   acc_mult};\n"
        f"  mdlc::qmlp_i8<{', '.join(str(v) for v in args)}>(g);\n}}\n")


def qconv_first_kernel(name: str, C: int, win: tuple, OC: int, dims: tuple, band: int, *, lo: int,
                       epi: int) -> tuple:
    """First int8 conv fused with its input quantization (float32 NCHW in,
    int8 NHWC out) on the matrix cores, in bands of ``band`` output rows of
    an image (workgroup b takes bands b, b + gridDim.x, ...); ``win`` = (KH,
    KW, SH, SW, PT, PL), ``dims`` = (H, W, OH, OW), compiled in. ``w`` is
    packed [block][step][lane] in 16-byte MFMA fragments.
    ABI: (x, float inv_s, w, bias, mult, table, y, int N, int H, int W, int OH, int OW)."""
    args = (C,) + tuple(int(v) for v in win) + (OC, int(lo), int(epi)) + tuple(int(v) for v in dims) \
        + (int(band),)
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, float inv_s, const int* __restrict__ w,\n"
        "    const int* __restrict__ bias, const float* __restrict__ mult,\n"
        "    const signed char* __restrict__ table, signed char* __restrict__ y,\n"
        "    int N, int H, int W, int OH, int OW) {\n"
        f"  mdlc::qconv_first<{', '.join(str(v) for v in args)}>(\n"
        "      x, inv_s, reinterpret_cast<const mdlc::intx4*>(w), bias, mult, table, y, N);\n}\n")


def qdwconv_kernel(name: str, win: tuple, *, cv: int, lo: int) -> tuple:
    """int8 depthwise conv over NHWC. ``win`` = (KH, KW, SH, SW, DH, DW).
    ABI: (x, w, bias, mult, y, int N, int C, int H, int W, int OH, int OW, int PT, int PL)."""
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ x, const signed char* __restrict__ w,\n"
        "    const int* __restrict__ bias, const float* __restrict__ mult, signed char* __restrict__ y,\n"
        "    int N, int C, int H, int W, int OH, int OW, int PT, int PL) {\n"
        f"  mdlc::qdwconv_nhwc<{', '.join(str(v) for v in win)}, {cv}, {int(lo)}>(x, w, bias, mult, y, "
        "N, C, H, W, OH, OW, PT, PL);\n}\n")


def quantize_kernel(name: str = "quantize_nchw_nhwc") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const float* __restrict__ x, signed char* __restrict__ y, int N, int C, int HW, float inv_s) {\n"
        "  mdlc::quantize_nchw_nhwc(x, y, N, C, HW, inv_s);\n}\n")


def qadd_kernel(name: str = "qadd") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ a, const signed char* __restrict__ b,\n"
        "    signed char* __restrict__ y, long long n, float ma, float mb) {\n"
        "  mdlc::qadd_i8(a, b, y, n, ma, mb);\n}\n")


def qlut_kernel(name: str = "qlut") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ x, const signed char* __restrict__ table,\n"
        "    signed char* __restrict__ y, long long n) {\n"
        "  mdlc::qlut_i8(x, table, y, n);\n}\n")


def qgap_kernel(name: str = "qgap", per_image: bool = False) -> tuple:
    """int8 global average pool; ``per_image``: one workgroup per image and
    channel block (grid y: C / block channels; C % 4 == 0).
    ABI: (x, y, int N, int C, int HW, float m)."""
    body = "mdlc::qgap_nhwc_wg(x, y, C, HW, m);" if per_image else "mdlc::qgap_nhwc(x, y, N, C, HW, m);"
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ x, signed char* __restrict__ y, int N, int C, int HW, float m) {\n"
        f"  {body}\n}}\n")


def dequantize_kernel(name: str = "dequantize") -> tuple:
    return name, (
        f'extern "C" __global__ __launch_bounds__(256) void {name}(\n'
        "    const signed char* __restrict__ x, float* __restrict__ y, long long n, int C, int HW,\n"
        "    float s) {\n"
        "  mdlc::dequantize_i8(x, y, n, C, HW, s);\n}\n")
