"""Host-side replay of a compiled plan's launches, as the device sees them.

Test infrastructure, no device needed. For each launch the packed argument
list (``launch_args``, the executor's own packing, over the executor's own
arena layout) is decoded the way ``hipModuleLaunchKernel`` reads a kernel
argument array: parameter i of the kernel's declaration takes argument i,
at the declared width. The GEMM/conv kernels' compile-time parameters
(tile shape, wave split, split-K form, output layout) are read from the
kernel's own template instantiation, not from the launch. The epilogue's
store index formulas of ``gemm_wsplit.hip`` and ``gemm_f32.hip`` are then
evaluated over the whole grid with those values, in 64-bit integers, so a
launch whose arguments do not match its kernel, or whose kernel was compiled
for another form than the one launched, shows up as stores outside the
tensor the kernel believes is its output.
"""

from __future__ import annotations

import re
import struct
from dataclasses import dataclass

import numpy as np

from mdlc_amd.codegen.hip.abi import declared_kinds
from mdlc_amd.codegen.hip.hip_executor import arena_layout, launch_args
from mdlc_amd.codegen.hip.hiprtc_runtime import Arg

BASE = 0x7F3A_1234_5000          # a plausible device address for the arena
WS_BASE = 0x7F3B_0000_0000       # and for a static workspace

_DECL = re.compile(r'extern "C"\s+__global__\s+(?:__launch_bounds__\(\s*\d+\s*(?:,\s*\d+\s*)?\)\s+)?void\s+'
                   r"(\w+)\s*\(([^)]*)\)")


def template_args(source: str, template: str):
    """The template arguments of the first ``template<...>`` in ``source``,
    split at top-level commas, or None."""
    i = source.find(template + "<")
    if i < 0:
        return None
    i += len(template) + 1
    depth, cur, out = 0, "", []
    while True:
        ch = source[i]
        if ch == "<":
            depth += 1
        elif ch == ">":
            if depth == 0:
                out.append(cur.strip())
                return out
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
        i += 1


def param_names(source: str) -> dict:
    """{kernel: [parameter names in order]}."""
    out = {}
    for m in _DECL.finditer(source):
        out[m.group(1)] = [p.split()[-1] for p in m.group(2).split(",") if p.strip()]
    return out


def _value(kind: str, data: bytes):
    data = data + bytes(max(0, 24 - len(data)))
    if kind == "p":
        return struct.unpack("<Q", data[:8])[0]
    if kind == "q":
        return struct.unpack("<q", data[:8])[0]
    if kind == "i":
        return struct.unpack("<i", data[:4])[0]
    if kind == "f":
        return struct.unpack("<f", data[:4])[0]
    return struct.unpack("<6i", data[:24])


@dataclass
class Tensor:
    name: str
    start: int
    nbytes: int


class PlanReplay:
    """The arena (or static workspace) of ``module`` laid out at ``BASE``, and
    every launch's kernel-side argument values."""

    def __init__(self, module, *, static_scratch: bool = False) -> None:
        self.module = module
        self.layout = arena_layout(module, static_scratch=static_scratch)
        src = "\n".join(module.kernels.values())
        self.kinds = declared_kinds(src)
        self.names = param_names(src)
        self.tensors = []
        for name, off in self.layout.offsets.items():
            self.tensors.append(Tensor(name, BASE + off, self.layout.nbytes(name)))
        for name, off in self.layout.ws_offsets.items():
            self.tensors.append(Tensor(name, WS_BASE + off, self.layout.nbytes(name)))
        self.by_name = {t.name: t for t in self.tensors}

    def arg_ptr(self, e: str) -> Arg:
        return Arg.ptr(self.by_name[e].start)

    def kernel_view(self, launch) -> dict:
        """Parameter name -> the value the kernel reads for this launch."""
        args = launch_args(launch, self.arg_ptr)
        kinds = self.kinds[launch.kernel_name]
        names = self.names[launch.kernel_name]
        return {n: _value(k, args[i].data if i < len(args) else b"")
                for i, (n, k) in enumerate(zip(names, kinds))}



def _cdiv(a, b):
    """C's truncating integer division (the kernels' int arithmetic)."""
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def _xcd_remap(b: np.ndarray, total: int) -> np.ndarray:
    q, r = _cdiv(total, 8), total - 8 * _cdiv(total, 8)
    x, j = b % 8, b // 8
    return x * q + np.minimum(x, r) + j


def _tile_origins(grid_x: int, tiles_m: int, total: int, TM: int, TN: int):
    b = np.arange(grid_x, dtype=np.int64)
    t = _xcd_remap(b, total)
    if tiles_m <= 0:
        return None
    return (t % tiles_m) * TM, (t // tiles_m) * TN, t


def store_ranges(rep: PlanReplay, launch) -> list:
    """[(pointer parameter, its value, lowest byte, one past the highest
    byte)] the launch's epilogue stores to, as the kernel computes them;
    None for a kernel this replay does not model."""
    if launch.kind == "conv_pair":
        # the first conv on workgroups 0 .. g0-1 with their own block indices,
        # the second's tiles t < nb in turn on the others: each stores what
        # its own launch would
        out = []
        for part in (launch.meta["first"], launch.meta["second"]):
            r = store_ranges(rep, part)
            if r is None:
                return None
            out += r
        return out
    src = rep.module.kernels[launch.kernel_name]
    v = rep.kernel_view(launch)
    gx, gy = launch.grid[0], launch.grid[1]
    w = template_args(src, "mdlc::gemm_f32_wsplit")
    if w:
        # <MI, NI, WK, UN, VA, BKN, Epi, SPLIT = false, Win = NoWin, CONV = false>
        MI, NI = int(w[0]), int(w[1])
        split = len(w) > 7 and w[7] == "true"
        conv = len(w) > 9 and w[9] == "true"
        TM, TN = 16 * MI, 16 * NI
        M, N = v["M"], v["N"]
        tiles_m = _cdiv(M + TM - 1, TM)
        total = tiles_m * _cdiv(N + TN - 1, TN)
        org = _tile_origins(gx, tiles_m, total, TM, TN)
        if org is None:
            return [("C", v["C"], 0, 0)]
        m0, n0, _ = org
        rows = m0[:, None] + np.arange(TM)[None, :]
        cols = n0[:, None] + np.arange(TN)[None, :]
        lo, hi = None, None
        for y in range(gy):
            for bi in range(gx):
                gr = rows[bi][rows[bi] < M]
                gc = cols[bi][cols[bi] < N]
                if gr.size == 0 or gc.size == 0:
                    continue
                gr, gc = gr[:, None], gc[None, :]
                if split:
                    idx = (y * M + gr) * v["ldc"] + gc
                elif conv:
                    ohw = v["OH"] * v["OW"]
                    img = gc // ohw
                    idx = (img * M + gr) * ohw + (gc - img * ohw)
                else:
                    idx = gr * v["ldc"] + gc
                a, b = int(idx.min()), int(idx.max())
                lo = a if lo is None else min(lo, a)
                hi = b if hi is None else max(hi, b)
        if lo is None:
            return [("C", v["C"], 0, 0)]
        return [("C", v["C"], v["C"] + 4 * lo, v["C"] + 4 * hi + 4)]
    w = template_args(src, "mdlc::gemm_f32_mfma")
    if w:
        # <BM, BN, BK, WGM, WGN, MS, DB, VA, BMODE, OUT, Epi, Win, SKW, UN>
        BM, BN = int(w[0]), int(w[1])
        out, skw = int(w[9]), int(w[12])
        if skw:
            return None                               # stream-K pieces: not modelled
        conv = "x" in v
        cname = "y" if conv else "C"
        M, N = v["M"], v["N"]
        ksplit = v["ksplit"]
        tiles_m = _cdiv(M + BM - 1, BM)
        tiles = tiles_m * _cdiv(N + BN - 1, BN)
        if tiles <= 0:
            return [(cname, v[cname], 0, 0)]
        b = np.arange(gx, dtype=np.int64)
        t = _xcd_remap(b, tiles * ksplit)
        ks = t // tiles
        tt = t - ks * tiles
        m0, n0 = (tt % tiles_m) * BM, (tt // tiles_m) * BN
        rmax = np.minimum(m0 + BM, M) - 1
        cmax = np.minimum(n0 + BN, N) - 1
        live = (m0 < M) & (n0 < N)
        if not live.any():
            return [(cname, v[cname], 0, 0)]
        m0, n0, rmax, cmax, ks = m0[live], n0[live], rmax[live], cmax[live], ks[live]
        if out == 2:
            lo = ks * M * N + m0 * N + n0
            hi = ks * M * N + rmax * N + cmax
        elif out == 1:
            hw = v["OH"] * v["OW"] if conv else v["hw"]
            cimg = v.get("cimg", M * hw)          # grouped: the whole output image
            # the column range of a tile may cross images: evaluate its ends
            # and every image boundary inside it
            lo_l, hi_l = [], []
            for c0, c1, r0, r1 in zip(n0, cmax, m0, rmax):
                cs = np.arange(c0, c1 + 1)
                n = cs // hw
                base = n * cimg + (cs - n * hw)
                lo_l.append(int(base.min()) + int(r0) * hw)
                hi_l.append(int(base.max()) + int(r1) * hw)
            lo, hi = np.array(lo_l), np.array(hi_l)
        else:
            lo = m0 * v["ldc"] + n0
            hi = rmax * v["ldc"] + cmax
        # a grouped conv: grid row g shifts the output base by g group planes
        shift = (gy - 1) * M * v["OH"] * v["OW"] if "cimg" in v else 0
        return [(cname, v[cname], v[cname] + 4 * int(lo.min()),
                 v[cname] + 4 * (int(hi.max()) + shift) + 4)]
    return None


def out_of_bounds(module, *, static_scratch: bool = False) -> list:
    """Every modelled store range that leaves the operand its pointer
    parameter holds (or whose pointer is none of the launch's operands), as
    readable strings. The operands of one launch are live together, so their
    start addresses are distinct (buffers the planner reuses hold other
    tensors at the same address at other times)."""
    rep = PlanReplay(module, static_scratch=static_scratch)
    bad = []
    for l in module.plan:
        ranges = store_ranges(rep, l)
        if ranges is None:
            continue
        at = {rep.by_name[e].start: rep.by_name[e] for e in list(l.inputs) + list(l.outputs)}
        for pname, ptr, lo, hi in ranges:
            if hi <= lo:
                continue
            t = at.get(ptr)
            if t is None or lo < t.start or hi > t.start + t.nbytes:
                where = "no operand" if t is None else f"{t.name!r} ({t.nbytes} bytes)"
                bad.append(f"{l.kernel_name}: {pname} stores [{lo - ptr}, {hi - ptr}) bytes from its "
                           f"base, past {where}")
    return bad


def modelled(module) -> int:
    """How many launches of ``module`` the store replay models."""
    rep = PlanReplay(module)
    return sum(store_ranges(rep, l) is not None for l in module.plan)


def operand_overlaps(module) -> list:
    """Launches whose output range overlaps one of their other operands'
    ranges in the arena (the planner never places a launch's output over a
    tensor the launch reads)."""
    rep = PlanReplay(module)
    bad = []
    for l in module.plan:
        outs = [rep.by_name[o] for o in l.outputs]
        for o in outs:
            for e in l.inputs:
                if e == o.name:
                    continue
                t = rep.by_name[e]
                if t.start < o.start + o.nbytes and o.start < t.start + t.nbytes:
                    bad.append(f"{l.kernel_name}: output {o.name!r} overlaps input {e!r}")
    return bad
