"""GEMM schedules for the CDNA4 matrix-core kernel: the autotuner's knobs.

The reference schedule is a CUDA thread-block tiling (BM, BN, BK, TM, TN;
mdlc/codegen/schedule.py:16-69). On gfx950 the same role is played by:

* the macro tile BM x BN x BK a workgroup owns,
* the wave grid WGM x WGN (64-lane wavefronts; the workgroup has
  64*WGM*WGN threads) and hence the wave tile (BM/WGM) x (BN/WGN),
* the MFMA shape MS: 32 for v_mfma_f32_32x32x2_f32, 16 for
  v_mfma_f32_16x16x4_f32 (int8 kernels use 32x32x32 / 16x16x64),
* LDS double buffering DB (one barrier per K step, twice the LDS),
* split-K SK: the K range is cut into SK slices computed by separate
  workgroups into a workspace, then reduced in slice order by an epilogue
  kernel — for deep layers whose M x N alone gives too few workgroups to
  fill 256 CUs.

Validity mirrors the kernel's static requirements; the space is the pruned
cross product of a few proven values, as in the reference.
"""

from __future__ import annotations

import math

import numpy as np

from dataclasses import asdict, dataclass, replace
from typing import Iterator, Optional

LDS_LIMIT = 160 * 1024         # bytes one workgroup may allocate (gfx950: 160 KB per CU)
MAX_ACC_REGS = 128             # fp32 accumulator registers per lane we allow
MAX_QACC_REGS = 256            # int8: a 128x128 wave tile, accumulators in AGPRs


@dataclass(frozen=True)
class MfmaSchedule:
    BM: int = 128
    BN: int = 128
    BK: int = 16
    WGM: int = 2
    WGN: int = 2
    MS: int = 32
    DB: bool = True
    SK: int = 1
    ST: bool = False        # stream-K remainder (fp32 GEMM/conv, SK == 1): see gemm_f32_mfma
    UN: int = 1             # K-loop unroll of the double-buffered fp32 loop (1 or 2); with
                            # WK > 1, the 16-deep K steps per register stage (1 .. 16)
    WK: int = 1             # > 1: the wave-split kernel (dense fp32 GEMM): WK waves share the
                            # K range of one BM x BN tile (BM, BN in 16, 32), one launch
    BT: bool = False        # wave-split only: constant B stored K-contiguous per column

    def threads_per_block(self) -> int:
        return 64 * self.WGM * self.WGN * self.WK

    def wave_tile(self) -> tuple:
        return self.BM // self.WGM, self.BN // self.WGN

    def acc_regs(self) -> int:
        wm, wn = self.wave_tile()
        per = 16 if self.MS == 32 else 4
        return (wm // self.MS) * (wn // self.MS) * per

    def lds_bytes(self, elem_bytes: int = 4, b_kmajor: bool = False) -> int:
        """LDS of the A and B tiles; ``b_kmajor`` for the convolution
        gathers, which keep B as [BN][BK + 4] instead of [BK][BN + 4]."""
        b = self.BN * (self.BK + 4) if b_kmajor else self.BK * (self.BN + 4)
        return (2 if self.DB else 1) * (self.BM * (self.BK + 4) + b) * elem_bytes

    def is_valid(self) -> bool:
        if self.WK != 1:
            return self.wsplit_valid()
        if self.BT:
            return False
        if min(self.BM, self.BN, self.BK, self.WGM, self.WGN, self.SK) <= 0 or self.MS not in (16, 32):
            return False
        if self.ST and self.SK != 1:
            return False
        if self.UN not in (1, 2) or (self.UN == 2 and not self.DB):
            return False
        wm, wn = self.wave_tile()
        if self.BM % self.WGM or self.BN % self.WGN:
            return False
        if wm % self.MS or wn % self.MS:
            return False
        kg = 64 // self.MS
        if self.BK % kg or (self.BK // kg) % 4:
            return False
        nt = self.threads_per_block()
        if nt > 1024 or self.BN % 4 or nt % (self.BN // 4):
            return False
        if self.lds_bytes() > LDS_LIMIT or self.acc_regs() > MAX_ACC_REGS:
            return False
        return True

    def wsplit_valid(self) -> bool:
        """The wave-split kernel: 16x16x4 MFMAs, a (BM x BN) tile of 16x16
        blocks per wave, WK waves over K, no LDS staging, one launch."""
        # two register stages of UN steps: 2 * UN * (MI + NI) * 4 operand VGPRs,
        # plus MI * NI * 4 accumulators; the partial tiles of all WK waves meet
        # in LDS (WK * MI * NI * 1 KB)
        mi, ni = self.BM // 16, self.BN // 16
        regs = 2 * self.UN * (mi + ni) * 4 + mi * ni * 4
        return (self.WK in (2, 4, 8, 16) and self.BM in (16, 32, 64) and self.BN in (16, 32, 64)
                and self.MS == 16 and self.WGM == 1 and self.WGN == 1 and self.BK == 16
                and not self.DB and self.SK >= 1 and not self.ST
                and self.UN in (1, 2, 4, 8, 16) and regs <= 200
                and self.WK * mi * ni * 1024 <= LDS_LIMIT)

    def conv_valid(self) -> bool:
        """Valid for the implicit-GEMM convolution kernels, whose gather gives
        each B column to NT / BN threads with BK / (NT / BN) k rows each."""
        if self.WK != 1 or not self.is_valid():
            return False
        nt = self.threads_per_block()
        if nt % self.BN or self.BK % (nt // self.BN):
            return False
        return self.lds_bytes(b_kmajor=True) <= LDS_LIMIT

    def key(self) -> str:
        if self.WK != 1:
            return (f"WS{self.WK}_BM{self.BM}_BN{self.BN}{f'_U{self.UN}' if self.UN > 1 else ''}"
                    f"{'_BT' if self.BT else ''}")
        return (f"BM{self.BM}_BN{self.BN}_BK{self.BK}_W{self.WGM}x{self.WGN}"
                f"_M{self.MS}{'_DB' if self.DB else ''}{'_U2' if self.UN == 2 else ''}")

    def key_full(self) -> str:
        return self.key() + (f"_SK{self.SK}" if self.SK > 1 else "") + ("_ST" if self.ST else "")

    @staticmethod
    def wsplit(bm: int, bn: int, wk: int, un: int = 1, bt: bool = False, sk: int = 1) -> "MfmaSchedule":
        return MfmaSchedule(bm, bn, 16, 1, 1, 16, False, sk, False, un, wk, bt)

    def with_split(self, sk: int) -> "MfmaSchedule":
        return MfmaSchedule(self.BM, self.BN, self.BK, self.WGM, self.WGN, self.MS, self.DB, sk,
                            False, self.UN)

    def with_stream_k(self) -> "MfmaSchedule":
        return MfmaSchedule(self.BM, self.BN, self.BK, self.WGM, self.WGN, self.MS, self.DB, 1, True,
                            self.UN)

    def with_unroll(self, un: int) -> "MfmaSchedule":
        return MfmaSchedule(self.BM, self.BN, self.BK, self.WGM, self.WGN, self.MS, self.DB, self.SK,
                            self.ST, un)

    def as_dict(self) -> dict:
        return asdict(self)


def gemm_search_space(splits=(1,)) -> Iterator[MfmaSchedule]:
    for bm in (32, 64, 128, 256):
        for bn in (32, 64, 128, 256):
            for bk in (8, 16, 32, 64):
                for wgm, wgn in ((1, 1), (2, 1), (1, 2), (2, 2), (4, 1), (1, 4), (4, 2), (2, 4)):
                    for ms in (32, 16):
                        for db in (True, False):
                            for sk in splits:
                                s = MfmaSchedule(bm, bn, bk, wgm, wgn, ms, db, sk)
                                if s.is_valid():
                                    yield s


def wsplit_search_space() -> Iterator[MfmaSchedule]:
    for bm in (16, 32, 64):
        for bn in (16, 32, 64):
            for wk in (4, 8, 16):
                for un in (1, 2, 4, 8, 16):
                    for bt in (False, True):
                        s = MfmaSchedule.wsplit(bm, bn, wk, un, bt)
                        if s.is_valid():
                            yield s
    # K also split over workgroups (a split-K workspace and the reduce launch)
    for bm in (16, 32, 64):
        for bn in (16, 32, 64):
            for wk in (4, 8):
                for un in (1, 2, 4):
                    for sk in (2, 4, 8, 16):
                        s = MfmaSchedule.wsplit(bm, bn, wk, un, True, sk)
                        if s.is_valid():
                            yield s


def wsplit_conv_search_space() -> Iterator[MfmaSchedule]:
    """Wave-split forms for tap-major implicit-GEMM convolutions (Cin % 16 ==
    0): the weights are dense K-contiguous rows, so no ``BT`` variants."""
    for bm in (16, 32, 64):
        for bn in (16, 32, 64):
            for wk in (4, 8, 16):
                for un in (1, 2):
                    for sk in (1, 2, 4, 8):
                        s = MfmaSchedule.wsplit(bm, bn, wk, un, False, sk)
                        if s.is_valid():
                            yield s


def split_slices(K: int, sched: MfmaSchedule) -> tuple:
    """(slices, chunk): K cut into chunks that are multiples of BK, with no
    empty slice."""
    if sched.SK <= 1:
        return 1, K
    chunk = -(-K // sched.SK)
    chunk = -(-chunk // sched.BK) * sched.BK
    return -(-K // chunk), chunk


def unsplit_if_one_slice(sched: MfmaSchedule, K: int) -> MfmaSchedule:
    """``sched`` with SK = 1 when its split leaves one slice of K. The
    kernels pick their split-K form (raw partial sums into the workspace, no
    bias or residual parameters) from the schedule, and the lowering picks
    the launch form from the slice count: they must agree, or the launch's
    arguments no longer match the kernel's parameters."""
    if sched.SK > 1 and split_slices(K, sched)[0] == 1:
        return replace(sched, SK=1)
    return sched


DEFAULT_GEMM = MfmaSchedule()
GemmSchedule = MfmaSchedule


CUS = 256


def default_schedule(M: int, N: int, K: int) -> MfmaSchedule:
    """A shape-aware default used when no tuned entry exists: shrink the
    tile until the grid covers the chip twice (or the tile is 64x64), then
    split K while slices stay at least 256 deep and the grid is short of
    two workgroups per CU."""
    bm = 128 if M > 64 else (64 if M > 32 else 32)
    bn = 128 if N > 64 else (64 if N > 32 else 32)
    tiles = lambda: -(-M // bm) * -(-N // bn)  # noqa: E731
    while tiles() < 2 * CUS and (bm > 64 or bn > 64):
        if bm >= bn and bm > 64:
            bm //= 2
        elif bn > 64:
            bn //= 2
        else:
            bm //= 2
    sk = 1
    while tiles() * sk < 2 * CUS and K // (2 * sk) >= 256 and sk < 8:
        sk *= 2
    wgm = 2 if bm >= 64 else 1
    wgn = 2 if bn >= 64 else 1
    ms = 32 if min(bm // wgm, bn // wgn) >= 32 else 16
    s = MfmaSchedule(bm, bn, 16, wgm, wgn, ms, True, sk)
    return s if s.conv_valid() else DEFAULT_GEMM


# ----- int8 schedules ---------------------------------------------------------
# The same MfmaSchedule fields describe the int8 kernel, with BK counted in
# bytes: MS = 32 selects v_mfma_i32_32x32x32_i8 (32 k per instruction), MS = 16
# v_mfma_i32_16x16x64_i8 (64 k); LDS rows are BK + 16 bytes, double buffered
# (DB) or single buffered.

def qsched_valid(s: MfmaSchedule) -> bool:
    """Valid for the int8 GEMM/conv kernel; ``UN == 2`` selects its
    interleaved pipeline (double-buffered only)."""
    if s.MS not in (16, 32) or s.SK != 1 or s.ST or s.WK != 1 or s.BT:
        return False
    if s.UN not in (1, 2) or (s.UN == 2 and not s.DB):
        return False
    wm, wn = s.wave_tile()
    if s.BM % s.WGM or s.BN % s.WGN or wm % s.MS or wn % s.MS:
        return False
    kg = 64 // s.MS
    if s.BK % (16 * kg):
        return False
    nt = s.threads_per_block()
    if nt > 1024 or nt % (s.BK // 16):
        return False
    if (2 if s.DB else 1) * (s.BM + s.BN) * (s.BK + 16) > LDS_LIMIT or s.acc_regs() > MAX_QACC_REGS:
        return False
    return True


def default_qschedule(M: int, N: int, K: int) -> MfmaSchedule:
    """Shape-aware int8 default: the largest of a few measured tiles whose
    grid still covers every CU once, else the smallest."""
    ladder = (MfmaSchedule(256, 256, 128, 4, 2, 32, True, 1),
              MfmaSchedule(256, 128, 128, 4, 2, 32, True, 1),
              MfmaSchedule(128, 128, 64, 2, 2, 32, True, 1),
              MfmaSchedule(128, 64, 64, 2, 2, 32, True, 1),
              MfmaSchedule(64, 64, 64, 2, 2, 32, True, 1),
              MfmaSchedule(64, 32, 64, 2, 1, 32, True, 1),
              MfmaSchedule(32, 32, 64, 1, 1, 32, True, 1))
    kpad = -(-K // 64) * 64
    for s in ladder:
        if s.BK <= kpad and s.BN <= max(32, N) * 2 and -(-M // s.BM) * -(-N // s.BN) >= CUS:
            return s
    return ladder[-1]


def qdw_valid(s: MfmaSchedule) -> bool:
    """Schedules of the block-diagonal depthwise int8 kernel: 16-channel
    column tiles on 16x16x64 MFMAs, one wave column."""
    return qsched_valid(s) and s.BN == 16 and s.MS == 16 and s.WGN == 1


def default_qdw_schedule(M: int) -> MfmaSchedule:
    return (MfmaSchedule(256, 16, 64, 4, 1, 16, True, 1) if M >= 256 * 64
            else MfmaSchedule(64, 16, 64, 1, 1, 16, True, 1))


def qdw_search_space():
    for bm in (64, 128, 256, 512):
        for bk in (64, 128, 256):
            for wgm in (1, 2, 4, 8):
                s = MfmaSchedule(bm, 16, bk, wgm, 1, 16, True, 1)
                if qdw_valid(s):
                    yield s


def qgemm_search_space():
    for bm in (32, 64, 128, 256):
        for bn in (32, 64, 128, 256):
            for bk in (64, 128, 256):
                for wgm, wgn in ((1, 1), (2, 1), (1, 2), (2, 2), (4, 1), (1, 4), (4, 2), (2, 4),
                                 (4, 4)):
                    for ms in (32, 16):
                        for db in (True, False):
                            s = MfmaSchedule(bm, bn, bk, wgm, wgn, ms, db, 1)
                            if qsched_valid(s):
                                yield s


# ----- the fused int8 channel-mixer kernel (QMlp) -------------------------------

@dataclass(frozen=True)
class QMlpLayout:
    """Tiling of the fused int8 MLP kernel: BM rows per 4-wave workgroup and,
    for each of its two GEMMs, a (WGM, WGN) wave grid with NI blocks of 16
    columns per wave per column chunk (g1: the hidden E columns, g2: the C
    output columns)."""
    BM: int
    g1: tuple
    g2: tuple

    def key(self) -> str:
        return "BM%d_%dx%dn%d_%dx%dn%d" % ((self.BM,) + tuple(self.g1) + tuple(self.g2))


def _round64(n: int) -> int:
    return -(-int(n) // 64) * 64


def qmlp_grid(ncols: int, k: int, bm: int) -> Optional[tuple]:
    """(WGM, WGN, NI) for one GEMM of the fused MLP: the widest wave grid
    along the columns that tiles (ncols, bm), then the largest NI whose B
    fragments for the whole K (16 bytes per lane per 64 K) stay within 96
    registers, with at most 12 accumulator blocks per wave."""
    ks = _round64(k) // 64
    for wgn in (4, 2, 1):
        wgm = 4 // wgn
        if ncols % (16 * wgn) or bm % (16 * wgm):
            continue
        blocks = ncols // (16 * wgn)
        mi = bm // wgm // 16
        for ni in range(blocks, 0, -1):
            if blocks % ni == 0 and ni * ks * 4 <= 96 and mi * ni <= 12:
                return (wgm, wgn, ni)
    return None


def qmlp_lds_bytes(C: int, E: int, bm: int, mixer_taps: int = 0) -> int:
    """LDS of the fused MLP: the X and hidden tiles, the lookup table, both
    GEMMs' bias and multipliers, and with a token mixer of ``mixer_taps``
    taps its block-diagonal weights (rows of KD + 16 bytes), bias and
    multipliers."""
    mixer = C * (_round64(mixer_taps * 16) + 16 + 8) if mixer_taps else 0
    return bm * (_round64(C) + 16 + _round64(E) + 16) + 256 + 8 * (C + E) + mixer


def qmlp_layout(C: int, E: int, M: int, bm: Optional[int] = None,
                mixer_taps: int = 0) -> Optional[QMlpLayout]:
    """The default tiling: 64-row workgroups when that still gives one per
    CU, else 32 rows when that gives 128, else 16 — or the next larger row
    count that tiles both GEMMs and fits LDS with a token mixer of
    ``mixer_taps`` taps; ``bm`` forces one. None when the channel counts admit
    no tiling (C and E must be multiples of 16)."""
    if C % 16 or E % 16:
        return None
    if bm is None:
        first = 64 if M >= 64 * CUS else (32 if M >= 32 * 128 else 16)
        rows = [r for r in (16, 32, 64) if r >= first]
    else:
        rows = [bm]
    for r in rows:
        g1, g2 = qmlp_grid(E, C, r), qmlp_grid(C, E, r)
        if g1 is not None and g2 is not None and qmlp_lds_bytes(C, E, r, mixer_taps) <= LDS_LIMIT:
            return QMlpLayout(r, g1, g2)
    return None


def qmlp_latency_form(C: int, E: int, M: int, layout: QMlpLayout, mixer) -> tuple:
    """(token-mixer tiles per load batch, fetch both weight sets at the
    start, token-mixer weights in registers) for the fused MLP. A launch with
    at most one workgroup per CU has one wave per SIMD, so registers cost no
    occupancy: every mixer tile of a wave is loaded in one batch (while its
    fragments fit in 160 registers), the second GEMM's weights come with the
    first's, and each wave holds the mixer weights of its channel blocks in
    registers (while they fit in QMIX_REG_MAX) instead of copying them to LDS
    behind a barrier. Larger grids keep batches of three, the second weights
    under the first GEMM's epilogue and the mixer weights in LDS."""
    if -(-M // layout.BM) > CUS:
        return 3, False, False
    tiles_per_wave = -(-(layout.BM // 16) * (C // 16) // 4)
    regs = False
    if mixer:
        steps = -(-mixer[0] * mixer[1] * 16 // 64)
        batch = tiles_per_wave if tiles_per_wave * steps * 8 <= 160 else 3
        cb = C // 16
        sets = min(cb // math.gcd(4, cb), max(tiles_per_wave, 1))
        regs = sets * (4 * steps + 8) <= QMIX_REG_MAX
    else:
        batch = 3
    return max(1, min(batch, max(tiles_per_wave, 1))), True, regs


QMIX_REG_MAX = 96         # registers a lane may give the token mixer's weights, bias and multipliers


# ----- direct convolution for few input channels ---------------------------

SMALLC_MAX_C = 4          # input channels up to which a conv takes the direct kernel
SMALLC_MAX_PAIRS = 96     # weight registers per lane it may hold (C * KH * KW / 2, rounded up)


def smallc_pairs(C: int, KH: int, KW: int) -> int:
    return (C * KH * KW + 1) // 2


def smallc_fits(C: int, KH: int, KW: int, DH: int, DW: int) -> bool:
    return C <= SMALLC_MAX_C and DH == 1 and DW == 1 and smallc_pairs(C, KH, KW) <= SMALLC_MAX_PAIRS


def smallc_tile(N: int, OC: int, OH: int, OW: int) -> tuple:
    """(TR, TC, OCW) of the direct small-channel convolution: 8x16 output
    blocks with two 32-channel blocks per workgroup, 4x16 blocks when that
    leaves fewer than two workgroups per CU; one channel block for OC <= 32."""
    ocw = 2 if OC > 32 else 1
    if ocw == 1:
        return 8, 16, 1
    wgs = N * -(-OH // 8) * -(-OW // 16) * -(-OC // 64)
    return (8, 16, 2) if wgs >= 2 * CUS else (4, 16, 2)


def smallc_lds_bytes(C: int, KH: int, KW: int, SH: int, SW: int, TR: int, TC: int) -> int:
    return 4 * C * ((TR - 1) * SH + KH) * ((TC - 1) * SW + KW)


# ----- small-channel convolution fused with the 3x3 stride-2 max pool -------

POOL_BAND_MAX = 7         # pooled rows per band at most (2R+1 conv-row accumulators of 4)
POOL_BAND_MIN = 4         # fewer, and the band's extra conv row outweighs the pool launch
CONV_POOL_LDS = 150 * 1024
CONV_POOL_MAX_K = 256     # weights (and their patch offsets) held in registers per k step


def conv_pool_band(C: int, KH: int, KW: int, SH: int, SW: int, DH: int, DW: int, N: int,
                   OH: int, OW: int) -> Optional[int]:
    """Pooled rows per workgroup band of the fused small-channel conv + max
    pool (3x3, stride 2, padding 1, pooled size OH/2 x OW/2): the largest R
    in [POOL_BAND_MIN, POOL_BAND_MAX] dividing OH/2 whose input patch (2R
    conv-row steps plus the kernel, every column) fits the LDS; None when the
    fused kernel does not apply — more than SMALLC_MAX_C input channels,
    dilation, OW not a multiple of 16 or odd OH, a patch row wider than the
    workgroup, or fewer bands than CUs (one band per CU is what keeps the
    chip busy; smaller batches run the two launches)."""
    if C > SMALLC_MAX_C or DH != 1 or DW != 1 or C * KH * KW > CONV_POOL_MAX_K:
        return None
    if OW % 16 or OH % 2 or OW <= 0 or OH <= 0:
        return None
    PC = (OW - 1) * SW + KW
    if PC > 256:
        return None
    PH = OH // 2
    for R in range(POOL_BAND_MAX, POOL_BAND_MIN - 1, -1):
        if PH % R:
            continue
        PR = 2 * R * SH + KH
        if 4 * C * PR * PC > CONV_POOL_LDS or 4 * (2 * R + 1) * SH * PC >= 65536:
            continue
        return R if N * (PH // R) >= CUS else None
    return None



QFIRST_LDS = 64 * 1024    # LDS of a first int8 conv's band: quantized patch + staged output
QFIRST_MAX_TAPS = 32      # two 16-tap MFMA steps
QFIRST_MAX_LOADS = 64     # input floats a thread holds while staging the patch
QFIRST_WG_PER_CU = 4      # workgroups of the first int8 conv a CU runs at once


def qconv_first_band(C: int, KH: int, KW: int, SH: int, SW: int, N: int, OH: int, OW: int,
                     OC: int) -> Optional[int]:
    """Output rows per workgroup of the first int8 conv with its input
    quantization: the largest of 8, 4, 2, 1 whose band (quantized patch of
    (R-1)*SH + KH input rows, staged R x OW x OC output bytes, lookup table)
    fits QFIRST_LDS and which still gives QFIRST_WG_PER_CU bands a CU; the
    smallest that fits where none does. None when the kernel does not apply:
    more than four input channels, more than QFIRST_MAX_TAPS taps, OC above
    64 or not a multiple of 4, or no band fits."""
    if C > 4 or KH * KW > QFIRST_MAX_TAPS or OC > 64 or OC % 4 or OW <= 0 or OH <= 0:
        return None
    PCW = (OW - 1) * SW + KW
    fits = []
    for R in (8, 4, 2, 1):
        words = ((R - 1) * SH + KH) * PCW
        rows = (R - 1) * SH + KH
        if (words + R * OW * OC // 4) * 4 + 256 <= QFIRST_LDS and rows * -(-PCW // 256) * C <= QFIRST_MAX_LOADS:
            fits.append(R)
    if not fits:
        return None
    for R in fits:
        if N * -(-OH // R) >= QFIRST_WG_PER_CU * CUS:
            return R
    return fits[-1]


def qconv_first_grid() -> int:
    """Workgroups of the first int8 conv at most (larger batches loop over
    their bands, the next band's input loads in flight under the current
    band's matrix and epilogue work). On RepViT's stem at batch 32 one band
    a workgroup (1792 workgroups, all resident at once) measured 8.3 us
    against 8.9 us for 1024 workgroups and 10.5 us for 512 taking bands in
    turn, so the cap only bounds the grid of large batches."""
    return 8 * CUS

# ----- Winograd F(2x2, 3x3) convolution -------------------------------------

WINO_BM = 64              # output channels per workgroup
WINO_BN = 64              # 2x2 output tiles per workgroup
WINO_BK = 8               # input channels per chunk
WINO_MIN_CHUNKS = 4       # chunks each channel slice keeps at least


WINO_PMAX = 704          # input patch floats per channel the kernel's LDS holds


def wino_patch(N: int, H: int, W: int, PT: int, OH: int, OW: int) -> int:
    """Largest input patch (floats per channel) over the Winograd kernel's
    workgroups: for the 64 tiles t0..t0+63 (2x2 output tiles in image-major
    raster order), in each image they touch the rows their 4x4 windows read
    (padding rows included), 2 TW + 2 columns wide (the kernel's own layout:
    the first image from its first tile's row, whole images 2 TH + 2 rows,
    the last up to its last tile's row)."""
    TH, TW = -(-OH // 2), -(-OW // 2)
    TT, P = TH * TW, N * TH * TW
    WP = 2 * TW + 2
    t0 = np.arange(0, P, WINO_BN)
    t1 = np.minimum(t0 + WINO_BN - 1, P - 1)
    nf, nl = t0 // TT, t1 // TT
    rlo0 = 2 * ((t0 - nf * TT) // TW) - PT
    rhil = 2 * ((t1 - nl * TT) // TW) + 3 - PT
    rows0 = np.where(nl == nf, rhil, 2 * TH + 1 - PT) - rlo0 + 1
    rows = rows0 + np.where(nl > nf, (nl - nf - 1) * (2 * TH + 2) + rhil + PT + 1, 0)
    return int((rows * WP).max())


def wino_pays(OC: int, tiles: int, C: int) -> bool:
    """Whether the Winograd kernel is expected to beat the implicit GEMM:
    its workgroups (one per CU at a time) must fill at least half the CUs
    with at least 8 chunks each (the two-stage pipeline's fill and the
    epilogue amortized); smaller problems (batch-1 layers) leave most of the
    chip idle, where the tuned GEMM schedules split the work finer."""
    blocks = -(-OC // WINO_BM) * -(-tiles // WINO_BN)
    s = wino_slices(OC, tiles, C)
    return blocks * s >= CUS // 2 and -(-C // WINO_BK) // s >= 8


def wino_fits(geo: dict) -> bool:
    """A plain 3x3 stride-1 undilated convolution whose workgroups' input
    patches fit the kernel's LDS."""
    if not (geo["group"] == 1 and geo["KH"] == 3 and geo["KW"] == 3 and geo["SH"] == 1
            and geo["SW"] == 1 and geo["DH"] == 1 and geo["DW"] == 1):
        return False
    return wino_patch(geo["N"], geo["H"], geo["W"], geo["PT"], geo["OH"], geo["OW"]) <= WINO_PMAX


def wino_slices(OC: int, tiles: int, C: int) -> int:
    """Channel slices of a Winograd convolution. One workgroup runs per CU
    (the LDS it stages), so the kernel takes about (rounds of workgroups) x
    (chunks per slice) chunk times; the slice count minimising that wins,
    the smallest on ties (each extra slice costs a workspace pass and the
    reduce), with at least WINO_MIN_CHUNKS chunks per slice."""
    blocks = -(-OC // WINO_BM) * -(-tiles // WINO_BN)
    chunks = -(-C // WINO_BK)
    best, best_cost = 1, None
    s = 1
    while s == 1 or -(-chunks // s) >= WINO_MIN_CHUNKS:
        cost = -(-blocks * s // CUS) * -(-chunks // s)
        if best_cost is None or cost < best_cost:
            best, best_cost = s, cost
        s *= 2
    return best
