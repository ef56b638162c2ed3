// INT8 quantized kernels for gfx950. Activations are channels-last (NHWC)
// on the device so both matrix operands are contiguous along K.
//
// Semantics (bit-exact contract): products of int8 codes accumulate in int32;
// requantization is clamp(rint(float(acc) * m), lo, 127) with a single
// correctly rounded float multiply, rint = round half to even, lo = 0 after
// a fused ReLU else -127. No fused multiply-add anywhere (-ffp-contract=off).
namespace mdlc {

typedef signed char i8;

// The clamp comes first (its bounds are integers, so clamping before or
// after the rounding gives the same code); adding 1.5 * 2^23 then rounds to
// the nearest integer with ties to even (the float addition's own rounding)
// and leaves that integer in the low mantissa bits: bits = 0x4B400000 + q,
// whose low byte is q in two's complement. Four instructions a code instead
// of a round, a convert and the byte packing of 32-bit integers.
__device__ __forceinline__ int requant_word(int acc, float m, float lo) {
  const float v = fminf(fmaxf((float)acc * m, lo), 127.0f);
  return __builtin_bit_cast(int, v + 12582912.0f);
}
__device__ __forceinline__ i8 requant(int acc, float m, float lo) {
  return (i8)requant_word(acc, m, lo);
}
// QuantizeLinear's code clamp(rint(v * inv_s), -127, 127) in the low byte,
// by the same clamp-then-round steps.
__device__ __forceinline__ int quantize_word(float v, float inv_s) {
  return __builtin_bit_cast(int, fminf(fmaxf(v * inv_s, -127.0f), 127.0f) + 12582912.0f);
}
// The low bytes of four words as one word (byte j from x_j): three byte
// permutes instead of masks, shifts and ors.
__device__ __forceinline__ int pack4(int x0, int x1, int x2, int x3) {
  const unsigned lo = __builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x0c0c0400u);
  const unsigned hi = __builtin_amdgcn_perm((unsigned)x3, (unsigned)x2, 0x0c0c0400u);
  return (int)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

template <int MS> struct MfmaI8;
template <> struct MfmaI8<32> {            // v_mfma_i32_32x32x32_i8: 32 k per step
  typedef intx16 acc_t;
  static constexpr int kAcc = 16;
  __device__ __forceinline__ static acc_t step(intx4 a, intx4 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaI8<16> {            // v_mfma_i32_16x16x64_i8: 64 k per step
  typedef intx4 acc_t;
  static constexpr int kAcc = 4;
  __device__ __forceinline__ static acc_t step(intx4 a, intx4 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

struct QGemmArgs {
  const i8* __restrict__ A;       // AMODE 0: [M][lda]; AMODE 1: NHWC conv input
  const i8* __restrict__ B;       // [N][ldb], K contiguous, zero padded to ldb
  const int* __restrict__ bias;   // [round16(N)], zero padded
  const float* __restrict__ mult; // [round16(N)], zero padded
  void* __restrict__ C;           // int8 [M][ldc] or float [M][ldc]
  const i8* __restrict__ aux;     // EPI 1: 256-entry table; EPI 2: residual [M][ldc]
  int M, N, K, lda, ldb, ldc;
  int Cin, H, W, OH, OW;          // conv geometry (AMODE 1); M = batch*OH*OW
  float res_mult, acc_mult;       // EPI 2 multipliers of the residual and of the codes
};

template <int BYTES> __device__ __forceinline__ void buffer_gather(__amdgpu_buffer_rsrc_t r, int off,
                                                                   i8* dst) {
  if (BYTES == 16) {
    *reinterpret_cast<intx4*>(dst) = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  } else if (BYTES == 8) {
    *reinterpret_cast<int2*>(dst) = __builtin_bit_cast(int2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  } else if (BYTES == 4) {
    *reinterpret_cast<int*>(dst) = (int)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else if (BYTES == 2) {
    *reinterpret_cast<short*>(dst) = (short)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  } else {
    *dst = (i8)__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
  }
}

// Epilogue shared by both staging paths: bias, requant (or dequant), the
// fused lookup or residual add, and the packed stores. ``acc`` is laid out
// as the operand-swapped MFMA leaves it (see qgemm_i8_mfma).
template <int BM, int BN, int WGM, int WGN, int MS, int OUT, int LO, int EPI, class Acc>
__device__ __forceinline__ void qgemm_epilogue(const QGemmArgs& g, Acc& acc, int m0, int n0) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MS, NI = WN / MS;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int li = lane % MS;
  const int lk = lane / MS;
  // acc[mi][ni][4q + j] is C[m0 + wm0 + mi*MS + li][n0 + wn0 + ni*MS + q*8 + lk*4 + j]
  // (MS = 32; for MS = 16 the single group is at lk*4 + j).
  constexpr int NG = MfmaI8<MS>::kAcc / 4;
  const bool vec_ok = (g.ldc & 3) == 0;
  // The tile's multipliers (and the lookup table) go through LDS: read from
  // global memory between the output stores, each would wait for the store
  // before it (the compiler cannot tell them apart from the output). The
  // bias is already in the accumulators (they start at it).
  __shared__ i8 table[EPI == 1 ? 256 : 1];
  __shared__ float mult_s[BN];
  for (int i = tid; i < BN; i += NT) {        // the K loop ended with a barrier: LDS is free
    const bool ok = n0 + i < g.N;
    mult_s[i] = ok ? g.mult[n0 + i] : 0.f;
  }
  if (EPI == 1)
    for (int i = tid; i < 256; i += NT) table[i] = g.aux[i];
  __syncthreads();
  auto finish = [&](i8 code, i8 res) -> i8 {
    if (EPI == 1) return table[(int)code + 128];
    if (EPI == 2) {
      const float v = (float)res * g.res_mult + (float)code * g.acc_mult;
      return (i8)(int)fminf(fmaxf(rintf(v), -127.0f), 127.0f);
    }
    return code;
  };
#pragma unroll
  for (int ni = 0; ni < NI; ++ni)
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const int col = n0 + wn0 + ni * MS + q * 8 + lk * 4;
      if (col >= g.N) continue;
      const floatx4 mv = *reinterpret_cast<const floatx4*>(&mult_s[col - n0]);
      const bool full = vec_ok && col + 4 <= g.N;
      // the residual words of all the group's rows before its first store
      int rw[MI];
      if (OUT == 0 && EPI == 2) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const int row = m0 + wm0 + mi * MS + li;
          const size_t off = (size_t)row * g.ldc + col;
          rw[mi] = (full && row < g.M) ? *reinterpret_cast<const int*>(g.aux + off) : 0;
        }
      }
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const int row = m0 + wm0 + mi * MS + li;
        if (row >= g.M) continue;
        if (OUT == 2) {
          int* cp = static_cast<int*>(g.C) + (size_t)row * g.ldc + col;
          int o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[mi][ni][4 * q + j];
          if (full) {
            *reinterpret_cast<intx4*>(cp) = intx4{o[0], o[1], o[2], o[3]};
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (col + j < g.N) cp[j] = o[j];
          }
        } else if (OUT == 1) {
          float* cp = static_cast<float*>(g.C) + (size_t)row * g.ldc + col;
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (float)acc[mi][ni][4 * q + j] * mv[j];
          if (full) {
            *reinterpret_cast<float4*>(cp) = make_float4(o[0], o[1], o[2], o[3]);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (col + j < g.N) cp[j] = o[j];
          }
        } else {
          const size_t off = (size_t)row * g.ldc + col;
          i8* cp = static_cast<i8*>(g.C) + off;
          union { int w; i8 b[4]; } o, r;
          r.w = 0;
          if (EPI == 2) {
            if (full) {
              r.w = rw[mi];
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (col + j < g.N) r.b[j] = g.aux[off + j];
            }
          }
          if (EPI == 0) {
            int wq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) wq[j] = requant_word(acc[mi][ni][4 * q + j], mv[j], (float)LO);
            o.w = pack4(wq[0], wq[1], wq[2], wq[3]);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              o.b[j] = finish(requant(acc[mi][ni][4 * q + j], mv[j], (float)LO), r.b[j]);
          }
          if (full) {
            *reinterpret_cast<int*>(cp) = o.w;
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (col + j < g.N) cp[j] = o.b[j];
          }
        }
      }
    }
}

// Scheduling hints for the interleaved int8 pipeline, as compile-time
// recursion (the hint's arguments must be constants): per sub-step, its
// MFS MFMAs each followed by one of EXTRA instructions of class MASK (LDS
// reads 0x100 or LDS writes 0x200), any surplus of those after the last.
template <int I, int MFS, int EXTRA, int MASK>
struct PipeInterleave {
  __device__ __forceinline__ static void emit() {
    if constexpr (I < MFS) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (I < EXTRA) __builtin_amdgcn_sched_group_barrier(MASK, 1, 0);
      PipeInterleave<I + 1, MFS, EXTRA, MASK>::emit();
    } else if constexpr (EXTRA > MFS) {
      __builtin_amdgcn_sched_group_barrier(MASK, EXTRA - MFS, 0);
    }
  }
};
template <int SUB, int SUBS, int MFS, int NFR, int NST>
struct PipeOrder {
  __device__ __forceinline__ static void emit() {
    if constexpr (SUB < SUBS) {
      PipeInterleave<0, MFS, SUB + 1 < SUBS ? NFR : NST, SUB + 1 < SUBS ? 0x100 : 0x200>::emit();
      PipeOrder<SUB + 1, SUBS, MFS, NFR, NST>::emit();
    }
  }
};

// C[m][n] = q(sum_k A[m][k] * B[n][k] + bias[n]).
//
// AMODE 0: dense A [M][lda] (lda % 16 == 0).
// AMODE 1: implicit im2col over an NHWC input (CIN channels, compile time)
//          with k = (kh, kw, c); the gather moves GV bytes at a time
//          (GV divides CIN: one tap's GV channels of one pixel).
// DWG 1:   depthwise conv as a block-diagonal GEMM: the input has g.Cin
//          channels, k = (kh, kw, c) runs over CIN = BN channels, and a
//          workgroup gathers the BN channels of its own output columns
//          (offset n0). B row n holds w[n][tap] at k = (tap, n - n0) and
//          zeros elsewhere, so the matrix cores do BN times the depthwise
//          arithmetic — cheap next to what the vector ALUs would take — and
//          each input byte is still fetched once per tap.
// OUT 0: int8 requantized output (LO = lower clamp); OUT 1: float32
//        float(acc) * mult[n] (dequantized logits); OUT 2: the int32
//        accumulators plus bias, as they are (the exactness check).
// EPI (OUT 0 only): 0 = the requantized codes; 1 = table[code + 128] (a
//        fused lookup, table staged in LDS); 2 = a fused residual add,
//        clamp(rint(f32(f32(r) * res_mult) + f32(f32(code) * acc_mult)))
//        with r read at the output's position. Both are the unfused ops'
//        arithmetic, so the fused kernel is bit-identical to the pair.
//
// Staging goes through raw buffer loads. The K tail needs no test: B is zero
// padded to ldb (a multiple of BK), so whatever A holds past K is multiplied
// by zero; rows past M or N and gathered pixels outside the image use an
// offset past the buffer end and load zeros. Each thread keeps one 16-byte
// k chunk (kc) of a few tile rows; for dense operands the per-tile k0 moves
// the buffer base (scalar work), so a load costs no vector ALU at all.
//
// The MFMA takes the B tile as its row operand: a lane then holds four
// consecutive output columns per accumulator group, stored as one 32-bit
// (int8) or 128-bit (float) write.
template <int BM, int BN, int BK, int WGM, int WGN, int MS, bool DB, int AMODE, int GV, int CIN, int OUT,
          int LO, int EPI, int DWG, class Win, bool PIPE = false>
__device__ __forceinline__ void qgemm_i8_mfma(const QGemmArgs& g) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MS, NI = WN / MS;
  constexpr int KG = 64 / MS;
  constexpr int KSUB = BK / KG;
  constexpr int LDS_ROW = BK + 16;
  constexpr int CPR = BK / 16;               // 16-byte chunks per tile row
  constexpr int RSTEP = NT / CPR;            // tile rows between one thread's slots
  constexpr int A_PT = (BM + RSTEP - 1) / RSTEP, B_PT = (BN + RSTEP - 1) / RSTEP;
  static_assert(KSUB % 16 == 0, "BK too small for this MFMA shape");
  static_assert(NT % CPR == 0, "rows must map to fixed threads");
  static_assert(AMODE == 0 || (CIN % GV == 0 && 16 % GV == 0), "gather width must divide Cin");
  static_assert(DWG == 0 || (AMODE == 1 && CIN == BN), "depthwise tiles span one channel block");
  typedef typename MfmaI8<MS>::acc_t acc_t;

  constexpr int NBUF = DB ? 2 : 1;
  __shared__ __attribute__((aligned(16))) i8 As[NBUF][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) i8 Bs[NBUF][BN * LDS_ROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int li = lane % MS;
  const int lk = lane / MS;

  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  int mt, nt;
  grouped_tile<8>(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, mt, nt);
  const int m0 = mt * BM;
  const int n0 = nt * BN;

  const int kc = tid % CPR;
  const int r0 = tid / CPR;

  // ---- per-thread row state, fixed across K tiles ---------------------------
  int b_off[B_PT];
#pragma unroll
  for (int i = 0; i < B_PT; ++i) {
    const int r = r0 + i * RSTEP;
    b_off[i] = (r < BN && n0 + r < g.N) ? (n0 + r) * g.ldb + kc * 16 : kOutside;
  }
  const int pix_stride = DWG ? g.Cin : CIN;   // bytes between neighbouring pixels (AMODE 1)
  int a_off[A_PT];                  // AMODE 0: row offset; AMODE 1: pixel (ih0, iw0) offset
  int a_ih[A_PT], a_iw[A_PT];
#pragma unroll
  for (int i = 0; i < A_PT; ++i) {
    const int r = r0 + i * RSTEP;
    const int p = m0 + r;
    const bool live = r < BM && p < g.M;
    if (AMODE == 0) {
      a_off[i] = live ? p * g.lda + kc * 16 : kOutside;
    } else {
      const int ohw = g.OH * g.OW;
      const int n = p / ohw;
      const int s = p - n * ohw;
      const int oh = s / g.OW;
      const int ow = s - oh * g.OW;
      const int ih0 = oh * Win::SH - Win::PT;
      a_ih[i] = live ? ih0 : -(1 << 28);
      a_iw[i] = ow * Win::SW - Win::PL;
      a_off[i] = live ? ((n * g.H + ih0) * g.W + a_iw[i]) * pix_stride + (DWG ? n0 : 0) : 0;
    }
  }
  const int a_bytes = AMODE == 0 ? g.M * g.lda : (g.M / (g.OH * g.OW)) * g.H * g.W * pix_stride;
  const int b_bytes = g.N * g.ldb;

  // byte offset in A of k for slot i (gather), or kOutside for padding
  auto gather_off = [&](int i, int k) -> int {
    const int tap = k / CIN;
    const int c = k - tap * CIN;
    const int kh = tap / Win::KW;
    const int kw = tap - kh * Win::KW;
    const int ih = a_ih[i] + kh * Win::DH;
    const int iw = a_iw[i] + kw * Win::DW;
    const bool ok = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
    return ok ? a_off[i] + (kh * Win::DH * g.W + kw * Win::DW) * pix_stride + c : kOutside;
  };

  // k0 may be up to two tiles past K (the loop prefetches unconditionally):
  // the clamped sizes keep every such load inside its operand or zero.
  auto load_tiles = [&](int k0, intx4 (&ra)[A_PT], intx4 (&rb)[B_PT]) {
    const __amdgpu_buffer_rsrc_t rB = buffer_over(g.B + k0, max(b_bytes - k0, 0));
#pragma unroll
    for (int i = 0; i < B_PT; ++i)
      rb[i] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rB, b_off[i], 0, 0));
    if (AMODE == 0) {
      const __amdgpu_buffer_rsrc_t rA = buffer_over(g.A + k0, max(a_bytes - k0, 0));
#pragma unroll
      for (int i = 0; i < A_PT; ++i)
        ra[i] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rA, a_off[i], 0, 0));
    } else {
      const __amdgpu_buffer_rsrc_t rA = buffer_over(g.A, a_bytes);
      const int kb = k0 + kc * 16;
#pragma unroll
      for (int i = 0; i < A_PT; ++i) {
        if (GV == 16) {
          ra[i] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rA, gather_off(i, kb), 0, 0));
        } else {
          union { intx4 v; i8 b[16]; } u;
#pragma unroll
          for (int j = 0; j < 16; j += GV) buffer_gather<GV>(rA, gather_off(i, kb + j), &u.b[j]);
          ra[i] = u.v;
        }
      }
    }
  };

  auto store_tiles = [&](int buf, const intx4 (&ra)[A_PT], const intx4 (&rb)[B_PT]) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      const int r = r0 + i * RSTEP;
      if (BM % RSTEP == 0 || r < BM) *reinterpret_cast<intx4*>(&As[buf][r * LDS_ROW + kc * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      const int r = r0 + i * RSTEP;
      if (BN % RSTEP == 0 || r < BN) *reinterpret_cast<intx4*>(&Bs[buf][r * LDS_ROW + kc * 16]) = rb[i];
    }
  };

  // The accumulators start at their columns' bias (the epilogue's layout:
  // acc[mi][ni][4q + j] is column n0 + wn0 + ni*MS + q*8 + lk*4 + j), so the
  // MFMAs leave the exact int32 acc + bias and the epilogue adds nothing. The
  // bias is zero padded to a multiple of 16 columns; four columns past that
  // read zeros through the buffer's range check.
  constexpr int NG = MfmaI8<MS>::kAcc / 4;
  acc_t acc[MI][NI];
  {
    const __amdgpu_buffer_rsrc_t rbias = buffer_over(g.bias, (g.N + 15) / 16 * 64);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        const int col = n0 + wn0 + ni * MS + q * 8 + lk * 4;
        const intx4 bv = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rbias, col * 4, 0, 0));
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[mi][ni][4 * q + j] = bv[j];
      }
  }

  auto compute = [&](int buf) {
    const i8* as = &As[buf][0];
    const i8* bs = &Bs[buf][0];
#pragma unroll
    for (int s = 0; s < KSUB / 16; ++s) {
      const int kk = lk * KSUB + s * 16;
      intx4 af[MI], bf[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        af[mi] = *reinterpret_cast<const intx4*>(as + (wm0 + mi * MS + li) * LDS_ROW + kk);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bf[ni] = *reinterpret_cast<const intx4*>(bs + (wn0 + ni * MS + li) * LDS_ROW + kk);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = MfmaI8<MS>::step(bf[ni], af[mi], acc[mi][ni]);
    }
  };

  // Global loads run ahead of the MFMAs through registers. With two
  // register sets (when the accumulators leave room) they run two K tiles
  // ahead: iteration kt issues tile kt+2's loads into the set tile kt
  // arrived in, computes tile kt from LDS, then stores tile kt+1 (loaded an
  // iteration earlier) into the idle LDS buffer. With one set, iteration kt
  // loads tile kt+1 and stores it at its end. Loads and stores are
  // unconditional (past the end they fetch zeros or stay inside the
  // operands, and land in a buffer nobody reads), so each iteration is one
  // basic block the scheduler can interleave with the MFMAs. The waves raise
  // their issue priority while they feed the matrix cores.
  constexpr bool kTwoSets = DB && MfmaI8<MS>::kAcc * MI * NI + 8 * (A_PT + B_PT) <= 192;
  static_assert(!PIPE || DB, "the interleaved pipeline needs two LDS buffers");
  intx4 ra0[A_PT], rb0[B_PT], ra1[kTwoSets && !PIPE ? A_PT : 1], rb1[kTwoSets && !PIPE ? B_PT : 1];
  const int nk = (g.K + BK - 1) / BK;
  auto kofs = [&](int kt) -> int { return kt * BK; };   // byte offset of K tile kt
  if constexpr (PIPE) {
    // Interleaved pipeline (double-buffered LDS, one register set for the
    // global staging): within one K tile the fragments of sub-step s + 1
    // are read from LDS while the MFMAs of sub-step s run, the next tile's
    // global loads are issued at the start, and written to the idle LDS
    // buffer between the MFMAs of the last sub-step. The scheduling hints
    // lay the iteration out in that order, so a wave keeps the matrix core
    // fed on its own, without a second wave on the SIMD to hide latency.
    constexpr int SUBS = KSUB / 16;
    constexpr int NFR = MI + NI;                 // LDS reads per sub-step
    constexpr int NST = A_PT + B_PT;             // LDS writes (and global loads) per tile
    constexpr int MFS = MI * NI;                 // MFMAs per sub-step
    auto read_frags = [&](intx4 (&fa)[MI], intx4 (&fb)[NI], const i8* as, const i8* bs, int sub) {
      const int kk = lk * KSUB + sub * 16;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        fa[mi] = *reinterpret_cast<const intx4*>(as + (wm0 + mi * MS + li) * LDS_ROW + kk);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        fb[ni] = *reinterpret_cast<const intx4*>(bs + (wn0 + ni * MS + li) * LDS_ROW + kk);
    };
    load_tiles(kofs(0), ra0, rb0);
    store_tiles(0, ra0, rb0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const i8* as = &As[kt & 1][0];
      const i8* bs = &Bs[kt & 1][0];
      intx4 fa[2][MI], fb[2][NI];
      read_frags(fa[0], fb[0], as, bs, 0);
      load_tiles(kofs(kt + 1), ra0, rb0);
#pragma unroll
      for (int sub = 0; sub < SUBS; ++sub) {
        if (sub + 1 < SUBS) read_frags(fa[(sub + 1) & 1], fb[(sub + 1) & 1], as, bs, sub + 1);
        else store_tiles((kt + 1) & 1, ra0, rb0);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = MfmaI8<MS>::step(fb[sub & 1][ni], fa[sub & 1][mi], acc[mi][ni]);
      }
      // order: first fragments, the global loads, then per sub-step its
      // MFMAs alternating with the next sub-step's reads (the last one's
      // with the LDS writes)
      __builtin_amdgcn_sched_group_barrier(0x100, NFR, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, NST, 0);
      PipeOrder<0, SUBS, MFS, NFR, NST>::emit();
      __syncthreads();
    }
  } else if constexpr (kTwoSets) {
    load_tiles(kofs(0), ra0, rb0);
    load_tiles(kofs(1), ra1, rb1);
    store_tiles(0, ra0, rb0);
    __syncthreads();
    auto step = [&](int kt, intx4 (&ra_in)[A_PT], intx4 (&rb_in)[B_PT], intx4 (&ra_nx)[A_PT],
                    intx4 (&rb_nx)[B_PT]) {
      load_tiles(kofs(kt + 2), ra_in, rb_in);
      __builtin_amdgcn_s_setprio(1);
      compute(kt & 1);
      __builtin_amdgcn_s_setprio(0);
      store_tiles((kt + 1) & 1, ra_nx, rb_nx);
      __syncthreads();
    };
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, ra0, rb0, ra1, rb1);
      if (kt + 1 < nk) step(kt + 1, ra1, rb1, ra0, rb0);
    }
  } else if constexpr (DB) {
    load_tiles(kofs(0), ra0, rb0);
    store_tiles(0, ra0, rb0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      load_tiles(kofs(kt + 1), ra0, rb0);
      __builtin_amdgcn_s_setprio(1);
      compute(kt & 1);
      __builtin_amdgcn_s_setprio(0);
      store_tiles((kt + 1) & 1, ra0, rb0);
      __syncthreads();
    }
  } else {
    // one LDS buffer (half the LDS, e.g. for 256-byte K tiles): the next
    // tile waits in registers while the current one is consumed
    load_tiles(kofs(0), ra0, rb0);
    for (int kt = 0; kt < nk; ++kt) {
      store_tiles(0, ra0, rb0);
      __syncthreads();
      load_tiles(kofs(kt + 1), ra0, rb0);
      __builtin_amdgcn_s_setprio(1);
      compute(0);
      __builtin_amdgcn_s_setprio(0);
      __syncthreads();
    }
  }

  qgemm_epilogue<BM, BN, WGM, WGN, MS, OUT, LO, EPI>(g, acc, m0, n0);
}

// Depthwise conv over NHWC int8 (one input channel per output channel),
// weights packed [KH][KW][C]; each thread owns one output pixel and CV
// consecutive channels (CV = 16 uses 128-bit loads and stores).
template <int KH, int KW, int SH, int SW, int DH, int DW, int CV, int LO>
__device__ __forceinline__ void qdwconv_nhwc(const i8* __restrict__ x, const i8* __restrict__ w,
                                             const int* __restrict__ bias,
                                             const float* __restrict__ mult, i8* __restrict__ y,
                                             int N, int C, int H, int W, int OH, int OW, int PT,
                                             int PL) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int cchunks = C / CV;
  const long long total = (long long)N * OH * OW * cchunks;
  if (i >= total) return;
  const int cc = (int)(i % cchunks);
  const long long pix = i / cchunks;
  const int ow = (int)(pix % OW);
  const int oh = (int)((pix / OW) % OH);
  const int n = (int)(pix / ((long long)OW * OH));
  const int c0 = cc * CV;
  int acc[CV];
#pragma unroll
  for (int j = 0; j < CV; ++j) acc[j] = 0;
#pragma unroll
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * SH - PT + kh * DH;
#pragma unroll
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * SW - PL + kw * DW;
      if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W) continue;
      const i8* xp = x + (((size_t)n * H + ih) * W + iw) * C + c0;
      const i8* wp = w + (size_t)(kh * KW + kw) * C + c0;
      if (CV == 16) {
        union { intx4 v; i8 b[16]; } xv, wv;
        xv.v = *reinterpret_cast<const intx4*>(xp);
        wv.v = *reinterpret_cast<const intx4*>(wp);
#pragma unroll
        for (int j = 0; j < CV; ++j) acc[j] += (int)xv.b[j] * (int)wv.b[j];
      } else {
#pragma unroll
        for (int j = 0; j < CV; ++j) acc[j] += (int)xp[j] * (int)wp[j];
      }
    }
  }
  i8* yp = y + (((size_t)n * OH + oh) * OW + ow) * C + c0;
  if (CV == 16) {
    union { intx4 v; i8 b[16]; } o;
#pragma unroll
    for (int j = 0; j < CV; ++j) o.b[j] = requant(acc[j] + bias[c0 + j], mult[c0 + j], (float)LO);
    *reinterpret_cast<intx4*>(yp) = o.v;
  } else {
#pragma unroll
    for (int j = 0; j < CV; ++j) yp[j] = requant(acc[j] + bias[c0 + j], mult[c0 + j], (float)LO);
  }
}

// First conv of an int8 network fused with its input quantization, on the
// matrix cores. x is the float32 NCHW network input with at most four
// channels; y is int8 channels-last. The work is split in bands of R output
// rows of one image, whose outputs are one contiguous range of y; workgroup
// b takes bands b, b + gridDim.x, ... and loads the next band's input while
// it computes the current one. For a band:
//  1. the input rows it reads are quantized into LDS with the QuantizeLinear
//     arithmetic (clamp(rint(x * inv_s), -127, 127); zeros where the window
//     leaves the image, as the conv pads the quantized tensor), one word per
//     input pixel holding its C codes (the bytes past C zero), so every input
//     value is read from HBM and quantized once;
//  2. v_mfma_i32_16x16x64_i8 forms 16 output channels x 16 output pixels a
//     step. The row operand is the weights (lane 16 lk + li: output channel
//     li of the block, taps 16 s + 4 lk .. 16 s + 4 lk + 3, one word per tap
//     packed like the input pixels, zero past the kernel's taps), the column
//     operand the same taps of pixel li, read from the LDS patch; K runs over
//     (tap, input channel) with every padding byte zero in the weights; the
//     accumulator starts at the bias, so the sum is the exact int32 acc + bias;
//  3. the accumulator holds channels 4 lk + r of pixel li in lane 16 lk + li:
//     the requant, the optional lookup, four channels packed into one word of
//     the band's output, which is staged in LDS and written with 16-byte
//     stores.
template <int C, int KH, int KW, int SH, int SW, int PT, int PL, int OC, int LO, int EPI,
          int H, int W, int OH, int OW, int R>
__device__ __forceinline__ void qconv_first(const float* __restrict__ x, float inv_s,
                                            const intx4* __restrict__ w,
                                            const int* __restrict__ bias,
                                            const float* __restrict__ mult,
                                            const i8* __restrict__ table, i8* __restrict__ y,
                                            int N) {
  constexpr int T = KH * KW;                   // taps
  constexpr int NS = (T + 15) / 16;            // MFMA steps of 16 taps
  constexpr int NOB = (OC + 15) / 16;          // 16-channel output blocks
  constexpr int PR = (R - 1) * SH + KH;        // patch rows
  constexpr int PCW = (OW - 1) * SW + KW;      // patch columns (padding included)
  constexpr int NE = PR * PCW;                 // patch words
  constexpr int NP = R * OW;                   // band pixels
  constexpr int NG = (NP + 15) / 16;           // 16-pixel groups
  constexpr int BANDS = (OH + R - 1) / R;
  static_assert(C <= 4 && OC % 4 == 0 && OC <= 64, "first convs with few channels only");
  static_assert((NE + NP * OC / 4) * 4 + 256 <= 64 * 1024, "band exceeds the LDS budget");
  __shared__ int patch[NE];
  __shared__ __attribute__((aligned(16))) int outs[NP * OC / 4];
  __shared__ unsigned char tab[256];           // tab[b] = table[code b + 128]
  const int total = N * BANDS;
  int band = blockIdx.x;

  // the band's input values of this thread's patch columns (column pc = t +
  // 256 q of every patch row; every load is issued before the first is
  // used), and their codes into the LDS patch. A row's offset is uniform
  // and goes in the scalar offset (clamped into the image); a row or column
  // outside the image reads zero through a vector offset past the buffer.
  constexpr int NQ = (PCW + 255) / 256;        // patch columns a thread stages
  float v[PR][NQ][C];
  auto load = [&](int b) {
    const int n = b / BANDS;
    const int ih0 = (b - n * BANDS) * R * SH - PT;
    const __amdgpu_buffer_rsrc_t rx = buffer_over(x + (size_t)n * C * H * W, C * H * W * 4);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int pc = (int)threadIdx.x + 256 * q;
      const int iw = pc - PL;
      const int voff = pc < PCW && (unsigned)iw < (unsigned)W ? iw * 4 : kOutside;
#pragma unroll
      for (int pr = 0; pr < PR; ++pr) {
        const int ih = ih0 + pr;
        const bool row_ok = (unsigned)ih < (unsigned)H;
        const int vo = row_ok ? voff : kOutside;
        const int ihc = row_ok ? ih : 0;
#pragma unroll
        for (int c = 0; c < C; ++c)
          v[pr][q][c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
              rx, vo, (c * H + ihc) * W * 4, 0));
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int pc = (int)threadIdx.x + 256 * q;
#pragma unroll
      for (int pr = 0; pr < PR; ++pr) {
        int qc[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < C; ++c) qc[c] = quantize_word(v[pr][q][c], inv_s);
        if (pc < PCW) patch[pr * PCW + pc] = pack4(qc[0], qc[1], qc[2], qc[3]);
      }
    }
  };
  load(band);
  if (EPI == 1) tab[threadIdx.x] = (unsigned char)table[threadIdx.x ^ 0x80];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lk = lane >> 4;
  intx4 wf[NOB][NS];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
    for (int s = 0; s < NS; ++s) wf[ob][s] = w[(ob * NS + s) * 64 + lane];
  intx4 bv[NOB];
  float mv[NOB][4];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int oc = 16 * ob + 4 * lk + r;
      bv[ob][r] = oc < OC ? bias[oc] : 0;
      mv[ob][r] = oc < OC ? mult[oc] : 0.f;
    }
  // the lane's patch offsets of taps 16 s + 4 lk + j (a tap past the kernel
  // reads offset 0: its weights are zero)
  int toff[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * s + 4 * lk + j;
      toff[s][j] = t < T ? (t / KW) * PCW + t % KW : 0;
    }
  stage();
  __syncthreads();

#pragma unroll 1
  for (; band < total; band += gridDim.x) {
    const int next = band + gridDim.x;
    if (next < total) load(next);            // in flight while this band computes

    // 2 + 3. 16-pixel groups, strided over the waves
#pragma unroll 1
    for (int g = wave; g < NG; g += 4) {
      const int p0 = 16 * g + li;
      const bool pv = p0 < NP;
      const int p = pv ? p0 : 0;
      const int r = p / OW, ow = p - r * OW;
      const int* pb = patch + r * SH * PCW + ow * SW;
      intx4 b[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        b[s] = intx4{pb[toff[s][0]], pb[toff[s][1]], pb[toff[s][2]], pb[toff[s][3]]};
#pragma unroll
      for (int ob = 0; ob < NOB; ++ob) {
        intx4 acc = bv[ob];
#pragma unroll
        for (int s = 0; s < NS; ++s)
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ob][s], b[s], acc, 0, 0, 0);
        if (pv && 16 * ob + 4 * lk < OC) {
          int c4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int word = requant_word(acc[j], mv[ob][j], (float)LO);
            c4[j] = EPI == 1 ? (int)tab[word & 0xff] : word;
          }
          outs[(p * OC + 16 * ob + 4 * lk) >> 2] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
      }
    }
    __syncthreads();

    // 4. the band's rows of y: one contiguous range
    const int n = band / BANDS;
    const int oh0 = (band - n * BANDS) * R;
    const int rows = OH - oh0 < R ? OH - oh0 : R;
    i8* yb = y + (size_t)(n * OH + oh0) * OW * OC;
    if constexpr ((OW * OC) % 16 == 0) {
      const int n16 = rows * (OW * OC / 16);
      for (int i = threadIdx.x; i < n16; i += 256)
        reinterpret_cast<intx4*>(yb)[i] = reinterpret_cast<const intx4*>(outs)[i];
    } else {
      const int n4 = rows * (OW * OC / 4);
      for (int i = threadIdx.x; i < n4; i += 256) reinterpret_cast<int*>(yb)[i] = outs[i];
    }
    if (next < total) stage();               // every wave has read the patch (barrier above)
    __syncthreads();
  }
}

// Quantize float32 NCHW -> int8 NHWC: clamp(rint(x * inv_s), -127, 127).
__device__ __forceinline__ void quantize_nchw_nhwc(const float* __restrict__ x, i8* __restrict__ y,
                                                   int N, int C, int HW, float inv_s) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * C * HW;
  if (i >= total) return;
  const int c = (int)(i % C);
  const long long p = i / C;
  const int hw = (int)(p % HW);
  const int n = (int)(p / HW);
  float r = rintf(x[((size_t)n * C + c) * HW + hw] * inv_s);
  y[i] = (i8)(int)fminf(fmaxf(r, -127.0f), 127.0f);
}

// Residual add of two int8 tensors with their own multipliers (same layout).
// Each thread handles 16 codes; the last n % 16 one per thread.
__device__ __forceinline__ void qadd_i8(const i8* __restrict__ a, const i8* __restrict__ b,
                                        i8* __restrict__ y, long long n, float ma, float mb) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long nq = n >> 4;
  auto one = [&](i8 av, i8 bv) -> i8 {
    const float s = (float)av * ma + (float)bv * mb;
    return (i8)(int)fminf(fmaxf(rintf(s), -127.0f), 127.0f);
  };
  if (i < nq) {
    union { intx4 v; i8 e[16]; } ua, ub, uy;
    ua.v = reinterpret_cast<const intx4*>(a)[i];
    ub.v = reinterpret_cast<const intx4*>(b)[i];
#pragma unroll
    for (int j = 0; j < 16; ++j) uy.e[j] = one(ua.e[j], ub.e[j]);
    reinterpret_cast<intx4*>(y)[i] = uy.v;
  } else {
    const long long j = nq * 16 + (i - nq);
    if (j < n) y[j] = one(a[j], b[j]);
  }
}

// Table lookup y = table[x + 128] (e.g. GELU between two scales).
__device__ __forceinline__ void qlut_i8(const i8* __restrict__ x, const i8* __restrict__ table,
                                        i8* __restrict__ y, long long n) {
  __shared__ i8 t[256];
  if (threadIdx.x < 256) t[threadIdx.x] = table[threadIdx.x];
  __syncthreads();
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long nq = n >> 4;
  if (i < nq) {
    union { intx4 v; i8 e[16]; } u;
    u.v = reinterpret_cast<const intx4*>(x)[i];
#pragma unroll
    for (int j = 0; j < 16; ++j) u.e[j] = t[(int)u.e[j] + 128];
    reinterpret_cast<intx4*>(y)[i] = u.v;
  } else {
    const long long j = nq * 16 + (i - nq);
    if (j < n) y[j] = t[(int)x[j] + 128];
  }
}

// Global average pool over NHWC int8: exact int32 sum over HW per (n, c),
// then requantize with m = s_in / (HW * s_out). Output [N][C].
__device__ __forceinline__ void qgap_nhwc(const i8* __restrict__ x, i8* __restrict__ y, int N,
                                          int C, int HW, float m) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * C) return;
  const int c = i % C;
  const int n = i / C;
  const i8* xp = x + (size_t)n * HW * C + c;
  int s = 0;
  for (int p = 0; p < HW; ++p) s += (int)xp[(size_t)p * C];
  y[i] = requant(s, m, -127.0f);
}

// Fused int8 channel mixer over channels-last rows:
//
//   h = table[q1(X W1^T + b1)]          [M][E], kept in LDS
//   Y = qadd(X, q2(h W2^T + b2))        [M][C]
//
// with q1/q2 the requantization of a QConv (lower clamps LO1/LO2) and qadd
// the residual add (res_mult on X, acc_mult on the codes), i.e. two 1x1
// QConvs with their fused lookup and residual epilogues in one launch: the
// hidden tensor never goes to HBM and X is read once (the residual comes
// from the LDS copy). Weights are [E][CP] and [C][EP], K zero padded to a
// multiple of 64 (CP, EP), so whatever sits in the padded K columns of the
// LDS tiles is multiplied by zero. With MIX = 1 the X rows are themselves
// computed in the prologue: a depthwise KHxKW stride-1 QConv (the block's
// token mixer, lower clamp LOD) over the input Z, so X never goes to HBM
// either.
//
// A workgroup of 4 waves owns BM rows. Each GEMM puts its waves on a
// WGM x WGN grid: a wave owns BM/WGM rows and, per column chunk, NI blocks
// of 16 columns; the chunks step over the output columns. A fragments come
// from the LDS tiles, B fragments (weight rows, 16 contiguous K bytes per
// lane) straight from global memory: the weights are small and L2 resident.
// MFMA v_mfma_i32_16x16x64_i8 with the weight fragment as the row operand,
// so a lane ends with 4 consecutive output columns of one row.
struct QMlpArgs {
  const i8* __restrict__ X;        // [M][C]; with a token mixer its input Z [N][H][W][C]
  const i8* __restrict__ Wd;       // token mixer: block-diagonal depthwise weights [C][KD]
  const int* __restrict__ bd;      // [C]
  const float* __restrict__ md;    // [C]
  const i8* __restrict__ W1;       // [E][CP]
  const int* __restrict__ b1;      // [E]
  const float* __restrict__ m1;    // [E]
  const i8* __restrict__ table;    // [256]
  const i8* __restrict__ W2;       // [C][EP]
  const int* __restrict__ b2;      // [C]
  const float* __restrict__ m2;    // [C]
  i8* __restrict__ Y;              // [M][C]
  int M, H, W;                     // rows; the token mixer's image size (stride 1, same size)
  float res_mult, acc_mult;
};

// Token mixer prologue: X rows [m0, m0 + BM) of a depthwise KHxKW stride-1
// QConv over the NHWC input Z, requantized with (bd, md, LOD), written to the
// LDS tile. It runs on the matrix cores as a block-diagonal GEMM per 16-row,
// 16-channel tile: k = (tap, channel in the block), so a lane's 16-byte A
// fragment is one tap's 16 channels of one pixel (loaded straight from Z,
// zeros outside the image and past M) and Wd is packed [C][KD] with
// Wd[n][tap*16 + n%16] = w[n][tap] and zeros elsewhere (KD = KH*KW*16
// rounded up to 64). The int32 sums are exact, so this equals the unfused
// depthwise conv bit for bit.
// A wave's tiles are handled in batches of MIXB (at most 3, or all of them):
// the loads of every tile of a batch (its Z fragments, KD / 64 steps each)
// are issued before the first MFMA, so a batch costs one memory round trip
// instead of one per tile. The block-diagonal weights, bias and multipliers
// come one of two ways:
//  * MIXW = 0: the workgroup copies them into LDS once (Wds rows padded to
//    KD + 16 bytes, so the 16 lanes reading one 16-byte column of 16 rows hit
//    distinct banks), the copy's global loads issued ahead of the first
//    batch's Z loads and its LDS stores and barrier after them;
//  * MIXW = 1 (launches with at most one workgroup per CU, where registers
//    cost no occupancy): tile u of wave w (t = w + 4u) takes channel block
//    (w + 4u) % CB, which repeats every P = CB / gcd(4, CB) tiles, so the
//    wave loads the fragments, bias and multipliers of its P channel blocks
//    once, straight from global memory into registers (the rows are small and
//    L2 resident) with the first batch's Z loads, and tile u uses set u % P:
//    no LDS copy, no barrier for the weights.
template <int C, int KH, int KW>
struct QMixDims {
  static constexpr int KD = (KH * KW * 16 + 63) / 64 * 64;   // Wd row (bytes) in global memory
  static constexpr int WS = KD + 16;                          // and in LDS
};

//
// `after_first` runs once the first batch's loads are issued, before any
// wait: the caller issues its own (later needed) loads there, so that the
// waits of the mixer, which count outstanding loads in issue order, do not
// wait for them.
template <int C, int BM, int XS, int KH, int KW, int PT, int PL, int LOD, int MIXB_MAX, int MIXW,
          int H, int W, class After>
__device__ __forceinline__ void qmlp_mixer(const QMlpArgs& g, i8* __restrict__ Xs, int m0,
                                           i8* __restrict__ Wds, int* __restrict__ bds,
                                           float* __restrict__ mds, After after_first) {
  constexpr int TAPS = KH * KW;
  constexpr int KD = QMixDims<C, KH, KW>::KD, WS = QMixDims<C, KH, KW>::WS;
  constexpr int NS = KD / 64;
  constexpr int CB = C / 16, TILES = (BM / 16) * CB;
  constexpr int TPW = (TILES + 3) / 4;                // tiles per wave
  constexpr int MIXB = TPW < MIXB_MAX ? TPW : MIXB_MAX;  // tiles per batch
  constexpr int WCH = C * KD / 16;                    // 16-byte chunks of Wd
  constexpr int WPT = MIXW ? 1 : (WCH + 255) / 256;
  constexpr int CPT = MIXW ? 1 : (C + 255) / 256;
  constexpr int G4 = CB % 4 == 0 ? 4 : (CB % 2 == 0 ? 2 : 1);   // gcd(4, CB)
  constexpr int P = !MIXW ? 1 : (CB / G4 < TPW ? CB / G4 : TPW);   // weight sets a wave holds
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // tiles are wave-uniform: scalar
  __builtin_assume(wave < 4);                         // 256 threads: with TILES % 4 == 0 every tile is real
  const int li = lane & 15, lk = lane >> 4;
  const __amdgpu_buffer_rsrc_t rZ = buffer_over(g.X, g.M * C);
  const __amdgpu_buffer_rsrc_t rW = buffer_over(g.Wd, C * KD);
  // the taps 4s + lk a lane reads at step s: row and column shifts, and the
  // neighbour's byte offset from the row's own pixel (rows are NHWC pixels,
  // so the pixel (n, oh + dy, ow + dx) is row m + dy W + dx)
  int dyv[NS], dxv[NS], dov[NS];
  bool tapv[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int tap = s * 4 + lk;
    dyv[s] = tap / KW - PT;
    dxv[s] = tap % KW - PL;
    dov[s] = (dyv[s] * W + dxv[s]) * C;
    tapv[s] = tap < TAPS;
  }
  intx4 wst[WPT];
  int bdv[CPT];
  float mdv[CPT];
  intx4 wf[P][NS], bf[P];
  floatx4 mf[P];
  if constexpr (MIXW) {
    // set p: channel block (wave + 4p) % CB; lane 16 lk + li holds row cb*16 + li
    // (taps 4s + lk) and channels cb*16 + 4lk .. +3 of the bias and multipliers
    const __amdgpu_buffer_rsrc_t rB = buffer_over(g.bd, C * 4);
    const __amdgpu_buffer_rsrc_t rM = buffer_over(g.md, C * 4);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int cb = (wave + 4 * p) % CB;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        wf[p][s] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(
            rW, (cb * 16 + li) * KD + lk * 16, s * 64, 0));
      bf[p] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rB, (cb * 16 + lk * 4) * 4, 0, 0));
      mf[p] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rM, (cb * 16 + lk * 4) * 4, 0, 0));
    }
  } else {
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int idx = tid + 256 * i;
      wst[i] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(
          rW, idx < WCH ? idx * 16 : kOutside, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      bdv[i] = c < C ? g.bd[c] : 0;
      mdv[i] = c < C ? g.md[c] : 0.f;
    }
  }
#pragma unroll
  for (int b0 = 0; b0 < TPW; b0 += MIXB) {
    intx4 a[MIXB][NS];
#pragma unroll
    for (int u = 0; u < MIXB; ++u) {
      // tile t of this wave (scalar); past the last tile (TILES % 4 != 0) a
      // tile with every load out of range, whose result is never stored
      const int t = wave + 4 * (b0 + u);
      const bool tile_ok = b0 + u < TPW && t < TILES;
      const int rb = t / CB, cb = t - (t / CB) * CB;
      const int m = m0 + rb * 16 + li;
      // H and W are compiled in: the divisions (of non-negative values) are
      // multiplies
      const int n = (int)((unsigned)m / (unsigned)(H * W));
      const int sp = m - n * (H * W);
      const int oh0 = (int)((unsigned)sp / (unsigned)W);
      const int ow = sp - oh0 * W;
      const int oh = tile_ok && m < g.M ? oh0 : -(1 << 20);
      const int base = m * C + cb * 16;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bool ok = tapv[s] && (unsigned)(oh + dyv[s]) < (unsigned)H && (unsigned)(ow + dxv[s]) < (unsigned)W;
        a[u][s] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(
            rZ, ok ? base + dov[s] : kOutside, 0, 0));
      }
    }
    if (b0 == 0) {
      after_first();
      __builtin_amdgcn_sched_barrier(0);              // every load above issues before the first wait
    }
    if (!MIXW && b0 == 0) {                           // the weights reach LDS (once)
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int idx = tid + 256 * i;
        if (WCH % 256 == 0 || idx < WCH)
          *reinterpret_cast<intx4*>(&Wds[(idx / (KD / 16)) * WS + (idx % (KD / 16)) * 16]) = wst[i];
      }
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = tid + 256 * i;
        if (c < C) {
          bds[c] = bdv[i];
          mds[c] = mdv[i];
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < MIXB; ++u) {
      // a tile past the last (TILES % 4 != 0) is computed from its zero
      // loads and not stored: no branch around its loads and MFMAs
      const int t = wave + 4 * (b0 + u);
      if (b0 + u >= TPW) continue;                    // compile time
      const int tt = t < TILES ? t : TILES - 1;
      const int rb = tt / CB, cb = tt - (tt / CB) * CB;
      // acc[j]: row rb*16 + li, channel cb*16 + lk*4 + j, starting at its bias
      const int c = cb * 16 + lk * 4;
      const int p = (b0 + u) % P;                     // compile time: b0 and u are unrolled
      intx4 acc = MIXW ? bf[p] : *reinterpret_cast<const intx4*>(&bds[c]);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const intx4 w = MIXW ? wf[p][s]
                             : *reinterpret_cast<const intx4*>(&Wds[(cb * 16 + li) * WS + s * 64 + lk * 16]);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, a[u][s], acc, 0, 0, 0);
      }
      const floatx4 mv = MIXW ? mf[p] : *reinterpret_cast<const floatx4*>(&mds[c]);
      const int o = pack4(requant_word(acc[0], mv[0], (float)LOD), requant_word(acc[1], mv[1], (float)LOD),
                          requant_word(acc[2], mv[2], (float)LOD), requant_word(acc[3], mv[3], (float)LOD));
      if (TILES % 4 == 0 || t < TILES) *reinterpret_cast<int*>(&Xs[(rb * 16 + li) * XS + c]) = o;
    }
  }
}

template <int NK, int LDB, int NI>
struct QMlpFrags {                   // B fragments of one column chunk, whole K
  intx4 f[NK / 64][NI];
  // One 32-bit lane offset; each fragment's place in the chunk (a constant)
  // goes in the scalar offset, so the loads cost no vector instructions.
  // Every fragment lies inside the weights (col0 + NI*16 <= their rows).
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rB, int col0) {
    const int lane = threadIdx.x & 63;
    const int vo = (col0 + (lane & 15)) * LDB + (lane >> 4) * 16;
#pragma unroll
    for (int s = 0; s < NK / 64; ++s)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        f[s][ni] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(
            rB, vo, ni * 16 * LDB + s * 64, 0));
  }
};

// the wave index as a scalar (it is uniform over the wave)
__device__ __forceinline__ int qmlp_wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

template <int WGN, int NI>
__device__ __forceinline__ int qmlp_col0(int c0) { return c0 + (qmlp_wave() % WGN) * NI * 16; }

// The accumulators of a column chunk start at the columns' bias (LDS), so
// the epilogue gets the exact int32 acc + bias.
template <int NK, int LDA, int LDB, int NCOLS, int BM, int WGM, int WGN, int NI, class Epi, class Hook>
__device__ __forceinline__ void qmlp_gemm(const i8* __restrict__ As, __amdgpu_buffer_rsrc_t rB,
                                          const QMlpFrags<NK, LDB, NI>& first,
                                          const int* __restrict__ bias_lds, Epi epi, Hook hook) {
  constexpr int MI = BM / WGM / 16;
  constexpr int CHUNK = WGN * NI * 16;
  static_assert(NCOLS % CHUNK == 0 && (BM / WGM) % 16 == 0, "column chunks must tile the output");
  const int lane = threadIdx.x & 63;
  const int wave = qmlp_wave();
  const int li = lane & 15, lk = lane >> 4;
  const int r0 = (wave / WGN) * (BM / WGM);
#pragma unroll
  for (int c0 = 0; c0 < NCOLS; c0 += CHUNK) {
    const int col0 = qmlp_col0<WGN, NI>(c0);
    QMlpFrags<NK, LDB, NI> fr;
    if (c0 == 0) fr = first; else fr.load(rB, col0);
    intx4 acc[MI][NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const intx4 bv = *reinterpret_cast<const intx4*>(&bias_lds[col0 + ni * 16 + lk * 4]);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) acc[mi][ni] = bv;
    }
#pragma unroll
    for (int s = 0; s < NK / 64; ++s) {
      intx4 af[MI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        af[mi] = *reinterpret_cast<const intx4*>(As + (r0 + mi * 16 + li) * LDA + s * 64 + lk * 16);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fr.f[s][ni], af[mi], acc[mi][ni], 0, 0, 0);
    }
    if (c0 + CHUNK >= NCOLS) hook();
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        epi(r0 + mi * 16 + li, col0 + ni * 16 + lk * 4, acc[mi][ni], c0 / CHUNK, ni);
  }
}

// MIXB_MAX: the token mixer's tiles per load batch; MIXW: its weights in
// registers (1) or in LDS (0), see qmlp_mixer. EW2: fetch the second
// GEMM's weight fragments at the start with the first's (registers for both
// sets; chosen where the launch has at most one workgroup per CU, so the
// registers cost no occupancy) instead of under the first GEMM's epilogue.
template <int C, int E, int BM, int WGM1, int WGN1, int NI1, int WGM2, int WGN2, int NI2, int LO1,
          int LO2, int MIX, int KH, int KW, int PT, int PL, int LOD, int MIXB_MAX = 3, bool EW2 = false,
          int MIXW = 0, int MH = 1, int MW = 1>
__device__ __forceinline__ void qmlp_i8(const QMlpArgs& g) {
  constexpr int CP = (C + 63) / 64 * 64, EP = (E + 63) / 64 * 64;
  constexpr int XS = CP + 16, HS = EP + 16;    // LDS row strides (bytes)
  constexpr int NT = 256;
  static_assert(C % 16 == 0 && E % 16 == 0, "channel counts must be multiples of 16");
  __shared__ __attribute__((aligned(16))) i8 Xs[BM * XS];
  __shared__ __attribute__((aligned(16))) i8 Hs[BM * HS];
  __shared__ i8 tab[256];
  // both GEMMs' bias and multipliers: staged with the table at the start, so
  // neither epilogue waits on a global load in the middle of the chain
  __shared__ __attribute__((aligned(16))) int b1s[E];
  __shared__ __attribute__((aligned(16))) float m1s[E];
  __shared__ __attribute__((aligned(16))) int b2s[C];
  __shared__ __attribute__((aligned(16))) float m2s[C];
  // the token mixer's weights, bias and multipliers in LDS (MIXW = 0; a few
  // bytes otherwise)
  constexpr bool kMixLds = MIX && !MIXW;
  __shared__ __attribute__((aligned(16))) i8 Wds[kMixLds ? C * QMixDims<C, KH, KW>::WS : 16];
  __shared__ __attribute__((aligned(16))) int bds[kMixLds ? C : 4];
  __shared__ __attribute__((aligned(16))) float mds[kMixLds ? C : 4];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.x * BM;

  // The lookup table (with its halves swapped: code q's entry sits at q's
  // low byte, (q + 128) ^ 0x80 = q & 0xff, which the requantized word holds)
  // and both GEMMs' bias and multipliers, loaded first into registers and
  // stored to LDS with the X tile: neither epilogue waits on a global load
  // in the middle of the chain, and the stores wait for these loads only.
  constexpr int EPT = (E + NT - 1) / NT, CPT2 = (C + NT - 1) / NT;
  const i8 tabv = g.table[tid ^ 0x80];
  int b1v[EPT], b2v[CPT2];
  float m1v[EPT], m2v[CPT2];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = tid + k * NT;
    b1v[k] = i < E ? g.b1[i] : 0;
    m1v[k] = i < E ? g.m1[i] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < CPT2; ++k) {
    const int i = tid + k * NT;
    b2v[k] = i < C ? g.b2[i] : 0;
    m2v[k] = i < C ? g.m2[i] : 0.f;
  }

  // The first weight chunk (with EW2 both GEMMs' fragments) is fetched while
  // the X tile comes in, issued after the X tile's loads (or the token
  // mixer's first batch): a wait counts outstanding loads in issue order, so
  // the X tile is then ready without waiting for the weights.
  const __amdgpu_buffer_rsrc_t rW1 = buffer_over(g.W1, E * CP);
  const __amdgpu_buffer_rsrc_t rW2 = buffer_over(g.W2, C * EP);
  QMlpFrags<CP, CP, NI1> w1f;
  QMlpFrags<EP, EP, NI2> w2f;
  const auto weights = [&]() {
    w1f.load(rW1, qmlp_col0<WGN1, NI1>(0));
    if constexpr (EW2) w2f.load(rW2, qmlp_col0<WGN2, NI2>(0));
  };
  if constexpr (MIX) {
    qmlp_mixer<C, BM, XS, KH, KW, PT, PL, LOD, MIXB_MAX, MIXW, MH, MW>(g, Xs, m0, Wds, bds, mds, weights);
  } else {
    const __amdgpu_buffer_rsrc_t rX = buffer_over(g.X, g.M * C);
    constexpr int CPR = CP / 16;
    constexpr int XPT = (BM * CPR + NT - 1) / NT;
    intx4 xr[XPT];
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int i = tid + k * NT;
      const int r = i / CPR, j = i - (i / CPR) * CPR;
      const int off = (i < BM * CPR && m0 + r < g.M && j * 16 < C) ? (m0 + r) * C + j * 16 : kOutside;
      xr[k] = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rX, off, 0, 0));
    }
    weights();
    __builtin_amdgcn_sched_barrier(0);                // every load above issues before the first wait
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int i = tid + k * NT;
      const int r = i / CPR, j = i - (i / CPR) * CPR;
      if ((BM * CPR) % NT == 0 || i < BM * CPR) *reinterpret_cast<intx4*>(&Xs[r * XS + j * 16]) = xr[k];
    }
  }
  tab[tid] = tabv;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = tid + k * NT;
    if (i < E) {
      b1s[i] = b1v[k];
      m1s[i] = m1v[k];
    }
  }
#pragma unroll
  for (int k = 0; k < CPT2; ++k) {
    const int i = tid + k * NT;
    if (i < C) {
      b2s[i] = b2v[k];
      m2s[i] = m2v[k];
    }
  }
  __syncthreads();

  qmlp_gemm<CP, XS, CP, E, BM, WGM1, WGN1, NI1>(Xs, rW1, w1f, b1s, [&](int r, int n, const intx4& acc,
                                                                      int, int) {
    const floatx4 mv = *reinterpret_cast<const floatx4*>(&m1s[n]);
    int o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = tab[requant_word(acc[j], mv[j], (float)LO1) & 0xff];
    *reinterpret_cast<int*>(&Hs[r * HS + n]) = pack4(o[0], o[1], o[2], o[3]);
  }, [&]() {
    if constexpr (!EW2) w2f.load(rW2, qmlp_col0<WGN2, NI2>(0));
  });
  __syncthreads();

  qmlp_gemm<EP, HS, EP, C, BM, WGM2, WGN2, NI2>(Hs, rW2, w2f, b2s, [&](int r, int n, const intx4& acc,
                                                                     int, int) {
    const int m = m0 + r;
    if (m >= g.M) return;
    const floatx4 mv = *reinterpret_cast<const floatx4*>(&m2s[n]);
    union { int w; i8 b[4]; } x;
    x.w = *reinterpret_cast<const int*>(&Xs[r * XS + n]);
    int o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // the requantized code as a float: clamp, then round half to even (the
      // clamp bounds are integers, so the order does not matter)
      const float code = rintf(fminf(fmaxf((float)acc[j] * mv[j], (float)LO2), 127.0f));
      const float v = (float)x.b[j] * g.res_mult + code * g.acc_mult;
      // clamp(rint(v), -127, 127) in the low byte, as requant_word forms it
      o[j] = __builtin_bit_cast(int, fminf(fmaxf(v, -127.0f), 127.0f) + 12582912.0f);
    }
    *reinterpret_cast<int*>(g.Y + (size_t)m * C + n) = pack4(o[0], o[1], o[2], o[3]);
  }, [] {});
}

// The same pool with one workgroup per image (blockIdx.x) and block of CB =
// C / gridDim.y channels (blockIdx.y; CB % 4 == 0, CB <= 1024): thread t sums
// channels c0 + [4g, 4g+4) (g = t % (CB/4)) over the pixels p = t / (CB/4)
// (mod R), R = 256 / (CB/4), with 32-bit loads coalesced along the channels;
// the R partial sums of each channel meet in LDS. Integer sums are exact, so
// the result equals qgap_nhwc's.
__device__ __forceinline__ void qgap_nhwc_wg(const i8* __restrict__ x, i8* __restrict__ y, int C,
                                             int HW, float m) {
  __shared__ int part[1024];
  const int n = blockIdx.x;
  const int CB = C / (int)gridDim.y, c0 = (int)blockIdx.y * CB;
  const int G = CB / 4, R = 256 / G;
  const int t = threadIdx.x, gi = t % G, r = t / G;
  int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  if (r < R) {
    const i8* xp = x + (size_t)n * HW * C + c0 + 4 * gi;
    for (int p = r; p < HW; p += R) {
      union { int w; i8 b[4]; } v;
      v.w = *reinterpret_cast<const int*>(xp + (size_t)p * C);
      s0 += v.b[0]; s1 += v.b[1]; s2 += v.b[2]; s3 += v.b[3];
    }
  }
  for (int c = t; c < CB; c += 256) part[c] = 0;
  __syncthreads();
  if (r < R) {
    atomicAdd(&part[4 * gi], s0);
    atomicAdd(&part[4 * gi + 1], s1);
    atomicAdd(&part[4 * gi + 2], s2);
    atomicAdd(&part[4 * gi + 3], s3);
  }
  __syncthreads();
  for (int c = t; c < CB; c += 256) y[(size_t)n * C + c0 + c] = requant(part[c], m, -127.0f);
}

// Dequantize: float(q) * s; an NHWC 4-D input is written back as NCHW.
__device__ __forceinline__ void dequantize_i8(const i8* __restrict__ x, float* __restrict__ y,
                                              long long n, int C, int HW, float s) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (HW > 1) {                       // i indexes NCHW output
    const int hw = (int)(i % HW);
    const int c = (int)((i / HW) % C);
    const long long nn = i / ((long long)HW * C);
    y[i] = (float)x[((size_t)nn * HW + hw) * C + c] * s;
  } else {
    y[i] = (float)x[i] * s;
  }
}

}  // namespace mdlc
