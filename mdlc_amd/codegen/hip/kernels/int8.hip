// INT8 quantized kernels for gfx950. Activations are channels-last (NHWC)
// on the device so both matrix operands are contiguous along K.
//
// Semantics (bit-exact contract): products of int8 codes accumulate in int32;
// requantization is clamp(rint(float(acc) * m), lo, 127) with a single
// correctly rounded float multiply, rint = round half to even, lo = 0 after
// a fused ReLU else -127. No fused multiply-add anywhere (-ffp-contract=off).
namespace mdlc {

typedef signed char i8;

__device__ __forceinline__ i8 requant(int acc, float m, float lo) {
  float r = rintf((float)acc * m);
  r = fminf(fmaxf(r, lo), 127.0f);
  return (i8)(int)r;
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
  const i8* __restrict__ A;       // AMODE 0: [M][lda]; AMODE 1/2: NHWC conv input
  const i8* __restrict__ B;       // [N][ldb], K contiguous, zero padded to ldb
  const int* __restrict__ bias;   // [N]
  const float* __restrict__ mult; // [N]
  void* __restrict__ C;           // int8 [M][ldc] or float [M][ldc]
  int M, N, K, lda, ldb, ldc;
  int Cin, H, W, OH, OW;          // conv geometry (AMODE 1/2); M = batch*OH*OW
};

// C[m][n] = q(sum_k A[m][k] * B[n][k] + bias[n]).
// AMODE 0: dense A, 16-byte loads (K % 16 == 0).
// AMODE 1: implicit im2col over an NHWC input with k = (kh, kw, c) and
//          Cin % 16 == 0: each 16-byte chunk is one tap's 16 channels of one
//          pixel, a single aligned load.
// AMODE 2: the same gather one byte at a time (any Cin).
// OUT 0: int8 requantized output (LO = lower clamp); OUT 1: float32
//        float(acc) * mult[n] (dequantized logits).
template <int BM, int BN, int BK, int WGM, int WGN, int MS, int AMODE, int OUT, int LO, class Win>
__device__ __forceinline__ void qgemm_i8_mfma(const QGemmArgs& g) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MS, NI = WN / MS;
  constexpr int KG = 64 / MS;
  constexpr int KSUB = BK / KG;
  constexpr int LDS_ROW = BK + 16;
  static_assert(KSUB % 16 == 0, "BK too small for this MFMA shape");
  typedef typename MfmaI8<MS>::acc_t acc_t;

  __shared__ __attribute__((aligned(16))) i8 As[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) i8 Bs[2][BN * LDS_ROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int li = lane % MS;
  const int lk = lane / MS;

  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int m0 = (t % tiles_m) * BM;
  const int n0 = (t / tiles_m) * BN;

  constexpr int CPR = BK / 16;               // 16-byte chunks per row
  constexpr int A_CH = BM * CPR, B_CH = BN * CPR;
  constexpr int A_PT = (A_CH + NT - 1) / NT, B_PT = (B_CH + NT - 1) / NT;
  static_assert(NT % CPR == 0, "rows must map to fixed threads");
  intx4 ra[A_PT], rb[B_PT];

  // per-thread conv rows (fixed across K tiles)
  int rbase[A_PT], rih[A_PT], riw[A_PT];
  if (AMODE != 0) {
    const int ohw = g.OH * g.OW;
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      const int p = m0 + (tid + i * NT) / CPR;
      if (p < g.M) {
        const int n = p / ohw;
        const int s = p - n * ohw;
        const int oh = s / g.OW;
        const int ow = s - oh * g.OW;
        rbase[i] = n * g.H * g.W;
        rih[i] = oh * Win::SH - Win::PT;
        riw[i] = ow * Win::SW - Win::PL;
      } else {
        rbase[i] = 0;
        rih[i] = -(1 << 28);
        riw[i] = 0;
      }
    }
  }

  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      const int idx = tid + i * NT;
      intx4 v = {0, 0, 0, 0};
      if (idx < A_CH) {
        const int r = idx / CPR, kc = idx % CPR;
        const int gm = m0 + r, gk = k0 + kc * 16;
        if (AMODE == 0) {
          if (gm < g.M && gk < g.K) v = *reinterpret_cast<const intx4*>(g.A + (size_t)gm * g.lda + gk);
        } else if (AMODE == 1) {
          if (gk < g.K) {
            const int tap = gk / g.Cin;
            const int c = gk - tap * g.Cin;
            const int kh = tap / Win::KW, kw = tap - (tap / Win::KW) * Win::KW;
            const int ih = rih[i] + kh * Win::DH, iw = riw[i] + kw * Win::DW;
            if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
              v = *reinterpret_cast<const intx4*>(g.A + ((size_t)rbase[i] + ih * g.W + iw) * g.Cin + c);
          }
        } else {
          union { intx4 v4; i8 b[16]; } u;
          u.v4 = v;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int k = gk + j;
            i8 e = 0;
            if (k < g.K) {
              const int tap = k / g.Cin;
              const int c = k - tap * g.Cin;
              const int kh = tap / Win::KW, kw = tap - (tap / Win::KW) * Win::KW;
              const int ih = rih[i] + kh * Win::DH, iw = riw[i] + kw * Win::DW;
              if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                e = g.A[((size_t)rbase[i] + ih * g.W + iw) * g.Cin + c];
            }
            u.b[j] = e;
          }
          v = u.v4;
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      const int idx = tid + i * NT;
      intx4 v = {0, 0, 0, 0};
      if (idx < B_CH) {
        const int r = idx / CPR, kc = idx % CPR;
        const int gn = n0 + r, gk = k0 + kc * 16;
        if (gn < g.N && gk < g.K) v = *reinterpret_cast<const intx4*>(g.B + (size_t)gn * g.ldb + gk);
      }
      rb[i] = v;
    }
  };

  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      const int idx = tid + i * NT;
      if (idx < A_CH)
        *reinterpret_cast<intx4*>(&As[buf][(idx / CPR) * LDS_ROW + (idx % CPR) * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      const int idx = tid + i * NT;
      if (idx < B_CH)
        *reinterpret_cast<intx4*>(&Bs[buf][(idx / CPR) * LDS_ROW + (idx % CPR) * 16]) = rb[i];
    }
  };

  acc_t acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int r = 0; r < MfmaI8<MS>::kAcc; ++r) acc[mi][ni][r] = 0;

  const int nk = (g.K + BK - 1) / BK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles((kt + 1) * BK);
    const i8* as = &As[cur][0];
    const i8* bs = &Bs[cur][0];
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
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = MfmaI8<MS>::step(af[mi], bf[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = n0 + wn0 + ni * MS + li;
    if (col >= g.N) continue;
    const int bv = g.bias[col];
    const float mv = g.mult[col];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < MfmaI8<MS>::kAcc; ++r) {
        const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
        if (row < g.M) {
          const int a = acc[mi][ni][r] + bv;
          if (OUT == 1)
            static_cast<float*>(g.C)[(size_t)row * g.ldc + col] = (float)a * mv;
          else
            static_cast<i8*>(g.C)[(size_t)row * g.ldc + col] = requant(a, mv, (float)LO);
        }
      }
  }
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
