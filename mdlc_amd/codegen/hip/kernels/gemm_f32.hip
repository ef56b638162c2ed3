// fp32 GEMM with a fused bias/activation epilogue on CDNA4 matrix cores.
//
//   C = epi(A[M x K] * B[K x N], bias)
//
// A is row-major with leading dimension lda. B comes from one of four
// sources (BMODE): 0 = dense row-major B[K][ldb] read as float4 (ldb % 4 == 0),
// 1 = dense row-major read as scalars, 2 = implicit im2col of an NCHW input x
// (B[k][p] = x[n][c][oh*SH-PT+kh*DH][ow*SW-PL+kw*DW], zero outside) with k
// ordered (c, kh, kw), 3 = the same gather with k ordered (kh, kw, c) — the
// weights are packed to match — for Cin % BK == 0: every K tile is then one
// filter tap, so a column's bounds check and pixel address are computed once
// per tile and each element costs one add and one load. Either way a
// convolution needs no column buffer. The output is row-major C[M][ldc]
// (OUT = 0) or, for convolutions, NCHW: column p = n*hw + s goes to
// C[(n*M + row)*hw + s] (OUT = 1). With split-K (OUT = 2) the grid holds
// ksplit slices of K; slice s writes its raw partial sums to the workspace
// C[(s*M + row)*N + col] and splitk_reduce_f32 adds the slices in order and
// applies the epilogue.
//
// Tiling: a workgroup of WGM x WGN waves (64 lanes each) owns a BM x BN tile;
// each wave owns (BM/WGM) x (BN/WGN) as a grid of MS x MS MFMA blocks
// (MS = 32: v_mfma_f32_32x32x2_f32, MS = 16: v_mfma_f32_16x16x4_f32).
// A and B tiles of depth BK are staged through LDS, double buffered: the next
// tile's global loads are in flight while the current tile feeds the MFMAs,
// with one barrier per K step (DB), or single buffered with two barriers
// per K step (!DB). LDS rows are padded by 4 floats so rows stay
// 16-byte aligned for ds_read_b128 and consecutive rows shift banks.
//
// K order inside a tile: the 64 lanes of an MFMA split into 64/MS groups that
// each supply one k of every instruction. Lane group g walks the contiguous
// k range [g*BK/(64/MS), (g+1)*BK/(64/MS)), so its A fragment is a run of
// consecutive floats (one ds_read_b128 per 4 k) and every k of the tile is
// covered exactly once.
namespace mdlc {

template <int MS> struct Mfma;
template <> struct Mfma<32> {
  typedef floatx16 acc_t;
  static constexpr int kAcc = 16;
  __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<16> {
  typedef floatx4 acc_t;
  static constexpr int kAcc = 4;
  __device__ __forceinline__ static acc_t step(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Compile-time convolution window (used when BMODE >= 2).
template <int KH_, int KW_, int SH_, int SW_, int DH_, int DW_, int PT_, int PL_>
struct ConvWin {
  static constexpr int KH = KH_, KW = KW_, SH = SH_, SW = SW_, DH = DH_, DW = DW_, PT = PT_, PL = PL_;
};
typedef ConvWin<1, 1, 1, 1, 1, 1, 0, 0> NoWin;

struct GemmArgs {
  const float* __restrict__ A;
  const float* __restrict__ B;   // dense B, or the NCHW conv input
  const float* __restrict__ bias;
  float* __restrict__ C;
  int M, N, K, lda, ldb, ldc, hw;
  int Cin, H, W, OH, OW;         // conv input / output geometry (BMODE >= 2)
  int ksplit, kchunk;            // K slices (grid = tiles * ksplit) and slice depth
};

template <int BM, int BN, int BK, int WGM, int WGN, int MS, bool DB, bool VA, int BMODE, int OUT,
          class Epi, class Win>
__device__ __forceinline__ void gemm_f32_mfma(const GemmArgs& g) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MS, NI = WN / MS;
  constexpr int KG = 64 / MS;          // lane groups along k
  constexpr int KSUB = BK / KG;        // k per lane group per tile
  constexpr int LDA_S = BK + 4, LDB_S = BN + 4;
  static_assert(WM % MS == 0 && WN % MS == 0, "wave tile must be a multiple of the MFMA");
  static_assert(KSUB % 4 == 0, "BK too small for this MFMA shape");
  static_assert(BN % 4 == 0 && BK % 4 == 0, "tile dims must be multiples of 4");
  typedef typename Mfma<MS>::acc_t acc_t;

  constexpr int NBUF = DB ? 2 : 1;
  __shared__ __attribute__((aligned(16))) float As[NBUF][BM * LDA_S];
  __shared__ __attribute__((aligned(16))) float Bs[NBUF][BK * LDB_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int li = lane % MS;
  const int lk = lane / MS;

  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  // Logical order (slice, n-block, m-block), m fastest: workgroups sharing a
  // B slab are consecutive and land on the same XCD.
  const int t = xcd_remap(blockIdx.x, tiles * g.ksplit);
  const int ks = t / tiles;
  const int tt = t - ks * tiles;
  const int m0 = (tt % tiles_m) * BM;
  const int n0 = (tt / tiles_m) * BN;
  const int kbeg = ks * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);

  // ---- A tile staging ----------------------------------------------------
  constexpr int A_ELEMS = VA ? BM * BK / 4 : BM * BK;
  constexpr int A_PT = (A_ELEMS + NT - 1) / NT;
  float4 ra[VA ? A_PT : 1];
  float rs[VA ? 1 : A_PT];

  // ---- B tile staging ----------------------------------------------------
  constexpr bool BQ = (BMODE != 1);    // quads of 4 consecutive columns
  constexpr int B_ELEMS = BQ ? BK * BN / 4 : BK * BN;
  constexpr int B_PT = (B_ELEMS + NT - 1) / NT;
  static_assert(!BQ || (NT % (BN / 4) == 0), "thread count must cover whole column quads");
  float4 rb[BQ ? B_PT : 1];
  float rbs[BQ ? 1 : B_PT];

  // Implicit-im2col state: the column quad each thread gathers is fixed.
  int cbase[4], cih[4], ciw[4];
  if (BMODE >= 2) {
    const int nq = tid % (BN / 4);
    const int ohw = g.OH * g.OW;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int p = n0 + nq * 4 + j;
      if (p < g.N) {
        int n = p / ohw;
        int s = p - n * ohw;
        int oh = s / g.OW;
        int ow = s - oh * g.OW;
        cbase[j] = n * g.Cin * g.H * g.W;
        cih[j] = oh * Win::SH - Win::PT;
        ciw[j] = ow * Win::SW - Win::PL;
      } else {
        cbase[j] = 0;
        cih[j] = -(1 << 28);
        ciw[j] = 0;
      }
    }
  }

  auto load_tiles = [&](int k0) {
    if (VA) {
#pragma unroll
      for (int i = 0; i < A_PT; ++i) {
        int idx = tid + i * NT;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (idx < A_ELEMS) {
          int r = idx / (BK / 4), kq = idx % (BK / 4);
          int gm = m0 + r, gk = k0 + kq * 4;
          if (gm < g.M && gk < kend) v = ld4(g.A + (size_t)gm * g.lda + gk);
        }
        ra[i] = v;
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_PT; ++i) {
        int idx = tid + i * NT;
        float v = 0.f;
        if (idx < A_ELEMS) {
          int r = idx / BK, kk = idx % BK;
          int gm = m0 + r, gk = k0 + kk;
          if (gm < g.M && gk < kend) v = g.A[(size_t)gm * g.lda + gk];
        }
        rs[i] = v;
      }
    }
    if (BMODE == 0) {
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (idx < B_ELEMS) {
          int kr = idx / (BN / 4), nq = idx % (BN / 4);
          int gk = k0 + kr, gn = n0 + nq * 4;
          if (gk < kend && gn < g.N) v = ld4(g.B + (size_t)gk * g.ldb + gn);
        }
        rb[i] = v;
      }
    } else if (BMODE == 1) {
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        float v = 0.f;
        if (idx < B_ELEMS) {
          int kr = idx / BN, nn = idx % BN;
          int gk = k0 + kr, gn = n0 + nn;
          if (gk < kend && gn < g.N) v = g.B[(size_t)gk * g.ldb + gn];
        }
        rbs[i] = v;
      }
    } else if (BMODE == 3) {
      // One filter tap per tile: k0 = tap * Cin + c0 with c0 % BK == 0.
      const int HW = g.H * g.W;
      const int tap = k0 / g.Cin;
      const int c0 = k0 - tap * g.Cin;
      const int kh = tap / Win::KW;
      const int kw = tap - kh * Win::KW;
      int pix[4];
      bool ok[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ih = cih[j] + kh * Win::DH;
        const int iw = ciw[j] + kw * Win::DW;
        ok[j] = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W && k0 < kend;
        pix[j] = cbase[j] + ih * g.W + iw;
      }
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        float e[4] = {0.f, 0.f, 0.f, 0.f};
        if (idx < B_ELEMS) {
          const int cofs = (c0 + idx / (BN / 4)) * HW;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (ok[j]) e[j] = g.B[pix[j] + cofs];
        }
        rb[i] = make_float4(e[0], e[1], e[2], e[3]);
      }
    } else {
      constexpr int KHW = Win::KH * Win::KW;
      const int HW = g.H * g.W;
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        float e[4] = {0.f, 0.f, 0.f, 0.f};
        if (idx < B_ELEMS) {
          int kr = idx / (BN / 4);
          int k = k0 + kr;
          if (k < kend) {
            int c = k / KHW;
            int rr = k - c * KHW;
            int kh = rr / Win::KW;
            int kw = rr - kh * Win::KW;
            int coff = c * HW;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              int ih = cih[j] + kh * Win::DH;
              int iw = ciw[j] + kw * Win::DW;
              if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                e[j] = g.B[cbase[j] + coff + ih * g.W + iw];
            }
          }
        }
        rb[i] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  };

  auto store_tiles = [&](int buf) {
    if (VA) {
#pragma unroll
      for (int i = 0; i < A_PT; ++i) {
        int idx = tid + i * NT;
        if (idx < A_ELEMS) {
          int r = idx / (BK / 4), kq = idx % (BK / 4);
          st4(&As[buf][r * LDA_S + kq * 4], ra[i]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_PT; ++i) {
        int idx = tid + i * NT;
        if (idx < A_ELEMS) As[buf][(idx / BK) * LDA_S + idx % BK] = rs[i];
      }
    }
    if (BQ) {
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        if (idx < B_ELEMS) {
          int kr = idx / (BN / 4), nq = idx % (BN / 4);
          st4(&Bs[buf][kr * LDB_S + nq * 4], rb[i]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_PT; ++i) {
        int idx = tid + i * NT;
        if (idx < B_ELEMS) Bs[buf][(idx / BN) * LDB_S + idx % BN] = rbs[i];
      }
    }
  };

  acc_t acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int r = 0; r < Mfma<MS>::kAcc; ++r) acc[mi][ni][r] = 0.f;

  auto compute = [&](int buf) {
    const float* as = &As[buf][0];
    const float* bs = &Bs[buf][0];
#pragma unroll
    for (int s4 = 0; s4 < KSUB / 4; ++s4) {
      const int kk = lk * KSUB + s4 * 4;
      float4 af[MI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) af[mi] = ld4(as + (wm0 + mi * MS + li) * LDA_S + kk);
      float bf[NI][4];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int q = 0; q < 4; ++q) bf[ni][q] = bs[(kk + q) * LDB_S + wn0 + ni * MS + li];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) {
            float a = q == 0 ? af[mi].x : q == 1 ? af[mi].y : q == 2 ? af[mi].z : af[mi].w;
            acc[mi][ni] = Mfma<MS>::step(a, bf[ni][q], acc[mi][ni]);
          }
    }
  };

  const int nk = (kend - kbeg + BK - 1) / BK;
  if (DB) {
    load_tiles(kbeg);
    store_tiles(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tiles(kbeg + (kt + 1) * BK);
      compute(cur);
      if (kt + 1 < nk) store_tiles(cur ^ 1);
      __syncthreads();
    }
  } else {
    for (int kt = 0; kt < nk; ++kt) {
      load_tiles(kbeg + kt * BK);
      store_tiles(0);
      __syncthreads();
      compute(0);
      __syncthreads();
    }
  }

  // ---- epilogue: bias + activation, scatter to the output layout ---------
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = n0 + wn0 + ni * MS + li;
    if (col >= g.N) continue;
    size_t cofs;
    int rstride;
    if (OUT == 2) {
      cofs = (size_t)ks * g.M * g.N + col;
      rstride = g.N;
    } else if (OUT == 1) {
      int n = col / g.hw;
      int s = col - n * g.hw;
      cofs = (size_t)n * g.M * g.hw + s;
      rstride = g.hw;
    } else {
      cofs = col;
      rstride = g.ldc;
    }
    const float bcol = (OUT != 2 && Epi::bias == 2) ? g.bias[col] : 0.f;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < Mfma<MS>::kAcc; ++r) {
        const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
        if (row < g.M) {
          if (OUT == 2) {
            g.C[cofs + (size_t)row * rstride] = acc[mi][ni][r];
          } else {
            const float bv = (Epi::bias == 1) ? g.bias[row] : bcol;
            g.C[cofs + (size_t)row * rstride] = Epi::apply(acc[mi][ni][r], bv);
          }
        }
      }
  }
}

// Split-K epilogue: out = epi(sum_s ws[s][row][col], bias) with the slices
// added in slice order, written row-major (ldc) or NCHW (hw > 0). One thread
// per output element, consecutive threads on consecutive columns.
template <class Epi>
__device__ __forceinline__ void splitk_reduce_f32(const float* __restrict__ ws,
                                                  const float* __restrict__ bias,
                                                  float* __restrict__ C, int S, int M, int N,
                                                  int ldc, int hw) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  const int row = (int)(i / N);
  const int col = (int)(i - (long long)row * N);
  float v = ws[i];
  for (int s = 1; s < S; ++s) v = v + ws[(size_t)s * M * N + i];
  const float b = Epi::bias == 1 ? bias[row] : (Epi::bias == 2 ? bias[col] : 0.f);
  v = Epi::apply(v, b);
  if (hw > 0) {
    const int n = col / hw;
    const int sidx = col - n * hw;
    C[((size_t)n * M + row) * hw + sidx] = v;
  } else {
    C[(size_t)row * ldc + col] = v;
  }
}

}  // namespace mdlc
