// fp32 GEMM with a fused bias/activation epilogue on CDNA4 matrix cores.
//
//   C = epi(A[M x K] * B[K x N], bias)
//
// A is row-major with leading dimension lda. B comes from one of four
// sources (BMODE): 0 = dense row-major B[K][ldb] read as float4 (ldb % 4 == 0),
// 1 = dense row-major read as scalars, 2 = implicit im2col of an NCHW input x
// (B[k][p] = x[n][c][oh*SH-PT+kh*DH][ow*SW-PL+kw*DW], zero outside) with k
// ordered (c, kh, kw), 3 = the same gather with k ordered (kh, kw, c) — the
// weights are packed to match — for Cin % BK == 0, so every K tile is one
// filter tap. Either way a convolution needs no column buffer. The output is
// row-major C[M][ldc] (OUT = 0) or, for convolutions, NCHW: column
// p = n*hw + s goes to C[(n*M + row)*hw + s] (OUT = 1). With split-K (OUT = 2)
// the grid holds ksplit slices of K; slice s writes its raw partial sums to
// the workspace C[(s*M + row)*N + col] and splitk_reduce_f32 adds the slices
// in order and applies the epilogue.
//
// Tiling: a workgroup of WGM x WGN waves (64 lanes each) owns a BM x BN tile;
// each wave owns (BM/WGM) x (BN/WGN) as a grid of MS x MS MFMA blocks
// (MS = 32: v_mfma_f32_32x32x2_f32, MS = 16: v_mfma_f32_16x16x4_f32).
// A and B tiles of depth BK are staged through LDS, double buffered (DB: the
// next tile's global loads are in flight while the current tile feeds the
// MFMAs, one barrier per K step) or single buffered (two barriers per step).
// A double-buffered loop may be unrolled by two (UN = 2) so that the two
// LDS buffers are compile-time operands.
// LDS rows are padded by 4 floats: rows stay 16-byte aligned for
// ds_read_b128 and consecutive rows start on different banks.
//
// Staging cost is kept off the K loop: every global and LDS address a thread
// touches is computed once before the loop and advanced by k0 per tile. For
// the convolution gathers each thread owns one output pixel (a B column) and
// a contiguous run of k rows, so the pixel's bounds check and address are
// computed once per tile and each element costs one address add and one load;
// B is then kept k-contiguous in LDS ([n][k]) so a lane's B fragment is one
// ds_read_b128, like A's.
//
// K order inside a tile: the 64 lanes of an MFMA split into 64/MS groups that
// each supply one k of every instruction. Lane group g walks the contiguous
// k range [g*BK/(64/MS), (g+1)*BK/(64/MS)), so its fragments are runs of
// consecutive floats and every k of the tile is covered exactly once.
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
  const float* __restrict__ R;   // folded residual, same layout as C (Epi::residual)
  float* __restrict__ C;
  int M, N, K, lda, ldb, ldc, hw;
  int Cin, H, W, OH, OW;         // conv input / output geometry (BMODE >= 2)
  int ksplit, kchunk;            // K slices (grid = tiles * ksplit) and slice depth; with
                                 // stream-K, ksplit = the tiles done whole (see gemm_f32_mfma)
  float* __restrict__ ws;        // stream-K partial-tile workspace [2 * SKW][BM * BN]
  int ximg;                      // floats per input image (conv gathers): Cin*H*W, or the
                                 // whole image's C*H*W for one group of a grouped conv
  int cimg;                      // floats per output image (OUT == 1): M*hw, or OC*hw for
                                 // one group of a grouped conv
};

__device__ __forceinline__ float pick(const float4& v, int q) {
  return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
}

// One output tile [m0, m0+BM) x [n0, n0+BN) over K range [kbeg, kend). slot < 0:
// the epilogue for OUT (slice ks of a split-K workspace for OUT == 2); slot
// >= 0: raw sums into the stream-K workspace, tile-local rows of BN.
template <int BM, int BN, int BK, int WGM, int WGN, int MS, bool DB, bool VA, int BMODE, int OUT,
          class Epi, class Win, int UN = 1>
__device__ __forceinline__ void gemm_f32_tile(const GemmArgs& g, int m0, int n0, int kbeg, int kend,
                                              int ks, int slot) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MS, NI = WN / MS;
  constexpr int KG = 64 / MS;          // lane groups along k
  constexpr int KSUB = BK / KG;        // k per lane group per tile
  constexpr bool BT = BMODE >= 2;      // B kept k-contiguous in LDS ([n][k])
  constexpr int LDA_S = BK + 4;
  constexpr int LDB_S = BT ? BK + 4 : BN + 4;
  constexpr int B_LDS = BT ? BN * LDB_S : BK * LDB_S;
  static_assert(WM % MS == 0 && WN % MS == 0, "wave tile must be a multiple of the MFMA");
  static_assert(KSUB % 4 == 0, "BK too small for this MFMA shape");
  static_assert(BN % 4 == 0 && BK % 4 == 0, "tile dims must be multiples of 4");
  typedef typename Mfma<MS>::acc_t acc_t;

  constexpr int NBUF = DB ? 2 : 1;
  __shared__ __attribute__((aligned(16))) float As[NBUF][BM * LDA_S];
  __shared__ __attribute__((aligned(16))) float Bs[NBUF][B_LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int li = lane % MS;
  const int lk = lane / MS;


  // ---- A staging: addresses fixed per thread, advanced by k0 --------------
  constexpr int A_ELEMS = VA ? BM * BK / 4 : BM * BK;
  constexpr int A_PT = (A_ELEMS + NT - 1) / NT;
  // A is read through a buffer resource: a masked element's offset is
  // kOutside, which reads zero, so the loads need no branches
  const __amdgpu_buffer_rsrc_t rsA = buffer_over(g.A, g.M * g.lda * 4);
  int a_off[A_PT], a_k[A_PT], a_lds[A_PT];
  bool a_ok[A_PT];
#pragma unroll
  for (int i = 0; i < A_PT; ++i) {
    const int idx = tid + i * NT;
    const int cpr = VA ? BK / 4 : BK;
    const int r = idx / cpr, kc = idx % cpr;
    const int kk = VA ? kc * 4 : kc;
    a_ok[i] = idx < A_ELEMS && m0 + r < g.M;
    a_off[i] = (min(m0 + r, g.M - 1) * g.lda + kk) * 4;
    a_k[i] = kk;
    a_lds[i] = r * LDA_S + kk;
  }
  float4 ra[VA ? A_PT : 1];
  float rs[VA ? 1 : A_PT];

  // ---- B staging ------------------------------------------------------------
  // dense: quads (BMODE 0) or scalars (BMODE 1) along n, LDS [k][n]
  constexpr int BD_ELEMS = BMODE == 0 ? BK * BN / 4 : BK * BN;
  constexpr int BD_PT = BT ? 1 : (BD_ELEMS + NT - 1) / NT;
  // dense B [K][ldb] through a buffer resource (masked elements read zero)
  const __amdgpu_buffer_rsrc_t rsD = buffer_over(g.B, BT ? 0 : g.K * g.ldb * 4);
  int b_off[BD_PT], b_k[BD_PT], b_lds[BD_PT];
  bool b_ok[BD_PT];
  float4 rb[BMODE == 0 ? BD_PT : 1];
  float rbs[BMODE == 1 ? BD_PT : 1];
  if (!BT) {
#pragma unroll
    for (int i = 0; i < BD_PT; ++i) {
      const int idx = tid + i * NT;
      const int cpr = BMODE == 0 ? BN / 4 : BN;
      const int kr = idx / cpr, nc = idx % cpr;
      const int nn = BMODE == 0 ? nc * 4 : nc;
      b_ok[i] = idx < BD_ELEMS && n0 + nn < g.N;
      b_off[i] = (kr * g.ldb + min(n0 + nn, g.N - 1)) * 4;
      b_k[i] = kr;
      b_lds[i] = kr * LDB_S + nn;
    }
  }
  // conv gather: one column (output pixel) per thread, RPT contiguous k rows
  constexpr int TPC = BT ? NT / BN : 1;           // threads per column
  constexpr int RPT = BT ? BK / TPC : 1;          // rows per thread per tile
  static_assert(!BT || (NT % BN == 0 && BK % (NT / BN) == 0), "conv gather needs NT % BN == 0");
  float rg[RPT];
  int g_base = 0, g_ih = -(1 << 28), g_iw = 0, g_row = 0, g_lds = 0;
  int g_pix = 0;                                  // BMODE 3: the thread's first row, tap (0, 0)
  // BMODE 3 reads the input through a buffer resource (out-of-image taps
  // read zero from offset kOutside, the rows of a thread one channel plane
  // apart through the scalar offset) and tracks the K tile's filter tap and
  // first channel in scalars: load_tiles is called once per K tile, in order
  const __amdgpu_buffer_rsrc_t rsB =
      buffer_over(g.B, BMODE == 3 ? g.N / (g.OH * g.OW) * g.ximg * 4 : 0);
  int g_tap = 0, g_c0 = 0;
  if (BMODE == 3) {
    g_tap = kbeg / g.Cin;
    g_c0 = kbeg - g_tap * g.Cin;
  }
  if (BT) {
    const int col = tid % BN;
    g_row = (tid / BN) * RPT;
    g_lds = col * LDB_S + g_row;
    const int p = n0 + col;
    if (p < g.N) {
      const int ohw = g.OH * g.OW;
      const int n = p / ohw;
      const int s = p - n * ohw;
      const int oh = s / g.OW;
      const int ow = s - oh * g.OW;
      g_base = n * g.ximg;
      g_ih = oh * Win::SH - Win::PT;
      g_iw = ow * Win::SW - Win::PL;
      g_pix = g_base + g_row * (g.H * g.W) + g_ih * g.W + g_iw;
    }
  }

  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      const int off = a_ok[i] && k0 + a_k[i] < kend ? a_off[i] + k0 * 4 : kOutside;
      if (VA) {
        ra[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsA, off, 0, 0));
      } else {
        rs[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsA, off, 0, 0));
      }
    }
    if (BMODE == 0) {
#pragma unroll
      for (int i = 0; i < BD_PT; ++i) {
        const int off = b_ok[i] && k0 + b_k[i] < kend ? b_off[i] + k0 * g.ldb * 4 : kOutside;
        rb[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsD, off, 0, 0));
      }
    } else if (BMODE == 1) {
#pragma unroll
      for (int i = 0; i < BD_PT; ++i) {
        const int off = b_ok[i] && k0 + b_k[i] < kend ? b_off[i] + k0 * g.ldb * 4 : kOutside;
        rbs[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsD, off, 0, 0));
      }
    } else if (BMODE == 3) {
      // the whole tile is one tap: k0 = tap * Cin + c0, c0 % BK == 0
      const int HW = g.H * g.W;
      const int kh = g_tap / Win::KW;
      const int dh = kh * Win::DH, dw = (g_tap - kh * Win::KW) * Win::DW;
      const bool ok = (unsigned)(g_ih + dh) < (unsigned)g.H && (unsigned)(g_iw + dw) < (unsigned)g.W &&
                      k0 < kend;
      const int off = ok ? (g_pix + (g_c0 * HW + dh * g.W + dw)) * 4 : kOutside;
#pragma unroll
      for (int i = 0; i < RPT; ++i)
        rg[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsB, off, i * HW * 4, 0));
      g_c0 += BK;
      if (g_c0 == g.Cin) {
        g_c0 = 0;
        ++g_tap;
      }
    } else {
      // general (c, kh, kw) order: walk the thread's rows incrementally
      constexpr int KHW = Win::KH * Win::KW;
      const int HW = g.H * g.W;
      const int k = k0 + g_row;
      int c = k / KHW;
      int rr = k - c * KHW;
      int kh = rr / Win::KW;
      int kw = rr - kh * Win::KW;
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int ih = g_ih + kh * Win::DH;
        const int iw = g_iw + kw * Win::DW;
        const bool ok = k + i < kend && (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
        rg[i] = ok ? g.B[g_base + c * HW + ih * g.W + iw] : 0.f;
        if (++kw == Win::KW) {
          kw = 0;
          if (++kh == Win::KH) {
            kh = 0;
            ++c;
          }
        }
      }
    }
  };

  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      if (A_ELEMS % NT == 0 || tid + i * NT < A_ELEMS) {   // (the block has NT threads)
        if (VA) st4(&As[buf][a_lds[i]], ra[i]);
        else As[buf][a_lds[i]] = rs[i];
      }
    }
    if (BMODE == 0) {
#pragma unroll
      for (int i = 0; i < BD_PT; ++i)
        if (BD_ELEMS % NT == 0 || tid + i * NT < BD_ELEMS) st4(&Bs[buf][b_lds[i]], rb[i]);
    } else if (BMODE == 1) {
#pragma unroll
      for (int i = 0; i < BD_PT; ++i)
        if (BD_ELEMS % NT == 0 || tid + i * NT < BD_ELEMS) Bs[buf][b_lds[i]] = rbs[i];
    } else if (RPT % 4 == 0) {
#pragma unroll
      for (int i = 0; i < RPT; i += 4)
        st4(&Bs[buf][g_lds + i], make_float4(rg[i], rg[i + 1], rg[i + 2], rg[i + 3]));
    } else if (RPT % 2 == 0) {
#pragma unroll
      for (int i = 0; i < RPT; i += 2)
        *reinterpret_cast<float2*>(&Bs[buf][g_lds + i]) = make_float2(rg[i], rg[i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < RPT; ++i) Bs[buf][g_lds + i] = rg[i];
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
      float4 bf[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        if (BT) {
          bf[ni] = ld4(bs + (wn0 + ni * MS + li) * LDB_S + kk);
        } else {
          const float* bp = bs + kk * LDB_S + wn0 + ni * MS + li;
          bf[ni] = make_float4(bp[0], bp[LDB_S], bp[2 * LDB_S], bp[3 * LDB_S]);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = Mfma<MS>::step(pick(af[mi], q), pick(bf[ni], q), acc[mi][ni]);
    }
  };

  const int nk = (kend - kbeg + BK - 1) / BK;
  if (DB) {
    // The next tile's loads and LDS stores are unconditional: past kend
    // every load is masked to zero and the stores go to the idle buffer,
    // which nobody reads again. The loop body is then one basic block the
    // scheduler can interleave with the MFMAs; the waves raise their issue
    // priority while they feed the matrix cores.
    load_tiles(kbeg);
    store_tiles(0);
    __syncthreads();
    if (UN == 2) {
      // K loop unrolled by two: both buffers are named at compile time, so
      // every LDS address is a constant offset from a base fixed per thread
      int kt = 0;
      for (; kt + 2 <= nk; kt += 2) {
        load_tiles(kbeg + (kt + 1) * BK);
        __builtin_amdgcn_s_setprio(1);
        compute(0);
        __builtin_amdgcn_s_setprio(0);
        store_tiles(1);
        __syncthreads();
        load_tiles(kbeg + (kt + 2) * BK);
        __builtin_amdgcn_s_setprio(1);
        compute(1);
        __builtin_amdgcn_s_setprio(0);
        store_tiles(0);
        __syncthreads();
      }
      if (kt < nk) {                   // odd step count: the last tile is in buffer 0
        __builtin_amdgcn_s_setprio(1);
        compute(0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();               // LDS free before a following piece's prologue
      }
    } else {
      for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        load_tiles(kbeg + (kt + 1) * BK);
        __builtin_amdgcn_s_setprio(1);
        compute(cur);
        __builtin_amdgcn_s_setprio(0);
        store_tiles(cur ^ 1);
        __syncthreads();
      }
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
  if (slot >= 0) {                     // stream-K piece: raw sums, tile-local
    float* wp = g.ws + (size_t)slot * BM * BN;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int c = wn0 + ni * MS + li;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int r = 0; r < Mfma<MS>::kAcc; ++r)
          wp[(wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4)) * BN + c] = acc[mi][ni][r];
    }
    return;
  }
  // Output offsets first, then every epilogue operand (bias, residual) is
  // loaded before the first store: the stores go through a pointer the
  // compiler cannot separate from the operands, so a load placed after a
  // store would wait out a full memory round trip per output.
  constexpr int KA = Mfma<MS>::kAcc;
  size_t cofs[NI];
  bool cok[NI];
  int rstride;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = n0 + wn0 + ni * MS + li;
    cok[ni] = col < g.N;
    if (OUT == 2) {
      cofs[ni] = (size_t)ks * g.M * g.N + col;
      rstride = g.N;
    } else if (OUT == 1) {
      const int n = col / g.hw;
      cofs[ni] = (size_t)n * g.cimg + (col - n * g.hw);
      rstride = g.hw;
    } else {
      cofs[ni] = col;
      rstride = g.ldc;
    }
  }
  float brow[MI][KA], bcol[NI], rv[NI][MI][KA];
  if (OUT != 2) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < KA; ++r) {
        const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
        brow[mi][r] = (Epi::bias == 1 && row < g.M) ? g.bias[row] : 0.f;
      }
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
      bcol[ni] = (Epi::bias == 2 && cok[ni]) ? g.bias[n0 + wn0 + ni * MS + li] : 0.f;
    if (Epi::residual) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int r = 0; r < KA; ++r) {
            const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
            rv[ni][mi][r] = (cok[ni] && row < g.M) ? g.R[cofs[ni] + (size_t)row * rstride] : 0.f;
          }
    }
  }
  // every output value is formed before the first store, and a tile that
  // lies wholly inside M x N stores without per-element branches, so no
  // store waits on an operand load or on the previous store
  float outv[NI][MI][KA];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni)
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < KA; ++r) {
        if (OUT == 2) {
          outv[ni][mi][r] = acc[mi][ni][r];
        } else {
          float v = Epi::apply(acc[mi][ni][r], Epi::bias == 1 ? brow[mi][r] : bcol[ni]);
          if (Epi::residual) v = Epi::post(v, rv[ni][mi][r]);
          outv[ni][mi][r] = v;
        }
      }
  if (m0 + BM <= g.M && n0 + BN <= g.N) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int r = 0; r < KA; ++r) {
          const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
          g.C[cofs[ni] + (size_t)row * rstride] = outv[ni][mi][r];
        }
  } else {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if (!cok[ni]) continue;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int r = 0; r < KA; ++r) {
          const int row = m0 + wm0 + mi * MS + (r / 4) * 8 + lk * 4 + (r % 4);
          if (row < g.M) g.C[cofs[ni] + (size_t)row * rstride] = outv[ni][mi][r];
        }
    }
  }
}

// Entry (``bid`` >= 0 stands in for blockIdx.x, for a launch that runs this
// GEMM on part of its grid). Without stream-K (SKW == 0) workgroup b owns one
// (K slice, tile):
// logical order (slice, n-block, m-block), m fastest, so workgroups sharing a
// B slab are consecutive and land on the same XCD.
//
// With stream-K (SKW > 0 workgroups): the first ksplit tiles (a multiple of
// the CU count) are done whole, one per workgroup; the remaining R tiles'
// R * KT K steps (KT = ceil(K / BK)) are cut into SKW equal contiguous
// ranges, one per extra workgroup, so every CU gets the same amount of work
// instead of some CUs one tile more than others. R < SKW, so a range covers
// at most two (partial) tiles; piece p of workgroup j writes its raw sums
// to workspace slot 2j + p and streamk_fixup_f32 adds each tile's pieces in
// K order and applies the epilogue.
template <int BM, int BN, int BK, int WGM, int WGN, int MS, bool DB, bool VA, int BMODE, int OUT,
          class Epi, class Win, int SKW = 0, int UN = 1>
__device__ __forceinline__ void gemm_f32_mfma(const GemmArgs& g, int bid = -1) {
  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  if (SKW == 0) {
    const int t = xcd_remap(bid < 0 ? (int)blockIdx.x : bid, tiles * g.ksplit);
    const int ks = t / tiles;
    const int tt = t - ks * tiles;
    const int kbeg = ks * g.kchunk;
    gemm_f32_tile<BM, BN, BK, WGM, WGN, MS, DB, VA, BMODE, OUT, Epi, Win, UN>(
        g, (tt % tiles_m) * BM, (tt / tiles_m) * BN, kbeg, min(g.K, kbeg + g.kchunk), ks, -1);
    return;
  }
  // One call site for whole tiles and pieces, so that the tile body is
  // inlined once: a whole tile is the step range [tt*KT, (tt+1)*KT).
  const int full = g.ksplit;
  const int b = bid < 0 ? (int)blockIdx.x : bid;
  const int KT = (g.K + BK - 1) / BK;
  long long it, it1;
  int slot = -1;
  if (b < full) {
    it = (long long)xcd_remap(b, full) * KT;
    it1 = it + KT;
  } else {
    const int j = b - full;
    const long long total = (long long)(tiles - full) * KT;
    it = (long long)full * KT + j * total / SKW;
    it1 = (long long)full * KT + (j + 1) * total / SKW;
    slot = 2 * j;
  }
  while (it < it1) {
    const int tt = (int)(it / KT);
    const int k0 = (int)(it - (long long)tt * KT);
    const int k1 = (int)min((long long)KT, k0 + (it1 - it));
    gemm_f32_tile<BM, BN, BK, WGM, WGN, MS, DB, VA, BMODE, OUT, Epi, Win, UN>(
        g, (tt % tiles_m) * BM, (tt / tiles_m) * BN, k0 * BK, min(g.K, k1 * BK), 0, slot);
    it += k1 - k0;
    if (slot >= 0) ++slot;
  }
}

// Stream-K fix-up: ``BM * BN / 1024`` workgroups per partially computed tile
// (the tiles after the first ``full``), four tile elements per thread. The
// pieces of tile u came from the consecutive workgroups whose K-step ranges
// overlap [u*KT, (u+1)*KT); up to eight of them are loaded at once and added
// in that (K) order, then bias, activation and the folded residual, and the
// elements are scattered like the main epilogue (row-major or NCHW).
template <class Epi, int BM, int BN, int BK, int SKW>
__device__ __forceinline__ void streamk_fixup_f32(const float* __restrict__ ws,
                                                  const float* __restrict__ bias,
                                                  const float* __restrict__ res,
                                                  float* __restrict__ C, int M, int N, int K,
                                                  int full, int ldc, int hw) {
  constexpr int CHUNKS = BM * BN / 1024;
  static_assert(BM * BN % 1024 == 0, "fix-up tile split");
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles = tiles_m * ((N + BN - 1) / BN);
  const int KT = (K + BK - 1) / BK;
  const long long total = (long long)(tiles - full) * KT;
  const int u = blockIdx.x / CHUNKS;
  const int e = ((blockIdx.x - u * CHUNKS) * 256 + threadIdx.x) * 4;
  const int tt = full + u;
  const int m0 = (tt % tiles_m) * BM, n0 = (tt / tiles_m) * BN;
  const long long lo = (long long)u * KT, hi = lo + KT;
  // contributors j0 .. j1 - 1: the workgroups whose ranges meet [lo, hi)
  int j0 = (int)(lo * SKW / total);
  while (j0 > 0 && j0 * total / SKW > lo) --j0;
  while ((j0 + 1) * total / SKW <= lo) ++j0;
  int j1 = (int)((hi - 1) * SKW / total) + 1;
  while (j1 < SKW && j1 * total / SKW < hi) ++j1;
  while (j1 - 1 > j0 && (j1 - 1) * total / SKW >= hi) --j1;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  bool first = true;
  for (int jb = j0; jb < j1; jb += 8) {
    float4 p[8];
    bool has[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {                        // issue the batch's loads together
      const int j = jb + q;
      const long long a = j * total / SKW, z = (j + 1) * total / SKW;
      has[q] = j < j1 && z > a;                          // skip empty ranges
      const int piece = (a >= lo) ? 0 : 1;               // which of j's pieces covers tile u
      if (has[q]) p[q] = ld4(ws + (size_t)(2 * j + piece) * BM * BN + e);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (!has[q]) continue;
      if (first) {
        v = p[q];
      } else {
        v.x += p[q].x; v.y += p[q].y; v.z += p[q].z; v.w += p[q].w;
      }
      first = false;
    }
  }
  const int r = e / BN, c = e - (e / BN) * BN;
  const int row = m0 + r;
  if (row >= M) return;
  const float vs[4] = {v.x, v.y, v.z, v.w};
  // offsets and epilogue operands for all four elements before any store
  size_t o[4];
  float b[4], rs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int col = n0 + c + i;
    const bool ok = col < N;
    if (hw > 0) {
      const int n = col / hw;
      o[i] = ((size_t)n * M + row) * hw + (col - n * hw);
    } else {
      o[i] = (size_t)row * ldc + col;
    }
    b[i] = Epi::bias == 1 ? bias[row] : ((Epi::bias == 2 && ok) ? bias[col] : 0.f);
    rs[i] = (Epi::residual && ok) ? res[o[i]] : 0.f;
  }
  float xs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xs[i] = Epi::apply(vs[i], b[i]);
    if (Epi::residual) xs[i] = Epi::post(xs[i], rs[i]);
  }
  if (n0 + c + 3 < N) {
#pragma unroll
    for (int i = 0; i < 4; ++i) C[o[i]] = xs[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + c + i < N) C[o[i]] = xs[i];
  }
}

// Split-K epilogue: out = epi(sum_s ws[s][row][col], bias) with the slices
// added in slice order (then a folded residual group, if any), written
// row-major (ldc) or NCHW (HW > 0: the plane size, col = n * HW + pixel).
// One thread per output element (V = 1) or per four consecutive columns
// (V = 4: N % 4 == 0 and HW % 4 == 0, or ldc % 4 == 0 row-major, so the four
// outputs are contiguous and 16-byte aligned and every access is 128-bit);
// consecutive threads on consecutive columns. Both forms do the same float
// operations per element. The slice count S and the plane size are
// compile-time constants, so a thread issues all S slice loads before the
// first addition, and the index arithmetic is 32-bit (M * N < 2^31, checked
// by the lowering).
template <class Epi, int V, int S, int HW>
__device__ __forceinline__ void splitk_reduce_f32(const float* __restrict__ ws,
                                                  const float* __restrict__ bias,
                                                  const float* __restrict__ res,
                                                  float* __restrict__ C, int M, int N, int ldc) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= M * N / V) return;
  const int i = q * V;
  const int row = i / N;
  const int col = i - row * N;
  const size_t plane = (size_t)M * N;
  int o;
  if (HW > 0) {
    const int n = col / HW;
    o = (n * M + row) * HW + (col - n * HW);
  } else {
    o = row * ldc + col;
  }
  if (V == 4) {
    float4 w[S];
#pragma unroll
    for (int s = 0; s < S; ++s) w[s] = ld4(ws + s * plane + i);
    float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
    if (Epi::bias == 1) b = make_float4(bias[row], bias[row], bias[row], bias[row]);
    if (Epi::bias == 2) b = ld4(bias + col);
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (Epi::residual) r = ld4(res + o);
    float4 v = w[0];
#pragma unroll
    for (int s = 1; s < S; ++s) {
      v.x = v.x + w[s].x; v.y = v.y + w[s].y; v.z = v.z + w[s].z; v.w = v.w + w[s].w;
    }
    v = make_float4(Epi::apply(v.x, b.x), Epi::apply(v.y, b.y), Epi::apply(v.z, b.z),
                    Epi::apply(v.w, b.w));
    if (Epi::residual)
      v = make_float4(Epi::post(v.x, r.x), Epi::post(v.y, r.y), Epi::post(v.z, r.z),
                      Epi::post(v.w, r.w));
    st4(C + o, v);
    return;
  }
  float w[S];
#pragma unroll
  for (int s = 0; s < S; ++s) w[s] = ws[s * plane + i];
  const float b = Epi::bias == 1 ? bias[row] : (Epi::bias == 2 ? bias[col] : 0.f);
  const float r = Epi::residual ? res[o] : 0.f;
  float v = w[0];
#pragma unroll
  for (int s = 1; s < S; ++s) v = v + w[s];
  v = Epi::apply(v, b);
  if (Epi::residual) v = Epi::post(v, r);
  C[o] = v;
}

// Convolution with few input channels (a network's stem, C <= 4) as a direct
// convolution on the matrix cores. A 4-wave workgroup computes 32 * OCW output
// channels of TR x TC blocks of one image's output pixels:
//  * the input patch of a block ((TR-1)*SH + KH rows by (TC-1)*SW + KW
//    columns of every channel, zero outside the image) is staged in LDS;
//  * each wave keeps its 32 channels' weights in registers for the whole K,
//    packed as [channel block][pair i][lane]: lane l holds w[oc0 + l%32][k],
//    k = 2i + l/32 in (c, kh, kw) order (K = C*KH*KW, one zero weight pads an
//    odd K);
//  * the K loop is v_mfma_f32_32x32x2f32 with the B operand read straight
//    from the patch: lane l's pixel (l%32 of a 32-pixel block) and k sit at
//    patch[c][SH*r + kh][SW*col + kw]. The second k of a pair is one column,
//    one row step or one channel step after the first (or, for the padding,
//    the same element), so each lane keeps one base address per step kind and
//    every read is such a base plus a compile-time offset: the loop has no
//    address arithmetic, global loads or barriers.
// The workgroups step through the pixel blocks (x = block index, stride
// gridDim.x; y = channel group), so the weights are loaded once per
// workgroup, and the next block's patch is fetched into registers while the
// current one is computed (two LDS patch buffers, one barrier per block).
// LDS offset of k = (c, kh, kw) in a C x PR x PC patch
template <int KH, int KW, int PR, int PC>
__device__ __forceinline__ constexpr int smallc_off(int k) {
  return (k / (KH * KW) * PR + k % (KH * KW) / KW) * PC + k % KW;
}
// how the pair's second k = 2i + 1 follows its first: 0 next column, 1 next
// row, 2 next channel, 3 padding past K (read the first k again)
template <int C, int KH, int KW>
__device__ __forceinline__ constexpr int smallc_step(int i) {
  return 2 * i + 1 >= C * KH * KW ? 3 : (2 * i + 1) % KW ? 0 : (2 * i + 1) % (KH * KW) ? 1 : 2;
}

template <class Epi, int C, int KH, int KW, int SH, int SW, int PT, int PL, int TR, int TC, int OCW>
__device__ __forceinline__ void conv_smallc_f32(const float* __restrict__ x,
                                                const float* __restrict__ wp,
                                                const float* __restrict__ bias,
                                                const float* __restrict__ res,
                                                float* __restrict__ y, int N, int H, int W, int OC,
                                                int OH, int OW) {
  constexpr int NPAIR = (C * KH * KW + 1) / 2;
  constexpr int PR = (TR - 1) * SH + KH;
  constexpr int PC = (TC - 1) * SW + KW;
  constexpr int PSZ = C * PR * PC;
  constexpr int NPT = (PSZ + 255) / 256;        // patch elements per thread
  constexpr int PXG = 4 / OCW;                  // wave groups along the pixels
  constexpr int NB = TR * TC / 32 / PXG;        // 32-pixel blocks per wave
  static_assert(4 % OCW == 0 && TR * TC == NB * 32 * PXG && NB >= 1, "tile split");
  static_assert(PSZ * 4 <= 65536, "patch exceeds the LDS offset range");
  __shared__ float patch[2][PSZ];

  const int tiles_w = (OW + TC - 1) / TC;
  const int tiles_h = (OH + TR - 1) / TR;
  const int ntiles = N * tiles_h * tiles_w;
  int t = blockIdx.x;
  if (t >= ntiles) return;

  // The patch elements a thread loads are fixed: element e = tid + 256 q is
  // channel c, row r, column col of the patch, at (c H + r) W + col from the
  // block's corner. Loads go through a buffer resource over the block's
  // image: taps outside it read zero from offset kOutside (no branches).
  int pe_off[NPT], pe_rc[NPT];
#pragma unroll
  for (int q = 0; q < NPT; ++q) {
    const int e = threadIdx.x + q * 256;
    const int c = e / (PR * PC);
    const int rem = e - c * (PR * PC);
    const int r = rem / PC, col = rem - r * PC;
    pe_off[q] = (c * H + r) * W + col;
    pe_rc[q] = e < PSZ ? r << 16 | col : 0x7fff0000;   // past the patch: a row no image has
  }
  auto load_patch = [&](int tile, float (&pr)[NPT]) {
    const int tw = tile % tiles_w;
    const int th = (tile / tiles_w) % tiles_h;
    const int n = tile / (tiles_w * tiles_h);
    const int ih0 = th * TR * SH - PT, iw0 = tw * TC * SW - PL;
    const __amdgpu_buffer_rsrc_t rx = buffer_over(x + (size_t)n * C * H * W, (N - n) * C * H * W * 4);
    const int corner = ih0 * W + iw0;
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int ih = ih0 + (pe_rc[q] >> 16), iw = iw0 + (pe_rc[q] & 0xffff);
      const bool ok = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
      pr[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
          rx, ok ? (pe_off[q] + corner) * 4 : kOutside, 0, 0));
    }
  };
  auto store_patch = [&](int buf, const float (&pr)[NPT]) {
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int e = threadIdx.x + q * 256;
      if (PSZ % 256 == 0 || e < PSZ) patch[buf][e] = pr[q];
    }
  };

  float pr[NPT];
  load_patch(t, pr);
  store_patch(0, pr);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ocb = blockIdx.y * OCW + wave % OCW;
  const int pg = wave / OCW;
  float a[NPAIR];
  const float* wl = wp + (size_t)ocb * NPAIR * 64 + lane;
#pragma unroll
  for (int i = 0; i < NPAIR; ++i) a[i] = wl[i * 64];

  const int li = lane & 31, lk = lane >> 5;
  // per block and step kind: the lane's pixel plus, for the upper half of the
  // lanes (the pair's second k), one column / one row / one channel
  int base[NB][4];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int p = (pg * NB + j) * 32 + li;
    const int r = p / TC, col = p - (p / TC) * TC;
    const int b0 = r * SH * PC + col * SW;
    base[j][0] = b0 + lk;
    base[j][1] = b0 + lk * (PC - KW + 1);
    base[j][2] = b0 + lk * ((PR - KH + 1) * PC - KW + 1);
    base[j][3] = b0;
  }
  // the workgroup's bias values in LDS: read between output stores from
  // global memory they would each wait for the store before them
  __shared__ float bias_s[32 * OCW];
  if (threadIdx.x < 32 * OCW) {
    const int oc = blockIdx.y * OCW * 32 + threadIdx.x;
    bias_s[threadIdx.x] = (Epi::bias && oc < OC) ? bias[oc] : 0.f;
  }
  __syncthreads();

  for (int cur = 0; t < ntiles; t += gridDim.x, cur ^= 1) {
    const int tn = t + gridDim.x;
    if (tn < ntiles) load_patch(tn, pr);
    const float* pt = patch[cur];
    floatx16 acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    // B operands run DIST pairs ahead of the MFMAs (a ring of registers);
    // the scheduling barriers keep the compiler from sinking each read next
    // to its MFMA, which would expose the LDS latency on every pair
    constexpr int DIST = 4;
    float bv[DIST][NB];
#pragma unroll
    for (int i = 0; i < DIST && i < NPAIR; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        bv[i][j] = pt[base[j][smallc_step<C, KH, KW>(i)] + smallc_off<KH, KW, PR, PC>(2 * i)];
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], bv[i % DIST][j], acc[j], 0, 0, 0);
      if (i + DIST < NPAIR) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
          bv[i % DIST][j] = pt[base[j][smallc_step<C, KH, KW>(i + DIST)] +
                               smallc_off<KH, KW, PR, PC>(2 * (i + DIST))];
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // lane l holds pixel l%32 of each block and channels (r/4)*8 + (l/32)*4 + r%4;
    // residual operands are all loaded before the first store
    const int tw = t % tiles_w;
    const int th = (t / tiles_w) % tiles_h;
    const int n = t / (tiles_w * tiles_h);
    const size_t cs = (size_t)OH * OW;
    size_t o0[NB];
    bool pok[NB];
    float rv[NB][16];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int p = (pg * NB + j) * 32 + li;
      const int oh = th * TR + p / TC, ow = tw * TC + p % TC;
      pok[j] = oh < OH && ow < OW;
      o0[j] = (((size_t)n * OC + ocb * 32 + lk * 4) * OH + oh) * OW + ow;
      if (Epi::residual) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int oc = ocb * 32 + (r / 4) * 8 + lk * 4 + (r % 4);
          rv[j][r] = (pok[j] && oc < OC) ? res[o0[j] + ((r / 4) * 8 + (r % 4)) * cs] : 0.f;
        }
      }
    }
    const float* bl = bias_s + (wave % OCW) * 32 + lk * 4;
    auto outval = [&](int j, int r) {
      float v = Epi::apply(acc[j][r], bl[(r / 4) * 8 + (r % 4)]);
      if (Epi::residual) v = Epi::post(v, rv[j][r]);
      return v;
    };
    const bool full = (ocb + 1) * 32 <= OC && (th + 1) * TR <= OH && (tw + 1) * TC <= OW;
    if (full) {                                  // no per-element branches
      // one 32-bit offset a block, the channel step in the scalar offset
      const __amdgpu_buffer_rsrc_t ry = buffer_over(y, N * OC * (int)cs * 4);
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, outval(j, r)), ry,
                                                (int)o0[j] * 4, ((r / 4) * 8 + (r % 4)) * (int)cs * 4, 0);
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (!pok[j]) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int oc = ocb * 32 + (r / 4) * 8 + lk * 4 + (r % 4);
          if (oc < OC) y[o0[j] + ((r / 4) * 8 + (r % 4)) * cs] = outval(j, r);
        }
      }
    }
    if (tn < ntiles) store_patch(cur ^ 1, pr);
    __syncthreads();
  }
}

}  // namespace mdlc
