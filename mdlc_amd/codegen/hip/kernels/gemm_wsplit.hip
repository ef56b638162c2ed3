// Small-output fp32 GEMM, one launch, K split across the waves of a
// workgroup:
//
//   C = epi(A[M x K] * B[K x N], bias)
//
// For GEMMs whose M x N gives few 64x64 tiles but whose K is deep (batch-1
// convolutions as GEMMs, a fully connected layer at small batch), a tile per
// workgroup leaves most CUs idle and a split-K grid needs a second launch to
// add the slices. Here a workgroup of WK waves owns one (16*MI) x (16*NI)
// output tile; wave w computes the partial sums of the whole tile over its
// own contiguous 1/WK of the K steps, straight from global memory into
// registers (no LDS staging: every operand element is used by exactly one
// wave), with the next steps' loads in flight while the current ones feed
// v_mfma_f32_16x16x4f32. The WK partial tiles then meet in LDS and are added
// in wave order (a fixed order: results do not depend on timing), the
// epilogue is applied and the tile is stored.
//
// Operand fragments: in each 16-deep K step, lane l = 16*g + i holds
// A[m0 + i][k0 + 4g + q] and B[k0 + 4g + q][n0 + i] for q = 0..3, and MFMA q
// takes element q, so lane group g supplies k = k0 + 4g + q: every k of the
// step exactly once, for A and B alike. A's four values are one 16-byte load
// when VA (K % 16 == 0 and lda % 4 == 0). B is either row-major [K][ldb]
// (four loads, each a 64-byte run of a B row across the 16 lanes of a
// group) or, BKN, stored K-contiguous per column as [N][ldb] (constant
// weights packed that way), when its four values are one 16-byte load too.
// Every vector memory instruction costs the CU's address pipeline the same
// whatever its width, so the 16-byte forms matter more than the bytes.
namespace mdlc {

// SPLIT: the K range is also cut over gridDim.y workgroups (kchunk values
// of K each, a multiple of 16); workgroup y writes its raw partial tile to
// slice y of the split-K workspace, C[(y * M + row) * ldc + col], for
// splitk_reduce_f32 to add in slice order and finish.
//
// CONV: B is the implicit-GEMM view of an NCHW convolution input (Win the
// window), K ordered (kh, kw, c) with Cin % 16 == 0, so the 16 k of a step
// share one tap and a lane's four are consecutive channels: per step and
// column block one bounds check and one base offset (the tap's pixel), the
// channels one plane (H*W floats) apart. A holds the weights as [OC][K] in
// that order; column p = (image, pixel) and the output goes to NCHW, with
// the folded residual (Epi::residual, read at the output's own position).
template <int MI, int NI, int WK, int UN, bool VA, bool BKN, class Epi, bool SPLIT = false,
          class Win = NoWin, bool CONV = false>
__device__ __forceinline__ void gemm_f32_wsplit(const float* __restrict__ A,
                                                const float* __restrict__ B,
                                                const float* __restrict__ bias,
                                                float* __restrict__ C, int M, int N, int K,
                                                int lda, int ldb, int ldc, int kchunk,
                                                const float* __restrict__ res = nullptr,
                                                int Cin = 0, int H = 0, int W = 0, int OH = 0,
                                                int OW = 0) {
  constexpr int TM = 16 * MI, TN = 16 * NI;
  __shared__ __attribute__((aligned(16))) floatx4 red[WK][MI][NI][64];

  // Logical tile t (m fastest) from an XCD-aware remap: each XCD runs a
  // contiguous range of tiles, so its L2 holds a few column blocks of B and
  // a range of A's rows instead of fetching all of both.
  const int tiles_m = (M + TM - 1) / TM;
  const int t = xcd_remap(blockIdx.x, tiles_m * ((N + TN - 1) / TN));
  const int m0 = (t % tiles_m) * TM;
  const int n0 = (t / tiles_m) * TN;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar K range
  const int li = lane & 15;
  const int lg = lane >> 4;

  // this wave's contiguous share of the workgroup's 16-deep K steps
  const int steps = (K + 15) / 16;
  const int sb = SPLIT ? (int)blockIdx.y * (kchunk / 16) : 0;
  const int sn = SPLIT ? min(steps, sb + kchunk / 16) - sb : steps;
  const int s0 = sb + (int)((long long)sn * w / WK);
  const int s1 = sb + (int)((long long)sn * (w + 1) / WK);

  // Loads go through buffer resources: a row past M or a column past N has
  // the out-of-range offset kOutside, k past K falls outside the resource's
  // range, and a step past this wave's share gets an empty range, so every
  // masked element reads zero and no load sits behind a branch. (Branches
  // around loads leave the number of loads in flight unknown to the
  // compiler, which then waits for all of them at each step.) The step's k0
  // moves the resource base (scalar work); the per-lane offsets stay fixed.
  const int a_bytes = M * lda * 4;
  const int b_bytes = CONV ? (N / (OH * OW)) * Cin * H * W * 4 : (BKN ? N * ldb * 4 : K * ldb * 4);
  const int HW = H * W;
  // CONV: per column block the lane's image offset and window corner; a
  // column past N gets image 0 and a corner row one above the highest any
  // tap reaches (ih <= -DH - 1 for every kh), so every tap fails the bounds
  // check and the address arithmetic stays small
  int cimg[CONV ? NI : 1], cih[CONV ? NI : 1], ciw[CONV ? NI : 1];
  if (CONV) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int p = n0 + ni * 16 + li;
      const int ohw = OH * OW;
      const int img = p / ohw;
      const int pix = p - img * ohw;
      const int oh = pix / OW;
      cimg[ni] = p < N ? (img * Cin + 4 * lg) * HW : 0;
      cih[ni] = p < N ? oh * Win::SH - Win::PT : -(Win::KH * Win::DH) - 1;
      ciw[ni] = (pix - oh * OW) * Win::SW - Win::PL;
    }
  }
  int aoff[MI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int row = m0 + mi * 16 + li;
    aoff[mi] = row < M ? (row * lda + 4 * lg) * 4 : kOutside;
  }
  int boff[NI][BKN ? 1 : 4];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = n0 + ni * 16 + li;
    if (BKN) {
      boff[ni][0] = col < N ? (col * ldb + 4 * lg) * 4 : kOutside;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) boff[ni][q] = col < N ? ((4 * lg + q) * ldb + col) * 4 : kOutside;
    }
  }

  floatx4 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};

  // UN steps per stage, two stages of registers: the loads of stage j + 1
  // are issued before the MFMAs of stage j
  float av[2][UN][MI][4];
  float bv[2][UN][NI][4];
  auto load = [&](int buf, int s) {
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int k0 = (s + u) * 16;
      const bool live = s + u < s1;
      const __amdgpu_buffer_rsrc_t rA = buffer_over(A + k0, live ? max(a_bytes - k0 * 4, 0) : 0);
      const __amdgpu_buffer_rsrc_t rB =
          CONV ? buffer_over(B, live ? b_bytes : 0)
               : BKN ? buffer_over(B + k0, live ? max(b_bytes - k0 * 4, 0) : 0)
                     : buffer_over(B + (size_t)k0 * ldb, live ? max(b_bytes - k0 * ldb * 4, 0) : 0);
      // k past K inside a row (only without VA): its element's offset is
      // pushed out of range per lane
      const int kl = k0 + 4 * lg;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        if (VA) {
          const floatx4 v = __builtin_bit_cast(
              floatx4, __builtin_amdgcn_raw_buffer_load_b128(rA, aoff[mi], 0, 0));
#pragma unroll
          for (int q = 0; q < 4; ++q) av[buf][u][mi][q] = v[q];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            av[buf][u][mi][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                rA, kl + q < K ? aoff[mi] + 4 * q : kOutside, 0, 0));
        }
      }
      // CONV: the step's tap and first channel (wave-uniform, scalar)
      const int tap = CONV ? k0 / Cin : 0;
      const int kh = tap / Win::KW, kw = tap - (tap / Win::KW) * Win::KW;
      const int cofs = (k0 - tap * Cin) * HW;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        if (CONV) {
          const int ih = cih[ni] + kh * Win::DH, iw = ciw[ni] + kw * Win::DW;
          const bool ok = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
          const int base = (cimg[ni] + cofs + ih * W + iw) * 4;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bv[buf][u][ni][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                rB, ok ? base + q * HW * 4 : kOutside, 0, 0));
        } else if (BKN && VA) {
          const floatx4 v = __builtin_bit_cast(
              floatx4, __builtin_amdgcn_raw_buffer_load_b128(rB, boff[ni][0], 0, 0));
#pragma unroll
          for (int q = 0; q < 4; ++q) bv[buf][u][ni][q] = v[q];
        } else if (BKN) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bv[buf][u][ni][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                rB, kl + q < K ? boff[ni][0] + 4 * q : kOutside, 0, 0));
        } else {
          // rows k >= K lie past the resource's range
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bv[buf][u][ni][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                rB, boff[ni][q], 0, 0));
        }
      }
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int u = 0; u < UN; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[buf][u][mi][q], bv[buf][u][ni][q],
                                                               acc[mi][ni], 0, 0, 0);
  };

  if (s0 < s1) {
    load(0, s0);
    int s = s0;
    // two stages per trip so both register sets are compile-time names
    for (; s + 2 * UN < s1; s += 2 * UN) {
      load(1, s + UN);
      compute(0);
      load(0, s + 2 * UN);
      compute(1);
    }
    if (s + UN < s1) {
      load(1, s + UN);
      compute(0);
      compute(1);
    } else {
      compute(0);
    }
  }

  // partial tiles meet in LDS; every thread then owns some tile elements
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) red[w][mi][ni][lane] = acc[mi][ni];
  __syncthreads();
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0][0]);
  for (int e = threadIdx.x; e < TM * TN; e += WK * 64) {
    const int row = e / TN, col = e - (e / TN) * TN;
    const int mi = row / 16, ni = col / 16;
    // 16x16x4 output layout: lane 16*(r/4) + c holds rows 4*(r/4) .. +3 of column c
    const int rr = row % 16, cc = col % 16;
    const int slot = ((mi * NI + ni) * 64 + (rr / 4) * 16 + cc) * 4 + (rr % 4);
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < WK; ++k) v += redf[k * MI * NI * 256 + slot];
    const int gr = m0 + row, gc = n0 + col;
    if (gr < M && gc < N) {
      if (SPLIT) {
        C[((size_t)blockIdx.y * M + gr) * ldc + gc] = v;
      } else if (CONV) {
        const int ohw = OH * OW;
        const int img = gc / ohw;
        const size_t o = ((size_t)img * M + gr) * ohw + (gc - img * ohw);
        const float b = Epi::bias == 1 ? bias[gr] : 0.f;
        float r = Epi::apply(v, b);
        if (Epi::residual) r = Epi::post(r, res[o]);
        C[o] = r;
      } else {
        const float b = Epi::bias == 2 ? bias[gc] : (Epi::bias == 1 ? bias[gr] : 0.f);
        C[(size_t)gr * ldc + gc] = Epi::apply(v, b);
      }
    }
  }
}

}  // namespace mdlc
