// 3x3 stride-1 convolution by Winograd F(2x2, 3x3), transforms fused into one
// matrix-core kernel (fp32 throughout).
//
// Each 2x2 block of output pixels (a "tile") is computed from the 4x4 input
// window around it:  Y = A^T [ sum_c (G g_c G^T) (.) (B^T d_c B) ] A,  where
// d_c is channel c's window (zeros outside the image), g_c the 3x3 filter of
// channel c and (.) the element-wise product of 4x4 matrices:
//
//   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//   G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//   A^T = [1 1 1 0; 0 1 -1 -1]
//
// For each of the 16 positions xi = 4a + b of the 4x4 matrices the channel
// sum is a GEMM, M_xi[oc][tile] = sum_c U_xi[oc][c] V_xi[c][tile], with 16/36
// of the direct convolution's multiply-adds.
//
// A workgroup of eight waves (two per SIMD) owns 64 output channels x 64
// tiles. Wave w = 4 h + tg owns the eight positions of rows a = 2h, 2h + 1
// of all 64 output channels x the 16 tiles 16 tg .. 16 tg + 15, on
// v_mfma_f32_16x16x4f32 (8 positions x 4 channel blocks of 16 = 32
// accumulators of 4, 128 registers a lane); waves tg and tg + 4 (the two
// halves of the same tiles) share a SIMD. In that instruction lane
// l = 16 lk + li supplies B[k = lk][li]; k-step j (0, 1) of an 8-channel
// chunk takes channel lk + 4 j, so a lane's B operands are V values of ONE
// window, tile 16 tg + li and channel lk + 4 j: the lane transforms that
// window itself, only the two rows of V its half needs (16 additions), and
// feeds the values straight to the matrix core. Its A operand is
// U[xi][oc = 16 blk + li][lk + 4 j]; the filters are transformed on the
// host (G g G^T, rounded once from float64) and packed per (channel block,
// chunk) as a 32 KB image in exactly the order the lanes read it,
// [h][blk][j][lane][8 positions], each lane's 8 values two 16-byte quartets
// in slots swizzled by lane so that any 8 or 16 consecutive lanes' reads hit
// distinct banks: one chunk's A operands are sixteen 16-byte LDS reads a
// lane, and the copy of the image into LDS is a linear 16-byte-per-thread
// stream. The output transform is linear in M, so each half forms its own
// partial Y_h = A^T M_h A in registers; after the channel loop the halves
// exchange partials through LDS (each finishes two of the four channel
// blocks, adding Y_0 + Y_1 in that order) and store the 2x2 pixels.
//
// The input reaches the windows through an LDS patch per channel of the
// rows the workgroup's 64 tiles read, filled with coalesced loads (wave w
// loads channel w of a chunk), zeros at the padding, so windows are read
// without bounds checks. The patch of one channel takes WINO_PSTR floats,
// 32 banks apart from the next channel's, so the four channels a window
// read touches at once hit distinct banks.
//
// Per chunk c, two phases around one barrier:
//   J0: transform window (c, j = 1), run the 32 j = 0 MFMAs;
//   barrier;
//   J1: transform window (c+1, j = 0), run the 32 j = 1 MFMAs.
// Each phase computes the V values the next phase needs into the registers
// the current phase does not read, so V takes 16 registers. The staging
// (a wave's channel of the patch and its pieces of the filter image, stored
// from registers into LDS, then the global loads of a later chunk) runs in
// J0 on waves 0-3 and in J1 on waves 4-7, their SIMD partners. Three
// filter stages and two patch buffers make the one barrier enough: a stage
// or buffer is rewritten only after the barrier that follows its last reads.
//
// With SPLIT the channel chunks are divided among gridDim.y slices and each
// writes its raw Y to the split-K workspace ws[(slice * OC + oc) * P + pixel],
// P = N*OH*OW, for splitk_reduce_f32 to add in slice order and finish.
namespace mdlc {

typedef unsigned v2u32_t __attribute__((ext_vector_type(2)));

struct WinoArgs {
  const float* __restrict__ U;     // packed filters, [OCP/64][CP/8][16][64][8]
  const float* __restrict__ x;     // [N][C][H][W]
  const float* __restrict__ bias;  // [OC] (Epi::bias == 1)
  const float* __restrict__ R;     // folded residual, NCHW like y (Epi::residual)
  float* __restrict__ y;           // [N][OC][OH][OW], or the split workspace
  int N, C, H, W, OC, OH, OW;
  int TH, TW;                      // tiles per image: ceil(OH / 2), ceil(OW / 2)
  int CP, OCP;                     // C and OC padded (U's layout)
  int PT, PL;                      // top / left padding
  int nchunk;                      // 8-channel chunks per slice
};

constexpr int WINO_NT = 512;
constexpr int WINO_USTAGE = 16 * 64 * 8;              // filter image floats per chunk (32 KB)
constexpr int WINO_PMAX = 704;                        // input patch floats per channel
constexpr int WINO_PSTR = WINO_PMAX + 32;             // patch stride per channel (banks apart)
constexpr int WINO_PBUF = 8 * WINO_PSTR;              // one chunk's patch

template <int V> struct WinoHalf { static constexpr int value = V; };

// n / d for 0 <= n < 2^21 and 0 < d < 2^21, given inv = rcp(d): the float
// quotient is within one of the true one, and one correction each way
// makes it exact (a 32-bit integer division costs some twenty VALU
// instructions, several at quarter rate).
__device__ __forceinline__ int wino_div(int n, int d, float inv) {
  int q = (int)((float)n * inv);
  const int r = n - __mul24(q, d);
  return q + (r >= d) - (r < 0);
}

// PL: patch loads per lane (one channel per wave), ceil(largest patch / 64)
// <= WINO_PMAX / 64.
// FULL: OH and OW are even, so every tile has its four pixels.
template <bool SPLIT, int PL, bool FULL, class Epi>
__device__ __forceinline__ void conv_wino_f32(const WinoArgs& g) {
  static_assert(PL * 64 <= WINO_PMAX, "patch larger than its LDS");
  __shared__ __attribute__((aligned(16))) float ust[3 * WINO_USTAGE];
  __shared__ __attribute__((aligned(16))) float pbuf[2 * WINO_PBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = wave >> 2;                          // position rows 2h, 2h + 1
  const int tg = wave & 3;
  const int li = lane & 15;
  const int lk = lane >> 4;

  const int P = g.N * g.TH * g.TW;                  // < 2^21 (checked by the host)
  const int tiles_n = (P + 63) >> 6;
  // Work item w = (ocb * slices + slice) * tiles_n + tile block, spread so
  // that each XCD (workgroups are dispatched to XCD linear id % 8) runs a
  // contiguous range of w: the workgroups that stream one channel block's
  // filter images share an XCD and its L2 instead of every XCD fetching
  // every block's filters.
  const int slices = SPLIT ? (int)gridDim.y : 1;
  const int w = xcd_remap(blockIdx.x + (int)gridDim.x * (int)blockIdx.y, (int)gridDim.x * slices);
  const int os = wino_div(w, tiles_n, __builtin_amdgcn_rcpf((float)tiles_n));
  const int t0 = (w - os * tiles_n) * 64;
  const int ocb = SPLIT ? os / slices : os;
  const int slice = SPLIT ? os - ocb * slices : 0;
  const int chunk0 = slice * g.nchunk;
  const int HW = g.H * g.W;
  const float* ublk = g.U + (size_t)ocb * (g.CP / 8) * WINO_USTAGE;

  // ---- input patch: the rows the workgroup's windows read -----------------
  // For each image its 64 tiles touch (segment s = image nfirst + s), the
  // rows its tiles' windows read (image coordinates, padding rows included),
  // each WP = 2 TW + 2 columns wide starting at column -PL; positions outside
  // the image hold zero. The segments are stacked: segment 0 holds rows
  // rlo0 .. (its last), the others rows -PT .. (their last), whole images
  // SR = 2 TH + 2 rows.
  const int TT = g.TH * g.TW;
  const int WP = 2 * g.TW + 2;
  const int SR = 2 * g.TH + 2;
  const float iTT = __builtin_amdgcn_rcpf((float)TT), iTW = __builtin_amdgcn_rcpf((float)g.TW);
  const float iWP = __builtin_amdgcn_rcpf((float)WP), iSR = __builtin_amdgcn_rcpf((float)SR);
  const int nfirst = wino_div(t0, TT, iTT);
  const int plast = min(t0 + 63, P - 1);
  const int nlast = wino_div(plast, TT, iTT);
  const int rlo0 = 2 * wino_div(t0 - nfirst * TT, g.TW, iTW) - g.PT;
  const int rhil = 2 * wino_div(plast - nlast * TT, g.TW, iTW) + 3 - g.PT;
  const int rows0 = (nlast == nfirst ? rhil : 2 * g.TH + 1 - g.PT) - rlo0 + 1;
  const int seg = SR * WP;
  const int PS = rows0 * WP + (nlast > nfirst ? (nlast - nfirst - 1) * seg + (rhil + g.PT + 1) * WP : 0);

  // the lane's tile: image n, tile row ty, tile column tx
  const int p = t0 + 16 * tg + li;
  const int pc = p < P ? p : t0;                    // tiles past the batch: any window, never stored
  const int n = wino_div(pc, TT, iTT);
  const int ty = wino_div(pc - n * TT, g.TW, iTW);
  const int tx = pc - n * TT - ty * g.TW;
  const int wbase = (n == nfirst ? (2 * ty - g.PT - rlo0) * WP
                                 : rows0 * WP + (n - nfirst - 1) * seg + 2 * ty * WP) + 2 * tx;
  // the lane's patch elements lane + 64 i: byte offset of the value from
  // the channel's plane in image 0, or kOutside (a zero) outside the image
  // or past the patch
  int poff[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    // element e is row q, column e - q WP of the stacked patch (segments
    // hold whole rows)
    const int e = i * 64 + lane;
    const int q = wino_div(e, WP, iWP);
    const int col = e - q * WP;
    int sg = 0, row = rlo0 + q;
    if (q >= rows0) {
      const int R = q - rows0;
      const int s1 = wino_div(R, SR, iSR);
      sg = 1 + s1;
      row = R - s1 * SR - g.PT;
    }
    const int ix = col - g.PL;
    const bool ok = e < PS && (unsigned)row < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
    poff[i] = ok ? ((nfirst + sg) * g.C * HW + row * g.W + ix) * 4 : kOutside;
  }
  const int xbytes = g.N * g.C * HW * 4;

  // staging registers: channel `wave` of a chunk's patch, four 16-byte
  // pieces of its filter image. The loads go through buffer resources: the
  // patch's zeros (padding, and every element of a channel past the last)
  // come back from out-of-range offsets, and the chunk's position is in the
  // resource, so the loop computes no addresses.
  float pv[PL];
  float4 ur[4];
  auto load_x = [&](int chunk) {
    const int c = chunk * 8 + wave;
    const __amdgpu_buffer_rsrc_t r = buffer_over(g.x + (size_t)min(c, g.C - 1) * HW,
                                                 c < g.C ? xbytes - c * HW * 4 : 0);
#pragma unroll
    for (int i = 0; i < PL; ++i)
      pv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, poff[i], 0, 0));
  };
  auto store_x = [&](int buf) {
    float* pw = pbuf + buf * WINO_PBUF + wave * WINO_PSTR;
#pragma unroll
    for (int i = 0; i < PL; ++i) pw[i * 64 + lane] = pv[i];
  };
  auto load_u = [&](int chunk) {
    const __amdgpu_buffer_rsrc_t r = buffer_over(ublk + (size_t)chunk * WINO_USTAGE, WINO_USTAGE * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ur[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (tid + i * WINO_NT) * 16, 0, 0));
  };
  auto store_u = [&](int stage) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st4(ust + stage * WINO_USTAGE + (tid + i * WINO_NT) * 4, ur[i]);
  };
  // Everything from here on depends on the half: it is compiled once per
  // half (H), so that the transform's formulas and the staging phase are
  // fixed in each copy instead of selected per instruction.
  auto run = [&](auto HC) {
    constexpr int H = decltype(HC)::value;
    // rows 2h, 2h + 1 of V = B^T d B of the lane's window for channel lk + 4 j
    // of a chunk (zero past the last channel: its patch is zeros); they need
    // window rows h .. h + 2
    auto window = [&](float (&v)[8], int buf, int j) {
      const float* pj = pbuf + buf * WINO_PBUF + (lk + 4 * j) * WINO_PSTR + wbase + H * WP;
      float d[12];
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
          const float2 q = *reinterpret_cast<const float2*>(pj + a * WP + b);
          d[4 * a + b] = q.x;
          d[4 * a + b + 1] = q.y;
        }
      float t[8];                                     // rows 2h, 2h + 1 of B^T d
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (H == 0) {
          t[b] = d[b] - d[8 + b];                     // d0 - d2
          t[4 + b] = d[4 + b] + d[8 + b];             // d1 + d2
        } else {
          t[b] = d[4 + b] - d[b];                     // d2 - d1
          t[4 + b] = d[b] - d[8 + b];                 // d1 - d3
        }
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        v[4 * a + 0] = t[4 * a] - t[4 * a + 2];
        v[4 * a + 1] = t[4 * a + 1] + t[4 * a + 2];
        v[4 * a + 2] = t[4 * a + 2] - t[4 * a + 1];
        v[4 * a + 3] = t[4 * a + 1] - t[4 * a + 3];
      }
    };

    // A operands: the lane's 8 positions of (blk, j) are two 16-byte
    // quartets of the filter image, quartet q in slot q ^ sw
    const int sw = ((lane >> 2) ^ (lane >> 3)) & 1;
    int qoff[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) qoff[q] = H * 8 * 512 + lane * 8 + ((q ^ sw) << 2);
    floatx4 acc[8][4];
#pragma unroll
    for (int x = 0; x < 8; ++x)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[x][blk][r] = 0.f;
    auto mfma_half = [&](const float* st, int j, const float (&v)[8]) {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        float4 a[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) a[q] = ld4(st + (blk * 2 + j) * 512 + qoff[q]);
#pragma unroll
        for (int x = 0; x < 8; ++x)
          acc[x][blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(pick(a[x >> 2], x & 3), v[x],
                                                              acc[x][blk], 0, 0, 0);
      }
    };

    // Waves 0-3 stage in J0, waves 4-7 (their SIMD partners) in J1, so that
    // on every SIMD one wave's stores and loads overlap the other's MFMAs. A
    // wave stores its own channel of the patch and its own pieces of the
    // filter image, so the two groups' stores of one chunk never overlap;
    // waves 4-7 run one chunk further ahead (they store chunk c+2 in J1 of
    // chunk c, into the patch buffer and filter stage the barrier before J1
    // has freed).
    constexpr bool early = H == 0;
    auto stage = [&](int buf, int ustage, int next) {
      __builtin_amdgcn_sched_barrier(0);
      store_x(buf);
      store_u(ustage);
      __builtin_amdgcn_sched_barrier(0);
      load_x(chunk0 + min(next, g.nchunk - 1));
      load_u(chunk0 + min(next, g.nchunk - 1));
      __builtin_amdgcn_sched_barrier(0);
    };
    load_x(chunk0);
    load_u(chunk0);
    store_x(0);
    store_u(0);
    load_x(chunk0 + min(1, g.nchunk - 1));
    load_u(chunk0 + min(1, g.nchunk - 1));
    if (!early) stage(1, 1, 2);
    __syncthreads();
    float v0[8], v1[8];
    window(v0, 0, 0);
    int us = 0;                                       // filter stage of chunk ch
    for (int ch = 0; ch < g.nchunk; ++ch) {
      const int pb = ch & 1;                          // patch buffer of chunk ch
      const int u1 = us == 2 ? 0 : us + 1;            // filter stage of chunk ch + 1
      const int u2 = u1 == 2 ? 0 : u1 + 1;            // and of chunk ch + 2
      if (early) stage(pb ^ 1, u1, ch + 2);           // chunk ch + 1 in, ch + 2 loaded
      window(v1, pb, 1);
      mfma_half(ust + us * WINO_USTAGE, 0, v0);
      __syncthreads();
      if (!early) stage(pb, u2, ch + 3);              // chunk ch + 2 in, ch + 3 loaded
      window(v0, pb ^ 1, 0);                          // past the last chunk: unused
      mfma_half(ust + us * WINO_USTAGE, 1, v1);
      us = u1;
    }

    // ---- output transform: partial Y of each half, summed through LDS --------
    // acc[4a' + b][blk][r] holds M at row a = 2h + a', column b, for
    // oc = 16 blk + 4 lk + r and the lane's tile (the 16x16x4 accumulator
    // layout). s = A^T M restricted to the half's two rows, Y_h = s A. Half h
    // finishes channel blocks 2h, 2h + 1: it hands its partials of the other
    // half's blocks over through LDS (the stages are no longer read).
    float y[4][4][4];                                 // [blk][r][pixel]
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s0[4], s1[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float m0 = acc[b][blk][r], m1 = acc[4 + b][blk][r];
          if (H == 0) {                               // rows 0, 1: A^T columns (1, 0), (1, 1)
            s0[b] = m0 + m1;
            s1[b] = m1;
          } else {                                    // rows 2, 3: (1, -1), (0, -1)
            s0[b] = m0;
            s1[b] = -m0 - m1;
          }
        }
        y[blk][r][0] = s0[0] + s0[1] + s0[2];
        y[blk][r][1] = s0[1] - s0[2] - s0[3];
        y[blk][r][2] = s1[0] + s1[1] + s1[2];
        y[blk][r][3] = s1[1] - s1[2] - s1[3];
      }
    // Epilogue operands (bias, folded residual) are loaded here, before any
    // store and ahead of the exchange: a load issued after a store waits for
    // that store too (one memory counter), which would serialize the stores.
    // Buffer resources give zeros for channels past OC and pixels past the
    // image, so the loads need no branches.
    const int OHW = g.OH * g.OW;
    const int oy = 2 * ty, ox = 2 * tx;
    const bool yok = oy + 1 < g.OH, xok = ox + 1 < g.OW;
    const int oc0 = ocb * 64 + 32 * H + 4 * lk;
    float bv[2][4] = {};
    float rv[2][4][4] = {};
    if (!SPLIT) {
      if (Epi::bias == 1) {
        const __amdgpu_buffer_rsrc_t rbias = buffer_over(g.bias, g.OC * 4);
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            bv[bb][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                rbias, (oc0 + 16 * bb + r) * 4, 0, 0));
      }
      if (Epi::residual) {
        const __amdgpu_buffer_rsrc_t rres = buffer_over(g.R, g.N * g.OC * OHW * 4);
        const int base = ((n * g.OC + oc0) * OHW + oy * g.OW + ox) * 4;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int o = oc0 + 16 * bb + r < g.OC ? base + (16 * bb + r) * OHW * 4 : kOutside;
            if (FULL) {
              const float2 r0 = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rres, o, 0, 0));
              const float2 r1 = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                  rres, o == kOutside ? kOutside : o + g.OW * 4, 0, 0));
              rv[bb][r][0] = r0.x; rv[bb][r][1] = r0.y; rv[bb][r][2] = r1.x; rv[bb][r][3] = r1.y;
            } else {
              const bool in = o != kOutside;
              rv[bb][r][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rres, o, 0, 0));
              rv[bb][r][1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                  rres, in && xok ? o + 4 : kOutside, 0, 0));
              rv[bb][r][2] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                  rres, in && yok ? o + g.OW * 4 : kOutside, 0, 0));
              rv[bb][r][3] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                  rres, in && xok && yok ? o + g.OW * 4 + 4 : kOutside, 0, 0));
            }
          }
      }
    }
    __syncthreads();
    float* xw = ust + H * 8192;                       // this half's partials for the other half
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int blk = 2 * (1 - H) + bb;
        st4(xw + (((tg * 2 + bb) * 4 + r) * 64 + lane) * 4,
            make_float4(y[blk][r][0], y[blk][r][1], y[blk][r][2], y[blk][r][3]));
      }
    __syncthreads();
    const float* xr = ust + (1 - H) * 8192;

    // Output channel oc0 + 16 bb + r of the lane's tile, channels a fixed
    // stride apart. The stores go through a buffer resource over the output
    // (or this slice of the workspace): a lane past the last tile, a channel
    // past OC or a pixel past the image gets the out-of-range offset and its
    // store is dropped, so the stores need no branches either. With FULL the
    // pixel pairs are 8-byte aligned.
    const int ocs = SPLIT ? g.N * OHW : OHW;          // stride between channels
    const int obase = (SPLIT ? oc0 * ocs + n * OHW : (n * g.OC + oc0) * OHW) + oy * g.OW + ox;
    const __amdgpu_buffer_rsrc_t rout =
        buffer_over(g.y + (SPLIT ? (size_t)slice * g.OC * g.N * OHW : 0), g.OC * g.N * OHW * 4);
    const bool live = p < P;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4 other = ld4(xr + (((tg * 2 + bb) * 4 + r) * 64 + lane) * 4);
        const float* mine = y[2 * H + bb][r];
        float out[4];                                 // Y_0 + Y_1
        if (H == 0) {
          out[0] = mine[0] + other.x; out[1] = mine[1] + other.y;
          out[2] = mine[2] + other.z; out[3] = mine[3] + other.w;
        } else {
          out[0] = other.x + mine[0]; out[1] = other.y + mine[1];
          out[2] = other.z + mine[2]; out[3] = other.w + mine[3];
        }
        if (!SPLIT) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            out[e] = Epi::apply(out[e], bv[bb][r]);
            if (Epi::residual) out[e] = Epi::post(out[e], rv[bb][r][e]);
          }
        }
        const bool ok = live && oc0 + 16 * bb + r < g.OC;
        const int o = (obase + (16 * bb + r) * ocs) * 4;
        if (FULL) {
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, make_float2(out[0], out[1])),
                                                rout, ok ? o : kOutside, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, make_float2(out[2], out[3])),
                                                rout, ok ? o + g.OW * 4 : kOutside, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out[0]), rout,
                                                ok ? o : kOutside, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out[1]), rout,
                                                ok && xok ? o + 4 : kOutside, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out[2]), rout,
                                                ok && yok ? o + g.OW * 4 : kOutside, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out[3]), rout,
                                                ok && xok && yok ? o + g.OW * 4 + 4 : kOutside, 0, 0);
        }
      }
  };
  if (h == 0) {
    run(WinoHalf<0>());
  } else {
    run(WinoHalf<1>());
  }
}

}  // namespace mdlc
