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
// tiles. Wave w = 4h + 2wm + wn owns the 32 x 32 block (wm, wn) of the eight
// positions of rows a = 2h, 2h + 1 (128 accumulator registers a lane). The
// output transform is linear in M, so each half h forms its own partial
// Y_h = A^T M_h A from its two rows; after the channel loop the halves meet
// in LDS and are added (Y_0 + Y_1, a fixed order) by the whole workgroup,
// which then applies bias, activation and the folded residual and stores
// the 2x2 pixels, consecutive threads on consecutive tiles.
//
// The channel sum runs in chunks of 8 channels through two LDS stages:
//
//   U stage  [16 xi][64 oc][8 k]: the filters, transformed on the host
//            (G g G^T, rounded once from float64) and packed per (channel
//            block, chunk) as exactly this 32 KB image, the two 16-byte
//            halves of row r swapped when bit 2 of r differs from bit 3, so
//            that any 8 (or 16) consecutive rows' 16-byte fragment reads hit
//            distinct banks of a 32 (or 64) bank LDS: the copy is a linear
//            16-byte-per-thread stream.
//   V stage  [16 xi][8 k][VLD]: the transformed input, tile-contiguous, so
//            that the transform's stores (64 consecutive tiles of one
//            channel per wave instruction) are conflict free.
//
// Chunk c's MFMAs read stage c % 2 while the waves also fill the other
// stage with chunk c+1 (loaded into registers one chunk earlier) and issue
// the global loads of chunk c+2: half 0 the input windows (two (tile,
// channel) windows a thread, transformed), half 1 the filter image, so each
// SIMD has one wave with the heavy staging and one with the light. One
// barrier per chunk. The input reaches the windows through a per-wave LDS
// patch of the rows the workgroup's tiles read, loaded with coalesced
// loads, zeros at the padding; windows are then read without bounds checks.
//
// MFMA k order: in v_mfma_f32_32x32x2f32 lane l = 32*lk + li supplies
// A[li][k] and B[k][li] for k = lk of the instruction's two; instruction q
// (q = 0..3) of a chunk takes k = 4*lk + q, so a lane's four A values are
// one 16-byte read and its B values four reads of one V row each. The
// instructions alternate between two positions so consecutive MFMAs are
// independent.
//
// With SPLIT the channel chunks are divided among gridDim.y slices and each
// writes its raw Y to the split-K workspace ws[(slice * OC + oc) * P + pixel],
// P = N*OH*OW, for splitk_reduce_f32 to add in slice order and finish.
namespace mdlc {

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
constexpr int WINO_VLD = 72;                          // V row: 64 tiles + 8 (bank offset of the k halves)
constexpr int WINO_USTAGE = 16 * 64 * 8;              // floats
constexpr int WINO_VSTAGE = 16 * 8 * WINO_VLD;
constexpr int WINO_STAGE = WINO_USTAGE + WINO_VSTAGE; // 68 KB
constexpr int WINO_PMAX = 704;                        // input patch floats per channel

// PL: patch loads per lane and channel, ceil(largest patch / 64) <= WINO_PMAX / 64.
template <bool SPLIT, int PL, class Epi>
__device__ __forceinline__ void conv_wino_f32(const WinoArgs& g) {
  static_assert(PL * 64 <= WINO_PMAX, "patch larger than its LDS");
  __shared__ __attribute__((aligned(16))) float lds[2 * WINO_STAGE];
  __shared__ float patch[4 * 2 * WINO_PMAX];         // per half-0 wave, two channels

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = wave >> 2;                          // position rows 2h, 2h + 1
  const int wm0 = ((wave >> 1) & 1) * 32;
  const int wn0 = (wave & 1) * 32;
  const int li = lane & 31;
  const int lk = lane >> 5;

  const int P = g.N * g.TH * g.TW;                  // tiles in the batch
  const int tiles_n = (P + 63) / 64;
  const int ocb = blockIdx.x / tiles_n;
  const int t0 = (blockIdx.x % tiles_n) * 64;
  const int slice = SPLIT ? blockIdx.y : 0;
  const int chunk0 = slice * g.nchunk;
  const int HW = g.H * g.W;
  const float* ublk = g.U + (size_t)ocb * (g.CP / 8) * WINO_USTAGE;

  // ---- input patch: the rows the workgroup's windows read -----------------
  // For each image its 64 tiles touch (segment s = image nfirst + s), the
  // rows its tiles' windows read (image coordinates, padding rows included),
  // each WP = 2 TW + 2 columns wide starting at column -PL; positions outside
  // the image hold zero, so windows are read without bounds checks. The
  // segments are stacked: segment 0 holds rows rlo0 .. (its last), the
  // others rows -PT .. (their last), whole images 2 TH + 2 rows.
  const int TT = g.TH * g.TW;
  const int WP = 2 * g.TW + 2;
  const int nfirst = t0 / TT;
  const int plast = min(t0 + 63, P - 1);
  const int nlast = plast / TT;
  const int rlo0 = 2 * ((t0 - nfirst * TT) / g.TW) - g.PT;
  const int rhil = 2 * ((plast - nlast * TT) / g.TW) + 3 - g.PT;
  const int rows0 = (nlast == nfirst ? rhil : 2 * g.TH + 1 - g.PT) - rlo0 + 1;
  const int seg = (2 * g.TH + 2) * WP;              // elements of a whole image's segment
  const int PS = rows0 * WP + (nlast > nfirst ? (nlast - nfirst - 1) * seg + (rhil + g.PT + 1) * WP : 0);

  // ---- staging: half 0 transforms the input windows, each thread those of
  // tile t0 + lane for channels wq and wq + 4 of a chunk, read from its
  // wave's patch of the two channels; half 1 copies the filter image, eight
  // 16-byte pieces a thread.
  const int wq = wave & 3;
  const int lt = tid & 255;
  int wbase;                                        // the lane's window in the patch
  {
    const int p = t0 + lane;
    const int pc = p < P ? p : t0;                  // tiles past the batch: any window, never stored
    const int n = pc / TT;
    const int r = pc - n * TT;
    const int ty = r / g.TW;
    const int tx = r - ty * g.TW;
    const int sg = n - nfirst;
    wbase = (sg == 0 ? (2 * ty - g.PT - rlo0) * WP : rows0 * WP + (sg - 1) * seg + 2 * ty * WP) + 2 * tx;
  }
  // the lane's patch elements lane + 64 i: offset of the channel-0 value, or
  // a zero (bit i of pzero) outside the image or past the patch
  int poff[PL];
  unsigned pzero = 0;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = i * 64 + lane;
    int sg, row, col;
    if (e < rows0 * WP) {
      sg = 0;
      row = rlo0 + e / WP;
      col = e - (e / WP) * WP;
    } else {
      const int e1 = e - rows0 * WP;
      sg = 1 + e1 / seg;
      const int e2 = e1 - (e1 / seg) * seg;
      row = e2 / WP - g.PT;
      col = e2 - (e2 / WP) * WP;
    }
    const int ix = col - g.PL;
    const bool ok = e < PS && (unsigned)row < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
    poff[i] = ok ? (nfirst + sg) * g.C * HW + row * g.W + ix : 0;
    pzero |= (ok ? 0u : 1u) << i;
  }

  // registers of the chunk in flight: half 0 the two channels' patch
  // elements, half 1 the filter image pieces
  float4 ur[8];
  float pv[2][PL];
  int held = chunk0;                                // chunk the patch registers hold
  float* pw = patch + wq * (2 * WINO_PMAX);
  auto load_x = [&](int chunk) {
    held = chunk;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float* src = g.x + (size_t)min(chunk * 8 + wq + 4 * j, g.C - 1) * HW;
#pragma unroll
      for (int i = 0; i < PL; ++i) pv[j][i] = src[(unsigned)poff[i]];
    }
  };
  auto store_x = [&](float* st) {
    // the patch, zeros written with a bit mask (no select: it would branch)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < PL; ++i)
        pw[j * WINO_PMAX + i * 64 + lane] =
            __uint_as_float(__float_as_uint(pv[j][i]) & ((pzero >> i & 1u) - 1u));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // V of channel wq + 4j; zero past the last channel (its filters are
      // zero too, but the window would repeat the last channel's values)
      float v[16];
      if (held * 8 + wq + 4 * j < g.C) {
        const float* pj = pw + j * WINO_PMAX + wbase;
        float d[16];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) d[4 * a + b] = pj[a * WP + b];
        float t[16];                                // t = B^T d, row by row
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          t[b] = d[b] - d[8 + b];
          t[4 + b] = d[4 + b] + d[8 + b];
          t[8 + b] = d[8 + b] - d[4 + b];
          t[12 + b] = d[4 + b] - d[12 + b];
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) {               // V = t B
          v[4 * a + 0] = t[4 * a] - t[4 * a + 2];
          v[4 * a + 1] = t[4 * a + 1] + t[4 * a + 2];
          v[4 * a + 2] = t[4 * a + 2] - t[4 * a + 1];
          v[4 * a + 3] = t[4 * a + 1] - t[4 * a + 3];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = 0.f;
      }
      // all 16 values in their own registers before the stores, so a store
      // waiting for the LDS does not hold up the transform of the next window
      float* vs = st + WINO_USTAGE + (wq + 4 * j) * WINO_VLD + lane;
#pragma unroll
      for (int e = 0; e < 16; ++e) vs[e * 8 * WINO_VLD] = v[e];
    }
  };
  auto load_u = [&](int chunk) {
    const float* us = ublk + (size_t)chunk * WINO_USTAGE;
#pragma unroll
    for (int i = 0; i < 8; ++i) ur[i] = ld4(us + (lt + i * 256) * 4);
  };
  auto store_u = [&](float* st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) st4(st + (lt + i * 256) * 4, ur[i]);
  };

  // acc[i] = M at position xi = 8h + i
  floatx16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  // fragment addresses within a stage (floats)
  const int arow = wm0 + li;
  const int a_off = arow * 8 + 4 * (lk ^ (((arow >> 2) ^ (arow >> 3)) & 1));
  const int b_off = WINO_USTAGE + (4 * lk) * WINO_VLD + wn0 + li;

  // MFMA fragments of one group of two positions: A as one 16-byte read,
  // B as two pairs of V rows per position
  struct Frag {
    float4 a[2];
    float b[2][4];
  };
  auto read_frags = [&](Frag& f, const float* st, int xg) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int xi = 8 * h + 2 * xg + x;
      f.a[x] = ld4(st + xi * 512 + a_off);
#pragma unroll
      for (int q = 0; q < 4; ++q) f.b[x][q] = st[b_off + xi * 8 * WINO_VLD + q * WINO_VLD];
    }
  };
  auto mfma_group = [&](const Frag& f, int xg) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const float a = q == 0 ? f.a[x].x : q == 1 ? f.a[x].y : q == 2 ? f.a[x].z : f.a[x].w;
        acc[2 * xg + x] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, f.b[x][q], acc[2 * xg + x], 0, 0, 0);
      }
  };

  // Staging is split by half: half 0 loads and transforms the input
  // windows (the heavy part), half 1 copies the filter image, each into the
  // stage of the next chunk while the current chunk's MFMAs run, and each
  // loading the chunk after that; so on every SIMD one wave's MFMAs keep the
  // matrix core busy while the other wave stages. The two halves run their
  // own copy of the loop (the same barriers), so each holds only its own
  // staging registers. Past the last chunk the stores and loads repeat the
  // last chunk (in bounds, never read); a stage is written only after the
  // barrier that ends its last reads. The scheduling barriers keep the
  // global loads ahead of the MFMAs (left to itself the compiler sinks them
  // to the end of the loop, where their latency shows).
  auto mfma_chunk = [&](const float* cur) {
    Frag f0, f1;
    read_frags(f0, cur, 0);
    read_frags(f1, cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f0, 0);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(f0, cur, 2);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f1, 1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(f1, cur, 3);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f0, 2);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f1, 3);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (h == 0) {
    load_x(chunk0);
    store_x(lds);
    load_x(chunk0 + min(1, g.nchunk - 1));
    __syncthreads();
    for (int ch = 0; ch < g.nchunk; ++ch) {
      __builtin_amdgcn_sched_barrier(0);
      store_x(lds + ((ch + 1) & 1) * WINO_STAGE);
      __builtin_amdgcn_sched_barrier(0);
      load_x(chunk0 + min(ch + 2, g.nchunk - 1));
      __builtin_amdgcn_sched_barrier(0);
      mfma_chunk(lds + (ch & 1) * WINO_STAGE);
      __syncthreads();
    }
  } else {
    load_u(chunk0);
    store_u(lds);
    load_u(chunk0 + min(1, g.nchunk - 1));
    __syncthreads();
    for (int ch = 0; ch < g.nchunk; ++ch) {
      __builtin_amdgcn_sched_barrier(0);
      store_u(lds + ((ch + 1) & 1) * WINO_STAGE);
      __builtin_amdgcn_sched_barrier(0);
      load_u(chunk0 + min(ch + 2, g.nchunk - 1));
      __builtin_amdgcn_sched_barrier(0);
      mfma_chunk(lds + (ch & 1) * WINO_STAGE);
      __syncthreads();
    }
  }

  // ---- output transform: partial Y of this half, through LDS -------------
  // acc[4a' + b][r] holds M at row a = 2h + a', column b, for
  // oc = wm0 + (r/4)*8 + lk*4 + r%4 and tile = wn0 + li (the 32x32x2
  // accumulator layout). s = A^T M restricted to the two rows, Y = s A.
  // Layout in LDS: Yp[h][oc][tile][4] (the stages are no longer read).
  float* yp = lds + h * (64 * 64 * 4);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int oc = wm0 + (r >> 2) * 8 + lk * 4 + (r & 3);
    float s0[4], s1[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float m0 = acc[b][r], m1 = acc[4 + b][r];
      if (h == 0) {                                 // rows 0, 1: A^T columns (1, 0), (1, 1)
        s0[b] = m0 + m1;
        s1[b] = m1;
      } else {                                      // rows 2, 3: (1, -1), (0, -1)
        s0[b] = m0;
        s1[b] = -m0 - m1;
      }
    }
    float4 yv;
    yv.x = s0[0] + s0[1] + s0[2];
    yv.y = s0[1] - s0[2] - s0[3];
    yv.z = s1[0] + s1[1] + s1[2];
    yv.w = s1[1] - s1[2] - s1[3];
    st4(yp + (oc * 64 + wn0 + li) * 4, yv);
  }
  __syncthreads();

  // ---- epilogue: Y = Y_0 + Y_1, 8 (channel, tile) pairs a thread ----------
  const int OHW = g.OH * g.OW;
  const bool pairs = (g.OW & 1) == 0;               // (ox, ox + 1) 8-byte aligned
#pragma unroll 2
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * WINO_NT;
    const int ocl = idx >> 6, tl = idx & 63;
    const int oc = ocb * 64 + ocl;
    const int p = t0 + tl;
    if (oc >= g.OC || p >= P) continue;
    const float4 y0 = ld4(lds + (ocl * 64 + tl) * 4);
    const float4 y1v = ld4(lds + 64 * 64 * 4 + (ocl * 64 + tl) * 4);
    float out[4] = {y0.x + y1v.x, y0.y + y1v.y, y0.z + y1v.z, y0.w + y1v.w};
    const int n = p / (g.TH * g.TW);
    const int rr = p - n * (g.TH * g.TW);
    const int ty = rr / g.TW;
    const int tx = rr - ty * g.TW;
    const int oy = 2 * ty, ox = 2 * tx;
    const bool yok = oy + 1 < g.OH, xok = ox + 1 < g.OW;
    float* dst;
    if (SPLIT) {
      dst = g.y + ((size_t)slice * g.OC + oc) * ((size_t)g.N * OHW) + (size_t)n * OHW;
    } else {
      dst = g.y + ((size_t)n * g.OC + oc) * OHW;
      const float b = Epi::bias == 1 ? g.bias[oc] : 0.f;
      const float* res = Epi::residual ? g.R + ((size_t)n * g.OC + oc) * OHW : nullptr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int py = oy + (e >> 1), px = ox + (e & 1);
        const bool ok = (e & 2 ? yok : true) && (e & 1 ? xok : true);
        float v = Epi::apply(out[e], b);
        if (Epi::residual) v = Epi::post(v, ok ? res[py * g.OW + px] : 0.f);
        out[e] = v;
      }
    }
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
      if (e2 == 1 && !yok) break;
      float* row = dst + (oy + e2) * g.OW + ox;
      if (pairs && xok) {
        *reinterpret_cast<float2*>(row) = make_float2(out[2 * e2], out[2 * e2 + 1]);
      } else {
        row[0] = out[2 * e2];
        if (xok) row[1] = out[2 * e2 + 1];
      }
    }
  }
}

}  // namespace mdlc
