// Direct convolution with few input channels (a network's stem) fused with
// the 3x3 stride-2 max pool (padding 1) that follows it, on the matrix cores.
// The convolution's output never leaves the chip: each workgroup computes
// a band of conv rows, takes the pool's maxima in registers and stores only
// the pooled rows.
//
// Pooled row p reads conv rows 2p-1, 2p, 2p+1 and pooled column q conv
// columns 2q-1, 2q, 2q+1 (row or column -1 is the pool's -inf padding). A
// workgroup owns R consecutive pooled rows of one image, all pooled columns,
// and 64 output channels: conv rows 2Rk-1 .. 2Rk+2R-1 of band k (2R+1 rows;
// band 0 skips row -1), every conv column. Its input patch (the rows those
// conv rows read, every column, zeros at the padding) is staged in LDS once.
//
// Wave w owns the 16 output channels of block 4 * blockIdx.y + w and walks
// the row's 16-pixel column blocks left to right. For one column block it
// runs v_mfma_f32_16x16x4f32 over the 4-deep k steps of K = C*KH*KW, A = the
// channel block's weights (registers, packed [block][step][lane]: lane
// 16 lk + li holds w[16 blk + li][4 s + lk], zeros past K), B = the patch
// values of the 2R+1 conv rows (lane 16 lk + li: pixel li of the block, k =
// 4 s + lk), one accumulator per conv row. The accumulator layout puts a
// pixel in lanes li and channel 4 lk + r in register r, so
//   * the vertical maxima over rows 2j, 2j+1, 2j+2 are register maxima;
//   * the horizontal maxima over columns 2q-1, 2q, 2q+1 are maxima over
//     neighbouring lanes of a 16-lane row, which DPP row shifts bring in
//     without a memory round trip; lane 0's left neighbour (column 16 b - 1)
//     is lane 15 of the previous block, kept in registers and rotated into
//     lane 0 the same way.
// The bias and the activation are applied to the pooled maximum: rounding
// an addition of the same bias and a non-decreasing activation (Relu, Clip)
// both preserve order, so act(max_i(acc_i) + b) is bit-identical to
// max_i(act(acc_i + b)), the pool of the conv's output.
namespace mdlc {

template <int V> struct PoolStep { static constexpr int value = V; };

// f(PoolStep<S>()), f(PoolStep<S + 1>()), ... up to N - 1
template <int S, int N, class F>
__device__ __forceinline__ void pool_steps(F&& f) {
  if constexpr (S < N) {
    f(PoolStep<S>());
    pool_steps<S + 1, N>(f);
  }
}

// Patch offset of k = (c, kh, kw) in a C x PR x PC patch; a padding k past K
// reads k = 0 (its weight is zero).
template <int K, int KH, int KW, int PR, int PC>
__device__ __forceinline__ constexpr int pool_koff(int k) {
  return k < K ? ((k / (KH * KW)) * PR + k % (KH * KW) / KW) * PC + k % KW : 0;
}

// The lane's patch offset for k = 4 S + lk: one addition where the step's
// four k are consecutive columns of one kernel row, else a choice of four
// constants.
template <int S, int K, int KH, int KW, int PR, int PC>
__device__ __forceinline__ int pool_lane_off(int lk) {
  constexpr int o0 = pool_koff<K, KH, KW, PR, PC>(4 * S), o1 = pool_koff<K, KH, KW, PR, PC>(4 * S + 1);
  constexpr int o2 = pool_koff<K, KH, KW, PR, PC>(4 * S + 2), o3 = pool_koff<K, KH, KW, PR, PC>(4 * S + 3);
  if constexpr (o1 == o0 + 1 && o2 == o0 + 2 && o3 == o0 + 3) {
    return o0 + lk;
  } else {
    return lk == 0 ? o0 : lk == 1 ? o1 : lk == 2 ? o2 : o3;
  }
}

// DPP moves within each row of 16 lanes: lane i takes lane i - 1 (row_shr:1),
// i + 1 (row_shl:1) or (i - 1) mod 16 (row_ror:1); a lane without a source
// keeps `old`.
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShl1 = 0x101;
constexpr int kDppRowRor1 = 0x121;
template <int CTRL>
__device__ __forceinline__ float row_dpp(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, old), __builtin_bit_cast(int, src), CTRL, 0xf, 0xf, false));
}

template <class Epi, int C, int KH, int KW, int SH, int SW, int PT, int PL, int R, int NBX>
__device__ __forceinline__ void conv_pool_f32(const float* __restrict__ x,
                                              const float* __restrict__ wp,
                                              const float* __restrict__ bias,
                                              float* __restrict__ y, int N, int H, int W, int OC,
                                              int OH) {
  constexpr int OW = NBX * 16;                  // conv columns (the host checks OW % 16 == 0)
  constexpr int PW = OW / 2;                    // pooled columns
  constexpr int NR = 2 * R + 1;                 // conv rows of a band
  constexpr int PR = (NR - 1) * SH + KH;        // input rows of the band's patch
  constexpr int PC = (OW - 1) * SW + KW;        // input columns of the patch (padding included)
  constexpr int K = C * KH * KW;
  constexpr int NS = (K + 3) / 4;               // 4-deep k steps
  constexpr int ROWS = C * PR;                  // patch rows over all channels
  static_assert(C * PR * PC * 4 <= 150 * 1024, "patch exceeds the LDS");
  static_assert(PC <= 256, "one patch column per thread");
  static_assert(NR * SH * PC * 4 < 65536, "row offsets exceed the LDS offset range");
  __shared__ float patch[C * PR * PC];

  const int PH = OH / 2;
  const int bands = PH / R;
  const int n = blockIdx.x / bands;
  const int kb = blockIdx.x - n * bands;
  const int ih0 = (2 * R * kb - 1) * SH - PT;   // input row of patch row 0

  // ---- the patch: thread t loads column t of every patch row -------------
  {
    const int pc = threadIdx.x;
    const int iw = pc - PL;
    const bool col_ok = pc < PC && (unsigned)iw < (unsigned)W;
    const __amdgpu_buffer_rsrc_t rx = buffer_over(x + (size_t)n * C * H * W, C * H * W * 4);
    constexpr int BATCH = 15;
#pragma unroll 1
    for (int r0 = 0; r0 < ROWS; r0 += BATCH) {
      float v[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int row = r0 + q;                 // channel row / PR, patch row row % PR
        const int c = row / PR;
        const int ih = ih0 + row - c * PR;
        const bool ok = col_ok && row < ROWS && (unsigned)ih < (unsigned)H;
        v[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
            rx, ok ? ((c * H + ih) * W + iw) * 4 : kOutside, 0, 0));
      }
#pragma unroll
      for (int q = 0; q < BATCH; ++q)
        if (pc < PC && r0 + q < ROWS) patch[(r0 + q) * PC + pc] = v[q];
    }
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int blk = blockIdx.y * 4 + wave;        // 16-channel block
  float wr[NS];
  {
    const float* wl = wp + (size_t)blk * NS * 64 + lane;
#pragma unroll
    for (int s = 0; s < NS; ++s) wr[s] = wl[s * 64];
  }
  float bv4[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int oc = blk * 16 + 4 * lk + r;
    bv4[r] = (Epi::bias && oc < OC) ? bias[oc] : 0.f;
  }
  const int PHW = PH * PW;
  const __amdgpu_buffer_rsrc_t ry = buffer_over(y, N * OC * PHW * 4);
  int obase[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int oc = blk * 16 + 4 * lk + r;
    obase[r] = oc < OC && (li & 1) == 0 ? ((n * OC + oc) * PH + R * kb) * PW + (li >> 1) : -1;
  }
  float vprev[R][4];                            // the previous block's vertical maxima
#pragma unroll
  for (int j = 0; j < R; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) vprev[j][r] = -__builtin_inff();
  __syncthreads();

#pragma unroll 1
  for (int bx = 0; bx < NBX; ++bx) {
    const float* pb = patch + (16 * bx + li) * SW;
    floatx4 acc[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float bv[2][NR];
    {
      const float* p0 = pb + pool_lane_off<0, K, KH, KW, PR, PC>(lk);
#pragma unroll
      for (int i = 0; i < NR; ++i) bv[0][i] = p0[i * SH * PC];
    }
    pool_steps<0, NS>([&](auto SC) {
      constexpr int s = decltype(SC)::value;
      if constexpr (s + 1 < NS) {
        const float* pn = pb + pool_lane_off<s + 1, K, KH, KW, PR, PC>(lk);
#pragma unroll
        for (int i = 0; i < NR; ++i) bv[(s + 1) & 1][i] = pn[i * SH * PC];
      }
#pragma unroll
      for (int i = 0; i < NR; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[s], bv[s & 1][i], acc[i], 0, 0, 0);
      // one read of the next step after each MFMA: every read has a whole
      // step of MFMAs to arrive in, and no wait stalls the matrix core
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
      }
      __builtin_amdgcn_sched_barrier(0);
    });

    // pooled rows R kb + j, columns 8 bx + li / 2 (even lanes)
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = fmaxf(acc[2 * j + 1][r], acc[2 * j + 2][r]);
        if (kb > 0 || j > 0) v = fmaxf(acc[2 * j][r], v);   // row -1 is padding
        const float carry = row_dpp<kDppRowRor1>(0.f, vprev[j][r]);   // lane 0: lane 15
        const float left = row_dpp<kDppRowShr1>(carry, v);
        const float right = row_dpp<kDppRowShl1>(v, v);
        const float m = fmaxf(fmaxf(left, v), right);
        vprev[j][r] = v;
        const int o = obase[r] < 0 ? kOutside : (obase[r] + j * PW + 8 * bx) * 4;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, Epi::apply(m, bv4[r])),
                                              ry, o, 0, 0);
      }
  }
}

}  // namespace mdlc
