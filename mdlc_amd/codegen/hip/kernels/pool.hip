// Pooling over NCHW planes.
namespace mdlc {

// Max pool, one thread per output element; out-of-range taps count as -inf
// (the padding value of the NumPy semantics).
__device__ __forceinline__ void maxpool_f32(const float* __restrict__ x, float* __restrict__ y,
                                            int planes, int H, int W, int OH, int OW, int KH,
                                            int KW, int SH, int SW, int PT, int PL, int DH, int DW) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)planes * OH * OW;
  if (i >= total) return;
  const int ow = (int)(i % OW);
  const int oh = (int)((i / OW) % OH);
  const long long plane = i / ((long long)OH * OW);
  const float* xp = x + plane * H * W;
  float m = -__builtin_inff();
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * SH - PT + kh * DH;
    if ((unsigned)ih >= (unsigned)H) continue;
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * SW - PL + kw * DW;
      if ((unsigned)iw >= (unsigned)W) continue;
      m = fmaxf(m, xp[ih * W + iw]);
    }
  }
  y[i] = m;
}

// Global average pool: one 64-lane wave per plane. Lanes accumulate a
// strided share in float32, a butterfly reduction combines them, and the
// plane mean is sum / HW.
__device__ __forceinline__ void gap_f32(const float* __restrict__ x, float* __restrict__ y,
                                        int planes, int HW) {
  const int lane = threadIdx.x & 63;
  const int plane = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (plane >= planes) return;
  const float* xp = x + (size_t)plane * HW;
  float s = 0.f;
  for (int i = lane; i < HW; i += 64) s += xp[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) y[plane] = s / (float)HW;
}

}  // namespace mdlc
