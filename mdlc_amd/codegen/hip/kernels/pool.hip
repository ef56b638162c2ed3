// Pooling over NCHW planes (max pooling is the window template in dwconv.hip).
namespace mdlc {

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
