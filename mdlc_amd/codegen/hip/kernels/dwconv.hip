// Direct depthwise convolution (group == C, one input channel per output
// channel, channel multiplier OC/C) with a fused bias/activation epilogue.
//
// Each thread computes VW horizontally adjacent outputs of one output row:
// it loads the input span those outputs share once per filter row (for a
// 3x3 stride-1 window, 6 loads serve 4 outputs instead of 12) and keeps the
// plane's KH*KW weights in registers. Indices are 32-bit (the host checks
// the sizes); the taps of each output accumulate in (kh, kw) order.
namespace mdlc {

template <int KH, int KW, int SH, int SW, int DH, int DW, int VW, class Epi>
__device__ __forceinline__ void dwconv_f32(const float* __restrict__ x, const float* __restrict__ w,
                                           const float* __restrict__ bias, float* __restrict__ y,
                                           int N, int C, int H, int W, int OC, int OH, int OW,
                                           int PT, int PL) {
  constexpr int SPAN = (VW - 1) * SW + (KW - 1) * DW + 1;
  const int segs = (OW + VW - 1) / VW;
  const int per_plane = OH * segs;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * OC * per_plane) return;
  const int plane = idx / per_plane;               // n * OC + oc
  const int rem = idx - plane * per_plane;
  const int oh = rem / segs;
  const int ow0 = (rem - oh * segs) * VW;
  const int oc = plane % OC;
  const int n = plane / OC;
  const int c = oc / (OC / C);
  const float* xp = x + ((size_t)n * C + c) * H * W;
  float wr[KH * KW];
#pragma unroll
  for (int t = 0; t < KH * KW; ++t) wr[t] = w[oc * KH * KW + t];
  float acc[VW];
#pragma unroll
  for (int v = 0; v < VW; ++v) acc[v] = 0.f;
  const int iw0 = ow0 * SW - PL;
#pragma unroll
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * SH - PT + kh * DH;
    const bool row_ok = (unsigned)ih < (unsigned)H;
    float xs[SPAN];
#pragma unroll
    for (int j = 0; j < SPAN; ++j) {
      const int iw = iw0 + j;
      xs[j] = (row_ok && (unsigned)iw < (unsigned)W) ? xp[ih * W + iw] : 0.f;
    }
#pragma unroll
    for (int v = 0; v < VW; ++v)
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) acc[v] = acc[v] + wr[kh * KW + kw] * xs[v * SW + kw * DW];
  }
  const float b = Epi::bias ? bias[oc] : 0.f;
  float* yp = y + ((size_t)plane * OH + oh) * OW + ow0;
  if constexpr (VW == 4) {
    if ((OW & 3) == 0) {            // rows and segments are 16-byte aligned
      *reinterpret_cast<float4*>(yp) = make_float4(Epi::apply(acc[0], b), Epi::apply(acc[1], b),
                                                   Epi::apply(acc[2], b), Epi::apply(acc[3], b));
      return;
    }
  }
#pragma unroll
  for (int v = 0; v < VW; ++v)
    if (ow0 + v < OW) yp[v] = Epi::apply(acc[v], b);
}

}  // namespace mdlc
