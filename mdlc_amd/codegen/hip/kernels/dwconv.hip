// Direct depthwise convolution (group == C, one input channel per output
// channel, channel multiplier OC/C) with a fused bias/activation epilogue.
// One thread per output element; taps accumulate in (kh, kw) order.
namespace mdlc {

template <int KH, int KW, int SH, int SW, int DH, int DW, class Epi>
__device__ __forceinline__ void dwconv_f32(const float* __restrict__ x, const float* __restrict__ w,
                                           const float* __restrict__ bias, float* __restrict__ y,
                                           int N, int C, int H, int W, int OC, int OH, int OW,
                                           int PT, int PL) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * OC * OH * OW;
  if (i >= total) return;
  const int ow = (int)(i % OW);
  const int oh = (int)((i / OW) % OH);
  const int oc = (int)((i / ((long long)OW * OH)) % OC);
  const int n = (int)(i / ((long long)OW * OH * OC));
  const int c = oc / (OC / C);
  const float* xp = x + ((size_t)n * C + c) * H * W;
  const float* wp = w + (size_t)oc * KH * KW;
  float acc = 0.f;
#pragma unroll
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * SH - PT + kh * DH;
#pragma unroll
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * SW - PL + kw * DW;
      const float xv = ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) ? xp[ih * W + iw] : 0.f;
      acc = acc + wp[kh * KW + kw] * xv;
    }
  }
  y[i] = Epi::apply(acc, Epi::bias ? bias[oc] : 0.f);
}

}  // namespace mdlc
