// Batched im2col: cols[k][p] for k = (c, kh, kw) with kw fastest and
// p = (n, oh, ow) with ow fastest, for an NCHW input x. Rows have leading
// dimension ldc (a multiple of 4); columns P..ldc-1 are written as zeros.
// Each thread writes 4 consecutive columns of one row with one 128-bit store.
// Grid: x covers ldc/4 quads in blocks of blockDim.x threads, y = row k.
namespace mdlc {

__device__ __forceinline__ void im2col_f32(const float* __restrict__ x, float* __restrict__ cols,
                                           int C, int H, int W, int KH, int KW, int OH, int OW,
                                           int SH, int SW, int PH, int PW, int DH, int DW,
                                           int N, int ldc) {
  const int k = blockIdx.y;
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  const int p0 = q * 4;
  if (p0 >= ldc || k >= C * KH * KW) return;
  const int ohw = OH * OW;
  const int P = N * ohw;
  const int c = k / (KH * KW);
  const int rr = k - c * KH * KW;
  const int kh = rr / KW;
  const int kw = rr - kh * KW;
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int p = p0 + j;
    float e = 0.f;
    if (p < P) {
      const int n = p / ohw;
      const int s = p - n * ohw;
      const int oh = s / OW;
      const int ow = s - oh * OW;
      const int ih = oh * SH - PH + kh * DH;
      const int iw = ow * SW - PW + kw * DW;
      if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
        e = x[((size_t)n * C + c) * H * W + ih * W + iw];
    }
    v[j] = e;
  }
  st4(cols + (size_t)k * ldc + p0, make_float4(v[0], v[1], v[2], v[3]));
}

}  // namespace mdlc
