// Per-plane sliding-window kernels over NCHW float32: depthwise convolution
// (group == C, channel multiplier OC/C, fused bias/activation epilogue), max
// pooling and average pooling share one template. Taps are combined in
// (kh, kw) order.
// Indices within a plane are 32-bit (the host checks the sizes).
namespace mdlc {

// Depthwise conv: acc = acc + w[kh][kw] * x, then the epilogue.
template <class Epi>
struct DwOp {
  static constexpr bool weights = true;
  static constexpr int average = 0;
  __device__ __forceinline__ static float pad() { return 0.f; }
  __device__ __forceinline__ static float init() { return 0.f; }
  __device__ __forceinline__ static float step(float acc, float x, float w) { return acc + w * x; }
  __device__ __forceinline__ static float finish(float acc, float b) { return Epi::apply(acc, b); }
};

// Max pool: out-of-range taps are -inf (the NumPy padding value).
struct MaxOp {
  static constexpr bool weights = false;
  static constexpr int average = 0;
  __device__ __forceinline__ static float pad() { return -__builtin_inff(); }
  __device__ __forceinline__ static float init() { return -__builtin_inff(); }
  __device__ __forceinline__ static float step(float acc, float x, float) { return fmaxf(acc, x); }
  __device__ __forceinline__ static float finish(float acc, float) { return acc; }
};

// Average pool: padding taps add zero; finish() divides the window sum by
// the divisor the template passes: KH*KW (average == 2, count_include_pad)
// or the number of taps inside the input (average == 1).
template <bool INCLUDE_PAD>
struct AvgOp {
  static constexpr bool weights = false;
  static constexpr int average = INCLUDE_PAD ? 2 : 1;
  __device__ __forceinline__ static float pad() { return 0.f; }
  __device__ __forceinline__ static float init() { return 0.f; }
  __device__ __forceinline__ static float step(float acc, float x, float) { return acc + x; }
  __device__ __forceinline__ static float finish(float acc, float den) { return acc / den; }
};

// Column-strip form: each thread owns VH vertically adjacent outputs of one
// output column and loads the (VH-1)*SH + (KH-1)*DH + 1 input rows x KW taps
// they need into registers, all loads issued before any arithmetic, so many
// bytes are in flight per wave. Consecutive threads own consecutive columns,
// so every load and store instruction is contiguous across the wave.
template <int KH, int KW, int SH, int SW, int DH, int DW, int VH, class Op>
__device__ __forceinline__ void window_column_f32(const float* __restrict__ x,
                                                  const float* __restrict__ w,
                                                  const float* __restrict__ bias,
                                                  float* __restrict__ y, int planes, int C, int H,
                                                  int W, int OC, int OH, int OW, int PT, int PL) {
  constexpr int NR = (VH - 1) * SH + (KH - 1) * DH + 1;
  const int strips = (OH + VH - 1) / VH;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= planes * strips * OW) return;
  const int ow = idx % OW;
  const int ps = idx / OW;                          // plane * strips + strip
  const int plane = ps / strips;
  const int oh0 = (ps - plane * strips) * VH;
  const int oc = plane % OC;
  const int n = plane / OC;
  const int c = oc / (OC / C);
  const float* xp = x + ((size_t)n * C + c) * H * W;
  const int ih0 = oh0 * SH - PT;
  const int iw0 = ow * SW - PL;
  float v[NR][KW];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int ih = ih0 + r;
    const bool row_ok = (unsigned)ih < (unsigned)H;
#pragma unroll
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = iw0 + kw * DW;
      v[r][kw] = (row_ok && (unsigned)iw < (unsigned)W) ? xp[ih * W + iw] : Op::pad();
    }
  }
  float wr[KH * KW];
#pragma unroll
  for (int k = 0; k < KH * KW; ++k) wr[k] = Op::weights ? w[oc * KH * KW + k] : 0.f;
  const float b = bias ? bias[oc] : 0.f;
  int cols_in = 0;                                  // taps of this column inside the input
  if (Op::average == 1) {
#pragma unroll
    for (int kw = 0; kw < KW; ++kw) cols_in += (unsigned)(iw0 + kw * DW) < (unsigned)W;
  }
  float* yp = y + (size_t)plane * OH * OW + ow;
#pragma unroll
  for (int j = 0; j < VH; ++j) {
    if (oh0 + j >= OH) break;
    float acc = Op::init();
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) acc = Op::step(acc, v[j * SH + kh * DH][kw], wr[kh * KW + kw]);
    float arg = b;
    if (Op::average == 2) {
      arg = (float)(KH * KW);
    } else if (Op::average == 1) {
      int rows_in = 0;
#pragma unroll
      for (int kh = 0; kh < KH; ++kh) rows_in += (unsigned)(ih0 + j * SH + kh * DH) < (unsigned)H;
      arg = (float)max(rows_in * cols_in, 1);
    }
    yp[(oh0 + j) * OW] = Op::finish(acc, arg);
  }
}

}  // namespace mdlc
