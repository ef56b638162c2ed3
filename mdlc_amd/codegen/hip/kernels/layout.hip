// Data-movement and row-reduction kernels for the ops the reference ran on
// the host: Softmax, Transpose, Pad and Concat (float32). Shapes of up to six
// dimensions are passed padded with leading ones. Element indices are 64-bit.
namespace mdlc {

struct Dims6 {
  int d[6];
};

// Softmax over an axis of length L, the tensor viewed as [outer][L][inner]:
// z = x - max, e = exp(z), y = e / sum(e), each step a float32 operation
// (the NumPy float32 order of mdlc/runtime/ops.py:188-191; expf is the
// correctly rounded-to-within-an-ulp device exponential).
//
// inner == 1 (the last axis): one 64-lane wave per row, strided lanes and a
// butterfly for the max and the sum.
__device__ __forceinline__ void softmax_rows_f32(const float* __restrict__ x, float* __restrict__ y,
                                                 long long rows, int L) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * L;
  float* yr = y + row * L;
  float m = -__builtin_inff();
  for (int i = lane; i < L; i += 64) m = fmaxf(m, xr[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  float s = 0.f;
  for (int i = lane; i < L; i += 64) s += expf(xr[i] - m);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  for (int i = lane; i < L; i += 64) yr[i] = expf(xr[i] - m) / s;
}

// inner > 1: one thread per (outer, inner) column, walking L with stride
// inner; neighbouring threads read neighbouring addresses.
__device__ __forceinline__ void softmax_cols_f32(const float* __restrict__ x, float* __restrict__ y,
                                                 long long outer, int L, int inner) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * inner) return;
  const long long o = t / inner;
  const int c = (int)(t - o * inner);
  const float* xc = x + o * L * inner + c;
  float* yc = y + o * L * inner + c;
  float m = -__builtin_inff();
  for (int i = 0; i < L; ++i) m = fmaxf(m, xc[(long long)i * inner]);
  float s = 0.f;
  for (int i = 0; i < L; ++i) s += expf(xc[(long long)i * inner] - m);
  for (int i = 0; i < L; ++i) yc[(long long)i * inner] = expf(xc[(long long)i * inner] - m) / s;
}

// Transpose: output element e (row-major over out dims) reads the input at
// sum_d idx_d * src_stride[d], src_stride[d] being the input stride of the
// axis that output axis d takes (perm).
__device__ __forceinline__ void transpose_f32(const float* __restrict__ x, float* __restrict__ y,
                                              long long total, Dims6 od, Dims6 ss) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  long long rem = e, src = 0;
#pragma unroll
  for (int d = 5; d >= 0; --d) {
    const long long i = rem % od.d[d];
    rem /= od.d[d];
    src += i * ss.d[d];
  }
  y[e] = x[src];
}

// Pad: MODE 0 constant (value), 1 edge (clamp), 2 reflect (mirror without
// repeating the edge element; each pad is shorter than its axis).
template <int MODE>
__device__ __forceinline__ void pad_f32(const float* __restrict__ x, float* __restrict__ y,
                                        long long total, Dims6 od, Dims6 id, Dims6 before,
                                        float value) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  long long rem = e, src = 0, stride = 1;
  bool inside = true;
#pragma unroll
  for (int d = 5; d >= 0; --d) {
    const int n = id.d[d];
    int j = (int)(rem % od.d[d]) - before.d[d];
    rem /= od.d[d];
    if (j < 0 || j >= n) {
      if (MODE == 0) {
        inside = false;
      } else if (MODE == 1) {
        j = j < 0 ? 0 : n - 1;
      } else {
        j = j < 0 ? -j : 2 * (n - 1) - j;
      }
    }
    src += (long long)j * stride;
    stride *= n;
  }
  y[e] = inside ? x[src] : value;
}

// One Concat operand: rows x run contiguous floats into the output at
// row stride dst_stride, starting dst_off floats into each row.
__device__ __forceinline__ void concat_part_f32(const float* __restrict__ x, float* __restrict__ y,
                                                long long rows, long long run, long long dst_stride,
                                                long long dst_off) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * run) return;
  const long long r = e / run;
  y[r * dst_stride + dst_off + (e - r * run)] = x[e];
}

}  // namespace mdlc
