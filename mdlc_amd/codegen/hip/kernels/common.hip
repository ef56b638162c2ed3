// Shared device helpers for the generated fused-group kernels (gfx950).
// Compiled by hipRTC as part of every generated module.
namespace mdlc {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Tile index remap so that consecutive logical tiles run on the same XCD.
// Workgroup b is dispatched to XCD (b % 8); XCD x owns a contiguous range of
// logical tiles. The map is a bijection on [0, total).
__device__ __forceinline__ int xcd_remap(int b, int total) {
  const int nx = 8;
  int q = total / nx, r = total % nx;
  int x = b % nx, j = b / nx;
  return x * q + (x < r ? x : r) + j;
}

}  // namespace mdlc
