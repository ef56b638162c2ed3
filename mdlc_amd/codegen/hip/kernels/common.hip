// Shared device helpers for the generated fused-group kernels (gfx950).
// Compiled by hipRTC as part of every generated module.
namespace mdlc {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Raw buffer resource over [p, p + bytes): a load whose offset is at or
// beyond `bytes` returns zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
constexpr int kOutside = 0x7ffffff0;   // an offset past every buffer (sizes < 2^31)

// Tile index remap so that consecutive logical tiles run on the same XCD.
// Workgroup b is dispatched to XCD (b % 8); XCD x owns a contiguous range of
// logical tiles. The map is a bijection on [0, total).
__device__ __forceinline__ int xcd_remap(int b, int total) {
  const int nx = 8;
  int q = total / nx, r = total % nx;
  int x = b % nx, j = b / nx;
  return x * q + (x < r ? x : r) + j;
}

// Logical tile t -> (m tile, n tile), down M in groups of GM rows of tiles:
// the tiles one XCD runs together then share GM row blocks of A and a few
// column blocks of B instead of every row block of A. With tiles_m <= GM this
// is plain column order. A bijection onto the tile grid.
template <int GM>
__device__ __forceinline__ void grouped_tile(int t, int tiles_m, int tiles_n, int& mt, int& nt) {
  const int grp = t / (GM * tiles_n);
  const int gsz = min(tiles_m - grp * GM, GM);
  const int tg = t - grp * GM * tiles_n;
  mt = grp * GM + tg % gsz;
  nt = tg / gsz;
}

}  // namespace mdlc
