// Byte-exact copy used for reshaping views (Flatten, Reshape, Identity,
// Squeeze/Unsqueeze): dst and src are 16-byte aligned arena tensors.
namespace mdlc {

__device__ __forceinline__ void copy_bytes(const unsigned char* __restrict__ src,
                                           unsigned char* __restrict__ dst, long long nbytes) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long nq = nbytes >> 4;
  if (i < nq) {
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    const long long b = nq * 16 + (i - nq);
    if (b < nbytes) dst[b] = src[b];
  }
}

}  // namespace mdlc
