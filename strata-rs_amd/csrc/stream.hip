// A plain streaming read: the HBM read-bandwidth ceiling the matvec is
// measured against. It reads n bytes with 16-byte loads, one load per lane
// per step of a grid-stride loop over kStreamBlocks workgroups of 256
// threads (consecutive lanes on consecutive 16 bytes: the fastest plain read
// pattern measured on MI355X for a 28 MB span), and folds them with XOR so
// no load is dead; workgroup b writes its fold to out[b]. No reference
// counterpart.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ p, uint64_t n16,
                                                          uint32_t* __restrict__ out) {
  __shared__ uint32_t part[256 / kWave];
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  uint32_t acc = 0;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, kWave);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

hipError_t launch_stream_read(const void* data, uint64_t nbytes, uint32_t* out, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(data) & 15u) || (nbytes & 15u)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(stream_read_kernel, dim3(kStreamBlocks), dim3(256), 0, s, static_cast<const u32x4*>(data),
                     nbytes / 16, out);
  return hipGetLastError();
}

// A byte copy for the host-slice entry points: between device memory and
// the context's mapped pinned staging (device-visible host memory), so a
// call's small input and output slices move in a kernel's loads and stores
// instead of a DMA-engine transfer each way. 16-byte accesses when both
// ends and the length allow, bytes otherwise (unaligned slices are small:
// routing ids and weights).
__global__ void __launch_bounds__(256) copy_bytes_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         uint64_t n, int vec) {
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  const uint64_t i0 = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (vec) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    u32x4* d = reinterpret_cast<u32x4*>(dst);
    for (uint64_t i = i0; i < n / 16; i += stride) d[i] = s[i];
  } else {
    for (uint64_t i = i0; i < n; i += stride) dst[i] = src[i];
  }
}

hipError_t launch_copy_bytes(const void* src, void* dst, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | n) & 15u) == 0;
  const uint64_t items = vec ? n / 16 : n;
  const uint64_t blocks = std::min<uint64_t>((items + 255) / 256, 1024);
  hipLaunchKernelGGL(copy_bytes_kernel, dim3(unsigned(blocks)), dim3(256), 0, s, static_cast<const uint8_t*>(src),
                     static_cast<uint8_t*>(dst), n, int(vec));
  return hipGetLastError();
}

}  // namespace sh
