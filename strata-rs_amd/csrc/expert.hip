// Expert gather-matvec in the reference orientation.
//
// crates/strata-core/src/ops.rs:169-195 (`expert_gemv`): an expert tensor is
// expert-major [n_expert][rows = in][cols = out] with quant blocks along the
// output axis (crates/strata-core/src/weights.rs:14-34), and
//   y[c] = sum_i x[i] * W_e[i][c]
// accumulated over input rows i, skipping rows with x[i] == 0.
//
// Because a packed row is one *input* element's coefficients for every
// output, the kernel is an axpy over rows with a split-K reduction:
//   * thread t of a 256-thread workgroup owns the 64-column unit u = t % U
//     (U = cols / 64) and visits rows r0 + t / U, r0 + t / U + RS, ... of its
//     workgroup's row chunk (RS = 256 / U row slots), keeping 64 column sums
//     in registers; per-block scales are folded into one coefficient per row
//     and sub-block (x[i]*d*sc), offsets (min, -32, +128 bias) are summed per
//     sub-block and subtracted once at the end;
//   * the row slots of a workgroup are summed through LDS, each workgroup
//     writes one partial vector, and a second kernel adds the partials in
//     chunk order, so results are deterministic.
#include "axpy.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

constexpr int kExpertThreads = 256;

// partial[blockIdx.x][c] for the row chunk [blockIdx.x*chunk, +chunk).
template <class F>
__global__ void __launch_bounds__(kExpertThreads)
    expert_partial_kernel(const uint8_t* __restrict__ w, int rows, int cols, int64_t row_bytes,
                          int chunk, const float* __restrict__ x, float* __restrict__ partial,
                          int q6_signed) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [RS][cols]
  const int U = cols >> 6;
  const int RS = kExpertThreads / U;
  const int t = threadIdx.x;
  const int u = t % U, slot = t / U;
  const int r0 = blockIdx.x * chunk;
  const int r1 = min(rows, r0 + chunk);
  float acc[1][64];
#pragma unroll
  for (int e = 0; e < 64; ++e) acc[0][e] = 0.f;
  float off[1][F::kOff];
#pragma unroll
  for (int k = 0; k < F::kOff; ++k) off[0][k] = 0.f;
  if (slot < RS) {
    for (int i = r0 + slot; i < r1; i += RS) {
      const float xi[1] = {x[i]};
      if (xi[0] == 0.f) continue;  // ops.rs:182-184
      F::template axpy<1>(w + int64_t(i) * row_bytes, u, xi, acc, off, q6_signed);
    }
    float* dst = red + slot * cols + 64 * u;
#pragma unroll
    for (int e = 0; e < 64; e += 4) {
      f32x4 v = {acc[0][e] - off[0][F::off_index(e)], acc[0][e + 1] - off[0][F::off_index(e + 1)],
                 acc[0][e + 2] - off[0][F::off_index(e + 2)], acc[0][e + 3] - off[0][F::off_index(e + 3)]};
      *reinterpret_cast<f32x4*>(dst + e) = v;
    }
  }
  __syncthreads();
  for (int c = t; c < cols; c += kExpertThreads) {
    float s = 0.f;
    for (int k = 0; k < RS; ++k) s += red[k * cols + c];
    partial[int64_t(blockIdx.x) * cols + c] = s;
  }
}

__global__ void sum_partials_kernel(const float* __restrict__ partial, int n_chunks, int cols,
                                    float* __restrict__ y) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int k = 0; k < n_chunks; ++k) s += partial[int64_t(k) * cols + c];
  y[c] = s;
}

bool expert_shape_ok(uint32_t quant, int64_t rows, int64_t cols) {
  if (!device_quant(quant) || rows <= 0 || cols <= 0) return false;
  if (cols % 64 != 0 || cols % geometry(quant).block != 0) return false;
  if (cols / 64 > kExpertThreads) return false;  // one thread per unit at least
  if (rows > (int64_t(1) << 31) - 1) return false;
  return true;
}

int expert_chunks(int64_t rows, int64_t cols) {
  const int U = int(cols / 64), RS = kExpertThreads / U;
  // enough row slots per chunk to amortise the reduction, at most 256 chunks
  int64_t chunk = int64_t(RS) * 4;
  int64_t n = (rows + chunk - 1) / chunk;
  if (n > 256) n = 256;
  return int(n);
}

size_t expert_workspace_bytes(int64_t rows, int64_t cols) {
  return size_t(expert_chunks(rows, cols)) * size_t(cols) * sizeof(float);
}

hipError_t launch_expert_gemv(uint32_t quant, const void* wv, int64_t rows, int64_t cols,
                              const float* x, float* y, float* workspace, int q6_signed,
                              hipStream_t stream) {
  if (!expert_shape_ok(quant, rows, cols)) return hipErrorInvalidValue;
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  if ((quant == kQ8_0 || quant == kIQ4_XS) && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
  const int64_t row_bytes = byte_size(quant, cols);
  const int n_chunks = expert_chunks(rows, cols);
  const int chunk = int((rows + n_chunks - 1) / n_chunks);
  const int U = int(cols / 64), RS = kExpertThreads / U;
  const size_t lds = size_t(RS) * size_t(cols) * sizeof(float);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  switch (quant) {
    case kQ4_K:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ4K>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    case kQ5_K:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ5K>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    case kQ8_0:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ8>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    case kIQ4_XS:  // the reading (reference or ggml qs bytes) is a template argument
      if (q6_signed)
        hipLaunchKernelGGL(expert_partial_kernel<AxIQ4XS<true>>, dim3(n_chunks), dim3(kExpertThreads), lds,
                           stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      else
        hipLaunchKernelGGL(expert_partial_kernel<AxIQ4XS<false>>, dim3(n_chunks), dim3(kExpertThreads), lds,
                           stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    case kQ6_K:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ6K>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    default:
      return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sum_partials_kernel, dim3(unsigned((cols + 255) / 256)), dim3(256), 0, stream,
                     workspace, n_chunks, int(cols), y);
  return hipGetLastError();
}

}  // namespace sh
