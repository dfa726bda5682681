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
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// Per-unit axpy for each format: acc[0..63] += coef * value and the offset
// terms per sub-block; 64 columns = one Q4_K group, one Q6_K quarter, or a
// pair of Q8_0 blocks (the same units as the matvec kernels).
struct AxQ4K {
  static constexpr int kOff = 2;
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, float xi, float* acc,
                                              float* off, int) {
    const uint8_t* sb = row + (u >> 2) * 144;
    const int g = u & 3;
    const u32x4 h = ld16(sb), a = ld16(sb + 16 + 32 * g), b = ld16(sb + 32 + 32 * g);
    const uint32_t sh = (g & 1) << 4;
    const uint32_t t1 = h.y >> sh, t2 = h.z >> sh, t3 = h.w >> sh;
    const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
    const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
    const float d = h2f(h.x), dm = h2f(h.x >> 16);
    const float c0 = xi * (d * ubyte<0>(scp));
    const float c1 = xi * (d * ubyte<1>(scp)) * 0.0625f;  // high nibbles read as 16 * q
    off[0] += xi * (dm * ubyte<0>(mp));
    off[1] += xi * (dm * ubyte<1>(mp));
    const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = q[k] & 0xF0F0F0F0u;
      acc[4 * k + 0] = __builtin_fmaf(c0, ubyte<0>(lo), acc[4 * k + 0]);
      acc[4 * k + 1] = __builtin_fmaf(c0, ubyte<1>(lo), acc[4 * k + 1]);
      acc[4 * k + 2] = __builtin_fmaf(c0, ubyte<2>(lo), acc[4 * k + 2]);
      acc[4 * k + 3] = __builtin_fmaf(c0, ubyte<3>(lo), acc[4 * k + 3]);
      acc[32 + 4 * k + 0] = __builtin_fmaf(c1, ubyte<0>(hi), acc[32 + 4 * k + 0]);
      acc[32 + 4 * k + 1] = __builtin_fmaf(c1, ubyte<1>(hi), acc[32 + 4 * k + 1]);
      acc[32 + 4 * k + 2] = __builtin_fmaf(c1, ubyte<2>(hi), acc[32 + 4 * k + 2]);
      acc[32 + 4 * k + 3] = __builtin_fmaf(c1, ubyte<3>(hi), acc[32 + 4 * k + 3]);
    }
  }
  // column e of the unit belongs to sub-block e / 32
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

struct AxQ8 {
  static constexpr int kOff = 2;
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, float xi, float* acc,
                                              float* off, int) {
    const uint8_t* p = row + u * 68;
    const u32x4 A = ld16(p), B = ld16(p + 16), C = ld16(p + 32), Dv = ld16(p + 48);
    const uint32_t E = ld4(p + 64);
    const uint32_t D[17] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w, C.x,
                            C.y, C.z, C.w, Dv.x, Dv.y, Dv.z, Dv.w, E};
    const float c0 = xi * h2f(D[0]), c1 = xi * h2f(D[8] >> 16);
    off[0] += 128.f * c0;
    off[1] += 128.f * c1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t q0 = realign(D[k], D[k + 1], 2) ^ 0x80808080u;
      const uint32_t q1 = D[9 + k] ^ 0x80808080u;
      acc[4 * k + 0] = __builtin_fmaf(c0, ubyte<0>(q0), acc[4 * k + 0]);
      acc[4 * k + 1] = __builtin_fmaf(c0, ubyte<1>(q0), acc[4 * k + 1]);
      acc[4 * k + 2] = __builtin_fmaf(c0, ubyte<2>(q0), acc[4 * k + 2]);
      acc[4 * k + 3] = __builtin_fmaf(c0, ubyte<3>(q0), acc[4 * k + 3]);
      acc[32 + 4 * k + 0] = __builtin_fmaf(c1, ubyte<0>(q1), acc[32 + 4 * k + 0]);
      acc[32 + 4 * k + 1] = __builtin_fmaf(c1, ubyte<1>(q1), acc[32 + 4 * k + 1]);
      acc[32 + 4 * k + 2] = __builtin_fmaf(c1, ubyte<2>(q1), acc[32 + 4 * k + 2]);
      acc[32 + 4 * k + 3] = __builtin_fmaf(c1, ubyte<3>(q1), acc[32 + 4 * k + 3]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

struct AxQ6K {
  static constexpr int kOff = 4;
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, float xi, float* acc,
                                              float* off, int q6_signed) {
    const uint8_t* blk = row + (u >> 2) * 210;
    const int j = u & 3, h = j >> 1;
    const uint32_t tp = uint32_t(j & 1);
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - s;
    const uint8_t* qlp = base + 64 * h;
    const u32x4 l0 = ld16(qlp), l1 = ld16(qlp + 16), l2 = ld16(qlp + 32), l3 = ld16(qlp + 48);
    const uint32_t l4 = ld4(qlp + 64);
    const uint8_t* qhp = base + 128 + 32 * h;
    const u32x4 h0 = ld16(qhp), h1 = ld16(qhp + 16);
    const uint32_t h2 = ld4(qhp + 32);
    const uint8_t* scp = base + 192 + 8 * h + 4 * tp;
    const uint32_t s0 = ld4(scp);
    const uint32_t s1 = s ? ld4(scp + 4) : 0u;
    const float d = h2f(*reinterpret_cast<const uint16_t*>(blk + 208));
    const uint32_t scw = realign(s0, s1, s);
    float sc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t byte = (scw >> (8 * k)) & 0xFFu;
      sc[k] = q6_signed ? float(int8_t(byte)) : float(byte);
    }
    float c[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      c[k] = xi * (d * sc[k]);
      off[k] += 32.f * c[k];
    }
    const uint32_t qlr[17] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w, l2.x,
                              l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w, l4};
    const uint32_t qhr[9] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w, h2};
    const uint32_t nib = 4u * tp;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t qh = realign(qhr[k], qhr[k + 1], s);
      const uint32_t qs = tp ? qh : (qh << 4);
      const uint32_t va = ((realign(qlr[k], qlr[k + 1], s) >> nib) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
      const uint32_t vb =
          ((realign(qlr[8 + k], qlr[9 + k], s) >> nib) & 0x0F0F0F0Fu) | ((qs >> 2) & 0x30303030u);
      const float ca = c[k >> 2], cb = c[2 + (k >> 2)];
      acc[4 * k + 0] = __builtin_fmaf(ca, ubyte<0>(va), acc[4 * k + 0]);
      acc[4 * k + 1] = __builtin_fmaf(ca, ubyte<1>(va), acc[4 * k + 1]);
      acc[4 * k + 2] = __builtin_fmaf(ca, ubyte<2>(va), acc[4 * k + 2]);
      acc[4 * k + 3] = __builtin_fmaf(ca, ubyte<3>(va), acc[4 * k + 3]);
      acc[32 + 4 * k + 0] = __builtin_fmaf(cb, ubyte<0>(vb), acc[32 + 4 * k + 0]);
      acc[32 + 4 * k + 1] = __builtin_fmaf(cb, ubyte<1>(vb), acc[32 + 4 * k + 1]);
      acc[32 + 4 * k + 2] = __builtin_fmaf(cb, ubyte<2>(vb), acc[32 + 4 * k + 2]);
      acc[32 + 4 * k + 3] = __builtin_fmaf(cb, ubyte<3>(vb), acc[32 + 4 * k + 3]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 4; }
};

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
  float acc[64];
#pragma unroll
  for (int e = 0; e < 64; ++e) acc[e] = 0.f;
  float off[F::kOff];
#pragma unroll
  for (int k = 0; k < F::kOff; ++k) off[k] = 0.f;
  if (slot < RS) {
    for (int i = r0 + slot; i < r1; i += RS) {
      const float xi = x[i];
      if (xi == 0.f) continue;  // ops.rs:182-184
      F::axpy(w + int64_t(i) * row_bytes, u, xi, acc, off, q6_signed);
    }
    float* dst = red + slot * cols + 64 * u;
#pragma unroll
    for (int e = 0; e < 64; e += 4) {
      f32x4 v = {acc[e] - off[F::off_index(e)], acc[e + 1] - off[F::off_index(e + 1)],
                 acc[e + 2] - off[F::off_index(e + 2)], acc[e + 3] - off[F::off_index(e + 3)]};
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
  if (quant == kQ8_0 && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
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
    case kQ8_0:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ8>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
      break;
    default:
      hipLaunchKernelGGL(expert_partial_kernel<AxQ6K>, dim3(n_chunks), dim3(kExpertThreads), lds,
                         stream, w, int(rows), int(cols), row_bytes, chunk, x, workspace, q6_signed);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sum_partials_kernel, dim3(unsigned((cols + 255) / 256)), dim3(256), 0, stream,
                     workspace, n_chunks, int(cols), y);
  return hipGetLastError();
}

}  // namespace sh
