// The rest of ComputeBackend on the device: rms_norm, rope_neox, softmax,
// l2_norm and add (crates/strata-core/src/backend.rs:38-50), with the CPU
// bodies' arithmetic (crates/strata-core/src/ops.rs:46-165):
//   rms_norm   ss = sum v*v (f64) / n; scale = 1 / sqrt(ss + eps);
//              out = (f32)((f64)x * scale * (f64)w)
//   l2_norm    inv = 1 / sqrt(sum v*v + eps); v = (f32)((f64)v * inv)
//   softmax    mx = max (f32); e = expf(v - mx) (f32); sum e (f64);
//              v = (f32)((f64)e * (1 / sum))
//   rope_neox  r = min(n_rot, head_dim) & ~1; pair (i, i + r/2):
//              theta = base^(-2i/r), angle = theta * pos, a' = (f32)(a cos -
//              b sin), b' = (f32)(a sin + b cos), all f64
//   add        a += b (f32)
// Every operation is a separate rounding, as in the Rust source (contraction
// is off in this file). Only the order of the f64 sums differs (a butterfly
// over the lanes instead of a sequential loop), and pow / sin / cos are the
// device library's f64 functions, within an ulp of the platform libm's; the
// f32 exponential of softmax is the f64 one rounded to f32.
//
// Batched over rows: x is [rows][n] (rope: [rows][head_dim], each row one
// head). A workgroup of 256 threads takes four rows of at most 1024
// elements (a wave each) or one longer row (all four waves), so the many
// short rows of per-head work (qk norms, rope) fill the chip as well as the
// few long rows of per-token work. Rows of up to 8192 floats (n % 4 == 0,
// 16-byte aligned) are held in registers between the reduction and the
// write; longer or unaligned rows are streamed twice (three times for
// softmax) through L2.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

constexpr int kRowThreads = 256;
constexpr int64_t kShortRow = 1024;

// Sums over the 64 lanes by butterfly: every lane ends with the same bits
// (each step adds the same two operands in both lanes).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma clang fp contract(off)
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Row-wide reductions for W waves per row (W = 4: the whole workgroup, so
// every thread must call them).
template <int W>
__device__ __forceinline__ double row_sum(double v, double* lds) {
#pragma clang fp contract(off)
  v = wave_sum_f64(v);
  if constexpr (W == 1) {
    return v;
  } else {
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    const double t = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    __syncthreads();  // the slots are reused by the next reduction
    return t;
  }
}

template <int W>
__device__ __forceinline__ float row_max(float v, float* lds) {
  v = wave_max_f32(v);
  if constexpr (W == 1) {
    return v;
  } else {
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
    __syncthreads();
    return t;
  }
}

// This thread's row and its index within the row's 64 * W threads.
template <int W>
__device__ __forceinline__ int64_t row_of_thread(int& t) {
  if constexpr (W == 1) {
    t = threadIdx.x & 63;
    return int64_t(blockIdx.x) * (kRowThreads / 64) + (threadIdx.x >> 6);
  } else {
    t = threadIdx.x;
    return blockIdx.x;
  }
}

template <int W>
__global__ void __launch_bounds__(kRowThreads) rms_norm_kernel(const float* x,  // may be out itself
                                                               const float* __restrict__ w, float* out,
                                                               int64_t rows, int64_t n, double eps) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  constexpr int T = 64 * W;
  const float* xr = x + row * n;
  double ss = 0.0;
  for (int64_t i = t; i < n; i += T) {
    const double v = xr[i];
    ss += v * v;
  }
  ss = row_sum<W>(ss, lds);
  const double scale = 1.0 / sqrt(ss / double(n) + eps);
  float* o = out + row * n;
  for (int64_t i = t; i < n; i += T) o[i] = float(double(xr[i]) * scale * double(w[i]));
}

template <int W>
__global__ void __launch_bounds__(kRowThreads) l2_norm_kernel(float* x, int64_t rows, int64_t n, double eps) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  constexpr int T = 64 * W;
  float* xr = x + row * n;
  double ss = 0.0;
  for (int64_t i = t; i < n; i += T) {
    const double v = xr[i];
    ss += v * v;
  }
  ss = row_sum<W>(ss, lds);
  const double inv = 1.0 / sqrt(ss + eps);
  for (int64_t i = t; i < n; i += T) xr[i] = float(double(xr[i]) * inv);
}

template <int W>
__global__ void __launch_bounds__(kRowThreads) softmax_kernel(float* x, int64_t rows, int64_t n) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  __shared__ float ldm[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  constexpr int T = 64 * W;
  float* xr = x + row * n;
  float mx = -__builtin_inff();
  for (int64_t i = t; i < n; i += T) mx = fmaxf(mx, xr[i]);
  mx = row_max<W>(mx, ldm);
  double sum = 0.0;
  for (int64_t i = t; i < n; i += T) {
    // the f32 exponential as the f64 one rounded once: within 0.5 ulp + a
    // hair, as close to a correctly rounded expf as the platform libm's
    const float e = float(exp(double(xr[i] - mx)));
    xr[i] = e;
    sum += double(e);
  }
  sum = row_sum<W>(sum, lds);
  const double inv = 1.0 / sum;
  for (int64_t i = t; i < n; i += T) xr[i] = float(double(xr[i]) * inv);
}

// ---- register-resident rows ---------------------------------------------
// Rows of n % 4 == 0 floats at 16-byte aligned addresses, up to 8192 floats:
// each thread loads its V float4 slots once (all loads in flight together),
// reduces, and writes from registers, so a row costs one read and one write
// and a single memory latency. Padding slots (past the row) are masked.
template <int W, int V>
__device__ __forceinline__ void load_slots(const float* row, int64_t n4, int t, f32x4 (&v)[V], float pad) {
  const f32x4* p = reinterpret_cast<const f32x4*>(row);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t i = t + int64_t(k) * 64 * W;
    v[k] = i < n4 ? p[i] : f32x4{pad, pad, pad, pad};
  }
}

template <int V>
__device__ __forceinline__ double sum_squares(const f32x4 (&v)[V]) {
#pragma clang fp contract(off)
  double ss = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const double a = v[k].x, b = v[k].y, c = v[k].z, d = v[k].w;
    ss += a * a;
    ss += b * b;
    ss += c * c;
    ss += d * d;
  }
  return ss;
}

template <int W, int V>
__global__ void __launch_bounds__(kRowThreads) rms_norm_reg_kernel(const float* x, const float* __restrict__ w,
                                                                   float* out, int64_t rows, int64_t n,
                                                                   double eps) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  const int64_t n4 = n >> 2;
  f32x4 v[V], g[V];
  load_slots<W, V>(x + row * n, n4, t, v, 0.f);
  load_slots<W, V>(w, n4, t, g, 0.f);
  const double ss = row_sum<W>(sum_squares(v), lds);
  const double scale = 1.0 / sqrt(ss / double(n) + eps);
  f32x4* o = reinterpret_cast<f32x4*>(out + row * n);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t i = t + int64_t(k) * 64 * W;
    if (i < n4)
      o[i] = f32x4{float(double(v[k].x) * scale * double(g[k].x)), float(double(v[k].y) * scale * double(g[k].y)),
                   float(double(v[k].z) * scale * double(g[k].z)), float(double(v[k].w) * scale * double(g[k].w))};
  }
}

template <int W, int V>
__global__ void __launch_bounds__(kRowThreads) l2_norm_reg_kernel(float* x, int64_t rows, int64_t n, double eps) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  const int64_t n4 = n >> 2;
  f32x4 v[V];
  load_slots<W, V>(x + row * n, n4, t, v, 0.f);
  const double ss = row_sum<W>(sum_squares(v), lds);
  const double inv = 1.0 / sqrt(ss + eps);
  f32x4* o = reinterpret_cast<f32x4*>(x + row * n);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t i = t + int64_t(k) * 64 * W;
    if (i < n4)
      o[i] = f32x4{float(double(v[k].x) * inv), float(double(v[k].y) * inv), float(double(v[k].z) * inv),
                   float(double(v[k].w) * inv)};
  }
}

template <int W, int V>
__global__ void __launch_bounds__(kRowThreads) softmax_reg_kernel(float* x, int64_t rows, int64_t n) {
#pragma clang fp contract(off)
  __shared__ double lds[4];
  __shared__ float ldm[4];
  int t;
  const int64_t row = row_of_thread<W>(t);
  if (W == 1 && row >= rows) return;
  const int64_t n4 = n >> 2;
  f32x4 v[V];
  load_slots<W, V>(x + row * n, n4, t, v, -__builtin_inff());  // padding leaves the max alone
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < V; ++k) mx = fmaxf(fmaxf(fmaxf(mx, v[k].x), fmaxf(v[k].y, v[k].z)), v[k].w);
  mx = row_max<W>(mx, ldm);
  double sum = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (t + int64_t(k) * 64 * W < n4) {
      v[k].x = float(exp(double(v[k].x - mx)));
      v[k].y = float(exp(double(v[k].y - mx)));
      v[k].z = float(exp(double(v[k].z - mx)));
      v[k].w = float(exp(double(v[k].w - mx)));
      sum += double(v[k].x);
      sum += double(v[k].y);
      sum += double(v[k].z);
      sum += double(v[k].w);
    }
  }
  sum = row_sum<W>(sum, lds);
  const double inv = 1.0 / sum;
  f32x4* o = reinterpret_cast<f32x4*>(x + row * n);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t i = t + int64_t(k) * 64 * W;
    if (i < n4)
      o[i] = f32x4{float(double(v[k].x) * inv), float(double(v[k].y) * inv), float(double(v[k].z) * inv),
                   float(double(v[k].w) * inv)};
  }
}

// Calls f(W, V) with compile-time waves per row W and float4 slots per
// thread V for a register-resident row of n floats; false when n does not
// fit (then the streaming kernels above take the row).
template <int A>
using ic = std::integral_constant<int, A>;
template <class F>
static bool with_reg_shape(int64_t n, F&& f) {
  if (n <= kShortRow) {
    const int64_t per = (n / 4 + 63) / 64;
    if (per <= 1) f(ic<1>{}, ic<1>{});
    else if (per <= 2) f(ic<1>{}, ic<2>{});
    else f(ic<1>{}, ic<4>{});
    return true;
  }
  const int64_t per = (n / 4 + 255) / 256;
  if (per <= 2) f(ic<4>{}, ic<2>{});
  else if (per <= 4) f(ic<4>{}, ic<4>{});
  else if (per <= 8) f(ic<4>{}, ic<8>{});
  else return false;
  return true;
}

static bool vec_row(int64_t n, const void* a, const void* b = nullptr, const void* c = nullptr) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  return n % 4 == 0 && al(a) && al(b) && al(c);
}

// One thread per (row, pair); row r is at position pos0 + r / heads_per_pos.
__global__ void __launch_bounds__(kRowThreads) rope_neox_kernel(float* x, int64_t rows, int64_t head_dim, int r,
                                                                uint64_t pos0, int64_t heads_per_pos,
                                                                double freq_base) {
#pragma clang fp contract(off)
  const int half = r >> 1;
  const int64_t gid = int64_t(blockIdx.x) * kRowThreads + threadIdx.x;
  if (gid >= rows * half) return;
  const int64_t row = gid / half;
  const int i = int(gid - row * half);
  const double p = double(pos0 + uint64_t(row / heads_per_pos));
  const double theta = pow(freq_base, -2.0 * double(i) / double(r));
  const double angle = theta * p;
  const double s = sin(angle), c = cos(angle);
  float* h = x + row * head_dim;
  const double a = h[i], b = h[i + half];
  const double ac = a * c, bs = b * s, as = a * s, bc = b * c;
  h[i] = float(ac - bs);
  h[i + half] = float(as + bc);
}

__global__ void __launch_bounds__(kRowThreads) add_kernel(float* __restrict__ a, const float* __restrict__ b,
                                                          int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kRowThreads;
  int64_t i = int64_t(blockIdx.x) * kRowThreads + threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(a) & 15u) == 0 && (reinterpret_cast<uintptr_t>(b) & 15u) == 0) {
    const int64_t n4 = n >> 2;
    f32x4* a4 = reinterpret_cast<f32x4*>(a);
    const f32x4* b4 = reinterpret_cast<const f32x4*>(b);
    for (int64_t k = i; k < n4; k += stride) a4[k] = a4[k] + b4[k];
    for (int64_t k = 4 * n4 + i; k < n; k += stride) a[k] = a[k] + b[k];
  } else {
    for (int64_t k = i; k < n; k += stride) a[k] = a[k] + b[k];
  }
}

// out = a + b (f32), out distinct from b.
__global__ void __launch_bounds__(kRowThreads) add_out_kernel(float* out, const float* a, const float* __restrict__ b,
                                                              int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kRowThreads;
  for (int64_t k = int64_t(blockIdx.x) * kRowThreads + threadIdx.x; k < n; k += stride) out[k] = a[k] + b[k];
}

static unsigned row_blocks(int64_t rows, int64_t n) {
  return unsigned(n <= kShortRow ? (rows + 3) / 4 : rows);
}

bool rowops_shape_ok(int64_t rows, int64_t n) {
  // grids of at most 2^31 workgroups; row offsets stay in int64
  return rows >= 0 && n >= 0 && rows <= (int64_t(1) << 31) - 1 && n <= (int64_t(1) << 31) - 1 &&
         (n == 0 || rows <= (int64_t(1) << 62) / n);
}

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t n, double eps,
                           hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  if (vec_row(n, x, w, out) && with_reg_shape(n, [&](auto w_, auto v_) {
        constexpr int W = decltype(w_)::value, V = decltype(v_)::value;
        hipLaunchKernelGGL((rms_norm_reg_kernel<W, V>), dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, w,
                           out, rows, n, eps);
      }))
    return hipGetLastError();
  if (n <= kShortRow)
    hipLaunchKernelGGL(rms_norm_kernel<1>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, w, out, rows, n,
                       eps);
  else
    hipLaunchKernelGGL(rms_norm_kernel<4>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, w, out, rows, n,
                       eps);
  return hipGetLastError();
}

hipError_t launch_l2_norm(float* x, int64_t rows, int64_t n, double eps, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  if (vec_row(n, x) && with_reg_shape(n, [&](auto w_, auto v_) {
        constexpr int W = decltype(w_)::value, V = decltype(v_)::value;
        hipLaunchKernelGGL((l2_norm_reg_kernel<W, V>), dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows,
                           n, eps);
      }))
    return hipGetLastError();
  if (n <= kShortRow)
    hipLaunchKernelGGL(l2_norm_kernel<1>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows, n, eps);
  else
    hipLaunchKernelGGL(l2_norm_kernel<4>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows, n, eps);
  return hipGetLastError();
}

hipError_t launch_softmax(float* x, int64_t rows, int64_t n, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  if (vec_row(n, x) && with_reg_shape(n, [&](auto w_, auto v_) {
        constexpr int W = decltype(w_)::value, V = decltype(v_)::value;
        hipLaunchKernelGGL((softmax_reg_kernel<W, V>), dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows,
                           n);
      }))
    return hipGetLastError();
  if (n <= kShortRow)
    hipLaunchKernelGGL(softmax_kernel<1>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows, n);
  else
    hipLaunchKernelGGL(softmax_kernel<4>, dim3(row_blocks(rows, n)), dim3(kRowThreads), 0, s, x, rows, n);
  return hipGetLastError();
}

hipError_t launch_rope_neox(float* x, int64_t rows, int64_t head_dim, int64_t n_rot, uint64_t pos0,
                            int64_t heads_per_pos, double freq_base, hipStream_t s) {
  int64_t r = n_rot < head_dim ? n_rot : head_dim;
  r &= ~int64_t(1);
  if (rows == 0 || r == 0) return hipSuccess;
  if (r > (int64_t(1) << 30) || heads_per_pos <= 0) return hipErrorInvalidValue;
  const int64_t threads = rows * (r / 2);
  const int64_t blocks = (threads + kRowThreads - 1) / kRowThreads;
  if (blocks > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rope_neox_kernel, dim3(unsigned(blocks)), dim3(kRowThreads), 0, s, x, rows, head_dim, int(r),
                     pos0, heads_per_pos, freq_base);
  return hipGetLastError();
}

hipError_t launch_add(float* a, const float* b, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int64_t blocks = ((n + 3) / 4 + kRowThreads - 1) / kRowThreads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(add_kernel, dim3(unsigned(blocks)), dim3(kRowThreads), 0, s, a, b, n);
  return hipGetLastError();
}

hipError_t launch_add_out(float* out, const float* a, const float* b, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int64_t blocks = (n + kRowThreads - 1) / kRowThreads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(add_out_kernel, dim3(unsigned(blocks)), dim3(kRowThreads), 0, s, out, a, b, n);
  return hipGetLastError();
}

}  // namespace sh
