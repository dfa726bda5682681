// The routed MoE FFN over out-major expert stacks.
//
// llama.cpp GGUF files store an expert stack as [n_expert][out][in] with the
// quant blocks along each row's input axis: gate / up [n_expert][n_ff]
// [n_embd], down [n_expert][n_embd][n_ff]. Each selected expert's product is
// then an ordinary matvec of its [out][in] slice (ops::gemv semantics,
// crates/strata-core/src/ops.rs:14-28), where the reference's own
// orientation (weights.rs:14-34, in-major) makes it ops::expert_gemv. The
// reference's GPU backend serves that orientation by transposing on upload
// (crates/strata-backend-wgpu/src/gpu.rs:287-303); here the packed rows are
// read in place.
//
// The route kernel, the work items (an expert's pairs two at a time), the
// pair tables and the combine are the in-major path's (moe.hip); only the
// two weight-streaming launches differ:
//   gate/up  workgroup (row block, matrix, item): rows [r0, r0 + rows) of
//            gate_e or up_e against the item's one or two token vectors,
//            staged in LDS with their per-16 sums; full dot products, so
//            each pair's h and p are written whole (one "chunk");
//   down     workgroup (row block, item): a = silu(h) * p staged for the
//            item's pairs (moe.rs:119-121), then rows of down_e against it.
// The vectors are staged per weight format for the most accurate dot: Q8_0
// against integer limbs (limb.hpp; exact per-block integer dots, free of the
// +128 code bias a float dot would cancel), the k-quants against the f32
// values themselves (fmt.hpp; their unsigned codes meet no such bias, and
// f32 x keeps the full 24 bits that limbs round to 22 below each block's
// maximum, which the silu(h) * p -> down -> weighted-sum chain amplifies
// where experts cancel). A row's 64-column units
// are spread over L lanes (L the power of two at or above the unit count, at
// most 64), so 64 / L rows share a wave and narrow rows (a 768-wide down
// input is 12 units) keep most lanes busy; the L lanes' sums are added with
// butterfly shuffles in a fixed order.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "fmt.hpp"
#include "kernels.hpp"
#include "limb.hpp"
#include "moe_items.hpp"

namespace sh {

constexpr int kOmThreads = 256;
constexpr int kOmWaves = kOmThreads / kWave;

// Q8_0 and IQ4_XS rows (signed codes) take limb activations; the k-quants
// f32 ones.
template <class F>
constexpr bool limb_x() {
  return std::is_same<F, LimbQ8>::value || std::is_same<F, LimbIQ4XS<false>>::value ||
         std::is_same<F, LimbIQ4XS<true>>::value;
}

// LDS bytes of one staged vector of `cols` values (either representation).
__host__ __device__ inline int om_vec_bytes(int cols) {
  return std::max(limb_lds_bytes(cols), int(sizeof(float)) * x_stride(cols));
}

// Stages nt vectors of `cols` values into LDS, vector t at lds + t *
// om_vec_bytes(cols); value(t, c) gives element c of vector t. Limbs: thread
// i converts 8-column group i (its quad of lanes holds one 32-column block,
// as limb_group8 needs; signed Q8_0 codes take the low-limb sums). f32: the
// x_stride layout with per-16 sums.
template <class F, class V>
__device__ __forceinline__ void stage_om(uint8_t* lds, int cols, int nt, V value) {
  const int vb = om_vec_bytes(cols);
  if constexpr (limb_x<F>()) {
    const int groups = cols / 8;  // a multiple of 4: whole quads are valid or not
    for (int t = 0; t < nt; ++t)
      for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = value(t, 8 * g + k);
        limb_group8<true>(lds + t * vb, cols, g, true, f32x4{v[0], v[1], v[2], v[3]},
                          f32x4{v[4], v[5], v[6], v[7]});
      }
  } else {
    const int groups = cols / 16;
    for (int i = threadIdx.x; i < nt * groups; i += blockDim.x) {
      const int t = i / groups, g = i - t * groups;
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = value(t, 16 * g + k);
      float* dst = reinterpret_cast<float*>(lds + t * vb);
      const int e0 = 16 * g;
      f32x4* d = reinterpret_cast<f32x4*>(dst + e0 + 4 * (e0 >> 6));
#pragma unroll
      for (int k = 0; k < 4; ++k) d[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
      // the sum in stage_x's order
      const float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])) +
                      (((v[8] + v[9]) + (v[10] + v[11])) + ((v[12] + v[13]) + (v[14] + v[15])));
      dst[cols + cols / 16 + g] = s;
    }
  }
}

template <class F>
struct OmX {
  using T = XSlice;
  __device__ static __forceinline__ void load(const uint8_t* lds, int cols, int u, T& o) {
    load_xslice(reinterpret_cast<const float*>(lds), cols, u, o);
  }
};
struct OmXLimbs {
  using T = XLimbs;
  __device__ static __forceinline__ void load(const uint8_t* lds, int cols, int u, T& o) {
    load_limbs(lds, cols, u, o);
  }
};
template <>
struct OmX<LimbQ8> : OmXLimbs {};
template <>
struct OmX<LimbIQ4XS<false>> : OmXLimbs {};
template <>
struct OmX<LimbIQ4XS<true>> : OmXLimbs {};

template <class F>
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, typename F::Load& ld) {
  if constexpr (limb_x<F>())
    F::load(row, F::offsets(u), ld);
  else
    F::load(row, u, ld);
}

// Rows [r0, r1) of one expert slice W (rows of `rb` bytes, `cols` inputs)
// against nt (<= NT) staged vectors: out_t[row] = W[row] . v_t.
// Rows at most 64 units wide (every lane one unit): the lane's x runs for
// all nt vectors stay in VGPRs, and the rows of the next passes are
// requested before the current one is computed. Wider rows loop over their
// units.
template <class F, int NT>
__device__ __forceinline__ void slice_rows(const uint8_t* __restrict__ W, int64_t rb, int cols, int r0, int r1,
                                           const uint8_t* xs, int nt, float* out0, float* out1, int q6) {
  using X = OmX<F>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int U = cols >> 6;
  int lg = 0;
  while ((1 << lg) < U && lg < 6) ++lg;
  const int L = 1 << lg, RW = kWave >> lg;  // lanes per row, rows per wave pass
  const int ul = lane & (L - 1), rr = lane >> lg;
  const int vb = om_vec_bytes(cols);
  const int step = kOmWaves * RW;
  auto finish = [&](float* acc, int row) {
    // the L lanes of a row, added in a fixed butterfly order
#pragma unroll
    for (int t = 0; t < NT; ++t)
      for (int off = L >> 1; off >= 1; off >>= 1) acc[t] += __shfl_xor(acc[t], off, kWave);
    if (row < r1 && ul == 0) {
      out0[row] = acc[0];
      if (NT > 1 && nt > 1) out1[row] = acc[NT - 1];
    }
  };
  if (U <= L) {
    // lanes past the row's units read a valid unit and discard it
    const int uc = min(ul, U - 1);
    const bool on = ul < U;
    typename X::T xv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < nt) X::load(xs + t * vb, cols, uc, xv[t]);
    auto row_ptr = [&](int base) { return W + int64_t(min(base + rr, r1 - 1)) * rb; };
    // a ring of D passes in flight (D from the size of a format's load, so
    // that two x runs and the ring stay within the VGPR budget)
    constexpr int D = sizeof(typename F::Load) <= 64 ? 4 : 2;
    typename F::Load ring[D];
    const int first = r0 + wave * RW;
#pragma unroll
    for (int k = 0; k < D; ++k)
      if (first + k * step < r1) load_unit<F>(row_ptr(first + k * step), uc, ring[k]);
    for (int base = first; base < r1; base += D * step) {
#pragma unroll
      for (int k = 0; k < D; ++k) {
        const int b = base + k * step;
        if (b < r1) {  // wave-uniform
          float acc[NT];
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t] = (t < nt && on) ? F::dot(ring[k], xv[t], uc, q6) : 0.f;
          finish(acc, b + rr);
          if (b + D * step < r1) load_unit<F>(row_ptr(b + D * step), uc, ring[k]);
        }
      }
    }
    return;
  }
  for (int base = r0 + wave * RW; base < r1; base += step) {
    const int row = base + rr;
    const uint8_t* wr = W + int64_t(min(row, r1 - 1)) * rb;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    for (int u = ul; u < U; u += L) {
      typename F::Load ld;
      load_unit<F>(wr, u, ld);
      // the unit's position in its super-block is u's (the limb formats
      // read it from their `lane` argument)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < nt) {
          typename X::T xt;
          X::load(xs + t * vb, cols, u, xt);
          acc[t] += F::dot(ld, xt, u, q6);
        }
      }
    }
    finish(acc, row);
  }
}

// Workgroup (row block b, matrix m: 0 gate / 1 up, work item s).
template <class F, int NT, bool ROUTE>
__global__ void __launch_bounds__(kOmThreads)
    moe_om_gateup_kernel(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, MoePlan plan,
                         const float* __restrict__ x, uint8_t* ws, int q6_gate, int q6_up,
                         const float* __restrict__ logits) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  const int b = blockIdx.x, m = blockIdx.y, s = blockIdx.z;
  MoeItem it;
  if (!moe_item<ROUTE>(plan, ws, logits, s, b == 0 && m == 0 && s == 0, it)) return;
  const int n_embd = plan.n_embd, n_ff = plan.n_ff;
  const int r0 = b * plan.om_rows_a, r1 = min(n_ff, r0 + plan.om_rows_a);
  const uint8_t* W = (m == 0 ? gate : up) + int64_t(it.e) * n_ff * plan.rb_a;
  float* part = reinterpret_cast<float*>(ws + plan.o_part_a);
  for (int j = 0; j < it.cnt; j += NT) {
    const int nt = min(NT, it.cnt - j);
    const int t0 = j == 0 ? it.tok0 : it.tok1;  // with NT == 1 the second pass takes the second token
    stage_om<F>(xs, n_embd, nt, [&](int t, int c) {
      return x[int64_t(t == 0 ? t0 : it.tok1) * n_embd + c];
    });
    __syncthreads();
    // part[(p * 2 + m) * n_ff + row]: one chunk
    float* o0 = part + (int64_t(it.p0 + j) * 2 + m) * n_ff;
    float* o1 = o0 + int64_t(2) * n_ff;
    slice_rows<F, NT>(W, plan.rb_a, n_embd, r0, r1, xs, nt, o0, o1, m == 0 ? q6_gate : q6_up);
    __syncthreads();
  }
}

// Workgroup (row block b, work item s): a = silu(h) * p for the item's
// pairs (h and p whole, from gate/up), then rows of down_e against it.
template <class F, int NT>
__global__ void __launch_bounds__(kOmThreads)
    moe_om_down_kernel(const uint8_t* __restrict__ down, MoePlan plan, uint8_t* ws, int q6_down) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  const int b = blockIdx.x, s = blockIdx.y;
  MoeItem it;
  if (!moe_item<false>(plan, ws, nullptr, s, false, it)) return;
  const int n_embd = plan.n_embd, n_ff = plan.n_ff;
  const int r0 = b * plan.om_rows_b, r1 = min(n_embd, r0 + plan.om_rows_b);
  const uint8_t* W = down + int64_t(it.e) * n_embd * plan.rb_b;
  const float* pa = reinterpret_cast<const float*>(ws + plan.o_part_a);
  float* part = reinterpret_cast<float*>(ws + plan.o_part_b);
  for (int j = 0; j < it.cnt; j += NT) {
    const int nt = min(NT, it.cnt - j);
    stage_om<F>(xs, n_ff, nt, [&](int t, int c) {
      const float* hp = pa + int64_t(it.p0 + j + t) * 2 * n_ff;
      const float h = hp[c], pv = hp[n_ff + c];
      return h / (1.f + expf(-h)) * pv;  // silu(h) * p (ops.rs:85-87, moe.rs:119-121)
    });
    __syncthreads();
    float* o0 = part + int64_t(it.p0 + j) * n_embd;  // part[p * n_embd + row]: one chunk
    float* o1 = o0 + n_embd;
    slice_rows<F, NT>(W, plan.rb_b, n_ff, r0, r1, xs, nt, o0, o1, q6_down);
    __syncthreads();
  }
}

// ------------------------------------------------------------------- host --
static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Rows per workgroup: about 1024 workgroups over the largest routing (s_max
// experts, `mats` matrices each), whole wave passes, at least one pass; 512
// when at most 8 experts are routed (one token): longer workgroups repeat
// the routing and the x staging less (1 token at 128 x 2048 x 768, top-8:
// 24.5 -> 23.0 us; 256 took 27.2 us, and 16 tokens run best at 1024).
static int om_rows(int rows, int cols, int mats, int s_max) {
  const int U = cols / 64;
  int L = 1;
  while (L < U && L < kWave) L <<= 1;
  const int pass = kOmWaves * (kWave / L);  // rows one pass of the workgroup covers
  const int target = s_max <= 8 ? 512 : 1024;
  const int per_matrix = std::max(1, target / (mats * s_max));
  int r = (rows + per_matrix - 1) / per_matrix;
  r = (r + pass - 1) / pass * pass;
  return std::max(r, pass);
}

bool moe_plan_out_major(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, uint32_t qa, uint32_t qb,
                        MoePlan* plan) {
  // gate / up rows are n_embd wide, down rows n_ff: whole 64-column units
  // of whole blocks, and the staged vectors fit LDS
  if (!device_quant(qa) || !device_quant(qb)) return false;
  if (n_embd % 64 != 0 || n_embd % geometry(qa).block != 0) return false;
  if (n_ff % 64 != 0 || n_ff % geometry(qb).block != 0) return false;
  if (n_embd > 8192 || n_ff > 8192) return false;
  MoePlan p{};
  p.out_major = true;
  p.n_tok = n_tok;
  p.top_k = top_k;
  p.n_expert = n_expert;
  p.n_embd = n_embd;
  p.n_ff = n_ff;
  p.rb_a = byte_size(qa, n_embd);
  p.rb_b = byte_size(qb, n_ff);
  const int pairs = n_tok * top_k;
  p.s_max = pairs < n_expert ? pairs : n_expert;
  p.z_max = (pairs + p.s_max + 1) / 2;
  p.nch_a = p.nch_b = 1;  // whole dot products: one chunk each
  p.om_rows_a = om_rows(n_ff, n_embd, 2, p.s_max);
  p.om_rows_b = om_rows(n_embd, n_ff, 1, p.s_max);
  const int nt = n_tok > 1 ? 2 : 1;
  p.lds_a = size_t(nt) * om_vec_bytes(n_embd);
  p.lds_b = size_t(nt) * om_vec_bytes(n_ff);
  if (p.lds_a > 160 * 1024 || p.lds_b > 160 * 1024) return false;
  p.route_lds = size_t(pairs) * 12;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  p.o_ids = take(sizeof(int) * pairs);
  p.o_wts = take(sizeof(float) * pairs);
  p.o_meta = take(sizeof(int) * 4);
  p.o_item_e = take(sizeof(int) * p.z_max);
  p.o_item_off = take(sizeof(int) * p.z_max);
  p.o_item_cnt = take(sizeof(int) * p.z_max);
  p.o_item_tok = take(sizeof(int) * 2 * p.z_max);
  p.o_tokpair = take(sizeof(int) * pairs);
  p.o_part_a = take(sizeof(float) * size_t(pairs) * 2 * n_ff);
  p.o_part_b = take(sizeof(float) * size_t(pairs) * n_embd);
  p.bytes = o;
  *plan = p;
  return true;
}

template <class F>
static void launch_om_gateup(const MoePlan& p, const void* gate, const void* up, const float* x, uint8_t* ws,
                             int q6g, int q6u, const float* logits, bool route, hipStream_t s) {
  const dim3 g(unsigned((p.n_ff + p.om_rows_a - 1) / p.om_rows_a), 2, p.z_max), b(kOmThreads);
  const uint8_t *gp = static_cast<const uint8_t*>(gate), *upp = static_cast<const uint8_t*>(up);
  if (route)
    hipLaunchKernelGGL((moe_om_gateup_kernel<F, 1, true>), g, b, p.lds_a, s, gp, upp, p, x, ws, q6g, q6u, logits);
  else if (p.n_tok == 1)
    hipLaunchKernelGGL((moe_om_gateup_kernel<F, 1, false>), g, b, p.lds_a, s, gp, upp, p, x, ws, q6g, q6u, logits);
  else
    hipLaunchKernelGGL((moe_om_gateup_kernel<F, 2, false>), g, b, p.lds_a, s, gp, upp, p, x, ws, q6g, q6u, logits);
}

template <class F>
static void launch_om_down(const MoePlan& p, const void* down, uint8_t* ws, int q6d, hipStream_t s) {
  const dim3 g(unsigned((p.n_embd + p.om_rows_b - 1) / p.om_rows_b), p.z_max), b(kOmThreads);
  const uint8_t* dp = static_cast<const uint8_t*>(down);
  if (p.n_tok == 1)
    hipLaunchKernelGGL((moe_om_down_kernel<F, 1>), g, b, p.lds_b, s, dp, p, ws, q6d);
  else
    hipLaunchKernelGGL((moe_om_down_kernel<F, 2>), g, b, p.lds_b, s, dp, p, ws, q6d);
}

void launch_moe_out_major(const MoePlan& p, uint32_t qg, uint32_t qd, const void* gate, const void* up,
                          const void* down, int q6g, int q6u, int q6d, const float* logits, const float* x,
                          void* workspace, bool fused_route, hipStream_t s) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  switch (qg) {
    case kQ4_K: launch_om_gateup<FmtQ4K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ5_K: launch_om_gateup<FmtQ5K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ8_0: launch_om_gateup<LimbQ8>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ6_K: launch_om_gateup<FmtQ6K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    default:  // kIQ4_XS: gate and up of one reading (checked by the caller)
      if (q6g) launch_om_gateup<LimbIQ4XS<true>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
      else launch_om_gateup<LimbIQ4XS<false>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
  }
  switch (qd) {
    case kQ4_K: launch_om_down<FmtQ4K>(p, down, ws, q6d, s); break;
    case kQ5_K: launch_om_down<FmtQ5K>(p, down, ws, q6d, s); break;
    case kQ8_0: launch_om_down<LimbQ8>(p, down, ws, q6d, s); break;
    case kQ6_K: launch_om_down<FmtQ6K>(p, down, ws, q6d, s); break;
    default:  // kIQ4_XS
      if (q6d) launch_om_down<LimbIQ4XS<true>>(p, down, ws, q6d, s);
      else launch_om_down<LimbIQ4XS<false>>(p, down, ws, q6d, s);
  }
}

}  // namespace sh
