// Routed mixture-of-experts FFN on the device.
//
// Semantics: crates/strata-core/src/moe.rs:48-127, routed part, starting from
// the router logits:
//   route   softmax over all experts (max-shifted, f32 exp, f64 sum,
//           inv = f32(1/sum), p *= inv), top-k by descending probability with
//           ties to the lower id, ids ascending, weights
//           f32(f64(p) / max(sum_f64(p), 2^-14)) (moe.rs:58-90);
//   combine for each selected expert in ascending id order with w != 0:
//           h = gate_e . x, p = up_e . x, h = silu(h) * p, d = down_e . h,
//           out += w * d (moe.rs:108-127).
// Expert tensors are in the reference orientation [n_expert][in][out]
// (crates/strata-core/src/weights.rs:14-34). The shared expert
// (moe.rs:129-143) is not part of this op.
//
// Four launches:
//   route    one workgroup routes every token and groups the (token, expert)
//            pairs by expert: the unique experts in ascending id order are
//            "slots", each with its tokens in ascending order ("pairs");
//   gate/up  workgroup (slot, matrix, row chunk) streams that expert's rows
//            once for all of the slot's tokens (one at a time; the repeat of
//            a chunk hits in L2) and writes one partial sum per pair;
//   down     workgroup (slot, row chunk) forms a = silu(h) * p for its rows
//            and the slot's tokens in LDS, then streams the down rows;
//   combine  out[t] = sum over t's experts in ascending id of w * d.
// Weight bytes cross HBM once per unique expert, however many tokens chose it.
#include "axpy.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

constexpr int kMoeThreads = 256;
constexpr int kMoeTok = 1;  // tokens sharing one decoded weight row (a chunk re-read for the next token hits in L2)

// ------------------------------------------------------------------ route --
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__global__ void __launch_bounds__(kMoeThreads) moe_route_kernel(const float* __restrict__ logits,
                                                                MoePlan plan, uint8_t* ws) {
  __shared__ int cnt[kMoeMaxExperts];
  __shared__ int eslot[kMoeMaxExperts];
  __shared__ int sel_id[kMoeThreads / kWave][kMoeMaxTopK];
  __shared__ float sel_p[kMoeThreads / kWave][kMoeMaxTopK];
  __shared__ int wave_nz[kMoeThreads / kWave], wave_sum[kMoeThreads / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = plan.n_expert, K = plan.top_k;
  int* ids = reinterpret_cast<int*>(ws + plan.o_ids);
  float* wts = reinterpret_cast<float*>(ws + plan.o_wts);
  constexpr int kPer = kMoeMaxExperts / kWave;  // experts per lane

  for (int t = wave; t < plan.n_tok; t += kMoeThreads / kWave) {
    const float* lg = logits + int64_t(t) * E;
    float p[kPer];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + kWave * j;
      p[j] = e < E ? lg[e] : -__builtin_inff();
      mx = fmaxf(mx, p[j]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + kWave * j;
      if (e < E) {
        p[j] = expf(p[j] - mx);
        sum += double(p[j]);
      }
    }
    sum = wave_sum_f64(sum);
    const float inv = float(1.0 / sum);
#pragma unroll
    for (int j = 0; j < kPer; ++j) p[j] *= inv;
    // top-k: k rounds of (largest p, then lowest id) over what is left
    uint32_t taken = 0;
    for (int r = 0; r < K; ++r) {
      // a NaN probability ranks below every number, so each round always
      // picks a valid id (k <= n_expert)
      float bp = -2.f;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = lane + kWave * j;
        const float pj = p[j] == p[j] ? p[j] : -1.f;
        if (e < E && !(taken >> j & 1u) && (pj > bp || (pj == bp && e < bi))) {
          bp = pj;
          bi = e;
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float op = __shfl_xor(bp, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (op > bp || (op == bp && oi < bi)) {
          bp = op;
          bi = oi;
        }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      if (lane == 0) {
        sel_id[wave][r] = bi;
        sel_p[wave][r] = bp;
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      // ids ascending (insertion sort of k <= 32), then the f64 renormalisation
      for (int a = 1; a < K; ++a) {
        const int id = sel_id[wave][a];
        const float pv = sel_p[wave][a];
        int b = a - 1;
        while (b >= 0 && sel_id[wave][b] > id) {
          sel_id[wave][b + 1] = sel_id[wave][b];
          sel_p[wave][b + 1] = sel_p[wave][b];
          --b;
        }
        sel_id[wave][b + 1] = id;
        sel_p[wave][b + 1] = pv;
      }
      double wsum = 0.0;
      for (int a = 0; a < K; ++a) wsum += double(sel_p[wave][a]);
      const double s = wsum > 6.103515625e-05 ? wsum : 6.103515625e-05;  // 2^-14
      for (int a = 0; a < K; ++a) {
        ids[t * K + a] = sel_id[wave][a];
        wts[t * K + a] = float(double(sel_p[wave][a]) / s);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();

  // group the pairs by expert: counts, then an exclusive scan over experts
  for (int e = tid; e < kMoeMaxExperts; e += kMoeThreads) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < plan.n_tok * K; i += kMoeThreads) atomicAdd(&cnt[ids[i]], 1);
  __syncthreads();
  constexpr int kEper = kMoeMaxExperts / kMoeThreads;  // experts per thread
  int nz = 0, tot = 0;
#pragma unroll
  for (int j = 0; j < kEper; ++j) {
    const int c = cnt[tid * kEper + j];
    nz += c > 0;
    tot += c;
  }
  // inclusive scans of (nz, tot) within the wave, then across waves
  int snz = nz, stot = tot;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int a = __shfl_up(snz, off, kWave), b = __shfl_up(stot, off, kWave);
    if (lane >= off) {
      snz += a;
      stot += b;
    }
  }
  if (lane == 63) {
    wave_nz[wave] = snz;
    wave_sum[wave] = stot;
  }
  __syncthreads();
  int base_nz = 0, base_tot = 0;
  for (int w2 = 0; w2 < wave; ++w2) {
    base_nz += wave_nz[w2];
    base_tot += wave_sum[w2];
  }
  int slot = base_nz + snz - nz, pos = base_tot + stot - tot;
  int* slot_e = reinterpret_cast<int*>(ws + plan.o_slot_e);
  int* slot_off = reinterpret_cast<int*>(ws + plan.o_slot_off);
  int* slot_cnt = reinterpret_cast<int*>(ws + plan.o_slot_cnt);
#pragma unroll
  for (int j = 0; j < kEper; ++j) {
    const int e = tid * kEper + j;
    const int c = cnt[e];
    if (c > 0) {
      slot_e[slot] = e;
      slot_off[slot] = pos;
      slot_cnt[slot] = c;
      eslot[e] = slot;
      ++slot;
      pos += c;
    }
  }
  if (tid == kMoeThreads - 1) reinterpret_cast<int*>(ws + plan.o_meta)[0] = slot;
  __syncthreads();
  // pairs of each expert in ascending token order
  int* pair_tok = reinterpret_cast<int*>(ws + plan.o_pair_tok);
  float* pair_w = reinterpret_cast<float*>(ws + plan.o_pair_w);
  int* tokpair = reinterpret_cast<int*>(ws + plan.o_tokpair);
  for (int e = tid; e < E; e += kMoeThreads) {
    if (cnt[e] == 0) continue;
    const int s = eslot[e];
    int p = slot_off[s];
    for (int t = 0; t < plan.n_tok; ++t)
      for (int a = 0; a < K; ++a)
        if (ids[t * K + a] == e) {
          pair_tok[p] = t;
          pair_w[p] = wts[t * K + a];
          tokpair[t * K + a] = p;
          ++p;
        }
  }
}

// Column sums of one row chunk for `nt` tokens, reduced over the workgroup's
// row slots through LDS and written to dst[t * cols + c].
template <class F>
__device__ __forceinline__ void chunk_axpy(const uint8_t* w, int64_t row_bytes, int cols, int r0,
                                           int r1, const float* const* xs, int xoff, int nt,
                                           float* red, float* dst, int64_t dst_stride, int q6_signed) {
  const int U = cols >> 6;
  const int RS = kMoeThreads / U;
  const int tid = threadIdx.x;
  const int u = tid % U, slot = tid / U;
  float acc[kMoeTok][64];
  float off[kMoeTok][F::kOff];
#pragma unroll
  for (int t = 0; t < kMoeTok; ++t) {
#pragma unroll
    for (int e = 0; e < 64; ++e) acc[t][e] = 0.f;
#pragma unroll
    for (int k = 0; k < F::kOff; ++k) off[t][k] = 0.f;
  }
  if (slot < RS) {
    for (int i = r0 + slot; i < r1; i += RS) {
      float xi[kMoeTok];
#pragma unroll
      for (int t = 0; t < kMoeTok; ++t) xi[t] = t < nt ? xs[t][i - xoff] : 0.f;
      F::template axpy<kMoeTok>(w + int64_t(i) * row_bytes, u, xi, acc, off, q6_signed);
    }
  }
  for (int t = 0; t < nt; ++t) {
    if (slot < RS) {
      float* d = red + slot * cols + 64 * u;
#pragma unroll
      for (int e = 0; e < 64; e += 4)
        *reinterpret_cast<f32x4*>(d + e) =
            f32x4{acc[t][e] - off[t][F::off_index(e)], acc[t][e + 1] - off[t][F::off_index(e + 1)],
                  acc[t][e + 2] - off[t][F::off_index(e + 2)], acc[t][e + 3] - off[t][F::off_index(e + 3)]};
    }
    __syncthreads();
    for (int c = tid; c < cols; c += kMoeThreads) {
      float s = 0.f;
      for (int k = 0; k < RS; ++k) s += red[k * cols + c];
      dst[int64_t(t) * dst_stride + c] = s;
    }
    __syncthreads();
  }
}

// -------------------------------------------------------------- gate / up --
template <class F>
__global__ void __launch_bounds__(kMoeThreads)
    moe_gateup_kernel(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, MoePlan plan,
                      const float* __restrict__ x, uint8_t* ws, int q6_gate, int q6_up) {
  extern __shared__ __attribute__((aligned(16))) float red[];
  const int s = blockIdx.x, m = blockIdx.y, c = blockIdx.z;
  const int n_slots = reinterpret_cast<const int*>(ws + plan.o_meta)[0];
  if (s >= n_slots) return;
  const int e = reinterpret_cast<const int*>(ws + plan.o_slot_e)[s];
  const int p0 = reinterpret_cast<const int*>(ws + plan.o_slot_off)[s];
  const int cnt = reinterpret_cast<const int*>(ws + plan.o_slot_cnt)[s];
  const int* pair_tok = reinterpret_cast<const int*>(ws + plan.o_pair_tok);
  const int64_t rb = plan.rb_a;
  const uint8_t* w = (m == 0 ? gate : up) + int64_t(e) * plan.n_embd * rb;
  const int r0 = c * plan.chunk_a, r1 = min(plan.n_embd, r0 + plan.chunk_a);
  float* part = reinterpret_cast<float*>(ws + plan.o_part_a);
  for (int tg = 0; tg < cnt; tg += kMoeTok) {
    const int nt = min(kMoeTok, cnt - tg);
    const float* xs[kMoeTok];
#pragma unroll
    for (int t = 0; t < kMoeTok; ++t) xs[t] = x + int64_t(pair_tok[p0 + tg + (t < nt ? t : 0)]) * plan.n_embd;
    // partial sums of pair p: part[((p * 2 + m) * nch_a + c) * n_ff + col]
    float* dst = part + ((int64_t(p0 + tg) * 2 + m) * plan.nch_a + c) * plan.n_ff;
    chunk_axpy<F>(w, rb, plan.n_ff, r0, r1, xs, 0, nt, red, dst, int64_t(2) * plan.nch_a * plan.n_ff,
                  m == 0 ? q6_gate : q6_up);
  }
}

// ------------------------------------------------------------------- down --
template <class F>
__global__ void __launch_bounds__(kMoeThreads)
    moe_down_kernel(const uint8_t* __restrict__ down, MoePlan plan, uint8_t* ws, int q6_down) {
  extern __shared__ __attribute__((aligned(16))) float red[];
  const int s = blockIdx.x, c = blockIdx.y;
  const int n_slots = reinterpret_cast<const int*>(ws + plan.o_meta)[0];
  if (s >= n_slots) return;
  const int e = reinterpret_cast<const int*>(ws + plan.o_slot_e)[s];
  const int p0 = reinterpret_cast<const int*>(ws + plan.o_slot_off)[s];
  const int cnt = reinterpret_cast<const int*>(ws + plan.o_slot_cnt)[s];
  const int r0 = c * plan.chunk_b, r1 = min(plan.n_ff, r0 + plan.chunk_b);
  const int nr = r1 - r0;
  // a = silu(h) * p for this chunk's rows and every token of the slot
  // (moe.rs:119-121), from the gate/up partials summed in chunk order
  float* a = red + kMoeThreads / (plan.n_embd >> 6) * plan.n_embd;  // after the reduction area
  const float* part = reinterpret_cast<const float*>(ws + plan.o_part_a);
  for (int idx = threadIdx.x; idx < cnt * nr; idx += kMoeThreads) {
    const int t = idx / nr, i = r0 + idx % nr;
    const float* hp = part + (int64_t(p0 + t) * 2 * plan.nch_a) * plan.n_ff + i;
    float h = 0.f, pv = 0.f;
    for (int k = 0; k < plan.nch_a; ++k) {
      h += hp[int64_t(k) * plan.n_ff];
      pv += hp[int64_t(plan.nch_a + k) * plan.n_ff];
    }
    a[t * nr + (i - r0)] = h / (1.f + expf(-h)) * pv;  // ops.rs:85-87
  }
  __syncthreads();
  const int64_t rb = plan.rb_b;
  const uint8_t* w = down + int64_t(e) * plan.n_ff * rb;
  float* out = reinterpret_cast<float*>(ws + plan.o_part_b);
  for (int tg = 0; tg < cnt; tg += kMoeTok) {
    const int nt = min(kMoeTok, cnt - tg);
    const float* xs[kMoeTok];
#pragma unroll
    for (int t = 0; t < kMoeTok; ++t) xs[t] = a + (tg + (t < nt ? t : 0)) * nr;
    // partial sums of pair p: out[(p * nch_b + c) * n_embd + col]
    float* dst = out + (int64_t(p0 + tg) * plan.nch_b + c) * plan.n_embd;
    chunk_axpy<F>(w, rb, plan.n_embd, r0, r1, xs, r0, nt, red, dst, int64_t(plan.nch_b) * plan.n_embd,
                  q6_down);
  }
}

// ---------------------------------------------------------------- combine --
__global__ void moe_combine_kernel(MoePlan plan, const uint8_t* ws, float* __restrict__ out) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= int64_t(plan.n_tok) * plan.n_embd) return;
  const int t = int(i / plan.n_embd), col = int(i - int64_t(t) * plan.n_embd);
  const int* tokpair = reinterpret_cast<const int*>(ws + plan.o_tokpair);
  const float* wts = reinterpret_cast<const float*>(ws + plan.o_wts);
  const float* part = reinterpret_cast<const float*>(ws + plan.o_part_b);
  float acc = 0.f;
  for (int a = 0; a < plan.top_k; ++a) {
    const float wv = wts[t * plan.top_k + a];
    if (wv == 0.f) continue;  // moe.rs:112-114
    const int p = tokpair[t * plan.top_k + a];
    float d = 0.f;
    for (int k = 0; k < plan.nch_b; ++k) d += part[(int64_t(p) * plan.nch_b + k) * plan.n_embd + col];
    acc = __fadd_rn(acc, __fmul_rn(wv, d));  // out += w * d, product then sum
  }
  out[i] = acc;
}

// ------------------------------------------------------------------- host --
static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

bool moe_plan(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, uint32_t qa, uint32_t qb,
              MoePlan* plan) {
  if (n_tok <= 0 || top_k <= 0 || top_k > kMoeMaxTopK || top_k > n_expert ||
      n_expert > kMoeMaxExperts || n_embd <= 0 || n_ff <= 0)
    return false;
  if (!expert_shape_ok(qa, n_embd, n_ff) || !expert_shape_ok(qb, n_ff, n_embd)) return false;
  if (n_tok > kMoeMaxTokens) return false;
  MoePlan p{};
  p.n_tok = n_tok;
  p.top_k = top_k;
  p.n_expert = n_expert;
  p.n_embd = n_embd;
  p.n_ff = n_ff;
  p.rb_a = byte_size(qa, n_ff);
  p.rb_b = byte_size(qb, n_embd);
  const int pairs = n_tok * top_k;
  p.s_max = pairs < n_expert ? pairs : n_expert;
  // row chunks: about 128 rows per gate/up chunk and 48 per down chunk,
  // enough workgroups to cover the chip even for a single token
  p.nch_a = (n_embd + 127) / 128;
  if (p.nch_a > 32) p.nch_a = 32;
  p.chunk_a = (n_embd + p.nch_a - 1) / p.nch_a;
  p.nch_b = (n_ff + 47) / 48;
  if (p.nch_b > 32) p.nch_b = 32;
  p.chunk_b = (n_ff + p.nch_b - 1) / p.nch_b;
  // the down kernel keeps its reduction rows and a = silu(h) * p for every
  // token of a slot in LDS
  const size_t lds_b = (size_t(kMoeThreads / (n_embd >> 6)) * n_embd + size_t(n_tok) * p.chunk_b) * 4;
  if (lds_b > 160 * 1024) return false;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  p.o_ids = take(sizeof(int) * pairs);
  p.o_wts = take(sizeof(float) * pairs);
  p.o_meta = take(sizeof(int) * 4);
  p.o_slot_e = take(sizeof(int) * p.s_max);
  p.o_slot_off = take(sizeof(int) * p.s_max);
  p.o_slot_cnt = take(sizeof(int) * p.s_max);
  p.o_pair_tok = take(sizeof(int) * pairs);
  p.o_pair_w = take(sizeof(float) * pairs);
  p.o_tokpair = take(sizeof(int) * pairs);
  p.o_part_a = take(sizeof(float) * size_t(pairs) * 2 * p.nch_a * n_ff);
  p.o_part_b = take(sizeof(float) * size_t(pairs) * p.nch_b * n_embd);
  p.bytes = o;
  *plan = p;
  return true;
}

template <class FA>
static void launch_gateup(const MoePlan& p, const void* gate, const void* up, const float* x,
                          uint8_t* ws, int q6g, int q6u, hipStream_t s) {
  const size_t lds = size_t(kMoeThreads / (p.n_ff >> 6)) * p.n_ff * sizeof(float);
  hipLaunchKernelGGL(moe_gateup_kernel<FA>, dim3(p.s_max, 2, p.nch_a), dim3(kMoeThreads), lds, s,
                     static_cast<const uint8_t*>(gate), static_cast<const uint8_t*>(up), p, x, ws, q6g,
                     q6u);
}

template <class FB>
static void launch_down(const MoePlan& p, const void* down, uint8_t* ws, int q6d, hipStream_t s) {
  const size_t lds = (size_t(kMoeThreads / (p.n_embd >> 6)) * p.n_embd +
                      size_t(p.n_tok) * p.chunk_b) *
                     sizeof(float);
  hipLaunchKernelGGL(moe_down_kernel<FB>, dim3(p.s_max, p.nch_b), dim3(kMoeThreads), lds, s,
                     static_cast<const uint8_t*>(down), p, ws, q6d);
}

hipError_t launch_moe(const MoePlan& p, uint32_t qg, uint32_t qu, uint32_t qd, const void* gate,
                      const void* up, const void* down, int q6g, int q6u, int q6d,
                      const float* logits, const float* x, float* out, void* workspace,
                      hipStream_t s) {
  if (qg != qu) return hipErrorInvalidValue;  // gate and up share one kernel
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kMoeThreads), 0, s, logits, p, ws);
  switch (qg) {
    case kQ4_K: launch_gateup<AxQ4K>(p, gate, up, x, ws, q6g, q6u, s); break;
    case kQ8_0: launch_gateup<AxQ8>(p, gate, up, x, ws, q6g, q6u, s); break;
    default: launch_gateup<AxQ6K>(p, gate, up, x, ws, q6g, q6u, s);
  }
  switch (qd) {
    case kQ4_K: launch_down<AxQ4K>(p, down, ws, q6d, s); break;
    case kQ8_0: launch_down<AxQ8>(p, down, ws, q6d, s); break;
    default: launch_down<AxQ6K>(p, down, ws, q6d, s);
  }
  const int64_t n = int64_t(p.n_tok) * p.n_embd;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, p, ws, out);
  return hipGetLastError();
}

// Routing alone (for the host-slice sh_moe_route): ids and weights per token.
hipError_t launch_moe_route(const MoePlan& p, const float* logits, void* workspace, hipStream_t s) {
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kMoeThreads), 0, s, logits, p,
                     static_cast<uint8_t*>(workspace));
  return hipGetLastError();
}

}  // namespace sh
