// Routing helpers and the work-item lookup shared by the MoE kernels of
// both expert-stack orientations (moe.hip, moe_om.hip).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// ------------------------------------------------------------------ route --
// Wave-wide max / min through DPP (quad swaps, row mirrors, row
// broadcasts; lane 63 ends with the result), returned to every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  const int id = __builtin_bit_cast(int, -__builtin_inff());
#define SH_DPP_MAX(ctrl, rm) \
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), ctrl, rm, 0xF, false)))
  SH_DPP_MAX(0xB1, 0xF);
  SH_DPP_MAX(0x4E, 0xF);
  SH_DPP_MAX(0x141, 0xF);
  SH_DPP_MAX(0x140, 0xF);
  SH_DPP_MAX(0x142, 0xA);
  SH_DPP_MAX(0x143, 0xC);
#undef SH_DPP_MAX
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ int wave_min_dpp(int v) {
#define SH_DPP_MIN(ctrl, rm) v = min(v, __builtin_amdgcn_update_dpp(0x7FFFFFFF, v, ctrl, rm, 0xF, false))
  SH_DPP_MIN(0xB1, 0xF);
  SH_DPP_MIN(0x4E, 0xF);
  SH_DPP_MIN(0x141, 0xF);
  SH_DPP_MIN(0x140, 0xF);
  SH_DPP_MIN(0x142, 0xA);
  SH_DPP_MIN(0x143, 0xC);
#undef SH_DPP_MIN
  return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Routes one token with one wave (moe.rs:58-90): max-shifted softmax (f32 exp,
// f64 sum, inv = f32(1 / sum)), k rounds of (largest probability, then lowest
// id), ids sorted ascending, weights f32(f64(p) / max(sum_f64(p), 2^-14)).
// sel_id / sel_p are the wave's LDS scratch (kMoeMaxTopK entries); on return
// they hold the ids ascending and their probabilities, and lane a < K holds
// id sel_id[a] and its weight in id_out, w_out. KPER experts per lane, with
// KPER * 64 >= E (a larger KPER gives the same result: experts past E are
// skipped everywhere).
template <int KPER>
__device__ __forceinline__ void route_token(const float* __restrict__ lg, int E, int K, int lane, int* sel_id,
                                            float* sel_p, int& id_out, float& w_out) {
  constexpr int kPer = KPER;
  float p[KPER];
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
  // top-k: k rounds of (largest p, then lowest id) over what is left; a
  // NaN probability ranks below every number, so each round picks a valid
  // id (k <= n_expert)
  uint32_t taken = 0;
  for (int r = 0; r < K; ++r) {
    // exact: the largest remaining probability, then the lowest id holding it
    float bp = -2.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + kWave * j;
      const float pj = p[j] == p[j] ? p[j] : -1.f;
      if (e < E && !(taken >> j & 1u)) bp = fmaxf(bp, pj);
    }
    bp = wave_max_dpp(bp);
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + kWave * j;
      const float pj = p[j] == p[j] ? p[j] : -1.f;
      if (e < E && !(taken >> j & 1u) && pj == bp) bi = min(bi, e);
    }
    bi = wave_min_dpp(bi);
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == 0) {
      sel_id[r] = bi;
      sel_p[r] = bp;
    }
  }
  __builtin_amdgcn_wave_barrier();
  // ids ascending: lane a < K goes to its rank among the selected ids
  int myid = 0, rank = 0;
  float myp = 0.f;
  if (lane < K) {
    myid = sel_id[lane];
    myp = sel_p[lane];
    for (int b = 0; b < K; ++b) rank += sel_id[b] < myid;
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < K) {
    sel_id[rank] = myid;
    sel_p[rank] = myp;
  }
  __builtin_amdgcn_wave_barrier();
  // f64 renormalisation in ascending-id order (moe.rs:80-90)
  double wsum = 0.0;
  for (int a = 0; a < K; ++a) wsum += double(sel_p[a]);
  const double sden = wsum > 6.103515625e-05 ? wsum : 6.103515625e-05;  // 2^-14
  id_out = 0;
  w_out = 0.f;
  if (lane < K) {
    id_out = sel_id[lane];
    w_out = float(double(sel_p[lane]) / sden);
  }
}

// One work item of a gate/up or down launch: expert e, its first pair p0,
// cnt (1 or 2) pairs, and their tokens.
struct MoeItem {
  int e, p0, cnt, tok0, tok1;
};

// Item s from the route kernel's tables; false (for the whole workgroup)
// when s is past the call's item count. ROUTE (one token, at most 256
// experts): the workgroup routes the token itself (route_token, the route
// kernel's own steps, so ids and weights are the same), its items being the
// token's k experts in ascending id; the `writer` workgroup also writes the
// ids, weights and item tables that later launches read. Contains a
// workgroup barrier when ROUTE is set.
template <bool ROUTE>
__device__ __forceinline__ bool moe_item(const MoePlan& plan, uint8_t* ws, const float* __restrict__ logits, int s,
                                         bool writer, MoeItem& it) {
  if constexpr (ROUTE) {
    __shared__ int r_id[kMoeMaxTopK];
    __shared__ float r_p[kMoeMaxTopK];
    const int K = plan.top_k;
    if (threadIdx.x < kWave) {
      const int a = threadIdx.x;
      int id;
      float wv;
      route_token<4>(logits, plan.n_expert, K, a, r_id, r_p, id, wv);
      if (writer && a < K) {
        reinterpret_cast<int*>(ws + plan.o_ids)[a] = id;
        reinterpret_cast<float*>(ws + plan.o_wts)[a] = wv;
        reinterpret_cast<int*>(ws + plan.o_item_e)[a] = id;
        reinterpret_cast<int*>(ws + plan.o_item_off)[a] = a;
        reinterpret_cast<int*>(ws + plan.o_item_cnt)[a] = 1;
        reinterpret_cast<int*>(ws + plan.o_item_tok)[2 * a] = 0;
        reinterpret_cast<int*>(ws + plan.o_item_tok)[2 * a + 1] = 0;
        reinterpret_cast<int*>(ws + plan.o_tokpair)[a] = a;
        if (a == 0) reinterpret_cast<int*>(ws + plan.o_meta)[0] = K;
      }
    }
    __syncthreads();
    if (s >= K) return false;
    it = MoeItem{r_id[s], s, 1, 0, 0};
    return true;
  } else {
    (void)logits;
    (void)writer;
    // all of the item's fields at once (the tables hold z_max entries, so
    // an item past the count reads allocated memory before returning)
    const int n_items = reinterpret_cast<const int*>(ws + plan.o_meta)[0];
    it.e = reinterpret_cast<const int*>(ws + plan.o_item_e)[s];
    it.p0 = reinterpret_cast<const int*>(ws + plan.o_item_off)[s];
    it.cnt = reinterpret_cast<const int*>(ws + plan.o_item_cnt)[s];
    it.tok0 = reinterpret_cast<const int*>(ws + plan.o_item_tok)[2 * s];
    it.tok1 = reinterpret_cast<const int*>(ws + plan.o_item_tok)[2 * s + 1];
    return s < n_items;
  }
}

}  // namespace sh
