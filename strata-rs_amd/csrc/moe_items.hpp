// Routing helpers and the work-item lookup shared by the MoE kernels of
// both expert-stack orientations (moe.hip, moe_om.hip).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// ------------------------------------------------------------------ route --
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Routes one token with one wave (moe.rs:58-90): max-shifted softmax (f32 exp,
// f64 sum, inv = f32(1 / sum)), then the top k by descending probability
// with ties to the lower id (the set the reference's k rounds of "largest
// probability, then lowest id" pick; a NaN probability ranks below every
// number), ids ascending, weights f32(f64(p) / max(sum_f64(p), 2^-14)).
// The k largest are found without k serial rounds: probabilities become
// order-preserving integer keys (p >= 0, so its bits; NaN and experts past E
// below them), a 32-step bisection over the key bits finds the k-th largest
// key T with wave ballots, every key above T is taken and the ties at T go
// to the lowest ids.
// sel_id / sel_p are the wave's LDS scratch (kMoeMaxTopK entries); on return
// they hold the ids ascending and their probabilities, and lane a < K holds
// id sel_id[a] and its weight in id_out, w_out. KPER experts per lane, with
// KPER * 64 >= E (a larger KPER gives the same result: experts past E are
// never selected, k <= E).
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
  uint32_t key[KPER];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    p[j] *= inv;
    const int e = lane + kWave * j;
    // p >= 0: its bits order like its value; NaN (1) below every number (>= 2)
    key[j] = e >= E ? 0u : (p[j] == p[j] ? __builtin_bit_cast(uint32_t, p[j]) + 2u : 1u);
  }
  // T: the largest key with at least K keys >= T (the K-th largest key)
  uint32_t T = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = T | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) cnt += __popcll(__ballot(key[j] >= c));
    if (cnt >= K) T = c;
  }
  // every key above T, then the ties at T in ascending id (id = lane + 64 j)
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));  // lanes under this one
  uint64_t sel[KPER];
  int need = K;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    sel[j] = __ballot(key[j] > T);
    need -= __popcll(sel[j]);
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint64_t eq = __ballot(key[j] == T);
    const int take = min(need, __popcll(eq));
    sel[j] |= __ballot(key[j] == T && __popcll(eq & below) < take);
    need -= take;
  }
  // the selected ids ascending (j-major, then lane) into the LDS scratch
  int base = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if ((sel[j] >> lane) & 1ull) {
      const int pos = base + __popcll(sel[j] & below);
      sel_id[pos] = lane + kWave * j;
      sel_p[pos] = p[j];
    }
    base += __popcll(sel[j]);
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
      // as few experts per lane as the expert count needs (the bisection's
      // ballots run per slot)
      if (plan.n_expert <= 64) route_token<1>(logits, plan.n_expert, K, a, r_id, r_p, id, wv);
      else if (plan.n_expert <= 128) route_token<2>(logits, plan.n_expert, K, a, r_id, r_p, id, wv);
      else route_token<4>(logits, plan.n_expert, K, a, r_id, r_p, id, wv);
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
