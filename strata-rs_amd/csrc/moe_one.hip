// The routed MoE FFN for one token (decode) over in-major expert stacks.
//
// Semantics as moe.hip (crates/strata-core/src/moe.rs:58-127, experts
// [n_expert][in][out], crates/strata-core/src/weights.rs:14-34): h = gate_e .
// x, p = up_e . x, a = silu(h) * p, d = down_e . a, out = sum over the
// selected experts in ascending id with w != 0 of w * d (f32 product, then
// f32 add), rows with x[i] == 0 skipped (ops.rs:182-184).
//
// One token leaves little work per expert, so the time is a chain of memory
// latencies rather than bandwidth. Two launches, each built to keep that
// chain short:
//   gate/up  workgroup (row chunk, column block, expert and matrix), 512
//            threads; a thread owns one 64-column unit of the matvec kernels
//            (the Ax units) and up to OneRows rows of the chunk, loads its
//            x values before the routing (which needs nothing of them) and
//            then every weight byte of its rows at once, straight into
//            registers, so a workgroup waits for memory about once; the
//            chunk's column sums go to the workspace;
//   down     workgroup (row chunk, column block, expert): a = silu(h) * p
//            for the chunk's rows from the gate/up chunk sums (loads issued
//            before the weight loads, so waiting for them does not wait for
//            the weights), then the same streaming into chunk sums;
// then moe.hip's combine launch adds the experts' sums in ascending id
// order. (A combine folded into down by its last workgroup per column
// block was measured slower: its reads of other XCDs' fresh sums at agent
// scope cost about 8 us against about 3 us for the extra launch.)
// The row slots' sums meet first within a quad of lanes (two DPP steps: the
// quad's four lanes hold four row slots of one unit), then in LDS, a
// quarter of the volume a per-thread LDS reduction moves (measured 4.2 ->
// 2.9 us at 512 threads x 64 sums before the quad step).
// Workgroups are sized for one per CU.
#include <algorithm>

#include "axpy.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "moe_items.hpp"

namespace sh {

constexpr int kOneThreads = 512;
constexpr int kOneRed = 68;  // floats per (slot group, unit) in the reduction's LDS: 64 sums + 4 pad

// Rows a thread can hold in flight: the Ax raw bytes of that many rows stay
// in registers next to the 64 sums and the 64 decoded codes.
template <class A>
struct OneRows {
  static constexpr int value = 4;
};
template <>
struct OneRows<AxQ6K> {
  static constexpr int value = 2;
};

// The column sums of one row chunk of one expert matrix, for the calling
// thread's unit `ug` (of the row) and row slot `sl`: rows r0 + sl + k * rs
// for k < MAXR inside [r0, r1), their bytes in raw[k], their inputs in
// xi[k]. Leaves acc - off in `acc`.
template <class A, int MAXR>
__device__ __forceinline__ void one_rows(int ug, bool active, int r0, int r1, int sl, int rs, const float* xi,
                                         typename A::Raw (&raw)[MAXR], float (&acc)[64], int q6s) {
  float a2[1][64];
  float off[1][A::kOff];
#pragma unroll
  for (int e = 0; e < 64; ++e) a2[0][e] = 0.f;
#pragma unroll
  for (int k = 0; k < A::kOff; ++k) off[0][k] = 0.f;
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const int r = r0 + sl + k * rs;
    if (active && r < r1 && xi[k] != 0.f) A::template apply<1>(raw[k], ug, &xi[k], a2, off, q6s);  // ops.rs:182-184
  }
#pragma unroll
  for (int e = 0; e < 64; ++e) acc[e] = a2[0][e] - off[0][A::off_index(e)];
}

constexpr int kOneMaxPer = 16;  // slot groups one thread adds in one_reduce (one_geometry keeps it within)

// Thread layout of a workgroup over a column block of cbu units: groups of
// cbu * 4 lanes, lane 4 u + q of group g holding unit u, row slot 4 g + q
// (a quad of lanes = four row slots of one unit).
struct OneLanes {
  int u, sl;
  bool in;  // a lane of a whole group
};
__device__ __forceinline__ OneLanes one_lanes(int cbu, int ngrp) {
  const int tid = threadIdx.x, G4 = cbu * 4;
  const int grp = tid / G4, rem = tid - grp * G4;
  return {rem >> 2, grp * 4 + (rem & 3), grp < ngrp};
}

__device__ __forceinline__ float quad_sum(float v) {  // the same sum in all four lanes of the quad
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}

// Sums over the 4 * ngrp row slots of each of the block's cbu * 64
// columns: each quad's four slots are added with DPP (every lane of the
// quad then holds the quad's 64 sums; its first lane writes them to LDS
// `red`, ngrp * cbu * kOneRed floats), then the G = cbu * 16 four-column groups
// are split over P parts, thread j * G + g adding slot groups j, j + P, ...
// of group g with 16-byte reads (the 16 lanes of an LDS pass read one
// contiguous run), and thread g adds the P parts in order (the same order
// on every call). store(col_in_block, v) is called once per column. Every
// lane of the workgroup calls this (the DPP steps read whole quads).
template <int P, class Store>
__device__ __forceinline__ void one_reduce(float (&acc)[64], const OneLanes& ln, int cbu, int ngrp, float* red,
                                           Store store) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 64; ++e) acc[e] = quad_sum(acc[e]);
  if (ln.in && (ln.sl & 3) == 0) {  // the quad's first lane writes its 64 sums
    float* dst = red + ((ln.sl >> 2) * cbu + ln.u) * kOneRed;
#pragma unroll
    for (int e = 0; e < 64; e += 4)
      *reinterpret_cast<f32x4*>(dst + e) = f32x4{acc[e], acc[e + 1], acc[e + 2], acc[e + 3]};
  }
  lds_barrier();
  const int G = cbu * 16;
  const int g = tid % G, j = tid / G;
  const int un = g >> 4, f = g & 15;
  const int per = (ngrp + P - 1) / P;
  float* tmp = red + ngrp * cbu * kOneRed;  // [P][G] float4
  if (j < P) {
    const float* base = red + un * kOneRed + 4 * f;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    f32x4 t[kOneMaxPer];
#pragma unroll
    for (int k = 0; k < kOneMaxPer; ++k) {
      if (k < per) {  // uniform; groups past ngrp read the last group and are not added
        const int grp = min(j + P * k, ngrp - 1);
        t[k] = *reinterpret_cast<const f32x4*>(base + grp * cbu * kOneRed);
      }
    }
#pragma unroll
    for (int k = 0; k < kOneMaxPer; ++k)
      if (k < per && j + P * k < ngrp) v = f32x4{v.x + t[k].x, v.y + t[k].y, v.z + t[k].z, v.w + t[k].w};
    *reinterpret_cast<f32x4*>(tmp + (j * G + g) * 4) = v;
  }
  lds_barrier();
  if (tid < G) {
    f32x4 v = *reinterpret_cast<const f32x4*>(tmp + g * 4);
#pragma unroll
    for (int k = 1; k < P; ++k) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(tmp + (k * G + g) * 4);
      v = f32x4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
    }
    const int col = 64 * un + 4 * f;
    store(col, v.x);
    store(col + 1, v.y);
    store(col + 2, v.z);
    store(col + 3, v.w);
  }
}

// ---------------------------------------------------------------- gate/up --
// Workgroup (row chunk c, column block b, item s * 2 + matrix m). ROUTE: the
// workgroup routes the token itself (moe_item<true>); workgroup (0, 0, 0)
// writes the routing tables down reads and clears down's block counters.
template <class A, bool ROUTE>
__global__ void __launch_bounds__(kOneThreads)
    moe1_gateup_kernel(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, MoePlan plan,
                       const float* __restrict__ x, uint8_t* ws, int q6_gate, int q6_up,
                       const float* __restrict__ logits) {
  constexpr int MAXR = OneRows<A>::value;
  extern __shared__ __attribute__((aligned(16))) float one_smem[];
  const int c = blockIdx.x, b = blockIdx.y, s = blockIdx.z >> 1, m = blockIdx.z & 1;
  const int cbu = plan.a1_cbu, rs = plan.a1_rs;
  const OneLanes ln = one_lanes(cbu, rs >> 2);
  const int u = ln.u, sl = ln.sl;
  const int units = plan.n_ff >> 6, ug = b * cbu + u;
  const bool active = ln.in && ug < units;
  const int r0 = c * plan.a1_rc, r1 = min(r0 + plan.a1_rc, plan.n_embd);
  // the rows' inputs first: they do not depend on the routing
  float xi[MAXR];
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const int r = r0 + sl + k * rs;
    const float v = x[min(r, plan.n_embd - 1)];
    xi[k] = (active && r < r1) ? v : 0.f;
  }
  const bool writer = c == 0 && b == 0 && blockIdx.z == 0;
  MoeItem it;
  if (!moe_item<ROUTE>(plan, ws, logits, s, writer, it)) return;
  const uint8_t* W = (m == 0 ? gate : up) + int64_t(it.e) * plan.n_embd * plan.rb_a;
  // every weight byte of the thread's rows in flight at once (rows past the
  // chunk load the chunk's last row again and are not applied)
  typename A::Raw raw[MAXR];
  const int ul = min(ug, units - 1);
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const int r = min(r0 + sl + k * rs, r1 - 1);
    raw[k] = A::load(W + int64_t(r) * plan.rb_a, ul);
  }
  float acc[64];
  one_rows<A, MAXR>(ug, active, r0, r1, sl, rs, xi, raw, acc, m == 0 ? q6_gate : q6_up);
  // part1_a[((s * 2 + m) * nrc_a + c) * n_ff + col]
  float* dst = reinterpret_cast<float*>(ws + plan.o_p1a) + (int64_t(s * 2 + m) * plan.a1_nrc + c) * plan.n_ff +
               int64_t(b) * cbu * 64;
  const int ncol = min(cbu, units - b * cbu) * 64;
  auto st = [&](int col, float v) {
    if (col < ncol) dst[col] = v;
  };
  switch (plan.a1_tpc) {
    case 1: one_reduce<1>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    case 2: one_reduce<2>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    case 4: one_reduce<4>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    default: one_reduce<8>(acc, ln, cbu, rs >> 2, one_smem, st);
  }
}

// ------------------------------------------------------------------- down --
// Workgroup (row chunk c over n_ff, column block b of n_embd, item s).
template <class A>
__global__ void __launch_bounds__(kOneThreads)
    moe1_down_kernel(const uint8_t* __restrict__ down, MoePlan plan, uint8_t* ws, int q6_down) {
  constexpr int MAXR = OneRows<A>::value;
  constexpr int kMaxA = 16;  // gate/up chunk sums per staged value (moe_plan keeps a1_nrc at most this)
  extern __shared__ __attribute__((aligned(16))) float one_smem[];
  const int c = blockIdx.x, b = blockIdx.y, s = blockIdx.z;
  const int tid = threadIdx.x;
  const int cbu = plan.b1_cbu, rs = plan.b1_rs, rc = plan.b1_rc;
  const OneLanes ln = one_lanes(cbu, rs >> 2);
  const int u = ln.u, sl = ln.sl;
  const int units = plan.n_embd >> 6, ug = b * cbu + u;
  const bool active = ln.in && ug < units;
  const int r0 = c * rc, r1 = min(r0 + rc, plan.n_ff), nrow = r1 - r0;
  MoeItem it;
  if (!moe_item<false>(plan, ws, nullptr, s, false, it)) return;
  // (1) the gate/up chunk sums of this chunk's rows: element tid is matrix
  // tid / rc, row tid % rc (loads first, so they complete before the weights)
  const int mm = tid >= rc ? 1 : 0, rr = tid - mm * rc;
  const bool stager = tid < 2 * rc && rr < nrow;
  const float* src = reinterpret_cast<const float*>(ws + plan.o_p1a) +
                     int64_t(s * 2 + mm) * plan.a1_nrc * plan.n_ff + r0 + min(rr, nrow - 1);
  float pv[kMaxA];
#pragma unroll
  for (int q = 0; q < kMaxA; ++q) pv[q] = src[int64_t(min(q, plan.a1_nrc - 1)) * plan.n_ff];
  // (2) every weight byte of the thread's rows
  const uint8_t* W = down + int64_t(it.e) * plan.n_ff * plan.rb_b;
  typename A::Raw raw[MAXR];
  const int ul = min(ug, units - 1);
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const int r = min(r0 + sl + k * rs, r1 - 1);
    raw[k] = A::load(W + int64_t(r) * plan.rb_b, ul);
  }
  // (3) h and p in chunk order, then a = silu(h) * p (ops.rs:85-87,
  // moe.rs:119-121) through LDS
  float* hp = one_smem + (rs >> 2) * cbu * kOneRed + plan.b1_tpc * cbu * 64;  // [2][rc], after the reduction's LDS
  if (stager) {
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxA; ++q)
      if (q < plan.a1_nrc) v += pv[q];
    hp[mm * rc + rr] = v;
  }
  lds_barrier();
  float xi[MAXR];
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const int r = sl + k * rs;
    float a = 0.f;
    if (active && r < nrow) {
      const float h = hp[r], pval = hp[rc + r];
      a = h / (1.f + expf(-h)) * pval;
    }
    xi[k] = a;
  }
  float acc[64];
  one_rows<A, MAXR>(ug, active, r0, r1, sl, rs, xi, raw, acc, q6_down);
  // (4) the chunk sums of the column block
  float* part = reinterpret_cast<float*>(ws + plan.o_p1b) + (int64_t(s) * plan.b1_nrc + c) * plan.n_embd +
                int64_t(b) * cbu * 64;
  const int ncol = min(cbu, units - b * cbu) * 64;
  auto st = [&](int col, float v) {
    if (col < ncol) part[col] = v;
  };
  switch (plan.b1_tpc) {
    case 1: one_reduce<1>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    case 2: one_reduce<2>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    case 4: one_reduce<4>(acc, ln, cbu, rs >> 2, one_smem, st); break;
    default: one_reduce<8>(acc, ln, cbu, rs >> 2, one_smem, st);
  }
}

// ------------------------------------------------------------------- host --
// Column blocks, row chunks and rows per thread of one phase (rows x cols
// per expert, `mats` matrices per item): the block is cbu 64-column units,
// rs = 512 / cbu row slots; chunks are chosen so the grid is about one
// workgroup per CU, with at most maxr rows a thread and at most max_chunks
// chunks. Returns false when no such split exists.
static bool one_geometry(int rows, int cols, int items, int mats, int cbu_max, int maxr, int max_chunks, int& cbu,
                         int& ncb, int& rs, int& rc, int& nrc, int& tpc) {
  constexpr int kTargetGroups = 256;  // MI355X CUs
  const int units = cols / 64;
  cbu = std::min(units, cbu_max);
  ncb = (units + cbu - 1) / cbu;
  rs = 4 * (kOneThreads / (4 * cbu));  // whole quads of row slots (OneLanes)
  const int per_chunk_groups = ncb * items * mats;
  nrc = std::min({std::max(1, kTargetGroups / per_chunk_groups), rows, max_chunks});
  // at most maxr rows a thread
  nrc = std::max(nrc, (rows + rs * maxr - 1) / (rs * maxr));
  if (nrc > max_chunks) return false;
  rc = (rows + nrc - 1) / nrc;
  nrc = (rows + rc - 1) / rc;
  // parts of the reduction's second step: as many as the threads allow (1
  // to 8), each adding at most kOneMaxPer slot groups
  tpc = 1;
  while (tpc < 8 && 2 * tpc * cbu * 16 <= kOneThreads) tpc *= 2;
  return rs >= 4 && tpc * cbu * 16 <= kOneThreads && (rs / 4 + tpc - 1) / tpc <= kOneMaxPer;
}

static int one_maxr(uint32_t q) { return q == kQ6_K ? OneRows<AxQ6K>::value : OneRows<AxQ4K>::value; }

bool moe_one_plan(MoePlan& p, uint32_t qa, uint32_t qb) {
  if (p.n_tok != 1 || p.out_major) return false;
  if (p.n_embd % 64 != 0 || p.n_ff % 64 != 0) return false;
  // gate / up: one column block when the row fits 16 units (n_ff <= 1024);
  // the chunk sums are staged by down, at most 16 per value
  if (!one_geometry(p.n_embd, p.n_ff, p.top_k, 2, 16, one_maxr(qa), 16, p.a1_cbu, p.a1_ncb, p.a1_rs, p.a1_rc,
                    p.a1_nrc, p.a1_tpc))
    return false;
  // down: 256-column blocks; the combine adds at most kMoeMaxChunks chunk
  // sums a column, and every staged value is a thread (2 * rows of a chunk
  // <= 512)
  if (!one_geometry(p.n_ff, p.n_embd, p.top_k, 1, 4, one_maxr(qb), kMoeMaxChunks, p.b1_cbu, p.b1_ncb, p.b1_rs,
                    p.b1_rc, p.b1_nrc, p.b1_tpc))
    return false;
  if (2 * p.b1_rc > kOneThreads) return false;
  p.lds1_a = (size_t(p.a1_rs / 4) * p.a1_cbu * kOneRed + size_t(p.a1_tpc) * p.a1_cbu * 64) * sizeof(float);
  p.lds1_b = (size_t(p.b1_rs / 4) * p.b1_cbu * kOneRed + size_t(p.b1_tpc) * p.b1_cbu * 64) * sizeof(float) +
             2 * size_t(p.b1_rc) * sizeof(float);
  if (p.lds1_a > 128 * 1024 || p.lds1_b > 128 * 1024) return false;
  p.one = true;
  return true;
}

template <class A>
static void launch_one_gateup(const MoePlan& p, const void* gate, const void* up, const float* x, uint8_t* ws,
                              int q6g, int q6u, const float* logits, bool route, hipStream_t s) {
  const dim3 g(p.a1_nrc, p.a1_ncb, 2 * p.top_k), blk(kOneThreads);
  const uint8_t *gp = static_cast<const uint8_t*>(gate), *upp = static_cast<const uint8_t*>(up);
  if (route)
    hipLaunchKernelGGL((moe1_gateup_kernel<A, true>), g, blk, p.lds1_a, s, gp, upp, p, x, ws, q6g, q6u, logits);
  else
    hipLaunchKernelGGL((moe1_gateup_kernel<A, false>), g, blk, p.lds1_a, s, gp, upp, p, x, ws, q6g, q6u, logits);
}

template <class A>
static void launch_one_down(const MoePlan& p, const void* down, uint8_t* ws, int q6d, hipStream_t s) {
  const dim3 g(p.b1_nrc, p.b1_ncb, p.top_k), blk(kOneThreads);
  hipLaunchKernelGGL((moe1_down_kernel<A>), g, blk, p.lds1_b, s, static_cast<const uint8_t*>(down), p, ws, q6d);
}

hipError_t launch_moe_one(const MoePlan& p, uint32_t qg, uint32_t qd, const void* gate, const void* up,
                          const void* down, int q6g, int q6u, int q6d, const float* logits, const float* x,
                          float* out, void* workspace, bool fused_route, hipStream_t s, const MoeShared* shared) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  switch (qg) {
    case kQ4_K: launch_one_gateup<AxQ4K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ5_K: launch_one_gateup<AxQ5K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ8_0: launch_one_gateup<AxQ8>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kQ6_K: launch_one_gateup<AxQ6K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
    case kIQ4_XS:  // gate and up of one reading (checked by launch_moe)
      if (q6g) launch_one_gateup<AxIQ4XS<true>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
      else launch_one_gateup<AxIQ4XS<false>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
      break;
    default: return hipErrorInvalidValue;
  }
  switch (qd) {
    case kQ4_K: launch_one_down<AxQ4K>(p, down, ws, q6d, s); break;
    case kQ5_K: launch_one_down<AxQ5K>(p, down, ws, q6d, s); break;
    case kQ8_0: launch_one_down<AxQ8>(p, down, ws, q6d, s); break;
    case kQ6_K: launch_one_down<AxQ6K>(p, down, ws, q6d, s); break;
    case kIQ4_XS:
      if (q6d) launch_one_down<AxIQ4XS<true>>(p, down, ws, q6d, s);
      else launch_one_down<AxIQ4XS<false>>(p, down, ws, q6d, s);
      break;
    default: return hipErrorInvalidValue;
  }
  // the combine over this path's sums: one pair per item, b1_nrc chunks
  MoePlan pc = p;
  pc.o_part_b = p.o_p1b;
  pc.nch_b = p.b1_nrc;
  return launch_moe_combine(pc, ws, out, shared, s, fused_route);
}

}  // namespace sh
