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
// Four launches (three for one token, whose gate/up workgroups route it
// themselves):
//   route    one workgroup routes every token (a wave per token) and groups
//            the (token, expert) pairs by expert, in ascending expert id;
//            each expert's pairs, two at a time, are "work items" (so every
//            workgroup below streams its rows once, and none runs twice as
//            long as the rest);
//   gate/up  workgroup (row chunk, matrix, item): the chunk's rows are
//            contiguous bytes, copied into an LDS ring of sub-tiles with
//            global_load_lds (the whole chunk, or two sub-tiles, in flight);
//            threads decode their 32-column half unit from LDS and apply each
//            row to the item's one or two tokens; row-slot sums reduce in
//            LDS to one chunk sum per pair;
//   down     workgroup (row chunk, item): a = silu(h) * p for its rows from
//            the gate/up chunk sums (fixed order), then the same streaming;
//   combine  out[t] = sum over t's experts in ascending id of w * d, with d
//            the sum of the down chunk sums.
// Chunk counts scale with the experts routed: a single token still spreads
// over the whole chip, and many tokens keep the chunk sums small. Each
// unique expert's weight bytes cross HBM once per call, however many tokens
// chose it.
#include <algorithm>
#include <type_traits>

#include "axpy.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "moe_items.hpp"

namespace sh {

constexpr int kMoeThreads = 256;
constexpr int kRouteThreads = 1024;  // one thread per expert in the grouping scan
static_assert(kRouteThreads == kMoeMaxExperts, "the scan gives each thread one expert");

// KPER: experts per lane (KPER * 64 >= n_expert)
template <int KPER>
__global__ void __launch_bounds__(kRouteThreads) moe_route_kernel(const float* __restrict__ logits,
                                                                  MoePlan plan, uint8_t* ws) {
  extern __shared__ __attribute__((aligned(16))) int rlds[];
  constexpr int kWaves = kRouteThreads / kWave;
  __shared__ int cnt[kMoeMaxExperts];
  __shared__ int cursor[kMoeMaxExperts];
  __shared__ int sel_id[kWaves][kMoeMaxTopK];
  __shared__ float sel_p[kWaves][kMoeMaxTopK];
  __shared__ int wave_nz[kWaves], wave_tot[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = plan.n_expert, K = plan.top_k;
  const int pairs = plan.n_tok * K;
  int* s_ids = rlds;                                     // [pairs]
  float* s_w = reinterpret_cast<float*>(rlds + pairs);   // [pairs]
  int* s_pt = rlds + 2 * pairs;                          // [pairs]: token of each grouped pair
  int* ids = reinterpret_cast<int*>(ws + plan.o_ids);
  float* wts = reinterpret_cast<float*>(ws + plan.o_wts);
  for (int e = tid; e < kMoeMaxExperts; e += kRouteThreads) cnt[e] = 0;

  for (int t = wave; t < plan.n_tok; t += kWaves) {
    int id;
    float wv;
    route_token<KPER>(logits + int64_t(t) * E, E, K, lane, sel_id[wave], sel_p[wave], id, wv);
    if (lane < K) {
      s_ids[t * K + lane] = id;
      s_w[t * K + lane] = wv;
      ids[t * K + lane] = id;
      wts[t * K + lane] = wv;
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();

  // group the pairs by expert: counts, an exclusive scan over experts (one
  // per thread), then each pair claims its position with an LDS atomic
  for (int i = tid; i < pairs; i += kRouteThreads) atomicAdd(&cnt[s_ids[i]], 1);
  __syncthreads();
  const int c = cnt[tid];
  const int nz = (c + 1) >> 1;  // this expert's work items: its pairs two at a time
  int snz = nz, stot = c;
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
    wave_tot[wave] = stot;
  }
  __syncthreads();
  int base_nz = 0, base_tot = 0;
  for (int w2 = 0; w2 < wave; ++w2) {
    base_nz += wave_nz[w2];
    base_tot += wave_tot[w2];
  }
  const int item = base_nz + snz - nz, pos = base_tot + stot - c;
  for (int i = 0; i < nz; ++i) {
    reinterpret_cast<int*>(ws + plan.o_item_e)[item + i] = tid;
    reinterpret_cast<int*>(ws + plan.o_item_off)[item + i] = pos + 2 * i;
    reinterpret_cast<int*>(ws + plan.o_item_cnt)[item + i] = min(2, c - 2 * i);
  }
  cursor[tid] = pos;
  if (tid == kRouteThreads - 1) reinterpret_cast<int*>(ws + plan.o_meta)[0] = base_nz + snz;
  __syncthreads();
  // a pair's position within its expert's run does not affect any result:
  // each pair's sums are computed on their own and found through tokpair
  int* tokpair = reinterpret_cast<int*>(ws + plan.o_tokpair);
  for (int i = tid; i < pairs; i += kRouteThreads) {
    const int q = atomicAdd(&cursor[s_ids[i]], 1);
    s_pt[q] = i / K;
    tokpair[i] = q;
  }
  __syncthreads();
  // each item's tokens, next to its other fields
  int* item_tok = reinterpret_cast<int*>(ws + plan.o_item_tok);
  for (int i = 0; i < nz; ++i) {
    item_tok[2 * (item + i)] = s_pt[pos + 2 * i];
    item_tok[2 * (item + i) + 1] = c - 2 * i > 1 ? s_pt[pos + 2 * i + 1] : 0;
  }
}

// ------------------------------------------------------- LDS row tiles --
// Copies bytes [src, src + n) of a weight tensor of `total` bytes into LDS
// at `dst` + (src & 15): whole 16-byte pieces from the 16-byte boundary at or
// below src, each thread a piece at a time; a piece that would run past the
// tensor's end is copied byte by byte. Returns the lead (src & 15). Loads
// are issued into registers first (`pieces` per thread at most), then
// stored, so they are all in flight together.
// 16-byte pieces per thread per tile (16 KiB tiles): small enough that
// four workgroups share a CU's LDS
constexpr int kTilePieces = 4;
constexpr int kRing = 3;  // sub-tile slots of the copy ring

template <int TP>
struct TileLoad {
  u32x4 v[TP];
  int n;     // pieces in the tile
  int lead;  // src & 15
};

template <int TP>
__device__ __forceinline__ void tile_issue(const uint8_t* base, int64_t src, int64_t n, int64_t total,
                                           TileLoad<TP>& t) {
  const int64_t a0 = src & ~int64_t(15);
  t.lead = int(src - a0);
  t.n = int((t.lead + n + 15) >> 4);
#pragma unroll
  for (int k = 0; k < TP; ++k) {
    const int pc = int(threadIdx.x) + kMoeThreads * k;
    const int64_t at = a0 + 16 * int64_t(pc);
    if (pc < t.n && at + 16 <= total) {
      t.v[k] = ld16(base + at);
    } else if (pc < t.n) {
      uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0;
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const uint32_t byte = at + b < total ? uint32_t(base[at + b]) : 0u;
        const uint32_t sh = 8 * (b & 3);
        if (b < 4) w0 |= byte << sh;
        else if (b < 8) w1 |= byte << sh;
        else if (b < 12) w2 |= byte << sh;
        else w3 |= byte << sh;
      }
      t.v[k] = u32x4{w0, w1, w2, w3};
    }
  }
}

template <int TP>
__device__ __forceinline__ void tile_store(uint8_t* dst, const TileLoad<TP>& t) {
#pragma unroll
  for (int k = 0; k < TP; ++k) {
    const int pc = int(threadIdx.x) + kMoeThreads * k;
    if (pc < t.n) *reinterpret_cast<u32x4*>(dst + 16 * pc) = t.v[k];
  }
}

// Column sums of one row chunk, for NT (1 or 2) input vectors at once
// (nt <= NT of them in use). The chunk (rows [r0, r0 + nrows) of W) is
// streamed through two LDS sub-tiles of `sr` rows; thread (half unit
// u = tid % U of 32 columns, slot sl = tid / U) applies rows sl, sl + RS, ...
// of each sub-tile to the inputs. The inputs' values for the chunk's rows are
// xs0[r], xs1[r]. The slots' sums are then reduced through the sub-tiles'
// LDS (`tiles`, `reg_bytes` of it, at least RS * U * 20 floats): all 32
// columns in one round when RS * U * 36 floats fit, else 16 a round; the
// column sums of input t go to out_t[col].
// `pre()` runs after the first sub-tile's loads are issued and before they
// are stored, so input staging overlaps the first weight bytes' latency.
constexpr int kRedStride = 20;  // floats per (slot, half unit) in a 16-column round: 16 sums + 4 pad

template <class F, int NT, bool DMA, class Pre>
__device__ __forceinline__ void chunk_sums(const uint8_t* W, int64_t rb, int64_t w_off, int64_t w_total, int cols,
                           int nrows, int sr, const float* xs0, const float* xs1, int nt, uint8_t* tiles,
                           int tile_cap, int64_t reg_bytes, float* out0, float* out1, int q6s, Pre pre) {
  const int tid = threadIdx.x;
  const int U = cols >> 5, RS = kMoeThreads / U;
  const int u = tid % U, sl = tid / U;
  const bool active = sl < RS;
  float acc[NT][32];
  float off[NT][F::kOff];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[t][e] = 0.f;
#pragma unroll
    for (int k = 0; k < F::kOff; ++k) off[t][k] = 0.f;
  }
  const int nsub = (nrows + sr - 1) / sr;
  // rows of sub-tile sb, applied by this thread
  auto apply_tile = [&](const uint8_t* tile, int sb) {
    const int rows_here = min(sr, nrows - sb * sr);
    if (!active) return;
    for (int r = sl; r < rows_here; r += RS) {
      const int rr = sb * sr + r;
      float xi[NT];
      xi[0] = xs0[rr];
      if constexpr (NT > 1) xi[1] = nt > 1 ? xs1[rr] : 0.f;
      if (xi[0] == 0.f && (NT == 1 || xi[NT - 1] == 0.f)) continue;  // ops.rs:182-184
      F::template apply<NT>(F::load(tile + int64_t(r) * rb, u), u, xi, acc, off, q6s);
    }
  };
  if constexpr (DMA) {
    // A ring of kRing sub-tile slots filled by global_load_lds copies (no
    // registers hold bytes in flight): kRing - 1 sub-tiles travel while one
    // is applied (all of them when the chunk has at most kRing). Sub-tile k is the 16-byte pieces from the boundary at or
    // below its first byte; piece p of it is copied by wave p / 64 % 4.
    const int wave = tid >> 6, lane = tid & 63;
    auto first = [&](int k) { return w_off + int64_t(k) * sr * rb; };
    auto pieces = [&](int k) {
      return int(((first(k) & 15) + int64_t(min(sr, nrows - k * sr)) * rb + 15) >> 4);
    };
    auto wave_copies = [&](int k) {  // this wave's copies of sub-tile k
      const int np = pieces(k), f = 64 * wave;
      return np > f ? (np - f + kMoeThreads - 1) / kMoeThreads : 0;
    };
    auto issue = [&](int k) {
      const int64_t a0 = first(k) & ~int64_t(15);
      const int np = pieces(k);
      uint8_t* dst = tiles + (k % kRing) * tile_cap;
      for (int p0 = 64 * wave; p0 < np; p0 += kMoeThreads)
        if (p0 + lane < np) copy16_to_lds(W + a0 + 16 * int64_t(p0 + lane), dst + 16 * p0);
    };
    // a chunk of at most kRing sub-tiles is requested whole up front
    int issued = 0;
    for (; issued < (nsub <= kRing ? nsub : kRing - 1); ++issued) issue(issued);
    pre();
    for (int sb = 0; sb < nsub; ++sb) {
      // sub-tile sb has landed once only this wave's later copies remain;
      // the barrier then covers every wave's (and, on the first pass, the
      // inputs pre() staged)
      int later = 0;
      for (int k = sb + 1; k < issued; ++k) later += wave_copies(k);
      wait_vmem(later);
      lds_barrier();
      // the slot of sub-tile sb - 1: every wave is past it
      if (issued < nsub) issue(issued++);
      apply_tile(tiles + (sb % kRing) * tile_cap + int(first(sb) & 15), sb);
    }
    lds_barrier();
  } else {
    (void)w_total;
    TileLoad<kTilePieces> tl;
    tile_issue(W, w_off, int64_t(min(sr, nrows)) * rb, w_total, tl);
    pre();
    tile_store(tiles, tl);
    int lead = tl.lead;
    __syncthreads();
    for (int sb = 0; sb < nsub; ++sb) {
      const bool more = sb + 1 < nsub;
      int next_lead = 0;
      if (more) {
        const int r1 = (sb + 1) * sr;
        tile_issue(W, w_off + int64_t(r1) * rb, int64_t(min(sr, nrows - r1)) * rb, w_total, tl);
        next_lead = tl.lead;
      }
      apply_tile(tiles + (sb & 1) * tile_cap + lead, sb);
      if (more) tile_store(tiles + ((sb + 1) & 1) * tile_cap, tl);
      lead = next_lead;
      __syncthreads();
    }
  }
  // the sub-tiles are free now: slot sums go through them, all 32 columns in
  // one round when `reg_bytes` holds them, else 16 a round; (slot, half
  // unit) rows are C + 4 floats apart so neighbouring threads' 16-byte
  // writes fall in different banks. Each column adds its slots in order, so
  // the result is the same either way.
  float* red = reinterpret_cast<float*>(tiles);
  auto reduce = [&](auto cols_c) {
    constexpr int C = decltype(cols_c)::value, stride = C + 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t >= nt) break;  // uniform: nt is the same for the whole workgroup
      float* o = t == 0 ? out0 : out1;
#pragma unroll
      for (int h = 0; h < 32 / C; ++h) {
        if (active) {
          float* dst = red + (sl * U + u) * stride;
#pragma unroll
          for (int e = 0; e < C; e += 4) {
            const int g = C * h + e;
            *reinterpret_cast<f32x4*>(dst + e) =
                f32x4{acc[t][g] - off[t][F::off_index(g)], acc[t][g + 1] - off[t][F::off_index(g + 1)],
                      acc[t][g + 2] - off[t][F::off_index(g + 2)], acc[t][g + 3] - off[t][F::off_index(g + 3)]};
          }
        }
        __syncthreads();
        for (int q = tid; q < U * C; q += kMoeThreads) {
          const int un = q / C, e = q - un * C;
          const float* src = red + un * stride + e;
          float v = 0.f;
#pragma unroll 8
          for (int k = 0; k < RS; ++k) v += src[k * U * stride];
          o[32 * un + C * h + e] = v;
        }
        __syncthreads();
      }
    }
  };
  if (int64_t(RS) * U * (32 + 4) * int64_t(sizeof(float)) <= reg_bytes)
    reduce(std::integral_constant<int, 32>{});
  else
    reduce(std::integral_constant<int, 16>{});
}

// -------------------------------------------------------------- gate / up --
// Workgroup (row chunk c, matrix m, work item s): chunk sums of gate_e . x_t
// or up_e . x_t for the item's pairs (token t, expert e), both tokens in one
// pass over the chunk's bytes.
// ROUTE (one token, at most 256 experts): the workgroup routes the token
// itself (route_token, the route kernel's own steps, so ids and weights are
// the same), its items being the token's k experts in ascending id;
// workgroup (0, 0, 0) writes the ids, weights and item tables that down and
// combine read, and no workgroup reads them here.
template <class F, int NT, bool DMA, bool ROUTE>
__global__ void __launch_bounds__(kMoeThreads)
    moe_gateup_kernel(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, MoePlan plan,
                      const float* __restrict__ x, uint8_t* ws, int q6_gate, int q6_up,
                      const float* __restrict__ logits) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int c = blockIdx.x, m = blockIdx.y, s = blockIdx.z;
  MoeItem it;
  if (!moe_item<ROUTE>(plan, ws, logits, s, c == 0 && m == 0 && s == 0, it)) return;
  const int e = it.e, p0 = it.p0, cnt = it.cnt, tok0 = it.tok0, tok1 = it.tok1;
  float* part = reinterpret_cast<float*>(ws + plan.o_part_a);
  const int r0 = c * plan.ca, nrows = min(plan.ca, plan.n_embd - r0);
  const int tile_cap = (plan.sr_a * int(plan.rb_a) + 31) & ~15;
  uint8_t* tiles = smem;
  float* xs = reinterpret_cast<float*>(smem + plan.reg_a);  // [2][ca]
  const uint8_t* W = m == 0 ? gate : up;
  const int64_t w_total = int64_t(plan.n_expert) * plan.n_embd * plan.rb_a;
  const int64_t w_off = (int64_t(e) * plan.n_embd + r0) * plan.rb_a;
  for (int j = 0; j < cnt; j += NT) {
    const int nt = min(NT, cnt - j);
    auto stage_x = [&]() {
      for (int i = threadIdx.x; i < nt * nrows; i += kMoeThreads) {
        const int t = i / nrows, r = i - t * nrows;
        const int tok = t == 0 ? tok0 : tok1;
        xs[t * plan.ca + r] = x[int64_t(tok) * plan.n_embd + r0 + r];
      }
    };
    // part[((p * 2 + m) * nch_a + c) * n_ff + col]
    float* o0 = part + ((int64_t(p0 + j) * 2 + m) * plan.nch_a + c) * plan.n_ff;
    float* o1 = o0 + int64_t(2) * plan.nch_a * plan.n_ff;
    // an item with one token takes the one-token pass (no FMAs for an absent second token)
    if (NT > 1 && nt == 1)
      chunk_sums<F, 1, DMA>(W, plan.rb_a, w_off, w_total, plan.n_ff, nrows, plan.sr_a, xs, xs + plan.ca, nt,
                            tiles, tile_cap, plan.reg_a, o0, o1, m == 0 ? q6_gate : q6_up, stage_x);
    else
      chunk_sums<F, NT, DMA>(W, plan.rb_a, w_off, w_total, plan.n_ff, nrows, plan.sr_a, xs, xs + plan.ca, nt,
                             tiles, tile_cap, plan.reg_a, o0, o1, m == 0 ? q6_gate : q6_up, stage_x);
  }
}

// ------------------------------------------------------------------- down --
// a = silu(h) * p for rows [r0, r0 + nrows) of the down chunk and tokens
// (pairs) q0 .. q0 + nt - 1, h and p summed over the gate/up chunk sums in a
// fixed order (ops.rs:85-87, moe.rs:119-121): 4 adjacent lanes load every 4th
// of the (at most 32) chunk sums, then a fixed shuffle tree adds the 4.
// Writes xs[t * cb + r]; hp ([2][2][cb] floats) is scratch.
__device__ __forceinline__ void stage_silu(const MoePlan& plan, const float* __restrict__ pa, int q0, int nt,
                                           int r0, int nrows, float* xs, float* hp) {
  const int tid = threadIdx.x, sub = tid & 3;
  const int n_el = nt * 2 * nrows;
  for (int i0 = 0; i0 < n_el * 4; i0 += kMoeThreads) {
    const int idx = i0 + tid, el = idx >> 2;
    const bool ok = el < n_el;
    const int elc = ok ? el : 0;
    const int t = elc / (2 * nrows), rem = elc - t * 2 * nrows, mm = rem / nrows, r = rem - mm * nrows;
    const float* src = pa + ((int64_t(q0 + t) * 2 + mm) * plan.nch_a) * plan.n_ff + r0 + r;
    float v[kMoeMaxChunks / 4];
#pragma unroll
    for (int q = 0; q < kMoeMaxChunks / 4; ++q) {
      const int k = sub + 4 * q;
      v[q] = ok && k < plan.nch_a ? src[int64_t(k) * plan.n_ff] : 0.f;
    }
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < kMoeMaxChunks / 4; ++q) sum += v[q];
    sum += __shfl_xor(sum, 1, kWave);
    sum += __shfl_xor(sum, 2, kWave);
    if (ok && sub == 0) hp[el] = sum;
  }
  __syncthreads();
  for (int i = tid; i < nt * nrows; i += kMoeThreads) {
    const int t = i / nrows, r = i - t * nrows;
    const float h = hp[(t * 2) * nrows + r], pv = hp[(t * 2 + 1) * nrows + r];
    xs[t * plan.cb + r] = h / (1.f + expf(-h)) * pv;
  }
}

// Workgroup (row chunk c over n_ff, work item s): first a = silu(h) * p for
// the chunk's rows and the item's tokens, h and p summed over the gate/up chunks
// in a fixed order (ops.rs:85-87, moe.rs:119-121); then chunk sums of
// down_e . a.
template <class F, int NT, bool DMA>
__global__ void __launch_bounds__(kMoeThreads)
    moe_down_kernel(const uint8_t* __restrict__ down, MoePlan plan, uint8_t* ws, int q6_down) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int c = blockIdx.x, s = blockIdx.y;
  MoeItem it;
  if (!moe_item<false>(plan, ws, nullptr, s, false, it)) return;
  const int e = it.e, p0 = it.p0, cnt = it.cnt;
  const float* pa = reinterpret_cast<const float*>(ws + plan.o_part_a);
  float* part = reinterpret_cast<float*>(ws + plan.o_part_b);
  const int r0 = c * plan.cb, nrows = min(plan.cb, plan.n_ff - r0);
  const int tile_cap = (plan.sr_b * int(plan.rb_b) + 31) & ~15;
  uint8_t* tiles = smem;
  float* xs = reinterpret_cast<float*>(smem + plan.reg_b);  // [2][cb]
  float* hp = xs + 2 * plan.cb;                                 // [2][2][cb]
  const int64_t w_total = int64_t(plan.n_expert) * plan.n_ff * plan.rb_b;
  const int64_t w_off = (int64_t(e) * plan.n_ff + r0) * plan.rb_b;
  for (int j = 0; j < cnt; j += NT) {
    const int nt = min(NT, cnt - j);
    auto stage_a = [&]() { stage_silu(plan, pa, p0 + j, nt, r0, nrows, xs, hp); };
    // part[(p * nch_b + c) * n_embd + col]
    float* o0 = part + (int64_t(p0 + j) * plan.nch_b + c) * plan.n_embd;
    float* o1 = o0 + int64_t(plan.nch_b) * plan.n_embd;
    if (NT > 1 && nt == 1)
      chunk_sums<F, 1, DMA>(down, plan.rb_b, w_off, w_total, plan.n_embd, nrows, plan.sr_b, xs, xs + plan.cb, nt,
                            tiles, tile_cap, plan.reg_b, o0, o1, q6_down, stage_a);
    else
      chunk_sums<F, NT, DMA>(down, plan.rb_b, w_off, w_total, plan.n_embd, nrows, plan.sr_b, xs, xs + plan.cb, nt,
                             tiles, tile_cap, plan.reg_b, o0, o1, q6_down, stage_a);
  }
}

// ---------------------------------------------------------------- combine --
// 32 columns of token t, by 256 threads as 32 columns x 8 expert lanes. Lane
// (col, a) sums the down chunk sums of the token's a-th expert (pair qa[a]);
// then the token's experts are added in ascending id order: out += w * d,
// skipping w == 0 (moe.rs:112-126). Every load a thread needs is issued
// before its first use (the pairs, weights and shared-expert values beside
// the chunk sums), so a workgroup waits for memory about twice.
__device__ __forceinline__ void combine_cols(const MoePlan& plan, const float* __restrict__ part,
                                             const int* qa, const float* wa, int t, int col0,
                                             float* __restrict__ out, float (*dsum)[32], float* wsh,
                                             const float* sh_d = nullptr, const float* sh_s = nullptr) {
  const int cl = threadIdx.x & 31, al = threadIdx.x >> 5;
  // the weights (one per expert lane) and the shared expert's terms, loaded
  // with everything else and passed on through LDS
  if (threadIdx.x < kMoeMaxTopK && int(threadIdx.x) < plan.top_k) wsh[threadIdx.x] = wa[threadIdx.x];
  float shd = 0.f, shs = 0.f;
  if (sh_d && al == 0) {
    shd = sh_d[int64_t(t) * plan.n_embd + col0 + cl];
    shs = sh_s[t];
  }
  for (int a = al; a < plan.top_k; a += 8) {
    const float* src = part + int64_t(qa[a]) * plan.nch_b * plan.n_embd + col0 + cl;
    // batches of 8 chunks (uniform), each batch's loads issued together
    // (indices clamped into the chunks, the extra values not added)
    float v[kMoeMaxChunks];
#pragma unroll
    for (int k8 = 0; k8 < kMoeMaxChunks; k8 += 8) {
      if (k8 < plan.nch_b) {
#pragma unroll
        for (int k = k8; k < k8 + 8; ++k) v[k] = src[int64_t(min(k, plan.nch_b - 1)) * plan.n_embd];
      }
    }
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < kMoeMaxChunks; ++k)
      if (k < plan.nch_b) sum += v[k];
    dsum[a][cl] = sum;
  }
  __syncthreads();
  if (al == 0) {
    float acc = 0.f;
    for (int a = 0; a < plan.top_k; ++a) {
      const float wv = wsh[a];
      if (wv != 0.f) acc = __fadd_rn(acc, __fmul_rn(wv, dsum[a][cl]));
    }
    if (sh_d) {
      // the shared expert: sigmoid(v) = 1 / (1 + exp(-v)) (ops.rs:90-92), then
      // one f32 product and one f32 add (moe.rs:139-142)
      const float gate = 1.f / (1.f + expf(-shs));
      acc = __fadd_rn(acc, __fmul_rn(gate, shd));
    }
    out[int64_t(t) * plan.n_embd + col0 + cl] = acc;
  }
}

// Block: 32 columns of one token.
// With sh_d set (the whole layer), the shared expert's gated output is added
// after the routed sum.
__global__ void __launch_bounds__(256) moe_combine_kernel(MoePlan plan, const uint8_t* ws,
                                                          float* __restrict__ out, const float* __restrict__ sh_d,
                                                          const float* __restrict__ sh_s, int pairs_in_order) {
  __shared__ float dsum[kMoeMaxTopK][32];
  __shared__ float wsh[kMoeMaxTopK];
  __shared__ int qsh[kMoeMaxTopK];
  const int blocks_per_tok = plan.n_embd / 32;
  const int t = blockIdx.x / blocks_per_tok, col0 = (blockIdx.x - t * blocks_per_tok) * 32;
  // the token's pairs, once for the workgroup (each expert lane reads its
  // own); in order, the table is not read: one memory round trip fewer
  const int* tp = reinterpret_cast<const int*>(ws + plan.o_tokpair) + t * plan.top_k;
  if (int(threadIdx.x) < plan.top_k)
    qsh[threadIdx.x] = pairs_in_order ? t * plan.top_k + int(threadIdx.x) : tp[threadIdx.x];
  __syncthreads();
  combine_cols(plan, reinterpret_cast<const float*>(ws + plan.o_part_b), qsh,
               reinterpret_cast<const float*>(ws + plan.o_wts) + t * plan.top_k, t, col0, out, dsum, wsh, sh_d,
               sh_s);
}

// ------------------------------------------------------------------- host --
static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

static int sub_rows(int64_t rb, int cols, int chunk, int tp) {
  const int rs = kMoeThreads / (cols >> 5);
  // rows that fit one tile with room for the 16-byte lead
  const int fit = int((int64_t(tp) * 16 * kMoeThreads - 16) / rb);
  if (chunk <= fit) return chunk;  // the whole chunk in one tile
  int sr = fit >= rs ? fit / rs * rs : fit;
  return sr < 1 ? 1 : sr;
}

bool moe_plan(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, uint32_t qa, uint32_t qb,
              MoePlan* plan, bool out_major) {
  if (n_tok <= 0 || top_k <= 0 || top_k > kMoeMaxTopK || top_k > n_expert ||
      n_expert > kMoeMaxExperts || n_embd <= 0 || n_ff <= 0 || n_tok > kMoeMaxTokens)
    return false;
  if (out_major) return moe_plan_out_major(n_tok, top_k, n_expert, n_embd, n_ff, qa, qb, plan);
  if (!expert_shape_ok(qa, n_embd, n_ff) || !expert_shape_ok(qb, n_ff, n_embd)) return false;
  if (n_tok > kMoeMaxTokens || n_embd % 32 != 0) return false;
  // one thread per 32-column half unit of a row at least
  if (n_ff > 32 * kMoeThreads || n_embd > 32 * kMoeThreads) return false;
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
  // work items (an expert's pairs two at a time): sum of ceil(cnt / 2) over
  // the experts routed to, at most (pairs + s_max) / 2
  p.z_max = (pairs + p.s_max + 1) / 2;
  // enough workgroups to cover the chip when few experts are routed, few
  // enough chunks that the partial sums stay small when many are
  const int rs_a = kMoeThreads / (n_ff >> 5), rs_b = kMoeThreads / (n_embd >> 5);
  p.nch_a = std::max(1, std::min({(4096 + 2 * p.s_max - 1) / (2 * p.s_max), (n_embd + rs_a - 1) / rs_a,
                                   kMoeMaxChunks}));
  p.ca = (n_embd + p.nch_a - 1) / p.nch_a;
  p.nch_a = (n_embd + p.ca - 1) / p.ca;
  p.nch_b = std::max(1, std::min({(2048 + p.s_max - 1) / p.s_max, (n_ff + rs_b - 1) / rs_b, kMoeMaxChunks}));
  p.cb = (n_ff + p.nch_b - 1) / p.nch_b;
  p.nch_b = (n_ff + p.cb - 1) / p.cb;
  const int tp = kTilePieces;
  p.sr_a = sub_rows(p.rb_a, n_ff, p.ca, tp);
  p.sr_b = sub_rows(p.rb_b, n_embd, p.cb, tp);
  const size_t cap_a = (size_t(p.sr_a) * p.rb_a + 31) & ~size_t(15);
  const size_t cap_b = (size_t(p.sr_b) * p.rb_b + 31) & ~size_t(15);
  // sub-tiles stream through a ring of copies when every 16-byte piece of a
  // tensor lies inside it (its size is a multiple of 16), else through
  // registers and two buffers; a chunk that fits one sub-tile needs one slot
  const int64_t total_a = int64_t(n_expert) * n_embd * p.rb_a, total_b = int64_t(n_expert) * n_ff * p.rb_b;
  p.staged = total_a % 16 == 0 && total_b % 16 == 0;
  const int nsub_a = (p.ca + p.sr_a - 1) / p.sr_a, nsub_b = (p.cb + p.sr_b - 1) / p.sr_b;
  const size_t nbuf_a = std::min(p.staged ? kRing : 2, nsub_a), nbuf_b = std::min(p.staged ? kRing : 2, nsub_b);
  // the sub-tiles' LDS is reused for the row-slot reduction (16 columns a
  // round at least; all 32 when the sub-tiles' bytes hold them)
  const size_t red_a = sizeof(float) * size_t(rs_a) * (n_ff / 32) * kRedStride;
  const size_t red_b = sizeof(float) * size_t(rs_b) * (n_embd / 32) * kRedStride;
  const size_t reg_a = std::max(nbuf_a * cap_a, red_a), reg_b = std::max(nbuf_b * cap_b, red_b);
  p.reg_a = int(reg_a);
  p.reg_b = int(reg_b);
  p.lds_a = reg_a + sizeof(float) * 2 * size_t(p.ca);
  p.lds_b = reg_b + sizeof(float) * 6 * size_t(p.cb);
  p.nbuf_a = int(nbuf_a);
  p.nbuf_b = int(nbuf_b);
  if (p.lds_a > 160 * 1024 || p.lds_b > 160 * 1024) return false;
  if (cap_a > size_t(tp) * 16 * kMoeThreads || cap_b > size_t(tp) * 16 * kMoeThreads) return false;
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
  p.o_part_a = take(sizeof(float) * size_t(pairs) * 2 * p.nch_a * n_ff);
  p.o_part_b = take(sizeof(float) * size_t(pairs) * p.nch_b * n_embd);
  // one token: the moe_one.hip launches and their sums instead
  if (moe_one_plan(p, qa, qb)) {
    p.o_p1a = take(sizeof(float) * size_t(top_k) * 2 * p.a1_nrc * n_ff);
    p.o_p1b = take(sizeof(float) * size_t(top_k) * p.b1_nrc * n_embd);
  }
  p.bytes = o;
  *plan = p;
  return true;
}

static bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// one token per pass when every expert has one token (decode), two otherwise;
// the copy ring when the plan allows it and the tensors start on 16 bytes
// `route`: one token routed inside gate/up (no route launch)
template <class FA>
static void launch_gateup(const MoePlan& p, const void* gate, const void* up, const float* x,
                          uint8_t* ws, int q6g, int q6u, const float* logits, bool route, hipStream_t s) {
  const dim3 g(p.nch_a, 2, p.z_max), b(kMoeThreads);
  const uint8_t *gp = static_cast<const uint8_t*>(gate), *upp = static_cast<const uint8_t*>(up);
  const bool dma = p.staged && aligned16(gate) && aligned16(up);
#define SH_GATEUP(NT, DMA, ROUTE) \
  hipLaunchKernelGGL((moe_gateup_kernel<FA, NT, DMA, ROUTE>), g, b, p.lds_a, s, gp, upp, p, x, ws, q6g, q6u, logits)
  if (route && dma) SH_GATEUP(1, true, true);
  else if (route) SH_GATEUP(1, false, true);
  else if (dma && p.n_tok == 1) SH_GATEUP(1, true, false);
  else if (dma) SH_GATEUP(2, true, false);
  else if (p.n_tok == 1) SH_GATEUP(1, false, false);
  else SH_GATEUP(2, false, false);
#undef SH_GATEUP
}

template <class FB>
static void launch_down(const MoePlan& p, const void* down, uint8_t* ws, int q6d, hipStream_t s) {
  const dim3 g(p.nch_b, p.z_max), b(kMoeThreads);
  const uint8_t* dp = static_cast<const uint8_t*>(down);
  const bool dma = p.staged && aligned16(down);
  if (dma && p.n_tok == 1) hipLaunchKernelGGL((moe_down_kernel<FB, 1, true>), g, b, p.lds_b, s, dp, p, ws, q6d);
  else if (dma) hipLaunchKernelGGL((moe_down_kernel<FB, 2, true>), g, b, p.lds_b, s, dp, p, ws, q6d);
  else if (p.n_tok == 1) hipLaunchKernelGGL((moe_down_kernel<FB, 1, false>), g, b, p.lds_b, s, dp, p, ws, q6d);
  else hipLaunchKernelGGL((moe_down_kernel<FB, 2, false>), g, b, p.lds_b, s, dp, p, ws, q6d);
}

hipError_t launch_moe(const MoePlan& p, uint32_t qg, uint32_t qu, uint32_t qd, const void* gate,
                      const void* up, const void* down, int q6g, int q6u, int q6d,
                      const float* logits, const float* x, float* out, void* workspace,
                      hipStream_t s, const MoeShared* shared) {
  if (qg != qu) return hipErrorInvalidValue;  // gate and up share one kernel
  if (qg == kIQ4_XS && (q6g != 0) != (q6u != 0)) return hipErrorInvalidValue;  // and one IQ4_XS reading
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  // one token (decode): gate/up routes it itself; otherwise the route kernel
  // groups every token's pairs by expert first
  const bool fused_route = p.n_tok == 1 && p.n_expert <= 4 * kWave;
  if (!fused_route) {
    hipError_t e = launch_moe_route(p, logits, workspace, s);
    if (e != hipSuccess) return e;
  }
  if (p.one) {
    // gate/up, down, then the combine (with the shared expert's add)
    return launch_moe_one(p, qg, qd, gate, up, down, q6g, q6u, q6d, logits, x, out, workspace, fused_route, s,
                          shared);
  }
  if (p.out_major) {
    launch_moe_out_major(p, qg, qd, gate, up, down, q6g, q6u, q6d, logits, x, workspace, fused_route, s);
  } else {
    switch (qg) {
      case kQ4_K: launch_gateup<HxQ4K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
      case kQ5_K: launch_gateup<HxQ5K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
      case kQ8_0: launch_gateup<HxQ8>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
      case kQ6_K: launch_gateup<HxQ6K>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s); break;
      default:  // kIQ4_XS: gate and up of one reading (checked by the caller)
        if (q6g) launch_gateup<HxIQ4XS<true>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
        else launch_gateup<HxIQ4XS<false>>(p, gate, up, x, ws, q6g, q6u, logits, fused_route, s);
    }
    switch (qd) {
      case kQ4_K: launch_down<HxQ4K>(p, down, ws, q6d, s); break;
      case kQ5_K: launch_down<HxQ5K>(p, down, ws, q6d, s); break;
      case kQ8_0: launch_down<HxQ8>(p, down, ws, q6d, s); break;
      case kQ6_K: launch_down<HxQ6K>(p, down, ws, q6d, s); break;
      default:  // kIQ4_XS
        if (q6d) launch_down<HxIQ4XS<true>>(p, down, ws, q6d, s);
        else launch_down<HxIQ4XS<false>>(p, down, ws, q6d, s);
    }
  }
  return launch_moe_combine(p, ws, out, shared, s, fused_route);
}

hipError_t launch_moe_combine(const MoePlan& p, const uint8_t* ws, float* out, const MoeShared* shared,
                              hipStream_t s, bool pairs_in_order) {
  if (shared && shared->join) {
    const hipError_t e = hipStreamWaitEvent(s, shared->join, 0);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(moe_combine_kernel, dim3(unsigned(p.n_tok * (p.n_embd / 32))), dim3(256), 0, s, p,
                     ws, out, shared ? shared->d : nullptr, shared ? shared->s : nullptr, int(pairs_in_order));
  return hipGetLastError();
}

// Routing alone (for the host-slice sh_moe_route): ids and weights per token.
hipError_t launch_moe_route(const MoePlan& p, const float* logits, void* workspace, hipStream_t s) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const dim3 g(1), b(kRouteThreads);
  if (p.n_expert <= 64) hipLaunchKernelGGL(moe_route_kernel<1>, g, b, p.route_lds, s, logits, p, ws);
  else if (p.n_expert <= 128) hipLaunchKernelGGL(moe_route_kernel<2>, g, b, p.route_lds, s, logits, p, ws);
  else if (p.n_expert <= 256) hipLaunchKernelGGL(moe_route_kernel<4>, g, b, p.route_lds, s, logits, p, ws);
  else if (p.n_expert <= 512) hipLaunchKernelGGL(moe_route_kernel<8>, g, b, p.route_lds, s, logits, p, ws);
  else hipLaunchKernelGGL(moe_route_kernel<16>, g, b, p.route_lds, s, logits, p, ws);
  return hipGetLastError();
}

}  // namespace sh
