// Fused dequant + matvec for Q8_0, Q4_K, Q5_K and Q6_K rows, read packed from
// HBM.
//
// Semantics: crates/strata-core/src/ops.rs:14-28 (`gemv`): y[r] = sum_c
// W[r][c] * x[c] with W[r][c] the strata-gguf dequantized value
// (crates/strata-gguf/src/dequant.rs:123-128, :208-234, :237-302). The sum is
// formed in f32 in a different order from the reference's sequential f64
// loop, and per-block scales are factored out:
//   Q4_K  sum_sub (d*sc) * sum(q*x) - (dmin*m) * sum(x)   (Q5_K alike, q 0..31)
//   Q8_0  sum_blk  d * (sum((q+128)*x) - 128 * sum(x))
//   Q6_K  sum_16   d*sc * (sum(q6*x) - 32 * sum(x))
// so the outputs agree with the reference to f32 rounding, not bit for bit.
//
// Work mapping (one design for all three formats):
//   * a lane "unit" is 64 consecutive columns of one row; a wave covers a
//     window of 64 units = 4096 columns, so a row of `cols` columns is
//     ceil(cols / 4096) windows;
//   * x (and per-16 partial sums of x) is staged once per workgroup in LDS,
//     with a 16-byte pad every 64 floats so each lane's 256-byte run is
//     read without bank conflicts; when a matrix has a single window each
//     lane keeps its x run in VGPRs for every row it visits;
//   * a wave takes R rows at a time, all windows of those rows in sequence,
//     and issues the next item's weight loads before computing the current
//     one; row sums are reduced across the wave with cross-lane shuffles.
// Weight bytes are read exactly once per launch with 16-byte loads of the
// block layout; nothing is dequantized to memory.
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "fmt.hpp"
#include "kernels.hpp"
#include "limb.hpp"

namespace sh {

// ---------------------------------------------------------------- kernel --
// One launch computes y[b][r] for all rows, b < NB. Each wave walks items
// (row group of F::kR rows, window) for the row groups
// wave_id, wave_id + total_waves, ...; the loads of the next item are in
// flight while the current one is computed.
template <class F, int NB>
__global__ void __launch_bounds__(512) gemv_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                   int64_t row_bytes, const float* __restrict__ x,
                                                   float* __restrict__ y, int q6_signed) {
  constexpr int R = (NB == 1) ? F::kR : 1;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  stage_x(lds, x, cols, NB);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wpg = blockDim.x >> 6;
  const int units = cols >> 6;            // 64-column units per row
  const int nwin = (units + 63) >> 6;     // 4096-column windows per row
  const int n_rg = (rows + R - 1) / R;    // row groups
  const int stride = gridDim.x * wpg;
  int rg = blockIdx.x * wpg + (threadIdx.x >> 6);
  if (rg >= n_rg) return;
  const int xs = x_stride(cols);

  int win = 0;
  typename F::Load cur[R], nxt[R];
  auto issue = [&](typename F::Load* L, int g, int wn) {
    const int u = (wn << 6) + lane;
    if (u < units) {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        int r = g * R + i;
        r = r < rows ? r : rows - 1;  // a short last group repeats its last row
        F::load(w + int64_t(r) * row_bytes, u, L[i]);
      }
    }
  };
  issue(cur, rg, win);

  float acc[R][NB];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[i][b] = 0.f;

  // batch 1: the lane's x run stays in VGPRs while the window is unchanged
  // (for a single-window matrix, for the whole launch); batches > 1 read each
  // vector's run from LDS per item.
  XSlice xv;
  int xwin = -1;
  while (true) {
    int nrg = rg, nwn = win + 1;
    if (nwn == nwin) {
      nwn = 0;
      nrg = rg + stride;
    }
    const bool more = nrg < n_rg;
    if (more) issue(nxt, nrg, nwn);

    const int u = (win << 6) + lane;
    if (u < units) {
      if constexpr (NB == 1) {
        if (xwin != win) {
          load_xslice(lds, cols, u, xv);
          xwin = win;
        }
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i][0] += F::dot(cur[i], xv, u, q6_signed);
      } else {
#pragma unroll 1
        for (int b = 0; b < NB; ++b) {
          load_xslice(lds + b * xs, cols, u, xv);
#pragma unroll
          for (int i = 0; i < R; ++i) acc[i][b] += F::dot(cur[i], xv, u, q6_signed);
        }
      }
    }
    if (win == nwin - 1) {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int r = rg * R + i;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float t = wave_sum(acc[i][b]);
          if (lane == 0 && r < rows) y[int64_t(b) * rows + r] = t;
          acc[i][b] = 0.f;
        }
      }
    }
    if (!more) break;
    rg = nrg;
    win = nwn;
#pragma unroll
    for (int i = 0; i < R; ++i) cur[i] = nxt[i];
  }
}

// ------------------------------------------------------- batch-1 kernel --
// Each wave owns `rg_per_wave` consecutive row groups (F::kR rows each) and
// walks their (row group, window) items in order. Loads are issued as early
// as the hardware allows:
//   1. the workgroup's share of x is loaded into registers,
//   2. the weight loads of the wave's first D items are issued,
//   3. x (and its per-16 sums) is written to LDS -- this waits only for the
//      x loads, which were issued first -- and the workgroup synchronises,
//   4. items are computed in order; the moment item i is consumed its D-slot
//      register set is refilled with item i + D.
// So every wave has D items of weight bytes in flight from the first cycle
// on, and x staging overlaps the first weight fetches instead of preceding
// them.
constexpr int kXRounds = 3;  // x groups held in registers per thread

// Loads are never under a branch: lanes past the last unit, items past the
// wave's last one and x groups past the end re-load a valid address whose
// result is discarded. Branch-free load sequences let the compiler count
// outstanding loads exactly (s_waitcnt vmcnt(N) with N > 0) instead of
// draining the whole queue at every control-flow merge.
template <class F, int D>
__global__ void __launch_bounds__(512) gemv1_kernel(const uint8_t* __restrict__ w, int rows,
                                                    int cols, int64_t row_bytes,
                                                    const float* __restrict__ x,
                                                    float* __restrict__ y, int q6_signed,
                                                    int rg_per_wave) {
  constexpr int R = F::kR;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wpg = blockDim.x >> 6;
  const int units = cols >> 6;
  const int nwin = (units + 63) >> 6;
  const int n_rg = (rows + R - 1) / R;
  const int wave_id = blockIdx.x * wpg + (tid >> 6);
  const int rg0 = wave_id * rg_per_wave;
  const int my_rg = max(0, min(rg_per_wave, n_rg - rg0));
  const int n_items = my_rg * nwin;  // wave-uniform

  // 1. x loads (16-float groups, round-robin over the workgroup)
  const int groups = cols >> 4;
  f32x4 xr[kXRounds][4];
#pragma unroll
  for (int k = 0; k < kXRounds; ++k) {
    const int g = min(tid + k * int(blockDim.x), groups - 1);
    const f32x4* src = reinterpret_cast<const f32x4*>(x + 16 * g);
#pragma unroll
    for (int j = 0; j < 4; ++j) xr[k][j] = src[j];
  }

  // 2. weight loads of the first D items
  typename F::Load slot[D][R];
  const int last = max(n_items - 1, 0);
  auto issue = [&](typename F::Load* L, int i) {
    i = min(i, last);
    const int q = i / nwin;
    const int win = i - q * nwin;
    const int u = min((win << 6) + lane, units - 1);
    const int rgq = min(rg0 + q, n_rg - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(rgq * R + r, rows - 1);
      typename F::Load v;
      F::load(w + int64_t(row) * row_bytes, u, v);
      L[r] = v;
    }
  };
#pragma unroll
  for (int s = 0; s < D; ++s) issue(slot[s], s);

  // 3. x -> LDS with per-16 sums (waits only for the x loads, issued first)
  const int sum_base = cols + cols / 16;
#pragma unroll
  for (int k = 0; k < kXRounds; ++k) {
    const int g = tid + k * int(blockDim.x);
    const f32x4 a = xr[k][0], b = xr[k][1], c = xr[k][2], e = xr[k][3];
    const float sum = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
                      (((c.x + c.y) + (c.z + c.w)) + ((e.x + e.y) + (e.z + e.w)));
    if (g < groups) {
      const int e0 = 16 * g;
      f32x4* d = reinterpret_cast<f32x4*>(lds + e0 + 4 * (e0 >> 6));
      d[0] = a;
      d[1] = b;
      d[2] = c;
      d[3] = e;
      lds[sum_base + g] = sum;
    }
  }
  // rows wider than kXRounds * blockDim * 16 columns (none of the configs)
  for (int g = tid + kXRounds * int(blockDim.x); g < groups; g += blockDim.x) {
    const f32x4* src = reinterpret_cast<const f32x4*>(x + 16 * g);
    const f32x4 a = src[0], b = src[1], c = src[2], e = src[3];
    const int e0 = 16 * g;
    f32x4* d = reinterpret_cast<f32x4*>(lds + e0 + 4 * (e0 >> 6));
    d[0] = a;
    d[1] = b;
    d[2] = c;
    d[3] = e;
    lds[sum_base + g] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
                        (((c.x + c.y) + (c.z + c.w)) + ((e.x + e.y) + (e.z + e.w)));
  }
  __syncthreads();
  if (n_items == 0) return;

  // 4. compute in order, refilling each slot as soon as it is consumed
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  XSlice xv;
  int xwin = -1;
  for (int base = 0; base < n_items; base += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int i = base + s;
      const int q = i / nwin;
      const int win = i - q * nwin;
      const int u = (win << 6) + lane;
      if (xwin != win) {
        load_xslice(lds, cols, min(u, units - 1), xv);
        xwin = win;
      }
      float part[R];
#pragma unroll
      for (int r = 0; r < R; ++r) part[r] = F::dot(slot[s][r], xv, u, q6_signed);
      // keep the refill below the last use of the slot, so the new loads land
      // in the same registers and the loop needs no register rotation (a
      // rotating copy of a pending load would drain the whole load queue)
      __builtin_amdgcn_sched_barrier(0);
      issue(slot[s], i + D);
      if (i < n_items) {
        if (u < units) {
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] += part[r];
        }
        if (win == nwin - 1) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float t = wave_sum(acc[r]);
            const int row = (rg0 + q) * R + r;
            if (lane == 0 && row < rows) y[row] = t;
            acc[r] = 0.f;
          }
        }
      }
    }
  }
}

// Batch-1 matvec on the integer path.
//
// Wave w owns row groups [w*per, w*per + per) of R rows. Items are
// (row group, window) pairs taken window-major, so each wave reads its x
// limbs from LDS once per window and keeps `per` (<= MAXQ) row sums per
// row in registers; rows of a single window are final after their one item
// and are stored at once (then `per` may exceed MAXQ: a wave streams its
// whole share of a tall matrix and x is staged once per workgroup). All item control is wave-uniform (scalar registers);
// per-lane byte offsets within a row are computed once. Loads are
// double-buffered (A/B ping-pong, both refills unconditional so the loop
// latch never drains the load queue), and the first item is requested
// before x is staged, so weight bytes are in flight from the first cycles
// (after every wave's x loads, when x takes more than one round).
//
// MODE bits (compile-time; 0 for the plain matvec) let the dense FFN run in
// two launches: kLimbTwoMat reads rows [0, rows1) from w and [rows1, rows)
// from w2 (gate and up in one launch, x staged once); kLimbSiluX stages
// silu(x) * xu, with silu(v) = v / (1 + exp(-v)) in f32 (qwen35.rs:120-124),
// instead of x; kLimbResid writes y = xres + sum (one f32 add, qwen35.rs:127-129);
// kLimbPairSilu (R = 2, rows of one 4096-column window) takes row group q
// as row q of w (gate) and row q of w2 (up) and stores y[q] = silu(g) * u,
// the same f32 expression kLimbSiluX stages, so the down launch stages one
// vector instead of two.
// kLimbFine stages x in the 23-bit limbs (limb.hpp), as the modes of the
// silu(g) * u chain (kLimbTwoMat, kLimbPairSilu, kLimbSiluX, kLimbResid, the
// shared expert's down) do.
constexpr int kLimbTwoMat = 1, kLimbSiluX = 2, kLimbResid = 4, kLimbPairSilu = 8, kLimbFine = 16;

// silu(g) * u in f32, g / (1 + exp(-g)) * u without contraction
// (qwen35.rs:120-124, ops.rs:85-87)
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  return g / (1.f + expf(-g)) * u;
}
constexpr int kLimbMaxRowsOneWin = 64;  // row groups a wave may take when rows are one window

template <class F, int R, int MAXQ, int MODE = 0, int NPRE = 1, bool SPREAD = false>
__global__ void __launch_bounds__(512) gemv_limb_kernel(const uint8_t* __restrict__ w, int rows,
                                                        int cols, int64_t row_bytes,
                                                        const float* __restrict__ x,
                                                        float* y, int per, int flags,
                                                        const uint8_t* __restrict__ w2, int rows1,
                                                        const float* __restrict__ xu,
                                                        const float* xres) {  // xres may be y (in place)
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  constexpr bool kLow = F::kQuant == kQ8_0 || F::kQuant == kIQ4_XS;  // signed codes: the low-limb sums
  // 23-bit limbs for every step of the silu(g) * u chain: the gate / up
  // inputs whose sums form it and the inputs formed from it
  constexpr bool kFine = (MODE & (kLimbTwoMat | kLimbPairSilu | kLimbSiluX | kLimbResid | kLimbFine)) != 0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (tid >> 6));
  const int units = cols >> 6;
  const int nwin = (units + 63) >> 6;
  const int n_rg = (rows + R - 1) / R;
  // Row groups of this wave: a run of `per` from wave * per; or, with
  // SPREAD (rows of one window), every W-th from the wave's index (W the
  // waves of the launch, per = ceil(n_rg / W)), so that the waves read one
  // stretch of the matrix at a time (the 151936-row Q6_K head: 111 -> 104
  // us). No division here: it would delay the first weight loads.
  static_assert(!SPREAD || NPRE == 1, "spread rows are single-window rows");
  const int W = int(gridDim.x) * int(blockDim.x >> 6);
  const int gstep = SPREAD ? W : 1;
  const int rg0 = SPREAD ? wave : wave * per;
  const int my = SPREAD ? max(0, per - (wave + (per - 1) * W >= n_rg ? 1 : 0)) : max(0, min(per, n_rg - rg0));
  const int n_items = my * nwin;

  // per-lane offsets: window 0, and the clamped unit of a partial last window
  const typename F::Off off0 = F::offsets(lane);
  const int ulast = min((nwin - 1) * 64 + lane, units - 1);
  const typename F::Off offl = F::offsets(ulast);
  const bool lane_valid_last = (nwin - 1) * 64 + lane < units;

  // the item sequence: window-major, row groups inner
  auto item_off = [&](int wn) -> typename F::Off {
    if (wn == nwin - 1) return offl;
    return {off0.h + wn * F::kWinBytes, off0.q};
  };
  int pw = 0, pq = 0;  // next item to request
  auto issue = [&](typename F::Load* L) {
    const bool past = pw >= nwin;  // past the end: re-request the last item
    const int wn = past ? nwin - 1 : pw;
    const int qq = past ? max(my - 1, 0) : pq;
    const typename F::Off o = item_off(wn);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min((rg0 + qq * gstep) * R + r, rows - 1);
      const uint8_t* base = w + int64_t(row) * row_bytes;
      if constexpr ((MODE & kLimbTwoMat) != 0)
        base = row >= rows1 ? w2 + int64_t(row - rows1) * row_bytes : base;
      if constexpr ((MODE & kLimbPairSilu) != 0)
        base = (r == 0 ? w : w2) + int64_t(row >> 1) * row_bytes;
      F::load(base, o, L[r]);
    }
    if (++pq == my) {
      pq = 0;
      ++pw;
    }
  };

  // x as limbs, 8 columns per thread and round (4096 columns a round). The
  // x loads of the first NPRE rounds are issued before the first weight
  // item's, so the wait for them does not wait for the weights; their
  // conversion is branch-free (a round's idle threads convert a clamped
  // copy and skip the write), which keeps the loads ahead of the weight
  // loads. Rounds past NPRE (rows wider than NPRE * 4096 columns) load and
  // convert in a loop after the first item is requested.
  const int n8 = cols >> 3;
  const int nthr = blockDim.x;
  f32x4 xv[NPRE][2], uv[NPRE][2];
#pragma unroll
  for (int k = 0; k < NPRE; ++k) {
    const int t = min(tid + k * nthr, n8 - 1);
    const f32x4* src = reinterpret_cast<const f32x4*>(x + 8 * t);
    xv[k][0] = src[0];
    xv[k][1] = src[1];
    if constexpr ((MODE & kLimbSiluX) != 0) {
      const f32x4* su = reinterpret_cast<const f32x4*>(xu + 8 * t);
      uv[k][0] = su[0];
      uv[k][1] = su[1];
    }
  }
  typename F::Load A[R], B[R];
  if constexpr (NPRE > 1) {
    // A CU returns vector loads about in the order they were issued, so a
    // weight load issued before another wave's x loads delays that wave's x
    // (and the barrier below) by a memory latency. An issue-only barrier
    // puts every x load of the workgroup ahead of its first weight load:
    // 4096x12288 Q4_K 8.16 -> 7.70 us. Rows of one window (one x round, 16
    // KiB) lose more to the barrier than they gain, and skip it.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
  issue(A);
  auto stage = [&](int t, f32x4 a, f32x4 b, f32x4 ua, f32x4 ub) {
    if constexpr ((MODE & kLimbSiluX) != 0) {
#pragma clang fp contract(off)
      const f32x4 h0{a.x / (1.f + expf(-a.x)) * ua.x, a.y / (1.f + expf(-a.y)) * ua.y,
                     a.z / (1.f + expf(-a.z)) * ua.z, a.w / (1.f + expf(-a.w)) * ua.w};
      const f32x4 h1{b.x / (1.f + expf(-b.x)) * ub.x, b.y / (1.f + expf(-b.y)) * ub.y,
                     b.z / (1.f + expf(-b.z)) * ub.z, b.w / (1.f + expf(-b.w)) * ub.w};
      limb_group8<kLow, kFine>(lds8, cols, t, t < n8, h0, h1);
    } else {
      limb_group8<kLow, kFine>(lds8, cols, t, t < n8, a, b);
    }
  };
#pragma unroll
  for (int k = 0; k < NPRE; ++k) stage(tid + k * nthr, xv[k][0], xv[k][1], uv[k][0], uv[k][1]);
  for (int t0 = NPRE * nthr; t0 < n8; t0 += nthr) {
    const int t = min(t0 + tid, n8 - 1);
    const f32x4* src = reinterpret_cast<const f32x4*>(x + 8 * t);
    f32x4 ua{}, ub{};
    if constexpr ((MODE & kLimbSiluX) != 0) {
      const f32x4* su = reinterpret_cast<const f32x4*>(xu + 8 * t);
      ua = su[0];
      ub = su[1];
    }
    stage(t0 + tid, src[0], src[1], ua, ub);
  }
  // LDS only: __syncthreads() would also wait for the first item's weight
  // loads, which keeps the second item's loads from issuing until they land
  lds_barrier();
  if (n_items == 0) return;

  float acc[MAXQ][R];
#pragma unroll
  for (int q = 0; q < MAXQ; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[q][r] = 0.f;
  typename LimbX<F>::T xl;
  int cw = 0, cq = 0;  // item being computed
  auto step = [&](const typename F::Load* L) {
    if (cq == 0) {
      const int u = cw == nwin - 1 ? ulast : cw * 64 + lane;
      LimbX<F>::load(lds8, cols, u, xl);
    }
    const bool ok = cw < nwin - 1 || lane_valid_last;
    if constexpr (NPRE == 1) {
      // a single window (NPRE == nwin): each item is whole rows, final at
      // once (so a wave may take any number of them, and fewer workgroups
      // stage x)
      if constexpr ((MODE & kLimbPairSilu) != 0) {
        static_assert(R == 2, "a gate row and an up row per item");
        const float g = wave_sum_dpp(ok ? F::dot(L[0], xl, lane, flags) : 0.f);
        const float u = wave_sum_dpp(ok ? F::dot(L[1], xl, lane, flags) : 0.f);
        const int q = rg0 + cq * gstep;
        if (lane == 63 && q < n_rg) y[q] = silu_mul(g, u);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float t = F::dot(L[r], xl, lane, flags);
          const float v = wave_sum_dpp(ok ? t : 0.f);
          const int row = (rg0 + cq * gstep) * R + r;
          if (lane == 63 && row < rows) y[row] = (MODE & kLimbResid) != 0 ? __fadd_rn(xres[row], v) : v;
        }
      }
    } else if constexpr ((MODE & kLimbPairSilu) == 0) {  // the pair mode takes one window only
      // one copy of the dot, its sum selected into row group cq's accumulator
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float t = F::dot(L[r], xl, lane, flags);
        const float v = ok ? t : 0.f;
#pragma unroll
        for (int q = 0; q < MAXQ; ++q) acc[q][r] = q == cq ? acc[q][r] + v : acc[q][r];
      }
    }
    if (++cq == my) {
      cq = 0;
      ++cw;
    }
  };
  for (int i = 0; i < n_items; i += 2) {
    issue(B);
    step(A);
    issue(A);
    if (i + 1 < n_items) step(B);
  }
  if constexpr (NPRE == 1 || (MODE & kLimbPairSilu) != 0) return;  // stored as computed
#pragma unroll
  for (int q = 0; q < MAXQ; ++q) {
    if (q < my) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float t = wave_sum_dpp(acc[q][r]);
        const int row = (rg0 + q) * R + r;
        if (lane == 63 && row < rows) y[row] = (MODE & kLimbResid) != 0 ? __fadd_rn(xres[row], t) : t;
      }
    }
  }
}

// ------------------------------------------------------- F32 / F16 / BF16 --
// Plain-float rows (quant.rs ids 0, 1, 30: the router and shared-expert gate
// tensors real files carry). As ops::gemv (ops.rs:14-28) every product
// w * x is exact in f64 and the row sum accumulates in f64 before the cast
// to f32; here a workgroup of 256 threads takes a row, thread t summing
// columns t, t + 256, ... (eight loads in flight before their products),
// and the 256 partial sums are added by wave butterflies and then in wave
// order through LDS, so only the order of the f64 additions differs from
// the sequential loop. Each weight is loaded once for all NB vectors.
template <int Q>
__device__ __forceinline__ float plain_at(const uint8_t* row, int c) {
  if constexpr (Q == kF32) return reinterpret_cast<const float*>(row)[c];
  const uint32_t h = reinterpret_cast<const uint16_t*>(row)[c];
  if constexpr (Q == kF16) return h2f(h);
  return __builtin_bit_cast(float, h << 16);  // BF16
}

constexpr int kPlainThreads = 256, kPlainUnroll = 8;

template <int Q, int NB, bool XB>
__global__ void __launch_bounds__(kPlainThreads) gemv_plain_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                                  int64_t row_bytes, const float* __restrict__ x,
                                                                  float* __restrict__ y, const uint8_t* __restrict__ w2,
                                                                  int rows2, float* __restrict__ y2) {
  __shared__ double part[kPlainThreads / kWave][NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // workgroups past `rows` take the rows of a second matrix of the same type
  // and width (the MoE layer's gate-input row beside its router), against x
  // as given (XB rounds only the first matrix's x) and into y2 [b][rows2]
  const bool tail = int(blockIdx.x) >= rows;
  const int r = tail ? int(blockIdx.x) - rows : int(blockIdx.x);
  const uint8_t* row = (tail ? w2 : w) + int64_t(r) * row_bytes;
  const bool round_x = XB && !tail;
  double acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0;
  constexpr int kStep = kPlainThreads * kPlainUnroll;
  for (int c0 = 0; c0 < cols; c0 += kStep) {
    float wv[kPlainUnroll], xv[kPlainUnroll][NB];
#pragma unroll
    for (int k = 0; k < kPlainUnroll; ++k) {
      const int c = min(c0 + k * kPlainThreads + tid, cols - 1);
      wv[k] = plain_at<Q>(row, c);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float v = x[int64_t(b) * cols + c];
        xv[k][b] = round_x ? bf16_rne(v) : v;  // XB: the matvec of bf16(x)
      }
    }
#pragma unroll
    for (int k = 0; k < kPlainUnroll; ++k) {
      if (c0 + k * kPlainThreads + tid < cols) {
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = __builtin_fma(double(wv[k]), double(xv[k][b]), acc[b]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    double v = acc[b];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    if (lane == 0) part[wave][b] = v;
  }
  __syncthreads();
  if (tid < NB) {
    double v = part[0][tid];
#pragma unroll
    for (int k = 1; k < kPlainThreads / kWave; ++k) v += part[k][tid];
    if (tail)
      y2[int64_t(tid) * rows2 + r] = float(v);
    else
      y[int64_t(tid) * rows + r] = float(v);
  }
}

template <int Q, bool XB>
static hipError_t launch_plain(int nb, const uint8_t* w, int rows, int cols, int64_t row_bytes, const float* x,
                               float* y, hipStream_t s, const uint8_t* w2 = nullptr, int rows2 = 0,
                               float* y2 = nullptr) {
  const dim3 grid = dim3(unsigned(rows + rows2)), block = dim3(kPlainThreads);
#define SH_PLAIN(N)                                                                                           \
  hipLaunchKernelGGL((gemv_plain_kernel<Q, N, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y, w2, rows2, \
                     y2)
  switch (nb) {
    case 1: SH_PLAIN(1); break;
    case 2: SH_PLAIN(2); break;
    case 3: SH_PLAIN(3); break;
    case 4: SH_PLAIN(4); break;
    case 5: SH_PLAIN(5); break;
    case 6: SH_PLAIN(6); break;
    case 7: SH_PLAIN(7); break;
    default: SH_PLAIN(8);
  }
#undef SH_PLAIN
  return hipGetLastError();
}

// --------------------------------------------------- Q8_0, odd blocks --
// Q8_0 rows with an odd number of 32-element blocks (cols % 64 == 32, e.g.
// the reference's one-block gemv case, ops_tests.rs:44-61): the 64-column
// lane units above do not fit them, and such rows start on 2-byte
// boundaries. A wave per row, lane l taking blocks l, l + 64, ... with
// 2-byte loads of the 34-byte block; each weight is dequantized as
// strata-gguf does (one f32 product q * d, dequant.rs:123-128) and the dot
// is summed in f64 as ops::gemv (ops.rs:14-28), the lanes' sums added by a
// butterfly: only the order of the f64 additions differs from the
// sequential loop.
template <int NB>
__global__ void __launch_bounds__(256) gemv_q8_odd_kernel(const uint8_t* __restrict__ w, int rows, int nblk,
                                                          int64_t row_bytes, const float* __restrict__ x,
                                                          float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform
  const uint8_t* row = w + int64_t(r) * row_bytes;
  const int64_t cols = int64_t(nblk) * 32;
  double acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0;
  for (int k = lane; k < nblk; k += kWave) {
    const uint8_t* blk = row + int64_t(k) * 34;
    const float d = h2f(*reinterpret_cast<const uint16_t*>(blk));
#pragma unroll 4
    for (int j = 0; j < 32; j += 2) {
      const uint32_t q2 = *reinterpret_cast<const uint16_t*>(blk + 2 + j);
      const float w0 = float(int8_t(q2 & 0xFFu)) * d, w1 = float(int8_t(q2 >> 8)) * d;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float* xb = x + b * cols + int64_t(k) * 32 + j;
        acc[b] = __builtin_fma(double(w0), double(xb[0]), acc[b]);
        acc[b] = __builtin_fma(double(w1), double(xb[1]), acc[b]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    double v = acc[b];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    if (lane == 0) y[int64_t(b) * rows + r] = float(v);
  }
}

template <int NB>
static hipError_t launch_q8_odd_nb(const uint8_t* w, int rows, int nblk, int64_t row_bytes, const float* x, float* y,
                                   hipStream_t s) {
  hipLaunchKernelGGL((gemv_q8_odd_kernel<NB>), dim3(unsigned((rows + 3) / 4)), dim3(256), 0, s, w, rows, nblk,
                     row_bytes, x, y);
  return hipGetLastError();
}

static hipError_t launch_q8_odd(int nb, const uint8_t* w, int rows, int cols, const float* x, float* y,
                                hipStream_t s) {
  const int nblk = cols / 32;
  const int64_t rb = int64_t(nblk) * 34;
  switch (nb) {
    case 1: return launch_q8_odd_nb<1>(w, rows, nblk, rb, x, y, s);
    case 2: return launch_q8_odd_nb<2>(w, rows, nblk, rb, x, y, s);
    case 3: return launch_q8_odd_nb<3>(w, rows, nblk, rb, x, y, s);
    case 4: return launch_q8_odd_nb<4>(w, rows, nblk, rb, x, y, s);
    case 5: return launch_q8_odd_nb<5>(w, rows, nblk, rb, x, y, s);
    case 6: return launch_q8_odd_nb<6>(w, rows, nblk, rb, x, y, s);
    case 7: return launch_q8_odd_nb<7>(w, rows, nblk, rb, x, y, s);
    default: return launch_q8_odd_nb<8>(w, rows, nblk, rb, x, y, s);
  }
}

// ---------------------------------------------------------------- launch --
// CU count of the current device, queried once per device. The cache is
// atomic: the entry points are called from several threads at once.
static int cu_count() {
  constexpr int kDevs = 64;
  static std::atomic<int> cache[kDevs];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  int n = dev < kDevs ? cache[dev].load(std::memory_order_relaxed) : 0;
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < kDevs) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

constexpr size_t kMaxLds = 160 * 1024;

static size_t lds_bytes(int cols, int nb) { return size_t(nb) * x_stride(cols) * sizeof(float); }

bool gemv_shape_ok(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  if (rows <= 0 || cols <= 0 || batch < 1 || batch > 8) return false;
  if (plain_quant(quant)) return rows <= (int64_t(1) << 31) - 1 && cols <= (int64_t(1) << 30);
  if (!gemv_quant(quant)) return false;
  if (rows > (int64_t(1) << 31) - 1 || cols > (int64_t(1) << 20)) return false;
  if (cols % geometry(quant).block != 0) return false;
  if (quant == kQ8_0 && cols % 64 == 32) return true;  // odd blocks: gemv_q8_odd_kernel
  if (cols % 64 != 0) return false;  // 64-column lane units (Q8_0 blocks in pairs)
  return lds_bytes(int(cols), 1) <= kMaxLds;
}

template <class F, int D>
static hipError_t launch_one(const uint8_t* w, int rows, int cols, int64_t row_bytes,
                             const float* x, float* y, int q6_signed, hipStream_t stream) {
  constexpr int R = F::kR;
  const int threads = 512, wpg = threads / 64;
  const int n_rg = (rows + R - 1) / R;
  // Spread the row groups over 8 waves per CU. For the decode shapes that is
  // at most D items per wave, so each wave fills its ring once and never
  // cycles; larger matrices (the lm_head) cycle the ring.
  const int min_waves = cu_count() * 8;
  const int per_wave = (n_rg + min_waves - 1) / min_waves;
  const int waves = (n_rg + per_wave - 1) / per_wave;
  const int blocks = (waves + wpg - 1) / wpg;
  const size_t lds = lds_bytes(cols, 1);
  hipLaunchKernelGGL((gemv1_kernel<F, D>), dim3(unsigned(blocks)), dim3(threads), lds, stream, w,
                     rows, cols, row_bytes, x, y, q6_signed, per_wave);
  return hipGetLastError();
}

// Row groups spread over `waves_per_cu` waves per CU; multi-window rows keep
// at most MAXQ row groups per wave (their sums live in registers).
template <class F, int R, int MAXQ, int MODE = 0>
static hipError_t launch_limb(const uint8_t* w, int rows, int cols, int64_t row_bytes,
                              const float* x, float* y, hipStream_t stream, int threads,
                              int waves_per_cu, int flags = 0, const uint8_t* w2 = nullptr, int rows1 = 0,
                              const float* xu = nullptr, const float* xres = nullptr, bool spread = false) {
  if constexpr (std::is_same<F, LimbQ6K>::value) {
    // Q6_K rows of whole 4096-column windows on 16-byte boundaries are read
    // a window at a time (LimbWin; 4096x12288: 13.5 -> 11.9 us)
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                         (w2 == nullptr || (reinterpret_cast<uintptr_t>(w2) & 15u) == 0) && row_bytes % 16 == 0;
    const size_t lds = size_t(limb_lds_bytes(cols)) + size_t(LimbX<LimbWin<LimbQ6K>>::kWaveLds) * (threads / 64);
    if (cols % 4096 == 0 && aligned && lds <= kMaxLds)
      return launch_limb<LimbWin<LimbQ6K>, R, MAXQ, MODE>(w, rows, cols, row_bytes, x, y, stream, threads,
                                                          waves_per_cu, flags, w2, rows1, xu, xres, spread);
  }
  const int wpg = threads / 64;
  const int n_rg = (rows + R - 1) / R;
  const int units = cols >> 6, nwin = (units + 63) >> 6;
  // 512 threads stage 4096 columns a round, so the kernel's x rounds NPRE
  // equal its windows when there is one (the single-window code is chosen
  // at compile time); the paired gate/up rows take one window only
  if (threads != 512 || ((MODE & kLimbPairSilu) != 0 && nwin != 1)) return hipErrorInvalidValue;
  // units that read whole windows through LDS take rows of whole windows
  if (LimbX<F>::kWaveLds > 0 && (cols % 4096 != 0 || row_bytes != int64_t(nwin) * F::kWinBytes))
    return hipErrorInvalidValue;
  const int min_waves = cu_count() * waves_per_cu;
  int per = (n_rg + min_waves - 1) / min_waves;
  // row sums in registers across windows: at most MAXQ row groups a wave;
  // single-window rows are stored as they complete, so a wave takes its
  // share of the rows in one pass of resident waves
  if (nwin > 1 && per > MAXQ) per = MAXQ;
  if (nwin == 1 && per > kLimbMaxRowsOneWin) per = kLimbMaxRowsOneWin;
  const int waves = (n_rg + per - 1) / per;
  const int blocks = (waves + wpg - 1) / wpg;
  // spread rows: each of the launch's waves takes every W-th row group
  if (spread && nwin == 1) per = (n_rg + blocks * wpg - 1) / (blocks * wpg);
  // x rounds (threads * 8 columns each) whose loads go ahead of the weights
  const int rounds = (cols + threads * 8 - 1) / (threads * 8);
  const dim3 grid = dim3(unsigned(blocks)), block = dim3(unsigned(threads));
  const size_t lds = size_t(limb_lds_bytes(cols)) + size_t(LimbX<F>::kWaveLds) * wpg;
  if (rounds <= 1 && spread)
    hipLaunchKernelGGL((gemv_limb_kernel<F, R, MAXQ, MODE, 1, true>), grid, block, lds, stream, w, rows, cols,
                       row_bytes, x, y, per, flags, w2, rows1, xu, xres);
  else if (rounds <= 1)
    hipLaunchKernelGGL((gemv_limb_kernel<F, R, MAXQ, MODE, 1>), grid, block, lds, stream, w, rows, cols, row_bytes, x,
                       y, per, flags, w2, rows1, xu, xres);
  else if (rounds == 2)
    hipLaunchKernelGGL((gemv_limb_kernel<F, R, MAXQ, MODE, 2>), grid, block, lds, stream, w, rows, cols, row_bytes, x,
                       y, per, flags, w2, rows1, xu, xres);
  else
    hipLaunchKernelGGL((gemv_limb_kernel<F, R, MAXQ, MODE, 3>), grid, block, lds, stream, w, rows, cols, row_bytes, x,
                       y, per, flags, w2, rows1, xu, xres);
  return hipGetLastError();
}

template <class F, int NB>
static hipError_t launch_fmt(const uint8_t* w, int rows, int cols, int64_t row_bytes,
                             const float* x, float* y, int q6_signed, hipStream_t stream) {
  constexpr int R = (NB == 1) ? F::kR : 1;
  const int threads = 512, wpg = threads / 64;
  const int n_rg = (rows + R - 1) / R;
  int64_t blocks = (n_rg + wpg - 1) / wpg;
  const int64_t cap = int64_t(cu_count()) * 2;
  if (blocks > cap) blocks = cap;
  const size_t lds = lds_bytes(cols, NB);
  hipLaunchKernelGGL((gemv_kernel<F, NB>), dim3(unsigned(blocks)), dim3(threads), lds, stream, w,
                     rows, cols, row_bytes, x, y, q6_signed);
  return hipGetLastError();
}

template <class F>
static hipError_t launch_nb(int nb, const uint8_t* w, int rows, int cols, int64_t row_bytes,
                            const float* x, float* y, int q6_signed, hipStream_t s) {
  switch (nb) {
    case 1: return launch_one<F, F::kRing>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 2: return launch_fmt<F, 2>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 3: return launch_fmt<F, 3>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 4: return launch_fmt<F, 4>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 5: return launch_fmt<F, 5>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 6: return launch_fmt<F, 6>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 7: return launch_fmt<F, 7>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    case 8: return launch_fmt<F, 8>(w, rows, cols, row_bytes, x, y, q6_signed, s);
    default: return hipErrorInvalidValue;
  }
}

// Batched Q4_K / Q5_K rows convert their activations once per call into the
// workspace (each workgroup then copies its window rather than converting
// it), and rows wider than one window run split-K over the windows.
size_t gemv_workspace_bytes(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  return batch >= 2 && gemv_mfma_ok(quant, rows, cols, batch) ? gemv_mfma_workspace_bytes(rows, cols) : 0;
}

hipError_t launch_gemv(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                       float* y, int batch, int q6_signed, hipStream_t stream, void* ws) {
  if (!gemv_shape_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  const int64_t row_bytes = byte_size(quant, cols);
  if (plain_quant(quant)) {
    // elements are read at their own alignment (4 bytes for F32, 2 otherwise)
    if (reinterpret_cast<uintptr_t>(w) & uintptr_t(quant == kF32 ? 3 : 1)) return hipErrorInvalidValue;
    switch (quant) {
      case kF32: return launch_plain<kF32, false>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
      case kF16: return launch_plain<kF16, false>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
      default: return launch_plain<kBF16, false>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
    }
  }
  // Q8_0 rows of an odd number of blocks (2-byte aligned rows, 2-byte loads)
  if (quant == kQ8_0 && cols % 64 == 32) {
    if ((reinterpret_cast<uintptr_t>(w) & 1u)) return hipErrorInvalidValue;
    return launch_q8_odd(batch, w, int(rows), int(cols), x, y, stream);
  }
  // Q8_0 reads 68-byte block pairs with dword loads: rows must start on a
  // dword boundary (row_bytes is 68 * cols/64, so only the base matters).
  if ((quant == kQ8_0 || quant == kIQ4_XS) && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(w) & 1u) || (reinterpret_cast<uintptr_t>(x) & 15u))
    return hipErrorInvalidValue;
  if (batch >= 2 && gemv_mfma_ok(quant, rows, cols, batch))
    return launch_gemv_mfma(quant, w, rows, cols, x, y, batch, cu_count(), stream, ws);
  // batch 1: 16 waves per CU for tall matrices whose rows are a single
  // 4096-column window (more waves hide more latency, and each still has
  // rows to stream); 8 otherwise (fewer workgroups stage x, and multi-window
  // rows keep the x limbs of every window they visit)
  const int wpc = (cols <= 4096 && rows >= 8192) ? 16 : 8;
  const bool spread = wpc == 16;  // tall single-window matrices: rows spread over the waves
  // x for all of the batch must fit in LDS; a larger batch runs in slices
  int per = int(kMaxLds / lds_bytes(int(cols), 1));
  if (per > 8) per = 8;
  for (int b0 = 0; b0 < batch; b0 += per) {
    const int nb = batch - b0 < per ? batch - b0 : per;
    const float* xb = x + int64_t(b0) * cols;
    float* yb = y + int64_t(b0) * rows;
    hipError_t e;
    switch (quant) {
      case kQ4_K:
        e = nb == 1 ? launch_limb<LimbQ4K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc, 0,
                                                  nullptr, 0, nullptr, nullptr, spread)
                    : launch_nb<FmtQ4K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kQ8_0:
        e = nb == 1 ? launch_limb<LimbQ8, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc, 0,
                                                 nullptr, 0, nullptr, nullptr, spread)
                    : launch_nb<FmtQ8>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kQ5_K:
        e = nb == 1 ? launch_limb<LimbQ5K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc, 0,
                                                  nullptr, 0, nullptr, nullptr, spread)
                    : launch_nb<FmtQ5K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kIQ4_XS:  // the reading (reference or ggml qs bytes) is a template argument
        if (q6_signed)
          e = nb == 1 ? launch_limb<LimbIQ4XS<true>, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512,
                                                            wpc, 0, nullptr, 0, nullptr, nullptr, spread)
                      : launch_nb<FmtIQ4XS<true>>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        else
          e = nb == 1 ? launch_limb<LimbIQ4XS<false>, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512,
                                                             wpc, 0, nullptr, 0, nullptr, nullptr, spread)
                      : launch_nb<FmtIQ4XS<false>>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      default:  // kQ6_K
        e = nb == 1 ? launch_limb<LimbQ6K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc,
                                                  q6_signed, nullptr, 0, nullptr, nullptr, spread)
                    : launch_nb<FmtQ6K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, q6_signed, stream);
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv_plain_bf16x(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                                   float* y, int batch, hipStream_t stream) {
  if (!plain_quant(quant) || !gemv_shape_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  if (reinterpret_cast<uintptr_t>(w) & uintptr_t(quant == kF32 ? 3 : 1)) return hipErrorInvalidValue;
  const int64_t row_bytes = byte_size(quant, cols);
  switch (quant) {
    case kF32: return launch_plain<kF32, true>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
    case kF16: return launch_plain<kF16, true>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
    default: return launch_plain<kBF16, true>(batch, w, int(rows), int(cols), row_bytes, x, y, stream);
  }
}

hipError_t launch_gemv_plain_pair(uint32_t quant, const void* w1, int64_t rows1, const void* w2, int64_t rows2,
                                  int64_t cols, const float* x, float* y1, float* y2, int batch, hipStream_t stream) {
  if (!plain_quant(quant) || !gemv_shape_ok(quant, rows1 + rows2, cols, batch) || rows2 < 0)
    return hipErrorInvalidValue;
  const uint8_t* a = static_cast<const uint8_t*>(w1);
  const uint8_t* b = static_cast<const uint8_t*>(w2);
  const uintptr_t al = uintptr_t(quant == kF32 ? 3 : 1);
  if ((reinterpret_cast<uintptr_t>(a) & al) || (reinterpret_cast<uintptr_t>(b) & al)) return hipErrorInvalidValue;
  const int64_t row_bytes = byte_size(quant, cols);
  switch (quant) {
    case kF32:
      return launch_plain<kF32, true>(batch, a, int(rows1), int(cols), row_bytes, x, y1, stream, b, int(rows2), y2);
    case kF16:
      return launch_plain<kF16, true>(batch, a, int(rows1), int(cols), row_bytes, x, y1, stream, b, int(rows2), y2);
    default:
      return launch_plain<kBF16, true>(batch, a, int(rows1), int(cols), row_bytes, x, y1, stream, b, int(rows2), y2);
  }
}

// The shared expert of a MoE layer for one token in two limb launches: [g; u]
// = [gate; up] . x (one launch, x staged once), then d = down . (silu(g) * u)
// with silu(g) * u formed as the down launch stages its x.
bool shexp_fused_ok(uint32_t q_gu, uint32_t q_d, int64_t n_embd, int64_t n_ff) {
  auto limb = [](uint32_t q) { return q == kQ4_K || q == kQ8_0 || q == kQ5_K || q == kQ6_K; };
  return limb(q_gu) && limb(q_d) && n_embd % 64 == 0 && n_ff % 64 == 0 &&
         gemv_shape_ok(q_gu, 2 * n_ff, n_embd, 1) && gemv_shape_ok(q_d, n_embd, n_ff, 1) &&
         2 * n_ff <= (int64_t(1) << 30);
}

hipError_t launch_shexp_one(uint32_t q_gu, uint32_t q_d, const void* gate, const void* up, const void* down,
                            int64_t n_embd, int64_t n_ff, const float* x, float* gu, float* d, int q6gu, int q6d,
                            hipStream_t s) {
  if (!shexp_fused_ok(q_gu, q_d, n_embd, n_ff)) return hipErrorInvalidValue;
  const auto* g = static_cast<const uint8_t*>(gate);
  const auto* u = static_cast<const uint8_t*>(up);
  const auto* w = static_cast<const uint8_t*>(down);
  const int64_t rb1 = byte_size(q_gu, n_embd), rb2 = byte_size(q_d, n_ff);
  const int E = int(n_embd), N = int(n_ff);
  hipError_t e;
  if (E <= 4096) {
    // gate and up in one launch, a gate row and an up row per item, storing
    // h = silu(g) * u (gu[0, N)); down stages h as its x
    switch (q_gu) {
      case kQ4_K: e = launch_limb<LimbQ4K, 2, 4, kLimbPairSilu>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
      case kQ8_0: e = launch_limb<LimbQ8, 2, 4, kLimbPairSilu>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
      case kQ5_K: e = launch_limb<LimbQ5K, 2, 4, kLimbPairSilu>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
      default: e = launch_limb<LimbQ6K, 2, 4, kLimbPairSilu>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N);
    }
    if (e != hipSuccess) return e;
    switch (q_d) {
      case kQ4_K: return launch_limb<LimbQ4K, 1, 4, kLimbFine>(w, E, N, rb2, gu, d, s, 512, 8, q6d);
      case kQ8_0: return launch_limb<LimbQ8, 1, 4, kLimbFine>(w, E, N, rb2, gu, d, s, 512, 8, q6d);
      case kQ5_K: return launch_limb<LimbQ5K, 1, 4, kLimbFine>(w, E, N, rb2, gu, d, s, 512, 8, q6d);
      default: return launch_limb<LimbQ6K, 1, 4, kLimbFine>(w, E, N, rb2, gu, d, s, 512, 8, q6d);
    }
  }
  // wider rows: [g; u] in one launch, silu(g) * u formed as down stages its x
  switch (q_gu) {
    case kQ4_K: e = launch_limb<LimbQ4K, 1, 4, kLimbTwoMat>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
    case kQ8_0: e = launch_limb<LimbQ8, 1, 4, kLimbTwoMat>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
    case kQ5_K: e = launch_limb<LimbQ5K, 1, 4, kLimbTwoMat>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N); break;
    default: e = launch_limb<LimbQ6K, 1, 4, kLimbTwoMat>(g, 2 * N, E, rb1, x, gu, s, 512, 8, q6gu, u, N);
  }
  if (e != hipSuccess) return e;
  switch (q_d) {
    case kQ4_K: return launch_limb<LimbQ4K, 1, 4, kLimbSiluX>(w, E, N, rb2, gu, d, s, 512, 8, q6d, nullptr, 0, gu + N);
    case kQ8_0: return launch_limb<LimbQ8, 1, 4, kLimbSiluX>(w, E, N, rb2, gu, d, s, 512, 8, q6d, nullptr, 0, gu + N);
    case kQ5_K: return launch_limb<LimbQ5K, 1, 4, kLimbSiluX>(w, E, N, rb2, gu, d, s, 512, 8, q6d, nullptr, 0, gu + N);
    default: return launch_limb<LimbQ6K, 1, 4, kLimbSiluX>(w, E, N, rb2, gu, d, s, 512, 8, q6d, nullptr, 0, gu + N);
  }
}

// One token through the dense FFN's two matvec launches (limb kernels):
// h = silu(gate . x) * (up . x) (both n_ff x n_embd, one launch, x staged
// once, each wave taking gate row q and up row q together), then
// out = xres + down . h (the residual add inside).
template <class F>
static hipError_t launch_ffn1(const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_embd, int n_ff,
                              const float* x, float* gu, const float* xres, float* out, int q6s, hipStream_t s) {
  const int64_t rb1 = byte_size(F::kQuant, n_embd), rb2 = byte_size(F::kQuant, n_ff);
  // gate and up: n_ff row pairs, one window when n_embd <= 4096: 16 waves
  // per CU as for other tall single-window matrices
  // a gate row and an up row per item, storing h = silu(g) * u into gu[0, n_ff);
  // down stages h as its x
  if (n_embd <= 4096) {
    hipError_t e = launch_limb<F, 2, 4, kLimbPairSilu>(gate, 2 * n_ff, n_embd, rb1, x, gu, s, 512, 16, q6s, up, n_ff);
    if (e != hipSuccess) return e;
    return launch_limb<F, 1, 4, kLimbResid>(down, n_embd, n_ff, rb2, gu, out, s, 512, 8, q6s, nullptr, 0, nullptr,
                                            xres);
  }
  // wider rows: [g; u] in one launch, silu(g) * u formed as down stages its x
  hipError_t e = launch_limb<F, 1, 4, kLimbTwoMat>(gate, 2 * n_ff, n_embd, rb1, x, gu, s, 512, 16, q6s, up, n_ff);
  if (e != hipSuccess) return e;
  return launch_limb<F, 1, 4, kLimbSiluX | kLimbResid>(down, n_embd, n_ff, rb2, gu, out, s, 512, 8, q6s, nullptr,
                                                       0, gu + n_ff, xres);
}

bool ffn_fused_ok(uint32_t quant, int64_t n_embd, int64_t n_ff) {
  return (quant == kQ4_K || quant == kQ8_0 || quant == kQ5_K || quant == kQ6_K) &&
         n_embd % 64 == 0 && n_ff % 64 == 0 &&  // the limb kernels' 64-column units
         gemv_shape_ok(quant, 2 * n_ff, n_embd, 1) && gemv_shape_ok(quant, n_embd, n_ff, 1) &&
         n_ff % 4 == 0 && 2 * n_ff <= (int64_t(1) << 30);
}

hipError_t launch_ffn_one(uint32_t quant, const void* gate, const void* up, const void* down, int64_t n_embd,
                          int64_t n_ff, const float* x, float* gu, const float* xres, float* out, int q6s,
                          hipStream_t s) {
  if (!ffn_fused_ok(quant, n_embd, n_ff)) return hipErrorInvalidValue;
  const auto* g = static_cast<const uint8_t*>(gate);
  const auto* u = static_cast<const uint8_t*>(up);
  const auto* d = static_cast<const uint8_t*>(down);
  switch (quant) {
    case kQ4_K: return launch_ffn1<LimbQ4K>(g, u, d, int(n_embd), int(n_ff), x, gu, xres, out, q6s, s);
    case kQ8_0: return launch_ffn1<LimbQ8>(g, u, d, int(n_embd), int(n_ff), x, gu, xres, out, q6s, s);
    case kQ5_K: return launch_ffn1<LimbQ5K>(g, u, d, int(n_embd), int(n_ff), x, gu, xres, out, q6s, s);
    default: return launch_ffn1<LimbQ6K>(g, u, d, int(n_embd), int(n_ff), x, gu, xres, out, q6s, s);
  }
}

}  // namespace sh
