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

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// ---------------------------------------------------------------- x slice --
struct XSlice {
  f32x4 v[16];  // the lane's 64 floats, in column order
  f32x4 s;      // sums of x over its four 16-column groups
};

// LDS layout of one x vector with `cols` columns: floats at e + 4*(e/64),
// then cols/16 partial sums.
__host__ __device__ inline int x_stride(int cols) { return cols + cols / 16 + cols / 16; }

__device__ __forceinline__ void load_xslice(const float* xs, int cols, int unit, XSlice& o) {
  const f32x4* p = reinterpret_cast<const f32x4*>(xs + 64 * unit + 4 * unit);
#pragma unroll
  for (int i = 0; i < 16; ++i) o.v[i] = p[i];
  const float* sums = xs + cols + cols / 16;
  o.s = *reinterpret_cast<const f32x4*>(sums + 4 * unit);
}

// Stage nb vectors of x (row-major [nb][cols]) into LDS with per-16 sums.
__device__ __forceinline__ void stage_x(float* lds, const float* __restrict__ x, int cols, int nb) {
  const int groups = cols / 16;
  for (int t = threadIdx.x; t < nb * groups; t += blockDim.x) {
    int b = t / groups, g = t - b * groups;
    const f32x4* src = reinterpret_cast<const f32x4*>(x + int64_t(b) * cols + 16 * g);
    f32x4 a = src[0], c = src[1], e = src[2], f = src[3];
    float* dst = lds + b * x_stride(cols);
    int e0 = 16 * g;
    f32x4* d = reinterpret_cast<f32x4*>(dst + e0 + 4 * (e0 >> 6));
    d[0] = a;
    d[1] = c;
    d[2] = e;
    d[3] = f;
    float s = ((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w)) +
              (((e.x + e.y) + (e.z + e.w)) + ((f.x + f.y) + (f.z + f.w)));
    dst[cols + cols / 16 + g] = s;
  }
}

// ------------------------------------------------------------------ Q4_K --
// Unit u of a row: super-block u/4, group g = u%4 (elements 64g..64g+63 of
// the super-block: low nibbles of qs[32g..32g+31] are sub-block 2g, high
// nibbles sub-block 2g+1).
struct FmtQ4K {
  static constexpr int kR = 2;
  static constexpr int kRing = 4;
  struct Load {
    u32x4 h, a, b;
  };
  __device__ static __forceinline__ void load(const uint8_t* row, int u, Load& o) {
    const uint8_t* sb = row + (u >> 2) * 144;
    int g = u & 3;
    o.h = ld16(sb);
    o.a = ld16(sb + 16 + 32 * g);
    o.b = ld16(sb + 32 + 32 * g);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XSlice& x, int u, int) {
    const int g = u & 3;
    // (scale, min) of sub-blocks 2g and 2g+1 in the two low bytes of scp/mp,
    // from the packed 12 bytes (dequant.rs:237-245).
    const uint32_t sh = (g & 1) << 4;
    const uint32_t t1 = L.h.y >> sh, t2 = L.h.z >> sh, t3 = L.h.w >> sh;
    const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
    const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
    const float d = h2f(L.h.x), dm = h2f(L.h.x >> 16);
    uint32_t q[8] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w};
    float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t lo = q[k] & 0x0F0F0F0Fu;  // nibble values
      const uint32_t hi = q[k] & 0xF0F0F0F0u;  // 16 * nibble values
      const f32x4 xl = x.v[k], xh = x.v[8 + k];
      lo0 = __builtin_fmaf(ubyte<0>(lo), xl.x, lo0);
      lo1 = __builtin_fmaf(ubyte<1>(lo), xl.y, lo1);
      lo0 = __builtin_fmaf(ubyte<2>(lo), xl.z, lo0);
      lo1 = __builtin_fmaf(ubyte<3>(lo), xl.w, lo1);
      hi0 = __builtin_fmaf(ubyte<0>(hi), xh.x, hi0);
      hi1 = __builtin_fmaf(ubyte<1>(hi), xh.y, hi1);
      hi0 = __builtin_fmaf(ubyte<2>(hi), xh.z, hi0);
      hi1 = __builtin_fmaf(ubyte<3>(hi), xh.w, hi1);
    }
    const float x0 = x.s.x + x.s.y, x1 = x.s.z + x.s.w;
    const float qsum = ubyte<0>(scp) * (lo0 + lo1) + (ubyte<1>(scp) * 0.0625f) * (hi0 + hi1);
    const float msum = ubyte<0>(mp) * x0 + ubyte<1>(mp) * x1;
    return d * qsum - dm * msum;
  }
};

// ------------------------------------------------------------------ Q5_K --
// Unit u of a row: super-block u/4, group g = u%4, as FmtQ4K, with the fifth
// code bit of q5k_codes. Every lane of a super-block reads its 16 header and
// 32 qh bytes.
struct FmtQ5K {
  static constexpr int kR = 2;
  static constexpr int kRing = 4;
  struct Load {
    u32x4 h, h0, h1, a, b;
  };
  __device__ static __forceinline__ void load(const uint8_t* row, int u, Load& o) {
    const uint8_t* sb = row + (u >> 2) * 176;
    const int g = u & 3;
    o.h = ld16(sb);
    o.h0 = ld16(sb + 16);
    o.h1 = ld16(sb + 32);
    o.a = ld16(sb + 48 + 32 * g);
    o.b = ld16(sb + 64 + 32 * g);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XSlice& x, int u, int) {
    const int g = u & 3;
    uint32_t scp, mp;
    k4_pair(L.h, g, scp, mp);
    const float d = h2f(L.h.x), dm = h2f(L.h.x >> 16);
    const uint32_t q[8] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w};
    const uint32_t qh[8] = {L.h0.x, L.h0.y, L.h0.z, L.h0.w, L.h1.x, L.h1.y, L.h1.z, L.h1.w};
    float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t lo, hi;
      q5k_codes(q[k], qh[k], uint32_t(g), lo, hi);
      const f32x4 xl = x.v[k], xh = x.v[8 + k];
      lo0 = __builtin_fmaf(ubyte<0>(lo), xl.x, lo0);
      lo1 = __builtin_fmaf(ubyte<1>(lo), xl.y, lo1);
      lo0 = __builtin_fmaf(ubyte<2>(lo), xl.z, lo0);
      lo1 = __builtin_fmaf(ubyte<3>(lo), xl.w, lo1);
      hi0 = __builtin_fmaf(ubyte<0>(hi), xh.x, hi0);
      hi1 = __builtin_fmaf(ubyte<1>(hi), xh.y, hi1);
      hi0 = __builtin_fmaf(ubyte<2>(hi), xh.z, hi0);
      hi1 = __builtin_fmaf(ubyte<3>(hi), xh.w, hi1);
    }
    const float x0 = x.s.x + x.s.y, x1 = x.s.z + x.s.w;
    const float qsum = ubyte<0>(scp) * (lo0 + lo1) + ubyte<1>(scp) * (hi0 + hi1);
    const float msum = ubyte<0>(mp) * x0 + ubyte<1>(mp) * x1;
    return d * qsum - dm * msum;
  }
};

// ------------------------------------------------------------------ Q8_0 --
// Unit u of a row: blocks 2u and 2u+1 (68 bytes, 4-byte aligned when the row
// start is, which the launcher checks).
struct FmtQ8 {
  static constexpr int kR = 2;
  static constexpr int kRing = 3;
  struct Load {
    u32x4 a, b, c, d;
    uint32_t e;
  };
  __device__ static __forceinline__ void load(const uint8_t* row, int u, Load& o) {
    const uint8_t* p = row + u * 68;
    o.a = ld16(p);
    o.b = ld16(p + 16);
    o.c = ld16(p + 32);
    o.d = ld16(p + 48);
    o.e = ld4(p + 64);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XSlice& x, int, int) {
    const uint32_t D[17] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w, L.c.x,
                            L.c.y, L.c.z, L.c.w, L.d.x, L.d.y, L.d.z, L.d.w, L.e};
    const float d0 = h2f(D[0]), d1 = h2f(D[8] >> 16);
    float s00 = 0.f, s01 = 0.f, s10 = 0.f, s11 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // signed bytes biased to unsigned: (q + 128)
      const uint32_t q0 = realign(D[k], D[k + 1], 2) ^ 0x80808080u;
      const uint32_t q1 = D[9 + k] ^ 0x80808080u;
      const f32x4 xa = x.v[k], xb = x.v[8 + k];
      s00 = __builtin_fmaf(ubyte<0>(q0), xa.x, s00);
      s01 = __builtin_fmaf(ubyte<1>(q0), xa.y, s01);
      s00 = __builtin_fmaf(ubyte<2>(q0), xa.z, s00);
      s01 = __builtin_fmaf(ubyte<3>(q0), xa.w, s01);
      s10 = __builtin_fmaf(ubyte<0>(q1), xb.x, s10);
      s11 = __builtin_fmaf(ubyte<1>(q1), xb.y, s11);
      s10 = __builtin_fmaf(ubyte<2>(q1), xb.z, s10);
      s11 = __builtin_fmaf(ubyte<3>(q1), xb.w, s11);
    }
    const float x0 = x.s.x + x.s.y, x1 = x.s.z + x.s.w;
    return d0 * ((s00 + s01) - 128.f * x0) + d1 * ((s10 + s11) - 128.f * x1);
  }
};

// ------------------------------------------------------------------ Q6_K --
// Unit u of a row: super-block u/4, quarter j = u%4 = (half h, pair tp):
// quadrants t0 = 2tp and t1 = 2tp+1 of half h (dequant.rs:217-229), i.e.
// elements 64j..64j+63 of the super-block:
//   t0, l = 0..31: low bits from ql[64h + l], high bits qh[32h + l] >> 2*t0
//   t1, l = 0..31: low bits from ql[64h + 32 + l], high bits >> 2*t1
//   the nibble is the low one for tp = 0 and the high one for tp = 1;
//   sub-block scales sc[8h + 4tp + {0,1,2,3}] cover 16 elements each.
// Super-blocks are 210 bytes, so a block starts at a 2-byte boundary: loads
// go through the dword-aligned address at or below it and are realigned by
// `shift` (0 or 2) bytes. No load leaves the block's own 210 bytes.
struct FmtQ6K {
  static constexpr int kR = 1;
  static constexpr int kRing = 4;
  struct Load {
    u32x4 l0, l1, l2, l3;
    uint32_t l4;
    u32x4 h0, h1;
    uint32_t h2;
    uint32_t s0, s1;
    uint32_t d;
    uint32_t shift;
  };
  __device__ static __forceinline__ void load(const uint8_t* row, int u, Load& o) {
    const uint8_t* blk = row + (u >> 2) * 210;
    const int j = u & 3, h = j >> 1, tp = j & 1;
    const uint32_t shift = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - shift;
    const uint8_t* ql = base + 64 * h;
    o.l0 = ld16(ql);
    o.l1 = ld16(ql + 16);
    o.l2 = ld16(ql + 32);
    o.l3 = ld16(ql + 48);
    o.l4 = ld4(ql + 64);  // ends at most at byte 131 of the block
    const uint8_t* qh = base + 128 + 32 * h;
    o.h0 = ld16(qh);
    o.h1 = ld16(qh + 16);
    o.h2 = ld4(qh + 32);  // ends at most at byte 195
    const uint8_t* sc = base + 192 + 8 * h + 4 * tp;
    o.s0 = ld4(sc);
    // a second dword is needed (and stays inside the block) only when the
    // block is misaligned; aligned, it could run 2 bytes past the block
    o.s1 = shift ? ld4(sc + 4) : 0u;
    o.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    o.shift = shift;
  }
  __device__ static __forceinline__ float dot(const Load& L, const XSlice& x, int u, int q6_signed) {
    const uint32_t tp = uint32_t(u) & 1u;
    const uint32_t s = L.shift;
    const uint32_t qlr[17] = {L.l0.x, L.l0.y, L.l0.z, L.l0.w, L.l1.x, L.l1.y, L.l1.z, L.l1.w, L.l2.x,
                              L.l2.y, L.l2.z, L.l2.w, L.l3.x, L.l3.y, L.l3.z, L.l3.w, L.l4};
    const uint32_t qhr[9] = {L.h0.x, L.h0.y, L.h0.z, L.h0.w, L.h1.x, L.h1.y, L.h1.z, L.h1.w, L.h2};
    const uint32_t scw = realign(L.s0, L.s1, s);
    const uint32_t nib = 4u * tp;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // one per 16-element sub-block
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t qh = realign(qhr[k], qhr[k + 1], s);
      // high 2 bits of quadrant t0 moved to bits 4-5 of each byte
      const uint32_t qs = tp ? qh : (qh << 4);
      const uint32_t a = ((realign(qlr[k], qlr[k + 1], s) >> nib) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
      const uint32_t b =
          ((realign(qlr[8 + k], qlr[9 + k], s) >> nib) & 0x0F0F0F0Fu) | ((qs >> 2) & 0x30303030u);
      const f32x4 xa = x.v[k], xb = x.v[8 + k];
      float& ca = acc[k >> 2];
      float& cb = acc[2 + (k >> 2)];
      ca = __builtin_fmaf(ubyte<0>(a), xa.x, ca);
      ca = __builtin_fmaf(ubyte<1>(a), xa.y, ca);
      ca = __builtin_fmaf(ubyte<2>(a), xa.z, ca);
      ca = __builtin_fmaf(ubyte<3>(a), xa.w, ca);
      cb = __builtin_fmaf(ubyte<0>(b), xb.x, cb);
      cb = __builtin_fmaf(ubyte<1>(b), xb.y, cb);
      cb = __builtin_fmaf(ubyte<2>(b), xb.z, cb);
      cb = __builtin_fmaf(ubyte<3>(b), xb.w, cb);
    }
    float sc0, sc1, sc2, sc3;
    if (q6_signed) {
      sc0 = float(int8_t(scw & 0xFFu));
      sc1 = float(int8_t((scw >> 8) & 0xFFu));
      sc2 = float(int8_t((scw >> 16) & 0xFFu));
      sc3 = float(int8_t(scw >> 24));
    } else {
      sc0 = ubyte<0>(scw);
      sc1 = ubyte<1>(scw);
      sc2 = ubyte<2>(scw);
      sc3 = ubyte<3>(scw);
    }
    const float t = sc0 * (acc[0] - 32.f * x.s.x) + sc1 * (acc[1] - 32.f * x.s.y) +
                    sc2 * (acc[2] - 32.f * x.s.z) + sc3 * (acc[3] - 32.f * x.s.w);
    return h2f(L.d) * t;
  }
};

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

// ================================================== batch-1 integer path ==
// x as three int8 limbs. Each workgroup converts the f32 activations once:
// per 32-column block a power-of-two scale 2^-k is chosen so that the block's
// largest |x| times 2^k is below 2^22, and every element becomes the integer
//   v = rne(x * 2^k) = a * 2^16 + b * 2^8 + c,  a in [-64, 64], b, c in [0, 255]
// (a is byte 2 of v, b byte 1, c byte 0, in two's complement). Each element
// is represented to within 2^-23 of its block's maximum, as close to x as the
// f32 activations themselves for elements near the maximum. Weight codes are
// small non-negative integers, so the per-block dot products are exact
// integer sums on v_dot4_i32_i8 (a) and v_dot4_u32_u8 (b, c), four weights
// per instruction:
//   sum_j q_j x_j = 2^-k (2^16 sum q a + (2^8 sum q b + sum q c)) + rounding of v
// and only the per-block scale epilogue is f32.
//
// LDS layout for `cols` columns (bytes): three limb planes, each with a
// 16-byte pad after every 64 bytes (so lanes reading 64-byte runs hit
// distinct banks), then per 32-column block 16 bytes:
//   {sum of x over columns 0-15, sum over 16-31, 2^-k, K}
// with K = sum of (v & 0xFFFF) = sum 2^8 b + c (an integer, for the bias of
// signed weights against the unsigned low limbs).
__host__ __device__ inline int plane_stride(int cols) { return cols + cols / 4; }
__host__ __device__ inline int limb_lds_bytes(int cols) { return 3 * plane_stride(cols) + (cols / 32) * 16; }

// Converts 8 consecutive columns held in registers (elements 8t .. 8t + 7,
// t the thread) and writes them to LDS. The four lanes of a 32-column block
// are t & ~3 .. t | 3, neighbours in one quad of the wave: they exchange the
// block's maximum and sums with DPP moves, and lane t & ~3 writes the block's
// record. K (the integer sum of the low limbs) is formed only when LOW is
// set: signed Q8_0 codes need it; the unsigned codes of the k-quants do not.
template <bool LOW>
__device__ __forceinline__ void limb_group8(uint8_t* lds, int cols, int t, bool valid, f32x4 a, f32x4 b) {
  const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float m = 0.f, s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m = fmaxf(m, fabsf(xs[i]));
    s += xs[i];
  }
  m = fmaxf(m, dpp_xor1(m));
  m = fmaxf(m, dpp_xor2(m));
  const float s16 = s + dpp_xor1(s);  // the lane pair's 16 columns
  const float s16_other = dpp_xor2(s16);
  // k with m * 2^k < 2^22; for m == 0 any k works
  // (clamped so 2^k stays finite for blocks whose maximum is below 2^-104)
  int e = 0;
  (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1)
  const int k = m > 0.f ? min(22 - e, 126) : 0;
  const float up = ldexpf(1.f, k);
  // a NaN or infinite block keeps its NaN through the scale
  const float down = (m - m == 0.f) ? ldexpf(1.f, -k) : __builtin_nanf("");
  uint32_t v[8];
  uint32_t low = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // rne(x * 2^k) through the 1.5 * 2^23 magic constant (|x * 2^k| < 2^22)
    const float tt = __builtin_fmaf(xs[i], up, 12582912.0f);
    v[i] = __builtin_bit_cast(uint32_t, tt) - 0x4B400000u;
    if constexpr (LOW) low += v[i] & 0xFFFFu;
  }
  if constexpr (LOW) {
    low += dpp_xor1(low);
    low += dpp_xor2(low);
  }
  if (!valid) return;
  const int e0 = 8 * t;
  const int off = e0 + 16 * (e0 >> 6);
  const int ps = plane_stride(cols);
  uint32_t pc[2], pb[2], pa[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) transpose_bytes(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3], pc[q], pb[q], pa[q]);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(lds + off) = u32x2{pa[0], pa[1]};
  *reinterpret_cast<u32x2*>(lds + ps + off) = u32x2{pb[0], pb[1]};
  *reinterpret_cast<u32x2*>(lds + 2 * ps + off) = u32x2{pc[0], pc[1]};
  if ((t & 3) == 0)
    *reinterpret_cast<u32x4*>(lds + 3 * ps + 16 * (t >> 2)) =
        u32x4{__builtin_bit_cast(uint32_t, s16), __builtin_bit_cast(uint32_t, s16_other),
              __builtin_bit_cast(uint32_t, down), low};
}

// The lane's 64 columns: limb dwords for elements 4j..4j+3 and the two
// 32-column blocks' {sum, scale}.
struct XLimbs {
  u32x4 a[4], b[4], c[4];
  u32x4 i0, i1;  // the two 32-column blocks: {sum 0-15, sum 16-31, 2^-k, K} as raw words
};

__device__ __forceinline__ float fw(uint32_t bits) { return __builtin_bit_cast(float, bits); }

__device__ __forceinline__ void load_limbs(const uint8_t* lds, int cols, int u, XLimbs& o) {
  const int ps = plane_stride(cols);
  const int off = 80 * u;  // 64 bytes + 16 pad per unit
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o.a[i] = *reinterpret_cast<const u32x4*>(lds + off + 16 * i);
    o.b[i] = *reinterpret_cast<const u32x4*>(lds + ps + off + 16 * i);
    o.c[i] = *reinterpret_cast<const u32x4*>(lds + 2 * ps + off + 16 * i);
  }
  o.i0 = *reinterpret_cast<const u32x4*>(lds + 3 * ps + 32 * u);
  o.i1 = *reinterpret_cast<const u32x4*>(lds + 3 * ps + 32 * u + 16);
}

__device__ __forceinline__ uint32_t limb_word(const u32x4* p, int j) {
  const u32x4 v = p[j >> 2];
  return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
}

// Exact sum over 4 weights (bytes of `q`, each 0..127) times 4 x elements
// (limb words a, b, c), accumulated into the three integer sums.
__device__ __forceinline__ void dot_limbs(uint32_t q, uint32_t a, uint32_t b, uint32_t c, int& sa,
                                          uint32_t& sb, uint32_t& sc) {
  sa = __builtin_amdgcn_sdot4(int(q), int(a), sa, false);
  sb = __builtin_amdgcn_udot4(q, b, sb, false);
  sc = __builtin_amdgcn_udot4(q, c, sc, false);
}

// sum q*v = 2^16 sa + 2^8 sb + sc as f32 (2^8 sb + sc < 2^25 is exact in u32)
__device__ __forceinline__ float limb_value(int sa, uint32_t sb, uint32_t sc) {
  return __builtin_fmaf(float(sa), 65536.f, float(sb * 256u + sc));
}

// Sum over the 64 lanes with DPP: quad swaps, half-row and row mirrors,
// then row broadcasts 15 and 31; lane 63 ends with the total.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // row_half_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)); // row_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false)); // row_bcast15
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false)); // row_bcast31
  return v;
}

// Q4_K with integer dots: unit u = (super-block u/4, group g = u%4) as in
// FmtQ4K; low nibbles are sub-block 2g (x block 2u), high nibbles 2g+1.
struct LimbQ4K {
  static constexpr uint32_t kQuant = kQ4_K;
  struct Load {
    u32x4 h, a, b;
  };
  static constexpr int kWinBytes = 16 * 144;  // one 4096-column window of a row
  struct Off {
    int h, q;
  };
  // h: the super-block's byte offset (advances by kWinBytes per window);
  // q: the lane's quant bytes relative to it
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 2) * 144, 16 + 32 * (u & 3)}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    L.h = ld16(row + o.h);
    L.a = ld16(row + o.h + o.q);
    L.b = ld16(row + o.h + o.q + 16);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbs& x, int lane, int) {
    const int g = lane & 3;
    const uint32_t sh = (g & 1) << 4;
    const uint32_t t1 = L.h.y >> sh, t2 = L.h.z >> sh, t3 = L.h.w >> sh;
    const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
    const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
    const float d = h2f(L.h.x), dm = h2f(L.h.x >> 16);
    const uint32_t q[8] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w};
    int a0 = 0, a1 = 0;
    uint32_t b0 = 0, b1 = 0, c0 = 0, c1 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t lo = q[k] & 0x0F0F0F0Fu;
      const uint32_t hi = (q[k] >> 4) & 0x0F0F0F0Fu;
      dot_limbs(lo, limb_word(x.a, k), limb_word(x.b, k), limb_word(x.c, k), a0, b0, c0);
      dot_limbs(hi, limb_word(x.a, 8 + k), limb_word(x.b, 8 + k), limb_word(x.c, 8 + k), a1, b1, c1);
    }
    const float s0 = limb_value(a0, b0, c0) * fw(x.i0.z);  // sum over sub-block 2g of q * x
    const float s1 = limb_value(a1, b1, c1) * fw(x.i1.z);  // sub-block 2g + 1
    const float qsum = ubyte<0>(scp) * s0 + ubyte<1>(scp) * s1;
    const float msum = ubyte<0>(mp) * (fw(x.i0.x) + fw(x.i0.y)) + ubyte<1>(mp) * (fw(x.i1.x) + fw(x.i1.y));
    return d * qsum - dm * msum;
  }
};

// Q5_K with integer dots: unit u as LimbQ4K; codes 0..31 (nibble plus the
// fifth bit, q5k_codes) go into the dots unchanged.
struct LimbQ5K {
  static constexpr uint32_t kQuant = kQ5_K;
  struct Load {
    u32x4 h, h0, h1, a, b;
  };
  static constexpr int kWinBytes = 16 * 176;
  struct Off {
    int h, q;
  };
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 2) * 176, 48 + 32 * (u & 3)}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    L.h = ld16(row + o.h);
    L.h0 = ld16(row + o.h + 16);
    L.h1 = ld16(row + o.h + 32);
    L.a = ld16(row + o.h + o.q);
    L.b = ld16(row + o.h + o.q + 16);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbs& x, int lane, int) {
    const int g = lane & 3;
    uint32_t scp, mp;
    k4_pair(L.h, g, scp, mp);
    const float d = h2f(L.h.x), dm = h2f(L.h.x >> 16);
    const uint32_t q[8] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w};
    const uint32_t qh[8] = {L.h0.x, L.h0.y, L.h0.z, L.h0.w, L.h1.x, L.h1.y, L.h1.z, L.h1.w};
    int a0 = 0, a1 = 0;
    uint32_t b0 = 0, b1 = 0, c0 = 0, c1 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t lo, hi;
      q5k_codes(q[k], qh[k], uint32_t(g), lo, hi);
      dot_limbs(lo, limb_word(x.a, k), limb_word(x.b, k), limb_word(x.c, k), a0, b0, c0);
      dot_limbs(hi, limb_word(x.a, 8 + k), limb_word(x.b, 8 + k), limb_word(x.c, 8 + k), a1, b1, c1);
    }
    const float s0 = limb_value(a0, b0, c0) * fw(x.i0.z);
    const float s1 = limb_value(a1, b1, c1) * fw(x.i1.z);
    const float qsum = ubyte<0>(scp) * s0 + ubyte<1>(scp) * s1;
    const float msum = ubyte<0>(mp) * (fw(x.i0.x) + fw(x.i0.y)) + ubyte<1>(mp) * (fw(x.i1.x) + fw(x.i1.y));
    return d * qsum - dm * msum;
  }
};

// Q8_0 with integer dots: unit u = blocks 2u and 2u+1 (68 bytes from a
// dword-aligned address). Codes are signed: the top limb (signed) takes them
// as they are; against the unsigned low limbs they are biased to q + 128 and
// the bias 128 * K is removed in integers before the one f32 conversion.
struct LimbQ8 {
  static constexpr uint32_t kQuant = kQ8_0;
  struct Load {
    u32x4 a, b, c, d;
    uint32_t e;
  };
  static constexpr int kWinBytes = 64 * 68;
  struct Off {
    int h, q;
  };
  __device__ static __forceinline__ Off offsets(int u) { return {u * 68, 0}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    const uint8_t* p = row + o.h;
    L.a = ld16(p);
    L.b = ld16(p + 16);
    L.c = ld16(p + 32);
    L.d = ld16(p + 48);
    L.e = ld4(p + 64);
  }
  __device__ static __forceinline__ float block(const uint32_t* q, const u32x4* xa, const u32x4* xb,
                                                const u32x4* xc, int j0, u32x4 info) {
    int sa = 0;
    uint32_t sb = 0, sc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t qb = q[k] ^ 0x80808080u;  // q + 128
      sa = __builtin_amdgcn_sdot4(int(q[k]), int(limb_word(xa, j0 + k)), sa, false);
      sb = __builtin_amdgcn_udot4(qb, limb_word(xb, j0 + k), sb, false);
      sc = __builtin_amdgcn_udot4(qb, limb_word(xc, j0 + k), sc, false);
    }
    const int bc = int(sb * 256u + sc) - 128 * int(info.w);
    return __builtin_fmaf(float(sa), 65536.f, float(bc)) * fw(info.z);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbs& x, int, int) {
    const uint32_t D[17] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w, L.c.x,
                            L.c.y, L.c.z, L.c.w, L.d.x, L.d.y, L.d.z, L.d.w, L.e};
    uint32_t q0[8], q1[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      q0[k] = realign(D[k], D[k + 1], 2);
      q1[k] = D[9 + k];
    }
    const float d0 = h2f(D[0]), d1 = h2f(D[8] >> 16);
    return d0 * block(q0, x.a, x.b, x.c, 0, x.i0) + d1 * block(q1, x.a, x.b, x.c, 8, x.i1);
  }
};

// IQ4_XS with integer dots: unit u = (super-block u/4, group g = u%4), the
// two 32-element sub-blocks 2g and 2g + 1 (elements 64g..64g+63). Each
// sub-block's codes are code-book values kvalues_iq4nl[nibble] in
// [-127, 113] (signed, so the dots are LimbQ8's: the top limb signed, the
// low limbs against codes biased by 128), its scale dl = d * (ls - 32) from
// the 6-bit ls. GGML: ggml's layout (sub-block ib reads qs[16 ib ..]); the
// default follows the reference, whose every sub-block reads qs[0..16]
// (dequant.rs:189-206).
__device__ __forceinline__ uint32_t iq4_lut(uint32_t idx) {  // four nibble indices -> four int8 codes
  const uint32_t i7 = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIq4Tab[1], kIq4Tab[0], i7);
  const uint32_t hi = __builtin_amdgcn_perm(kIq4Tab[3], kIq4Tab[2], i7);
  const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}

template <bool GGML>
struct LimbIQ4XS {
  static constexpr uint32_t kQuant = kIQ4_XS;
  struct Load {
    uint32_t h0, h1;  // d | scales_h, scales_l
    u32x4 a, b;       // the qs bytes of sub-blocks 2g and 2g + 1
  };
  static constexpr int kWinBytes = 16 * 136;
  struct Off {
    int h, q;
  };
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 2) * 136, GGML ? 8 + 32 * (u & 3) : 8}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    L.h0 = ld4(row + o.h);
    L.h1 = ld4(row + o.h + 4);
    L.a = ld16u(row + o.h + o.q);
    L.b = ld16u(row + o.h + o.q + (GGML ? 16 : 0));
  }
  __device__ static __forceinline__ float block(const u32x4 q, const u32x4* xa, const u32x4* xb, const u32x4* xc,
                                                int j0, u32x4 info) {
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    int sa = 0;
    uint32_t sb = 0, sc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {  // elements 4k..4k+3: low nibbles of bytes 4k.. (k < 4), high nibbles after
      const uint32_t idx = k < 4 ? (qw[k] & 0x0F0F0F0Fu) : ((qw[k - 4] >> 4) & 0x0F0F0F0Fu);
      const uint32_t v = iq4_lut(idx);
      const uint32_t vb = v ^ 0x80808080u;  // v + 128
      sa = __builtin_amdgcn_sdot4(int(v), int(limb_word(xa, j0 + k)), sa, false);
      sb = __builtin_amdgcn_udot4(vb, limb_word(xb, j0 + k), sb, false);
      sc = __builtin_amdgcn_udot4(vb, limb_word(xc, j0 + k), sc, false);
    }
    const int bc = int(sb * 256u + sc) - 128 * int(info.w);
    return __builtin_fmaf(float(sa), 65536.f, float(bc)) * fw(info.z);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbs& x, int lane, int) {
    const uint32_t g = uint32_t(lane) & 3u;
    const float d = h2f(L.h0);
    const uint32_t shb = L.h0 >> 16;                     // scales_h
    const uint32_t slb = (L.h1 >> (8 * g)) & 0xFFu;      // scales_l[g]: ls of sub-blocks 2g (low) and 2g + 1
    const uint32_t ls0 = (slb & 0x0Fu) | (((shb >> (4 * g)) & 3u) << 4);
    const uint32_t ls1 = (slb >> 4) | (((shb >> (4 * g + 2)) & 3u) << 4);
    const float dl0 = d * (float(ls0) - 32.f), dl1 = d * (float(ls1) - 32.f);
    return dl0 * block(L.a, x.a, x.b, x.c, 0, x.i0) + dl1 * block(L.b, x.a, x.b, x.c, 8, x.i1);
  }
};

// Q6_K with integer dots: unit u = (super-block u/4, quarter j = u%4) as in
// FmtQ6K; the 6-bit codes 0..63 go straight into the dots and the -32
// offset is taken off with the per-16 sums of x.
struct LimbQ6K {
  static constexpr uint32_t kQuant = kQ6_K;
  using Load = FmtQ6K::Load;
  static constexpr int kWinBytes = 16 * 210;
  struct Off {
    int h, q;
  };
  // h: the super-block's byte offset, q: the quarter 0..3
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 2) * 210, u & 3}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    FmtQ6K::load(row + o.h, o.q, L);
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbs& x, int lane, int q6_signed) {
    const uint32_t tp = uint32_t(lane) & 1u;
    const uint32_t s = L.shift;
    const uint32_t qlr[17] = {L.l0.x, L.l0.y, L.l0.z, L.l0.w, L.l1.x, L.l1.y, L.l1.z, L.l1.w, L.l2.x,
                              L.l2.y, L.l2.z, L.l2.w, L.l3.x, L.l3.y, L.l3.z, L.l3.w, L.l4};
    const uint32_t qhr[9] = {L.h0.x, L.h0.y, L.h0.z, L.h0.w, L.h1.x, L.h1.y, L.h1.z, L.h1.w, L.h2};
    const uint32_t scw = realign(L.s0, L.s1, s);
    const uint32_t nib = 4u * tp;
    int sa[4] = {0, 0, 0, 0};
    uint32_t sb[4] = {0, 0, 0, 0}, sc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t qh = realign(qhr[k], qhr[k + 1], s);
      const uint32_t qs = tp ? qh : (qh << 4);
      const uint32_t va = ((realign(qlr[k], qlr[k + 1], s) >> nib) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
      const uint32_t vb =
          ((realign(qlr[8 + k], qlr[9 + k], s) >> nib) & 0x0F0F0F0Fu) | ((qs >> 2) & 0x30303030u);
      const int ga = k >> 2, gb = 2 + (k >> 2);
      dot_limbs(va, limb_word(x.a, k), limb_word(x.b, k), limb_word(x.c, k), sa[ga], sb[ga], sc[ga]);
      dot_limbs(vb, limb_word(x.a, 8 + k), limb_word(x.b, 8 + k), limb_word(x.c, 8 + k), sa[gb], sb[gb], sc[gb]);
    }
    float scf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t byte = (scw >> (8 * i)) & 0xFFu;
      scf[i] = q6_signed ? float(int8_t(byte)) : float(byte);
    }
    const float xs[4] = {fw(x.i0.x), fw(x.i0.y), fw(x.i1.x), fw(x.i1.y)};
    const float ks[4] = {fw(x.i0.z), fw(x.i0.z), fw(x.i1.z), fw(x.i1.z)};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) t += scf[i] * (limb_value(sa[i], sb[i], sc[i]) * ks[i] - 32.f * xs[i]);
    return h2f(L.d) * t;
  }
};

// Batch-1 matvec on the integer path.
//
// Wave w owns row groups [w*per, w*per + per) of R rows. Items are
// (row group, window) pairs taken window-major, so each wave reads its x
// limbs from LDS once per window and keeps `per` (<= MAXQ) row sums per
// row in registers. All item control is wave-uniform (scalar registers);
// per-lane byte offsets within a row are computed once. Loads are
// double-buffered (A/B ping-pong, both refills unconditional so the loop
// latch never drains the load queue), and the first item is requested
// before x is staged, so weight bytes are in flight from the first cycles.
//
// MODE bits (compile-time; 0 for the plain matvec) let the dense FFN run in
// two launches: kLimbTwoMat reads rows [0, rows1) from w and [rows1, rows)
// from w2 (gate and up in one launch, x staged once); kLimbSiluX stages
// silu(x) * xu, with silu(v) = v / (1 + exp(-v)) in f32 (qwen35.rs:120-124),
// instead of x; kLimbResid writes y = xres + sum (one f32 add, qwen35.rs:127-129).
constexpr int kLimbTwoMat = 1, kLimbSiluX = 2, kLimbResid = 4;

template <class F, int R, int MAXQ, int MODE = 0, int NPRE = 1>
__global__ void __launch_bounds__(512) gemv_limb_kernel(const uint8_t* __restrict__ w, int rows,
                                                        int cols, int64_t row_bytes,
                                                        const float* __restrict__ x,
                                                        float* y, int per, int flags,
                                                        const uint8_t* __restrict__ w2, int rows1,
                                                        const float* __restrict__ xu,
                                                        const float* xres) {  // xres may be y (in place)
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  constexpr bool kLow = F::kQuant == kQ8_0 || F::kQuant == kIQ4_XS;  // signed codes: the low-limb sums
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (tid >> 6));
  const int units = cols >> 6;
  const int nwin = (units + 63) >> 6;
  const int n_rg = (rows + R - 1) / R;
  const int rg0 = wave * per;
  const int my = max(0, min(per, n_rg - rg0));  // row groups of this wave
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
      const int row = min((rg0 + qq) * R + r, rows - 1);
      const uint8_t* base = w + int64_t(row) * row_bytes;
      if constexpr ((MODE & kLimbTwoMat) != 0)
        base = row >= rows1 ? w2 + int64_t(row - rows1) * row_bytes : base;
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
  issue(A);
  auto stage = [&](int t, f32x4 a, f32x4 b, f32x4 ua, f32x4 ub) {
    if constexpr ((MODE & kLimbSiluX) != 0) {
#pragma clang fp contract(off)
      const f32x4 h0{a.x / (1.f + expf(-a.x)) * ua.x, a.y / (1.f + expf(-a.y)) * ua.y,
                     a.z / (1.f + expf(-a.z)) * ua.z, a.w / (1.f + expf(-a.w)) * ua.w};
      const f32x4 h1{b.x / (1.f + expf(-b.x)) * ub.x, b.y / (1.f + expf(-b.y)) * ub.y,
                     b.z / (1.f + expf(-b.z)) * ub.z, b.w / (1.f + expf(-b.w)) * ub.w};
      limb_group8<kLow>(lds8, cols, t, t < n8, h0, h1);
    } else {
      limb_group8<kLow>(lds8, cols, t, t < n8, a, b);
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
  __syncthreads();
  if (n_items == 0) return;

  float acc[MAXQ][R];
#pragma unroll
  for (int q = 0; q < MAXQ; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[q][r] = 0.f;
  XLimbs xl;
  int cw = 0, cq = 0;  // item being computed
  auto step = [&](const typename F::Load* L) {
    if (cq == 0) {
      const int u = cw == nwin - 1 ? ulast : cw * 64 + lane;
      load_limbs(lds8, cols, u, xl);
    }
    const bool ok = cw < nwin - 1 || lane_valid_last;
#pragma unroll
    for (int q = 0; q < MAXQ; ++q) {
      if (q == cq) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float t = F::dot(L[r], xl, lane, flags);
          acc[q][r] += ok ? t : 0.f;
        }
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
                                                                  float* __restrict__ y) {
  __shared__ double part[kPlainThreads / kWave][NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = blockIdx.x;
  const uint8_t* row = w + int64_t(r) * row_bytes;
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
        xv[k][b] = XB ? bf16_rne(v) : v;  // XB: the matvec of bf16(x)
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
    y[int64_t(tid) * rows + r] = float(v);
  }
}

template <int Q, bool XB>
static hipError_t launch_plain(int nb, const uint8_t* w, int rows, int cols, int64_t row_bytes, const float* x,
                               float* y, hipStream_t s) {
  const dim3 grid = dim3(unsigned(rows)), block = dim3(kPlainThreads);
  switch (nb) {
    case 1: hipLaunchKernelGGL((gemv_plain_kernel<Q, 1, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 2: hipLaunchKernelGGL((gemv_plain_kernel<Q, 2, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 3: hipLaunchKernelGGL((gemv_plain_kernel<Q, 3, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 4: hipLaunchKernelGGL((gemv_plain_kernel<Q, 4, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 5: hipLaunchKernelGGL((gemv_plain_kernel<Q, 5, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 6: hipLaunchKernelGGL((gemv_plain_kernel<Q, 6, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    case 7: hipLaunchKernelGGL((gemv_plain_kernel<Q, 7, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y); break;
    default: hipLaunchKernelGGL((gemv_plain_kernel<Q, 8, XB>), grid, block, 0, s, w, rows, cols, row_bytes, x, y);
  }
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
                              const float* xu = nullptr, const float* xres = nullptr) {
  const int wpg = threads / 64;
  const int n_rg = (rows + R - 1) / R;
  const int units = cols >> 6, nwin = (units + 63) >> 6;
  const int min_waves = cu_count() * waves_per_cu;
  int per = (n_rg + min_waves - 1) / min_waves;
  if (nwin > 1 && per > MAXQ) per = MAXQ;
  if (nwin == 1 && per > MAXQ) per = MAXQ;
  const int waves = (n_rg + per - 1) / per;
  const int blocks = (waves + wpg - 1) / wpg;
  // x rounds (threads * 8 columns each) whose loads go ahead of the weights
  const int rounds = (cols + threads * 8 - 1) / (threads * 8);
  const dim3 grid = dim3(unsigned(blocks)), block = dim3(unsigned(threads));
  const size_t lds = size_t(limb_lds_bytes(cols));
  if (rounds <= 1)
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

// Batches of rows wider than one 4096-column window run split-K over the
// windows with their activations converted once per call (the workspace);
// narrower rows gain nothing from the extra launch and take none.
size_t gemv_workspace_bytes(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  return batch >= 2 && cols > 4096 && gemv_mfma_ok(quant, rows, cols, batch) ? gemv_mfma_workspace_bytes(rows, cols)
                                                                               : 0;
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
        e = nb == 1 ? launch_limb<LimbQ4K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc)
                    : launch_nb<FmtQ4K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kQ8_0:
        e = nb == 1 ? launch_limb<LimbQ8, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc)
                    : launch_nb<FmtQ8>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kQ5_K:
        e = nb == 1 ? launch_limb<LimbQ5K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc)
                    : launch_nb<FmtQ5K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream);
        break;
      case kIQ4_XS:  // batch-1 launches, one vector each
        e = hipSuccess;
        for (int b = 0; b < nb && e == hipSuccess; ++b)
          e = q6_signed ? launch_limb<LimbIQ4XS<true>, 1, 4>(w, int(rows), int(cols), row_bytes, xb + int64_t(b) * cols,
                                                             yb + int64_t(b) * rows, stream, 512, wpc)
                        : launch_limb<LimbIQ4XS<false>, 1, 4>(w, int(rows), int(cols), row_bytes,
                                                              xb + int64_t(b) * cols, yb + int64_t(b) * rows, stream,
                                                              512, wpc);
        break;
      default:
        e = nb == 1 ? launch_limb<LimbQ6K, 1, 4>(w, int(rows), int(cols), row_bytes, xb, yb, stream, 512, wpc,
                                                  q6_signed)
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

// One token through the dense FFN's two matvec launches (limb kernels):
// [g; u] = [gate; up] . x (both n_ff x n_embd, one launch, x staged once),
// then out = xres + down . (silu(g) * u) (silu and the residual add inside).
template <class F>
static hipError_t launch_ffn1(const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_embd, int n_ff,
                              const float* x, float* gu, const float* xres, float* out, int q6s, hipStream_t s) {
  const int64_t rb1 = byte_size(F::kQuant, n_embd), rb2 = byte_size(F::kQuant, n_ff);
  hipError_t e = launch_limb<F, 1, 4, kLimbTwoMat>(gate, 2 * n_ff, n_embd, rb1, x, gu, s, 512, 8, q6s, up, n_ff);
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
