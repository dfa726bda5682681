// Fused dequant + matvec for Q8_0, Q4_K and Q6_K rows, read packed from HBM.
//
// Semantics: crates/strata-core/src/ops.rs:14-28 (`gemv`): y[r] = sum_c
// W[r][c] * x[c] with W[r][c] the strata-gguf dequantized value
// (crates/strata-gguf/src/dequant.rs:123-128, :208-234, :237-270). The sum is
// formed in f32 in a different order from the reference's sequential f64
// loop, and per-block scales are factored out:
//   Q4_K  sum_sub (d*sc) * sum(q*x) - (dmin*m) * sum(x)
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

// ------------------------------------------------------------------ Q8_0 --
// Unit u of a row: blocks 2u and 2u+1 (68 bytes, 4-byte aligned when the row
// start is, which the launcher checks).
struct FmtQ8 {
  static constexpr int kR = 2;
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

// ---------------------------------------------------------------- launch --
static int g_cu_count = 0;

static int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_cu_count = n;
    else
      g_cu_count = 256;
  }
  return g_cu_count;
}

constexpr size_t kMaxLds = 160 * 1024;

static size_t lds_bytes(int cols, int nb) { return size_t(nb) * x_stride(cols) * sizeof(float); }

bool gemv_shape_ok(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  if (!device_quant(quant) || rows <= 0 || cols <= 0 || batch < 1 || batch > 8) return false;
  if (rows > (int64_t(1) << 31) - 1 || cols > (int64_t(1) << 20)) return false;
  if (cols % 64 != 0) return false;  // 64-column lane units (Q8_0 blocks in pairs)
  if (cols % geometry(quant).block != 0) return false;
  return lds_bytes(int(cols), 1) <= kMaxLds;
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
    case 1: return launch_fmt<F, 1>(w, rows, cols, row_bytes, x, y, q6_signed, s);
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

hipError_t launch_gemv(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                       float* y, int batch, int q6_signed, hipStream_t stream) {
  if (!gemv_shape_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  const int64_t row_bytes = byte_size(quant, cols);
  // Q8_0 reads 68-byte block pairs with dword loads: rows must start on a
  // dword boundary (row_bytes is 68 * cols/64, so only the base matters).
  if (quant == kQ8_0 && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(w) & 1u) || (reinterpret_cast<uintptr_t>(x) & 15u))
    return hipErrorInvalidValue;
  // x for all of the batch must fit in LDS; a larger batch runs in slices
  int per = int(kMaxLds / lds_bytes(int(cols), 1));
  if (per > 8) per = 8;
  for (int b0 = 0; b0 < batch; b0 += per) {
    const int nb = batch - b0 < per ? batch - b0 : per;
    const float* xb = x + int64_t(b0) * cols;
    float* yb = y + int64_t(b0) * rows;
    hipError_t e;
    switch (quant) {
      case kQ4_K: e = launch_nb<FmtQ4K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream); break;
      case kQ8_0: e = launch_nb<FmtQ8>(nb, w, int(rows), int(cols), row_bytes, xb, yb, 0, stream); break;
      default: e = launch_nb<FmtQ6K>(nb, w, int(rows), int(cols), row_bytes, xb, yb, q6_signed, stream);
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace sh
