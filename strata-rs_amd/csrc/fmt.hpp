// Matvec units over f32 activations: a 64-column unit of a packed row
// (one Q4_K / Q5_K group, one Q6_K quarter, a pair of Q8_0 blocks) against
// the lane's 64 staged x values and their per-16 sums. Shared by the general
// matvec kernel and the out-major (ggml orientation) MoE kernels.
#pragma once

#include "common.hpp"

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
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // one per 16-element sub-block
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t a, b;
      q6_code_words(qlr[k], qlr[k + 1], qlr[8 + k], qlr[9 + k], qhr[k], qhr[k + 1], s, tp, a, b);
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

// ---------------------------------------------------------------- IQ4_XS --
// Unit u of a row: super-block u/4 (136 bytes), group g = u%4 = sub-blocks
// 2g and 2g + 1, the qs bytes as AxIQ4XS reads them (the reference's
// qs[0..16] for every sub-block, or ggml's qs[16 ib ..] with GGML). The
// signed code-book values are biased to v + 128 (as FmtQ8).
template <bool GGML>
struct FmtIQ4XS {
  static constexpr int kR = 2;
  static constexpr int kRing = 3;
  struct Load {
    uint32_t h0, h1;
    u32x4 a, b;
  };
  __device__ static __forceinline__ void load(const uint8_t* row, int u, Load& o) {
    const uint8_t* sb = row + (u >> 2) * 136;
    const int g = u & 3;
    o.h0 = ld4(sb);
    o.h1 = ld4(sb + 4);
    o.a = ld16u(sb + 8 + (GGML ? 32 * g : 0));
    o.b = ld16u(sb + 8 + (GGML ? 32 * g + 16 : 0));
  }
  __device__ static __forceinline__ float dot(const Load& L, const XSlice& x, int u, int) {
    const int g = u & 3;
    const uint32_t qa[4] = {L.a.x, L.a.y, L.a.z, L.a.w}, qb[4] = {L.b.x, L.b.y, L.b.z, L.b.w};
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;  // columns 0-15, 16-31, 32-47, 48-63
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t v0 = iq4_lut(qa[k] & 0x0F0F0F0Fu) ^ 0x80808080u;
      const uint32_t v1 = iq4_lut((qa[k] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u;
      const uint32_t v2 = iq4_lut(qb[k] & 0x0F0F0F0Fu) ^ 0x80808080u;
      const uint32_t v3 = iq4_lut((qb[k] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u;
      const f32x4 x0 = x.v[k], x1 = x.v[4 + k], x2 = x.v[8 + k], x3 = x.v[12 + k];
      s0 = __builtin_fmaf(ubyte<0>(v0), x0.x, s0);
      s0 = __builtin_fmaf(ubyte<1>(v0), x0.y, s0);
      s0 = __builtin_fmaf(ubyte<2>(v0), x0.z, s0);
      s0 = __builtin_fmaf(ubyte<3>(v0), x0.w, s0);
      s1 = __builtin_fmaf(ubyte<0>(v1), x1.x, s1);
      s1 = __builtin_fmaf(ubyte<1>(v1), x1.y, s1);
      s1 = __builtin_fmaf(ubyte<2>(v1), x1.z, s1);
      s1 = __builtin_fmaf(ubyte<3>(v1), x1.w, s1);
      s2 = __builtin_fmaf(ubyte<0>(v2), x2.x, s2);
      s2 = __builtin_fmaf(ubyte<1>(v2), x2.y, s2);
      s2 = __builtin_fmaf(ubyte<2>(v2), x2.z, s2);
      s2 = __builtin_fmaf(ubyte<3>(v2), x2.w, s2);
      s3 = __builtin_fmaf(ubyte<0>(v3), x3.x, s3);
      s3 = __builtin_fmaf(ubyte<1>(v3), x3.y, s3);
      s3 = __builtin_fmaf(ubyte<2>(v3), x3.z, s3);
      s3 = __builtin_fmaf(ubyte<3>(v3), x3.w, s3);
    }
    const float d = h2f(L.h0);
    const float dl0 = d * iq4xs_scale(L.h0, L.h1, 2 * g), dl1 = d * iq4xs_scale(L.h0, L.h1, 2 * g + 1);
    return dl0 * ((s0 + s1) - 128.f * (x.s.x + x.s.y)) + dl1 * ((s2 + s3) - 128.f * (x.s.z + x.s.w));
  }
};

}  // namespace sh
