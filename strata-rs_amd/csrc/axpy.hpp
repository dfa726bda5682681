// Per-unit "axpy" of one packed row into column sums, for the expert
// (in-major) matvec and the MoE FFN: a thread owns one 64-column unit (one
// Q4_K / Q5_K / IQ4_XS group, one Q6_K quarter, or a pair of Q8_0 blocks --
// the units of the matvec kernels) and adds x[i] * W[i][unit columns] for a row i into 64
// f32 accumulators per token. Block scales are folded into one coefficient
// per sub-block and token (x[i] * d * sc); the constant parts of the codes
// (Q4_K min, Q6_K -32, Q8_0 +128 bias) are summed per sub-block in `off` and
// subtracted once when the sums are read out. The weight codes are decoded
// once per row and applied to NT tokens.
#pragma once

#include "common.hpp"

namespace sh {

// Per-unit axpy for each format: acc[0..63] += coef * value and the offset
// terms per sub-block; 64 columns = one Q4_K group, one Q6_K quarter, or a
// pair of Q8_0 blocks (the same units as the matvec kernels).
struct AxQ4K {
  static constexpr int kOff = 2;
  struct Raw {
    u32x4 h, a, b;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int u) {
    const uint8_t* sb = row + (u >> 2) * 144;
    const int g = u & 3;
    return {ld16u(sb), ld16u(sb + 16 + 32 * g), ld16u(sb + 32 + 32 * g)};
  }
  template <int NT>
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, const float* xi,
                                              float (*acc)[64], float (*off)[kOff], int q6s) {
    apply<NT>(load(row, u), u, xi, acc, off, q6s);
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int u, const float* xi, float (*acc)[64],
                                               float (*off)[kOff], int) {
    const int g = u & 3;
    const u32x4 h = r.h, a = r.a, b = r.b;
    const uint32_t sh = (g & 1) << 4;
    const uint32_t t1 = h.y >> sh, t2 = h.z >> sh, t3 = h.w >> sh;
    const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
    const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
    const float d = h2f(h.x), dm = h2f(h.x >> 16);
    const float dsc0 = d * ubyte<0>(scp), dsc1 = d * ubyte<1>(scp) * 0.0625f;  // high nibbles read as 16 * q
    const float dmm0 = dm * ubyte<0>(mp), dmm1 = dm * ubyte<1>(mp);
    const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float wv[64];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = q[k] & 0xF0F0F0F0u;
      wv[4 * k + 0] = ubyte<0>(lo);
      wv[4 * k + 1] = ubyte<1>(lo);
      wv[4 * k + 2] = ubyte<2>(lo);
      wv[4 * k + 3] = ubyte<3>(lo);
      wv[32 + 4 * k + 0] = ubyte<0>(hi);
      wv[32 + 4 * k + 1] = ubyte<1>(hi);
      wv[32 + 4 * k + 2] = ubyte<2>(hi);
      wv[32 + 4 * k + 3] = ubyte<3>(hi);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (xi[t] == 0.f) continue;  // ops.rs:182-184
      const float c0 = xi[t] * dsc0, c1 = xi[t] * dsc1;
      off[t][0] += xi[t] * dmm0;
      off[t][1] += xi[t] * dmm1;
#pragma unroll
      for (int e = 0; e < 32; ++e) acc[t][e] = __builtin_fmaf(c0, wv[e], acc[t][e]);
#pragma unroll
      for (int e = 32; e < 64; ++e) acc[t][e] = __builtin_fmaf(c1, wv[e], acc[t][e]);
    }
  }
  // column e of the unit belongs to sub-block e / 32
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

// Q5_K: unit u is group g = u & 3 of super-block u >> 2 (176 bytes), as
// AxQ4K, with each code's fifth bit from the super-block's 32 qh bytes
// (q5k_codes; codes 0..31, dequant.rs:272-302).
struct AxQ5K {
  static constexpr int kOff = 2;
  struct Raw {
    u32x4 h, h0, h1, a, b;  // header, qh, the group's 32 code bytes
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int u) {
    const uint8_t* sb = row + (u >> 2) * 176;
    const int g = u & 3;
    return {ld16u(sb), ld16u(sb + 16), ld16u(sb + 32), ld16u(sb + 48 + 32 * g), ld16u(sb + 64 + 32 * g)};
  }
  template <int NT>
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, const float* xi,
                                              float (*acc)[64], float (*off)[kOff], int q6s) {
    apply<NT>(load(row, u), u, xi, acc, off, q6s);
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int u, const float* xi, float (*acc)[64],
                                               float (*off)[kOff], int) {
    const int g = u & 3;
    uint32_t scp, mp;
    k4_pair(r.h, g, scp, mp);
    const float d = h2f(r.h.x), dm = h2f(r.h.x >> 16);
    const float dsc0 = d * ubyte<0>(scp), dsc1 = d * ubyte<1>(scp);
    const float dmm0 = dm * ubyte<0>(mp), dmm1 = dm * ubyte<1>(mp);
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    float wv[64];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t lo, hi;
      q5k_codes(q[k], qh[k], uint32_t(g), lo, hi);
      wv[4 * k + 0] = ubyte<0>(lo);
      wv[4 * k + 1] = ubyte<1>(lo);
      wv[4 * k + 2] = ubyte<2>(lo);
      wv[4 * k + 3] = ubyte<3>(lo);
      wv[32 + 4 * k + 0] = ubyte<0>(hi);
      wv[32 + 4 * k + 1] = ubyte<1>(hi);
      wv[32 + 4 * k + 2] = ubyte<2>(hi);
      wv[32 + 4 * k + 3] = ubyte<3>(hi);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (xi[t] == 0.f) continue;  // ops.rs:182-184
      const float c0 = xi[t] * dsc0, c1 = xi[t] * dsc1;
      off[t][0] += xi[t] * dmm0;
      off[t][1] += xi[t] * dmm1;
#pragma unroll
      for (int e = 0; e < 32; ++e) acc[t][e] = __builtin_fmaf(c0, wv[e], acc[t][e]);
#pragma unroll
      for (int e = 32; e < 64; ++e) acc[t][e] = __builtin_fmaf(c1, wv[e], acc[t][e]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

struct AxQ8 {
  static constexpr int kOff = 2;
  struct Raw {
    u32x4 a, b, c, d;
    uint32_t e;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int u) {
    const uint8_t* p = row + u * 68;
    return {ld16u(p), ld16u(p + 16), ld16u(p + 32), ld16u(p + 48), ld4(p + 64)};
  }
  template <int NT>
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, const float* xi,
                                              float (*acc)[64], float (*off)[kOff], int q6s) {
    apply<NT>(load(row, u), u, xi, acc, off, q6s);
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int, const float* xi, float (*acc)[64],
                                               float (*off)[kOff], int) {
    const u32x4 A = r.a, B = r.b, C = r.c, Dv = r.d;
    const uint32_t E = r.e;
    const uint32_t D[17] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w, C.x,
                            C.y, C.z, C.w, Dv.x, Dv.y, Dv.z, Dv.w, E};
    const float d0 = h2f(D[0]), d1 = h2f(D[8] >> 16);
    float wv[64];  // q + 128 for both blocks
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t q0 = realign(D[k], D[k + 1], 2) ^ 0x80808080u;
      const uint32_t q1 = D[9 + k] ^ 0x80808080u;
      wv[4 * k + 0] = ubyte<0>(q0);
      wv[4 * k + 1] = ubyte<1>(q0);
      wv[4 * k + 2] = ubyte<2>(q0);
      wv[4 * k + 3] = ubyte<3>(q0);
      wv[32 + 4 * k + 0] = ubyte<0>(q1);
      wv[32 + 4 * k + 1] = ubyte<1>(q1);
      wv[32 + 4 * k + 2] = ubyte<2>(q1);
      wv[32 + 4 * k + 3] = ubyte<3>(q1);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (xi[t] == 0.f) continue;  // ops.rs:182-184
      const float c0 = xi[t] * d0, c1 = xi[t] * d1;
      off[t][0] += 128.f * c0;
      off[t][1] += 128.f * c1;
#pragma unroll
      for (int e = 0; e < 32; ++e) acc[t][e] = __builtin_fmaf(c0, wv[e], acc[t][e]);
#pragma unroll
      for (int e = 32; e < 64; ++e) acc[t][e] = __builtin_fmaf(c1, wv[e], acc[t][e]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

struct AxQ6K {
  static constexpr int kOff = 4;
  struct Raw {
    u32x4 l0, l1, l2, l3, h0, h1;
    uint32_t l4, h2, s0, s1, d, s;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int u) {
    const uint8_t* blk = row + (u >> 2) * 210;
    const int j = u & 3, h = j >> 1;
    const uint32_t tp = uint32_t(j & 1);
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - s;
    const uint8_t* qlp = base + 64 * h;
    const uint8_t* qhp = base + 128 + 32 * h;
    const uint8_t* scp = base + 192 + 8 * h + 4 * tp;
    Raw r;
    r.l0 = ld16u(qlp);
    r.l1 = ld16u(qlp + 16);
    r.l2 = ld16u(qlp + 32);
    r.l3 = ld16u(qlp + 48);
    r.l4 = ld4(qlp + 64);
    r.h0 = ld16u(qhp);
    r.h1 = ld16u(qhp + 16);
    r.h2 = ld4(qhp + 32);
    r.s0 = ld4(scp);
    r.s1 = s ? ld4(scp + 4) : 0u;
    r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    r.s = s;
    return r;
  }
  template <int NT>
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, const float* xi,
                                              float (*acc)[64], float (*off)[kOff], int q6_signed) {
    apply<NT>(load(row, u), u, xi, acc, off, q6_signed);
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int u, const float* xi, float (*acc)[64],
                                               float (*off)[kOff], int q6_signed) {
    const uint32_t tp = uint32_t(u & 1);
    const uint32_t s = r.s;
    const u32x4 l0 = r.l0, l1 = r.l1, l2 = r.l2, l3 = r.l3, h0 = r.h0, h1 = r.h1;
    const uint32_t l4 = r.l4, h2 = r.h2;
    const float d = h2f(r.d);
    const uint32_t scw = realign(r.s0, r.s1, s);
    float sc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t byte = (scw >> (8 * k)) & 0xFFu;
      sc[k] = q6_signed ? float(int8_t(byte)) : float(byte);
    }
    float dsc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) dsc[k] = d * sc[k];
    const uint32_t qlr[17] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w, l2.x,
                              l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w, l4};
    const uint32_t qhr[9] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w, h2};
    float wv[64];  // 6-bit codes 0..63
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t va, vb;
      q6_code_words(qlr[k], qlr[k + 1], qlr[8 + k], qlr[9 + k], qhr[k], qhr[k + 1], s, tp, va, vb);
      wv[4 * k + 0] = ubyte<0>(va);
      wv[4 * k + 1] = ubyte<1>(va);
      wv[4 * k + 2] = ubyte<2>(va);
      wv[4 * k + 3] = ubyte<3>(va);
      wv[32 + 4 * k + 0] = ubyte<0>(vb);
      wv[32 + 4 * k + 1] = ubyte<1>(vb);
      wv[32 + 4 * k + 2] = ubyte<2>(vb);
      wv[32 + 4 * k + 3] = ubyte<3>(vb);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (xi[t] == 0.f) continue;  // ops.rs:182-184
      float c[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        c[k] = xi[t] * dsc[k];
        off[t][k] += 32.f * c[k];
      }
#pragma unroll
      for (int e = 0; e < 64; ++e) acc[t][e] = __builtin_fmaf(c[e >> 4], wv[e], acc[t][e]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 4; }
};

// IQ4_XS: unit u is group g = u & 3 of super-block u >> 2 (136 bytes), the
// 32-element sub-blocks 2g and 2g + 1. Element i of sub-block ib takes the
// code-book value of the low (i < 16) or high nibble of qs byte i % 16; the
// sub-block's 16 qs bytes are qs[0..16] in the reference's reading (its
// slice is never advanced, dequant.rs:189-206) and qs[16 ib ..] in ggml's
// (GGML). Scale d * (ls - 32). The signed codes are biased to v + 128 for
// the unsigned conversion, 128 * coefficient going to the offset (as Q8_0).
template <bool GGML>
struct AxIQ4XS {
  static constexpr int kOff = 2;
  struct Raw {
    uint32_t h0, h1;  // d | scales_h, scales_l
    u32x4 a, b;       // the qs bytes of sub-blocks 2g and 2g + 1
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int u) {
    const uint8_t* sb = row + (u >> 2) * 136;
    const int g = u & 3;
    return {ld4(sb), ld4(sb + 4), ld16u(sb + 8 + (GGML ? 32 * g : 0)), ld16u(sb + 8 + (GGML ? 32 * g + 16 : 0))};
  }
  template <int NT>
  __device__ static __forceinline__ void axpy(const uint8_t* row, int u, const float* xi,
                                              float (*acc)[64], float (*off)[kOff], int q6s) {
    apply<NT>(load(row, u), u, xi, acc, off, q6s);
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int u, const float* xi, float (*acc)[64],
                                               float (*off)[kOff], int) {
    const int g = u & 3;
    const float d = h2f(r.h0);
    const float dl0 = d * iq4xs_scale(r.h0, r.h1, 2 * g), dl1 = d * iq4xs_scale(r.h0, r.h1, 2 * g + 1);
    const uint32_t qa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, qb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    float wv[64];  // v + 128
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t v[4] = {iq4_lut(qa[k] & 0x0F0F0F0Fu) ^ 0x80808080u,
                             iq4_lut((qa[k] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u,
                             iq4_lut(qb[k] & 0x0F0F0F0Fu) ^ 0x80808080u,
                             iq4_lut((qb[k] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u};
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // columns 16 q + 4 k ..
        wv[16 * q + 4 * k + 0] = ubyte<0>(v[q]);
        wv[16 * q + 4 * k + 1] = ubyte<1>(v[q]);
        wv[16 * q + 4 * k + 2] = ubyte<2>(v[q]);
        wv[16 * q + 4 * k + 3] = ubyte<3>(v[q]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (xi[t] == 0.f) continue;  // ops.rs:182-184
      const float c0 = xi[t] * dl0, c1 = xi[t] * dl1;
      off[t][0] += 128.f * c0;
      off[t][1] += 128.f * c1;
#pragma unroll
      for (int e = 0; e < 32; ++e) acc[t][e] = __builtin_fmaf(c0, wv[e], acc[t][e]);
#pragma unroll
      for (int e = 32; e < 64; ++e) acc[t][e] = __builtin_fmaf(c1, wv[e], acc[t][e]);
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 5; }
};

// ------------------------------------------------------- half units --
// The same axpy for 32-column half units (one Q4_K sub-block, one Q8_0
// block, half a Q6_K quarter), with the codes decoded four at a time next to
// the FMAs that use them: 32 column sums per token instead of 64, and no
// decoded row held in registers, so that several waves fit per SIMD.
// Half unit hu covers columns [32 hu, 32 hu + 32).
struct HxQ4K {
  static constexpr int kOff = 1;
  struct Raw {
    u32x4 h, a, b;  // header, the group's 32 code bytes
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int hu) {
    const int u = hu >> 1;
    const uint8_t* sb = row + (u >> 2) * 144;
    const int g = u & 3;
    return {ld16u(sb), ld16u(sb + 16 + 32 * g), ld16u(sb + 32 + 32 * g)};
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int hu, const float* xi, float (*acc)[32],
                                               float (*off)[kOff], int) {
    const int u = hu >> 1, g = u & 3;
    const uint32_t hi = uint32_t(hu & 1);  // high nibbles: sub-block 2g + 1
    const u32x4 h = r.h;
    const uint32_t sh = (g & 1) << 4;
    const uint32_t t1 = h.y >> sh, t2 = h.z >> sh, t3 = h.w >> sh;
    // get_scale_min_k4 for sub-blocks 2g (byte 0) and 2g + 1 (byte 1)
    const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
    const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
    const float d = h2f(h.x), dm = h2f(h.x >> 16);
    const float scf = float((scp >> (8 * hi)) & 0xFFu), mf = float((mp >> (8 * hi)) & 0xFFu);
    // high nibbles are read in place as 16 * q, so their scale carries 1/16 (exact)
    const float dsc = d * scf * (hi ? 0.0625f : 1.f), dmm = dm * mf;
    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    float c[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // a zero input contributes nothing, whatever the scales hold (ops.rs:182-184)
      c[t] = xi[t] == 0.f ? 0.f : xi[t] * dsc;
      off[t][0] += xi[t] == 0.f ? 0.f : xi[t] * dmm;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t v = q[k] & mask;
      const float w0 = ubyte<0>(v), w1 = ubyte<1>(v), w2 = ubyte<2>(v), w3 = ubyte<3>(v);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[t][4 * k + 0] = __builtin_fmaf(c[t], w0, acc[t][4 * k + 0]);
        acc[t][4 * k + 1] = __builtin_fmaf(c[t], w1, acc[t][4 * k + 1]);
        acc[t][4 * k + 2] = __builtin_fmaf(c[t], w2, acc[t][4 * k + 2]);
        acc[t][4 * k + 3] = __builtin_fmaf(c[t], w3, acc[t][4 * k + 3]);
      }
    }
  }
  __device__ static __forceinline__ int off_index(int) { return 0; }
};

// Q5_K: half unit hu is sub-block 2g + (hu & 1) of group g = (hu >> 1) & 3
// of super-block hu >> 3, as HxQ4K; its 32 codes take the nibble (hu & 1)
// of the group's code bytes and bit 2g + (hu & 1) of qh[l] as 16.
struct HxQ5K {
  static constexpr int kOff = 1;
  struct Raw {
    u32x4 h, h0, h1, a, b;  // header, qh, the group's 32 code bytes
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int hu) {
    const int u = hu >> 1;
    const uint8_t* sb = row + (u >> 2) * 176;
    const int g = u & 3;
    return {ld16u(sb), ld16u(sb + 16), ld16u(sb + 32), ld16u(sb + 48 + 32 * g), ld16u(sb + 64 + 32 * g)};
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int hu, const float* xi, float (*acc)[32],
                                               float (*off)[kOff], int) {
    const int u = hu >> 1, g = u & 3;
    const uint32_t hi = uint32_t(hu & 1);
    uint32_t scp, mp;
    k4_pair(r.h, g, scp, mp);
    const float d = h2f(r.h.x), dm = h2f(r.h.x >> 16);
    const float dsc = d * float((scp >> (8 * hi)) & 0xFFu), dmm = dm * float((mp >> (8 * hi)) & 0xFFu);
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    const uint32_t bit = 2u * uint32_t(g) + hi;
    float c[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      c[t] = xi[t] == 0.f ? 0.f : xi[t] * dsc;  // ops.rs:182-184
      off[t][0] += xi[t] == 0.f ? 0.f : xi[t] * dmm;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t v = ((q[k] >> (4 * hi)) & 0x0F0F0F0Fu) | (((qh[k] >> bit) & 0x01010101u) << 4);
      const float w0 = ubyte<0>(v), w1 = ubyte<1>(v), w2 = ubyte<2>(v), w3 = ubyte<3>(v);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[t][4 * k + 0] = __builtin_fmaf(c[t], w0, acc[t][4 * k + 0]);
        acc[t][4 * k + 1] = __builtin_fmaf(c[t], w1, acc[t][4 * k + 1]);
        acc[t][4 * k + 2] = __builtin_fmaf(c[t], w2, acc[t][4 * k + 2]);
        acc[t][4 * k + 3] = __builtin_fmaf(c[t], w3, acc[t][4 * k + 3]);
      }
    }
  }
  __device__ static __forceinline__ int off_index(int) { return 0; }
};

// Q8_0: half unit hu is block hu (34 bytes from a 2-byte boundary), read as
// nine dwords from the dword boundary at or below it. The codes are biased to
// q + 128 for the unsigned conversion; 128 * coefficient goes to the offset.
struct HxQ8 {
  static constexpr int kOff = 1;
  struct Raw {
    u32x4 a, b;
    uint32_t c, s;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int hu) {
    const uint8_t* blk = row + hu * 34;
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - s;
    return {ld16u(base), ld16u(base + 16), ld4(base + 32), s};
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int, const float* xi, float (*acc)[32],
                                               float (*off)[kOff], int) {
    const uint32_t D[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
    const bool s2 = r.s != 0;  // the block starts at byte 2 of D[0]
    const float d = h2f(s2 ? (D[0] >> 16) : D[0]);
    float c[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      c[t] = xi[t] == 0.f ? 0.f : xi[t] * d;  // ops.rs:182-184
      off[t][0] += 128.f * c[t];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // codes are bytes 2..33 of the block
      const uint32_t v = (s2 ? D[k + 1] : realign(D[k], D[k + 1], 2)) ^ 0x80808080u;
      const float w0 = ubyte<0>(v), w1 = ubyte<1>(v), w2 = ubyte<2>(v), w3 = ubyte<3>(v);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[t][4 * k + 0] = __builtin_fmaf(c[t], w0, acc[t][4 * k + 0]);
        acc[t][4 * k + 1] = __builtin_fmaf(c[t], w1, acc[t][4 * k + 1]);
        acc[t][4 * k + 2] = __builtin_fmaf(c[t], w2, acc[t][4 * k + 2]);
        acc[t][4 * k + 3] = __builtin_fmaf(c[t], w3, acc[t][4 * k + 3]);
      }
    }
  }
  __device__ static __forceinline__ int off_index(int) { return 0; }
};

// Q6_K: half unit hu is half p = hu & 1 of quarter j = (hu >> 1) & 3 of
// super-block hu >> 3 (the quarters as in AxQ6K: half hh = j >> 1, nibble
// tp = j & 1). Its 32 columns take code bytes ql[64 hh + 32 p + l] (nibble
// tp) and qh[32 hh + l] bits 4 tp + 2 p (l < 32), and the two 16-column
// scales sc[8 hh + 4 tp + 2 p + {0, 1}].
struct HxQ6K {
  static constexpr int kOff = 2;
  struct Raw {
    u32x4 l0, l1, h0, h1;
    uint32_t l2, h2, sc, d, s;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int hu) {
    const int u = hu >> 1, p = hu & 1;
    const uint8_t* blk = row + (u >> 2) * 210;
    const int j = u & 3, hh = j >> 1, tp = j & 1;
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - s;
    const uint8_t* qlp = base + 64 * hh + 32 * p;
    const uint8_t* qhp = base + 128 + 32 * hh;
    Raw r;
    r.l0 = ld16u(qlp);
    r.l1 = ld16u(qlp + 16);
    r.l2 = ld4(qlp + 32);  // ends at most at byte 131 of the block
    r.h0 = ld16u(qhp);
    r.h1 = ld16u(qhp + 16);
    r.h2 = ld4(qhp + 32);  // ends at most at byte 195
    // sc[8 hh + 4 tp + 2 p] and the next byte: bytes [s + 192 + off, +2) of base
    const int so = int(s) + 192 + 8 * hh + 4 * tp + 2 * p;  // even, <= 208
    const uint32_t sw = ld4(base + (so & ~3));
    r.sc = (so & 2) ? (sw >> 16) : (sw & 0xFFFFu);
    r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    r.s = s;
    return r;
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int hu, const float* xi, float (*acc)[32],
                                               float (*off)[kOff], int q6_signed) {
    const int u = hu >> 1, p = hu & 1, tp = u & 1;
    const uint32_t s = r.s;
    const float d = h2f(r.d);
    const uint32_t b0 = r.sc & 0xFFu, b1 = (r.sc >> 8) & 0xFFu;
    const float sc0 = q6_signed ? float(int8_t(b0)) : float(b0);
    const float sc1 = q6_signed ? float(int8_t(b1)) : float(b1);
    const float ds0 = d * sc0, ds1 = d * sc1;
    const uint32_t qlr[9] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w, r.l1.x, r.l1.y, r.l1.z, r.l1.w, r.l2};
    const uint32_t qhr[9] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w, r.h2};
    const uint32_t nib = 4u * uint32_t(tp);
    const uint32_t hsh = uint32_t(4 * tp + 2 * p);  // qh bits of this half
    float c0[NT], c1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      c0[t] = xi[t] == 0.f ? 0.f : xi[t] * ds0;  // ops.rs:182-184
      c1[t] = xi[t] == 0.f ? 0.f : xi[t] * ds1;
      off[t][0] += 32.f * c0[t];
      off[t][1] += 32.f * c1[t];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // realignment and shift in one funnel shift each (s <= 3, so 8 s + 6 < 32)
      const uint32_t v = (__builtin_amdgcn_alignbit(qlr[k + 1], qlr[k], 8u * s + nib) & 0x0F0F0F0Fu) |
                         ((__builtin_amdgcn_alignbit(qhr[k + 1], qhr[k], 8u * s + hsh) & 0x03030303u) << 4);
      const float w0 = ubyte<0>(v), w1 = ubyte<1>(v), w2 = ubyte<2>(v), w3 = ubyte<3>(v);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float cc = k < 4 ? c0[t] : c1[t];  // columns 0-15: sc0, 16-31: sc1
        acc[t][4 * k + 0] = __builtin_fmaf(cc, w0, acc[t][4 * k + 0]);
        acc[t][4 * k + 1] = __builtin_fmaf(cc, w1, acc[t][4 * k + 1]);
        acc[t][4 * k + 2] = __builtin_fmaf(cc, w2, acc[t][4 * k + 2]);
        acc[t][4 * k + 3] = __builtin_fmaf(cc, w3, acc[t][4 * k + 3]);
      }
    }
  }
  __device__ static __forceinline__ int off_index(int e) { return e >> 4; }
};

// IQ4_XS: half unit hu is sub-block ib = hu & 7 of super-block hu >> 3, its
// 16 qs bytes read as AxIQ4XS (columns 0-15 the low nibbles, 16-31 the high).
template <bool GGML>
struct HxIQ4XS {
  static constexpr int kOff = 1;
  struct Raw {
    uint32_t h0, h1;
    u32x4 a;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int hu) {
    const uint8_t* sb = row + (hu >> 3) * 136;
    return {ld4(sb), ld4(sb + 4), ld16u(sb + 8 + (GGML ? 16 * (hu & 7) : 0))};
  }
  template <int NT>
  __device__ static __forceinline__ void apply(const Raw& r, int hu, const float* xi, float (*acc)[32],
                                               float (*off)[kOff], int) {
    const float dl = h2f(r.h0) * iq4xs_scale(r.h0, r.h1, hu & 7);
    const uint32_t q[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    float c[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      c[t] = xi[t] == 0.f ? 0.f : xi[t] * dl;  // ops.rs:182-184
      off[t][0] += 128.f * c[t];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t idx = k < 4 ? (q[k] & 0x0F0F0F0Fu) : ((q[k - 4] >> 4) & 0x0F0F0F0Fu);
      const uint32_t v = iq4_lut(idx) ^ 0x80808080u;  // v + 128
      const float w0 = ubyte<0>(v), w1 = ubyte<1>(v), w2 = ubyte<2>(v), w3 = ubyte<3>(v);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[t][4 * k + 0] = __builtin_fmaf(c[t], w0, acc[t][4 * k + 0]);
        acc[t][4 * k + 1] = __builtin_fmaf(c[t], w1, acc[t][4 * k + 1]);
        acc[t][4 * k + 2] = __builtin_fmaf(c[t], w2, acc[t][4 * k + 2]);
        acc[t][4 * k + 3] = __builtin_fmaf(c[t], w3, acc[t][4 * k + 3]);
      }
    }
  }
  __device__ static __forceinline__ int off_index(int) { return 0; }
};

}  // namespace sh
