// Per-unit "axpy" of one packed row into column sums, for the expert
// (in-major) matvec and the MoE FFN: a thread owns one 64-column unit (one
// Q4_K group, one Q6_K quarter, or a pair of Q8_0 blocks -- the units of the
// matvec kernels) and adds x[i] * W[i][unit columns] for a row i into 64
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
    const uint32_t nib = 4u * tp;
    float wv[64];  // 6-bit codes 0..63
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t qh = realign(qhr[k], qhr[k + 1], s);
      const uint32_t qs = tp ? qh : (qh << 4);
      const uint32_t va = ((realign(qlr[k], qlr[k + 1], s) >> nib) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
      const uint32_t vb =
          ((realign(qlr[8 + k], qlr[9 + k], s) >> nib) & 0x0F0F0F0Fu) | ((qs >> 2) & 0x30303030u);
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

}  // namespace sh
