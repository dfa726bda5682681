// Integer-limb activations and the matvec units that dot them exactly:
// shared by the batch-1 matvec kernels and the out-major MoE kernels.
#pragma once

#include "common.hpp"
#include "fmt.hpp"

namespace sh {

// ================================================== batch-1 integer path ==
// x as three int8 limbs. Each workgroup converts the f32 activations once:
// per 32-column block a power-of-two scale 2^-k is chosen so that the block's
// largest |x| times 2^k is below 2^22 (2^23 with FINE), and every element
// becomes the integer
//   v = rne(x * 2^k) = a * 2^16 + b * 2^8 + c,  b, c in [0, 255]
// (a is byte 2 of v, b byte 1, c byte 0, in two's complement): a in [-64, 64],
// each element within 2^-23 of its block's maximum; with FINE a in
// [-128, 127] (a value that rounds up to 2^23 is held at 2^23 - 1), within
// 2^-24, at two more instructions per element. Near the block maximum either
// is as close to x as the f32 activations themselves; FINE serves the steps
// of a chain of products (the gate / up sums that form silu(g) * u and the
// matvec that takes it), whose rounding the next matvec passes on. Weight
// codes are
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
template <bool LOW, bool FINE = false>
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
  // k with m * 2^k < 2^22 (2^23 FINE); for m == 0 any k works
  // (clamped so 2^k stays finite for blocks whose maximum is below 2^-104)
  int e = 0;
  (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1)
  const int k = m > 0.f ? min((FINE ? 23 : 22) - e, 126) : 0;
  const float up = ldexpf(1.f, k);
  // a NaN or infinite block keeps its NaN through the scale
  const float down = (m - m == 0.f) ? ldexpf(1.f, -k) : __builtin_nanf("");
  uint32_t v[8];
  uint32_t low = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (FINE) {
      // rne(x * 2^k), |x * 2^k| < 2^23 (exact: 2^k is a power of two); the
      // one value that can round up to 2^23 is held below it
      v[i] = uint32_t(min(int(__builtin_rintf(xs[i] * up)), 0x7FFFFF));
    } else {
      // rne(x * 2^k) through the 1.5 * 2^23 magic constant (|x * 2^k| < 2^22)
      const float tt = __builtin_fmaf(xs[i], up, 12582912.0f);
      v[i] = __builtin_bit_cast(uint32_t, tt) - 0x4B400000u;
    }
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
  // unit `lane` of a window copied to LDS (blocks on 16-byte boundaries)
  __device__ static __forceinline__ void load_lds(const uint8_t* win, int lane, Load& L) {
    load(win, offsets(lane), L);
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
  // unit `lane` of a window copied to LDS (blocks on 16-byte boundaries)
  __device__ static __forceinline__ void load_lds(const uint8_t* win, int lane, Load& L) {
    load(win, offsets(lane), L);
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

// Q6_K with integer dots. Unit u covers half h = (u >> 1) & 1 of super-block
// u / 4 split between the lanes of a pair by t = u & 1: the lane takes the
// 16 positions l in [16 t, 16 t + 16) of the half's four 32-element groups
// i (elements 128 h + 32 i + l, dequant.rs:208-234), so each of its four
// 16-element sub-blocks (scale 8 h + 2 i + t) is whole and it reads only its
// own 16 bytes of ql[l], ql[l + 32] and qh[l] (the quarter-per-lane split
// has both lanes of a pair read all 96 of them). The codes 0..63 go straight
// into the dots and the -32 offset is taken off with the per-16 sums of x.
struct XLimbsQ6 {
  u32x4 a[4], b[4], c[4];  // limb words of group i's 16 columns
  uint32_t xs[4], ks[4];   // group i's sum of those 16 x, and its block's 2^-k
};

struct LimbQ6K {
  static constexpr uint32_t kQuant = kQ6_K;
  struct Load {
    u32x4 a;       // ql[l .. l + 16) of the lane, from the dword below
    uint32_t a4;   // the dword after (bytes past 16 when misaligned)
    u32x4 b;       // ql[l + 32 ..]
    uint32_t b4;
    u32x4 h;       // qh[l ..]
    uint32_t h4;
    uint32_t s0, s1, s2;  // scales[8 h .. 8 h + 8) from the dword below
    uint32_t d;           // d | misalignment << 16
  };
  static constexpr int kWinBytes = 16 * 210;
  struct Off {
    int h, q;
  };
  // h: the super-block's byte offset, q: 2 * half + lane of the pair
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 2) * 210, u & 3}; }
  // Rows start on even bytes (the entry points check it), so a block's
  // misalignment is 0 or 2 and every dword read below ends inside the block;
  // s2 is read only when misaligned (aligned, it would run 2 bytes past).
  // `base` is the dword boundary `shift` bytes below the block; LDS sources
  // take 16-byte reads that promise 4-byte alignment only.
  template <bool LDS>
  __device__ static __forceinline__ void load_at(const uint8_t* base, uint32_t shift, int h, int t, Load& L) {
    const uint8_t* ql = base + 64 * h + 16 * t;
    L.a = LDS ? ld16u(ql) : ld16(ql);
    L.a4 = ld4(ql + 16);
    L.b = LDS ? ld16u(ql + 32) : ld16(ql + 32);
    L.b4 = ld4(ql + 48);  // ends at most at byte 133 of the block
    const uint8_t* qh = base + 128 + 32 * h + 16 * t;
    L.h = LDS ? ld16u(qh) : ld16(qh);
    L.h4 = ld4(qh + 16);  // ends at most at byte 195
    const uint8_t* sc = base + 192 + 8 * h;
    L.s0 = ld4(sc);
    L.s1 = ld4(sc + 4);
    L.s2 = shift ? ld4(sc + 8) : 0u;
    L.d = uint32_t(*reinterpret_cast<const uint16_t*>(base + shift + 208)) | (shift << 16);
  }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    const uint8_t* blk = row + o.h;
    const uint32_t shift = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    load_at<false>(blk - shift, shift, o.q >> 1, o.q & 1, L);
  }
  // unit `lane` of a window copied to LDS from a 16-byte boundary
  __device__ static __forceinline__ void load_lds(const uint8_t* win, int lane, Load& L) {
    const int sbo = (lane >> 2) * 210;
    const uint32_t shift = uint32_t(sbo) & 3u;
    load_at<true>(win + sbo - int(shift), shift, (lane >> 1) & 1, lane & 1, L);
  }
  // Limb words and sums of unit u's columns: group i lies in the 64-column
  // LDS unit 2 (u >> 1) + (i >> 1), at byte 32 (i & 1) + 16 t of it, and
  // in x block 4 (u >> 1) + i (half t of its two 16-column sums).
  __device__ static __forceinline__ void load_x(const uint8_t* lds, int cols, int u, XLimbsQ6& o) {
    const int ps = plane_stride(cols);
    const int p = u >> 1, t = u & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int off = 80 * (2 * p + (i >> 1)) + 32 * (i & 1) + 16 * t;
      o.a[i] = *reinterpret_cast<const u32x4*>(lds + off);
      o.b[i] = *reinterpret_cast<const u32x4*>(lds + ps + off);
      o.c[i] = *reinterpret_cast<const u32x4*>(lds + 2 * ps + off);
      const u32x4 rec = *reinterpret_cast<const u32x4*>(lds + 3 * ps + 16 * (4 * p + i));
      o.xs[i] = t ? rec.y : rec.x;
      o.ks[i] = rec.z;
    }
  }
  __device__ static __forceinline__ float dot(const Load& L, const XLimbsQ6& x, int lane, int q6_signed) {
    const uint32_t t = uint32_t(lane) & 1u;
    const uint32_t s = L.d >> 16;
    const uint32_t qa[5] = {L.a.x, L.a.y, L.a.z, L.a.w, L.a4};
    const uint32_t qb[5] = {L.b.x, L.b.y, L.b.z, L.b.w, L.b4};
    const uint32_t qh[5] = {L.h.x, L.h.y, L.h.z, L.h.w, L.h4};
    // scales 8 h + 2 i + t: bytes t and t + 2 of the first realigned word
    // (groups 0, 1) and of the second (groups 2, 3)
    const uint32_t sw[2] = {realign(L.s0, L.s1, s), realign(L.s1, L.s2, s)};
    constexpr uint32_t kLo = 0x0F0F0F0Fu, kHi = 0x30303030u;
    float t_sum = 0.f;
    // one group at a time (three live sums): group i's codes are the low
    // (i < 2) or high nibbles of ql[l] (i even) or ql[l + 32] (i odd) under
    // bits 4-5 from qh bit pair i; the realignment and the nibble shift are
    // one funnel shift
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t* q = (i & 1) ? qb : qa;
      int sa = 0;
      uint32_t sb = 0, sc = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = __builtin_amdgcn_alignbit(q[w + 1], q[w], 8u * s + 4u * uint32_t(i >> 1)) & kLo;
        const uint32_t hb = __builtin_amdgcn_alignbyte(qh[w + 1], qh[w], s);
        const uint32_t hi = (i == 0 ? hb << 4 : i == 1 ? hb << 2 : i == 2 ? hb : hb >> 2) & kHi;
        dot_limbs(lo | hi, limb_word(x.a, 4 * i + w), limb_word(x.b, 4 * i + w), limb_word(x.c, 4 * i + w), sa, sb,
                  sc);
      }
      const uint32_t byte = (sw[i >> 1] >> (8u * t + 16u * uint32_t(i & 1))) & 0xFFu;
      const float scf = q6_signed ? float(int8_t(byte)) : float(byte);
      t_sum += scf * (limb_value(sa, sb, sc) * fw(x.ks[i]) - 32.f * fw(x.xs[i]));
    }
    return h2f(L.d) * t_sum;
  }
};

// A unit F read a whole 4096-column window at a time: the wave's loads take
// the window's bytes in contiguous 16-byte pieces (lane i: bytes 16 i +
// 1024 k), which the memory system serves as whole lines, and each lane then
// reads its unit's bytes (F::load_lds) from a per-wave LDS copy of the window.
// F's own per-unit loads touch partial lines: Q6_K's are ten reads a row (the
// 151936x4096 head: 103 -> 92 us). Rows of whole windows on 16-byte
// boundaries only (the launcher checks).
template <class F>
struct LimbWin {
  static constexpr uint32_t kQuant = F::kQuant;
  static constexpr int kWinBytes = F::kWinBytes;
  static constexpr int kPieces = (kWinBytes + 1023) / 1024;
  static_assert(kWinBytes % 16 == 0, "windows of whole 16-byte pieces");
  struct Load {
    u32x4 p[kPieces];
  };
  using Off = typename F::Off;
  // h: the window's byte offset in the row, q: the lane's unit in it
  __device__ static __forceinline__ Off offsets(int u) { return {(u >> 6) * kWinBytes, u & 63}; }
  __device__ static __forceinline__ void load(const uint8_t* row, Off o, Load& L) {
    const uint8_t* win = row + o.h;
#pragma unroll
    for (int k = 0; k < kPieces; ++k) L.p[k] = ld16(win + min(16 * o.q + 1024 * k, kWinBytes - 16));
  }
  template <class X>
  __device__ static __forceinline__ float dot(const Load& L, const X& x, int lane, int flags) {
    // the window into LDS (a wave's LDS operations run in order, so the
    // reads below see every lane's piece, and the next window's writes come
    // after them), then the unit's bytes from it
#pragma unroll
    for (int k = 0; k < kPieces; ++k) {
      const int off = 16 * lane + 1024 * k;
      if (off < kWinBytes) *reinterpret_cast<u32x4*>(x.buf + off) = L.p[k];
    }
    typename F::Load q;
    F::load_lds(x.buf, lane, q);
    return F::dot(q, x, lane, flags);
  }
};

template <class XT>
struct XWithBuf : XT {
  uint8_t* buf;  // the wave's window buffer in LDS
};

// The x limbs a unit of F reads, and how it reads them; LDS bytes per wave
// that F needs beyond the limbs.
template <class F>
struct LimbX {
  using T = XLimbs;
  static constexpr int kWaveLds = 0;
  __device__ static __forceinline__ void load(const uint8_t* lds, int cols, int u, T& o) { load_limbs(lds, cols, u, o); }
};
template <>
struct LimbX<LimbQ6K> {
  using T = XLimbsQ6;
  static constexpr int kWaveLds = 0;
  __device__ static __forceinline__ void load(const uint8_t* lds, int cols, int u, T& o) {
    LimbQ6K::load_x(lds, cols, u, o);
  }
};
template <class F>
struct LimbX<LimbWin<F>> {
  using T = XWithBuf<typename LimbX<F>::T>;
  static constexpr int kWaveLds = F::kWinBytes;
  __device__ static __forceinline__ void load(const uint8_t* lds, int cols, int u, T& o) {
    LimbX<F>::load(lds, cols, u, o);
    o.buf = const_cast<uint8_t*>(lds) + limb_lds_bytes(cols) + int(threadIdx.x >> 6) * F::kWinBytes;
  }
};

}  // namespace sh
