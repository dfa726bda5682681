// Batched prefill matmul on MFMA: Y[t][r] = sum_c W[r][c] * X[t][c] for m
// tokens, W packed Q4_K / Q5_K / Q8_0 / Q6_K / IQ4_XS [rows][cols], X and Y
// f32 row-major.
//
// The reference has no matmul: prefill runs one forward per token
// (crates/strata-core/src/generate.rs:116-117), so the op is defined as m
// independent ops::gemv calls (crates/strata-core/src/ops.rs:14-28).
//
// Two modes:
//   bf16  X is rounded to bf16; each workgroup dequantizes its weight rows
//         chunk by chunk into a bf16 LDS tile and runs
//         v_mfma_f32_32x32x16_bf16 with f32 accumulation.
//   q8    X is quantized to Q8 blocks (32 elements, f32 scale max|x| / 127,
//         int8 codes rounded to nearest even); the weight codes go to LDS as
//         int8 and v_mfma_i32_32x32x32_i8 computes one exact integer dot per
//         32-element block, which the VALU scales by the weight block's scale
//         and the activation block's scale (and subtracts the Q4_K min term).
//
// Workgroup tile: 256 tokens x 96 weight rows, K in 64-element chunks.
// bf16 (mm_bf16_ws_kernel): 8 waves by role -- 4 consumers (wave w owns
// tokens [64w, 64w + 64) and all 96 rows: 2 x 3 MFMA tiles of 32 x 32),
// 3 stagers dequantizing each weight chunk into a double-buffered bf16 LDS
// tile, one barrier per chunk; each consumer loads its activation fragments
// from a fragment-ordered bf16 copy written by a pre-pass (1 KiB contiguous
// a wave load) into registers two chunks ahead. q8 (mm_q8_kernel): 4 waves
// stacked along the tokens, the weight codes staged through LDS, activation
// fragments loaded from the pre-pass's tiled int8 copy. The MFMA's k order
// is free as long as A and B agree, so lane half h of k-step s holds chunk
// elements [32h + 8s, +8) (bf16) or [32s + 16h, +16) (int8) of both
// operands, which keeps every fragment one 16-byte load. Tiles are numbered
// so that the 8 XCDs (workgroup i runs on XCD i % 8) each get a contiguous
// run of weight rows, and the token tiles of one weight tile share that
// XCD's L2.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Four bytes each times a small factor f (every product < 256, so no byte
// carries into the next): one v_pk_mul_lo_u16 over the word's two halves.
__device__ __forceinline__ uint32_t bytes_times(uint32_t w, uint32_t f) {
  const u16x2 v = __builtin_bit_cast(u16x2, w);
  const u16x2 k = {static_cast<unsigned short>(f), static_cast<unsigned short>(f)};
  return __builtin_bit_cast(uint32_t, v * k);
}
// Bytes p (0..255) less k (0..127, the same in every byte), each mod 256:
// with bit 7 set first no byte borrows from the next; the xor restores it.
__device__ __forceinline__ uint32_t bytes_minus(uint32_t p, uint32_t k4) {
  return ((p | 0x80808080u) - k4) ^ (~p & 0x80808080u);
}

constexpr int kMmBM = 256;                  // tokens per workgroup
constexpr int kMmBN = 96;                   // weight rows per workgroup
constexpr int kMmKC = 64;                   // K elements per chunk
constexpr int kMmRowB = kMmKC * 2 + 16;     // bytes per bf16 LDS row (padded)
constexpr int kMmRowQ = kMmKC + 16;         // bytes per int8 LDS row (padded)

// Two floats -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// ------------------------------------------------------------ weight stagers --
// A stager turns one row's 64-element chunk c of packed blocks into values
// for the LDS tile. The chunk is split into kPieces pieces per row, each a
// thread's task: `load` issues the global loads (so they can be in flight a
// chunk ahead), `emit_bf16` writes two runs of 16 bf16 at chunk offsets
// o0 and o1, `emit_q8` writes the same runs as int8 codes plus the block
// scale (and min) for the int8 path.

// Q4_K: chunk c is group g = c % 4 of super-block c / 4; piece hb holds qs
// bytes [16hb, 16hb + 16) of the group, whose low nibbles are elements
// [16hb, +16) (sub-block 2g) and high nibbles [32 + 16hb, +16) (sub-block
// 2g + 1). dequant.rs:247-270 and get_scale_min_k4 (dequant.rs:237-245).
struct StQ4K {
  static constexpr int kPieces = 2;
  static constexpr bool kQ8 = true;
  static constexpr bool kQ8K = true;  // int8 mode on 256-element activation blocks
  static constexpr bool kMin = true;  // value d * q - m
  struct Raw {
    u32x4 h, q;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int c, int hb) {
    const uint8_t* sb = row + (c >> 2) * 144;
    return {ld16(sb), ld16(sb + 16 + 32 * (c & 3) + 16 * hb)};
  }
  // 6-bit scales (scp) and mins (mp) of sub-blocks 2g and 2g + 1 in bytes 0, 1
  __device__ static __forceinline__ void scale_bytes(const u32x4& h, int g, uint32_t& scp, uint32_t& mp) {
    const uint32_t s = (g & 1) << 4;
    const uint32_t t1 = h.y >> s, t2 = h.z >> s, t3 = h.w >> s;
    // both readings, then a mask select: no branch on the wave-uniform g, so
    // staging stays in the MFMAs' basic block
    const uint32_t hi_sel = 0u - uint32_t(g >> 1);  // all ones for g >= 2
    scp = ((t1 & 0x3F3Fu) & ~hi_sel) | (((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u)) & hi_sel);
    mp = ((t2 & 0x3F3Fu) & ~hi_sel) | ((((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u)) & hi_sel);
  }
  // all eight 6-bit scales and mins of the super-block, four per word
  // (get_scale_min_k4, dequant.rs:237-245)
  __device__ static __forceinline__ void all_scale_bytes(const u32x4& h, uint32_t& sc03, uint32_t& sc47,
                                                         uint32_t& m03, uint32_t& m47) {
    sc03 = h.y & 0x3F3F3F3Fu;
    m03 = h.z & 0x3F3F3F3Fu;
    sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  }
  // d * sc and dmin * m of sub-blocks 2g and 2g + 1
  __device__ static __forceinline__ void scales(const u32x4& h, int g, float& d0, float& m0, float& d1,
                                                float& m1) {
    uint32_t scp, mp;
    scale_bytes(h, g, scp, mp);
    const float d = h2f(h.x), dm = h2f(h.x >> 16);
    d0 = d * ubyte<0>(scp);
    d1 = d * ubyte<1>(scp);
    m0 = dm * ubyte<0>(mp);
    m1 = dm * ubyte<1>(mp);
  }
  // d * sc_j and dmin * m_j of all eight sub-blocks: the products scales()
  // forms, for a stager that decodes them once per super-block
  __device__ static __forceinline__ void sb_scales(const u32x4& h, float* d8, float* m8) {
    uint32_t sc03, sc47, m03, m47;
    all_scale_bytes(h, sc03, sc47, m03, m47);
    const float d = h2f(h.x), dm = h2f(h.x >> 16);
    d8[0] = d * ubyte<0>(sc03); d8[1] = d * ubyte<1>(sc03); d8[2] = d * ubyte<2>(sc03); d8[3] = d * ubyte<3>(sc03);
    d8[4] = d * ubyte<0>(sc47); d8[5] = d * ubyte<1>(sc47); d8[6] = d * ubyte<2>(sc47); d8[7] = d * ubyte<3>(sc47);
    m8[0] = dm * ubyte<0>(m03); m8[1] = dm * ubyte<1>(m03); m8[2] = dm * ubyte<2>(m03); m8[3] = dm * ubyte<3>(m03);
    m8[4] = dm * ubyte<0>(m47); m8[5] = dm * ubyte<1>(m47); m8[6] = dm * ubyte<2>(m47); m8[7] = dm * ubyte<3>(m47);
  }
  __device__ static __forceinline__ void emit_bf16(const Raw& r, int c, int hb, uint32_t* run0,
                                                   uint32_t* run1, int& o0, int& o1, int) {
    float d0, m0, d1, m1;
    scales(r.h, c & 3, d0, m0, d1, m1);
    emit_bf16_sc(r, c, hb, d0, m0, d1, m1, run0, run1, o0, o1);
  }
  __device__ static __forceinline__ void emit_bf16_sc(const Raw& r, int, int hb, float d0, float m0, float d1,
                                                      float m1, uint32_t* run0, uint32_t* run1, int& o0,
                                                      int& o1) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
      // keep the masked words whole, so each byte converts with one
      // v_cvt_f32_ubyteN instead of an extract and a convert
      asm volatile("" : "+v"(lo), "+v"(hi));
      run0[2 * k] = pack_bf16(__builtin_fmaf(d0, ubyte<0>(lo), -m0), __builtin_fmaf(d0, ubyte<1>(lo), -m0));
      run0[2 * k + 1] =
          pack_bf16(__builtin_fmaf(d0, ubyte<2>(lo), -m0), __builtin_fmaf(d0, ubyte<3>(lo), -m0));
      run1[2 * k] = pack_bf16(__builtin_fmaf(d1, ubyte<0>(hi), -m1), __builtin_fmaf(d1, ubyte<1>(hi), -m1));
      run1[2 * k + 1] =
          pack_bf16(__builtin_fmaf(d1, ubyte<2>(hi), -m1), __builtin_fmaf(d1, ubyte<3>(hi), -m1));
    }
    o0 = 16 * hb;
    o1 = 32 + 16 * hb;
  }
  // K-quant int8 path: the codes times the two limbs of their sub-block's
  // scale, sc = 8 sh + sl (sh, sl <= 7: products <= 105 fit int8), for
  // sub-blocks 2g (h0, l0) and 2g + 1 (h1, l1)
  static constexpr int kCenter = 0;  // codes enter unshifted
  __device__ static __forceinline__ void emit_q8k(const Raw& r, int c, uint32_t* h0, uint32_t* l0,
                                                  uint32_t* h1, uint32_t* l1) {
    uint32_t scp, mp;
    scale_bytes(r.h, c & 3, scp, mp);
    const uint32_t sh0 = (scp >> 3) & 7u, sl0 = scp & 7u, sh1 = (scp >> 11) & 7u, sl1 = (scp >> 8) & 7u;
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t a = q[k] & 0x0F0F0F0Fu, b = (q[k] >> 4) & 0x0F0F0F0Fu;
      h0[k] = bytes_times(a, sh0);
      l0[k] = bytes_times(a, sl0);
      h1[k] = bytes_times(b, sh1);
      l1[k] = bytes_times(b, sl1);
    }
  }
  // int8 codes 0..15; run k lies in block jb_k of the chunk, whose values
  // are dj[k] * q - mj[k]
  __device__ static __forceinline__ void emit_q8(const Raw& r, int c, int hb, uint32_t* run0,
                                                 uint32_t* run1, int& o0, int& o1, int& jb0, int& jb1,
                                                 float* dj, float* mj) {
    scales(r.h, c & 3, dj[0], mj[0], dj[1], mj[1]);
    jb0 = 0;
    jb1 = 1;
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      run0[k] = q[k] & 0x0F0F0F0Fu;
      run1[k] = (q[k] >> 4) & 0x0F0F0F0Fu;
    }
    o0 = 16 * hb;
    o1 = 32 + 16 * hb;
  }
};

// Q5_K: chunk c and piece hb as StQ4K (176-byte super-blocks, codes at byte
// 48); each code takes its fifth bit from the qh bytes of the same element
// positions [16hb, +16): bit 2g for the low nibbles, 2g + 1 for the high
// (q5k_codes; dequant.rs:272-302), so codes run 0..31.
struct StQ5K {
  static constexpr int kPieces = 2;
  static constexpr bool kQ8 = true;
  static constexpr bool kQ8K = true;
  static constexpr bool kMin = true;  // value d * q - m
  struct Raw {
    u32x4 h, q, qh;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int c, int hb) {
    const uint8_t* sb = row + (c >> 2) * 176;
    return {ld16(sb), ld16(sb + 48 + 32 * (c & 3) + 16 * hb), ld16(sb + 16 + 16 * hb)};
  }
  __device__ static __forceinline__ void codes(const Raw& r, int c, uint32_t* lo, uint32_t* hi) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) q5k_codes(q[k], qh[k], uint32_t(c & 3), lo[k], hi[k]);
  }
  __device__ static __forceinline__ void sb_scales(const u32x4& h, float* d8, float* m8) {
    StQ4K::sb_scales(h, d8, m8);
  }
  __device__ static __forceinline__ void emit_bf16(const Raw& r, int c, int hb, uint32_t* run0,
                                                   uint32_t* run1, int& o0, int& o1, int) {
    float d0, m0, d1, m1;
    StQ4K::scales(r.h, c & 3, d0, m0, d1, m1);
    emit_bf16_sc(r, c, hb, d0, m0, d1, m1, run0, run1, o0, o1);
  }
  __device__ static __forceinline__ void emit_bf16_sc(const Raw& r, int c, int hb, float d0, float m0, float d1,
                                                      float m1, uint32_t* run0, uint32_t* run1, int& o0,
                                                      int& o1) {
    uint32_t lo[4], hi[4];
    codes(r, c, lo, hi);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      run0[2 * k] = pack_bf16(__builtin_fmaf(d0, ubyte<0>(lo[k]), -m0), __builtin_fmaf(d0, ubyte<1>(lo[k]), -m0));
      run0[2 * k + 1] =
          pack_bf16(__builtin_fmaf(d0, ubyte<2>(lo[k]), -m0), __builtin_fmaf(d0, ubyte<3>(lo[k]), -m0));
      run1[2 * k] = pack_bf16(__builtin_fmaf(d1, ubyte<0>(hi[k]), -m1), __builtin_fmaf(d1, ubyte<1>(hi[k]), -m1));
      run1[2 * k + 1] =
          pack_bf16(__builtin_fmaf(d1, ubyte<2>(hi[k]), -m1), __builtin_fmaf(d1, ubyte<3>(hi[k]), -m1));
    }
    o0 = 16 * hb;
    o1 = 32 + 16 * hb;
  }
  // K-quant int8 path as StQ4K::emit_q8k, on the codes less 16 (-16..15,
  // so that sh * (q - 16) and sl * (q - 16) fit int8); the 16 * sc part
  // returns through the code sums
  static constexpr int kCenter = 16;
  __device__ static __forceinline__ void emit_q8k(const Raw& r, int c, uint32_t* h0, uint32_t* l0,
                                                  uint32_t* h1, uint32_t* l1) {
    uint32_t scp, mp;
    StQ4K::scale_bytes(r.h, c & 3, scp, mp);
    const uint32_t sh0 = (scp >> 3) & 7u, sl0 = scp & 7u, sh1 = (scp >> 11) & 7u, sl1 = (scp >> 8) & 7u;
    uint32_t lo[4], hi[4];
    codes(r, c, lo, hi);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // codes <= 31 times <= 7: products <= 217, one byte each
      h0[k] = bytes_minus(bytes_times(lo[k], sh0), 0x10101010u * sh0);
      l0[k] = bytes_minus(bytes_times(lo[k], sl0), 0x10101010u * sl0);
      h1[k] = bytes_minus(bytes_times(hi[k], sh1), 0x10101010u * sh1);
      l1[k] = bytes_minus(bytes_times(hi[k], sl1), 0x10101010u * sl1);
    }
  }
  // int8 codes 0..31, blocks as StQ4K::emit_q8
  __device__ static __forceinline__ void emit_q8(const Raw& r, int c, int hb, uint32_t* run0,
                                                 uint32_t* run1, int& o0, int& o1, int& jb0, int& jb1,
                                                 float* dj, float* mj) {
    StQ4K::scales(r.h, c & 3, dj[0], mj[0], dj[1], mj[1]);
    jb0 = 0;
    jb1 = 1;
    codes(r, c, run0, run1);
    o0 = 16 * hb;
    o1 = 32 + 16 * hb;
  }
};

// Q8_0: chunk c is blocks 2c and 2c + 1 (68 bytes from 68c, 4-byte aligned);
// piece hb is block hb, read through the aligned 36-byte window at
// 68c + 32hb. dequant.rs:123-128: value = q * d (exact in f32).
struct StQ8 {
  static constexpr int kPieces = 2;
  static constexpr bool kQ8 = true;
  static constexpr bool kQ8K = false;  // 32-element activation blocks, as its own scales
  static constexpr bool kMin = false;  // value d * q
  struct Raw {
    u32x4 a, b;
    uint32_t e;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int c, int hb) {
    const uint8_t* p = row + 68 * c + 32 * hb;
    return {ld16(p), ld16(p + 16), ld4(p + 32)};
  }
  __device__ static __forceinline__ void codes(const Raw& r, int hb, uint32_t* q, float& d) {
    const uint32_t w[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.e};
    d = h2f(hb ? (w[0] >> 16) : w[0]);
#pragma unroll
    for (int k = 0; k < 8; ++k) q[k] = hb ? w[k + 1] : realign(w[k], w[k + 1], 2);
  }
  __device__ static __forceinline__ void emit_bf16(const Raw& r, int, int hb, uint32_t* run0,
                                                   uint32_t* run1, int& o0, int& o1, int) {
    uint32_t q[8];
    float d;
    codes(r, hb, q, d);
    const float bias = -128.f * d;  // (q ^ 0x80) - 128 = q: d * q exactly
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t u = q[k] ^ 0x80808080u;
      uint32_t* dst = k < 4 ? run0 + 2 * k : run1 + 2 * (k - 4);
      dst[0] = pack_bf16(__builtin_fmaf(d, ubyte<0>(u), bias), __builtin_fmaf(d, ubyte<1>(u), bias));
      dst[1] = pack_bf16(__builtin_fmaf(d, ubyte<2>(u), bias), __builtin_fmaf(d, ubyte<3>(u), bias));
    }
    o0 = 32 * hb;
    o1 = 32 * hb + 16;
  }
  __device__ static __forceinline__ void emit_q8(const Raw& r, int, int hb, uint32_t* run0,
                                                 uint32_t* run1, int& o0, int& o1, int& jb0, int& jb1,
                                                 float* dj, float* mj) {
    uint32_t q[8];
    float d;
    codes(r, hb, q, d);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      run0[k] = q[k];
      run1[k] = q[k + 4];
    }
    // both runs are block hb
    jb0 = jb1 = hb;
    dj[0] = dj[1] = d;
    mj[0] = mj[1] = 0.f;
    o0 = 32 * hb;
    o1 = 32 * hb + 16;
  }
};

// IQ4_XS: chunk c is sub-blocks 2g and 2g + 1 (g = c % 4) of super-block
// c / 4 (136 bytes); piece hb is sub-block 2g + hb, whose 16 qs bytes (the
// reference's qs[0..16], or ggml's qs[16 ib ..] with GGML; dequant.rs:189-206)
// give elements [32 hb, +16) from their low nibbles and [32 hb + 16, +16)
// from their high ones: code-book values v (int8) scaled by dl = d * (ls - 32).
template <bool GGML>
struct StIQ4XS {
  static constexpr int kPieces = 2;
  static constexpr bool kQ8 = true;
  static constexpr bool kQ8K = false;  // 32-element activation blocks, as its own scales
  static constexpr bool kMin = false;  // value dl * v
  struct Raw {
    uint32_t h0, h1;
    u32x4 q;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int c, int hb) {
    const uint8_t* sb = row + (c >> 2) * 136;
    const int ib = 2 * (c & 3) + hb;
    return {ld4(sb), ld4(sb + 4), ld16u(sb + 8 + (GGML ? 16 * ib : 0))};
  }
  __device__ static __forceinline__ float scale(const Raw& r, int c, int hb) {
    return h2f(r.h0) * iq4xs_scale(r.h0, r.h1, 2 * (c & 3) + hb);
  }
  __device__ static __forceinline__ void emit_bf16(const Raw& r, int c, int hb, uint32_t* run0,
                                                   uint32_t* run1, int& o0, int& o1, int) {
    const float dl = scale(r, c, hb);
    const float bias = -128.f * dl;  // dl * ((v ^ 0x80) - 128) = dl * v, one rounding
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = iq4_lut(q[k] & 0x0F0F0F0Fu) ^ 0x80808080u;
      const uint32_t hi = iq4_lut((q[k] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u;
      run0[2 * k] = pack_bf16(__builtin_fmaf(dl, ubyte<0>(lo), bias), __builtin_fmaf(dl, ubyte<1>(lo), bias));
      run0[2 * k + 1] = pack_bf16(__builtin_fmaf(dl, ubyte<2>(lo), bias), __builtin_fmaf(dl, ubyte<3>(lo), bias));
      run1[2 * k] = pack_bf16(__builtin_fmaf(dl, ubyte<0>(hi), bias), __builtin_fmaf(dl, ubyte<1>(hi), bias));
      run1[2 * k + 1] = pack_bf16(__builtin_fmaf(dl, ubyte<2>(hi), bias), __builtin_fmaf(dl, ubyte<3>(hi), bias));
    }
    o0 = 32 * hb;
    o1 = 32 * hb + 16;
  }
  // int8 codes: the code-book values themselves; both runs are block hb
  __device__ static __forceinline__ void emit_q8(const Raw& r, int c, int hb, uint32_t* run0,
                                                 uint32_t* run1, int& o0, int& o1, int& jb0, int& jb1,
                                                 float* dj, float* mj) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      run0[k] = iq4_lut(q[k] & 0x0F0F0F0Fu);
      run1[k] = iq4_lut((q[k] >> 4) & 0x0F0F0F0Fu);
    }
    jb0 = jb1 = hb;
    dj[0] = dj[1] = scale(r, c, hb);
    mj[0] = mj[1] = 0.f;
    o0 = 32 * hb;
    o1 = 32 * hb + 16;
  }
};

// Q6_K: chunk c is quarter j = c % 4 of super-block c / 4 (half h = j / 2,
// nibble tp = j % 2); piece hb holds elements [16hb, +16) and
// [32 + 16hb, +16) of the quarter. dequant.rs:208-234: value
// d * sc * (q - 32) with q = (ql nibble) | (qh 2 bits << 4); sc read as u8
// (dequant.rs:211,224-227) or, with the signed-scale flag, as i8.
struct StQ6K {
  static constexpr int kPieces = 2;
  static constexpr bool kQ8 = false;  // 16-element scales: its own int8 kernel (mm_i8q6_kernel)
  static constexpr bool kQ8K = false;
  struct Raw {
    u32x4 l0, l1, qh;
    uint32_t l0e, l1e, qhe, s0, s1;
    uint32_t d;
  };
  __device__ static __forceinline__ Raw load(const uint8_t* row, int c, int hb) {
    const uint8_t* blk = row + (c >> 2) * 210;
    const int j = c & 3, h = j >> 1, tp = j & 1;
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* base = blk - s;  // rows are 2-byte aligned: s is 0 or 2
    const uint8_t* p0 = base + 64 * h + 16 * hb;
    const uint8_t* p1 = p0 + 32;
    const uint8_t* ph = base + 128 + 32 * h + 16 * hb;
    const uint8_t* ps = base + 192 + 8 * h + 4 * tp;
    Raw r;
    r.l0 = ld16(p0);
    r.l0e = ld4(p0 + 16);
    r.l1 = ld16(p1);
    r.l1e = ld4(p1 + 16);
    r.qh = ld16(ph);
    r.qhe = ld4(ph + 16);
    r.s0 = ld4(ps);
    r.s1 = s ? ld4(ps + 4) : 0u;  // ends at blk + 210; with s = 0 it is not needed
    r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    return r;
  }
  // 6-bit codes of the two runs (4 per word) and the scale bytes of the piece
  __device__ static __forceinline__ void decode(const Raw& r, int c, uint32_t shift, uint32_t* va,
                                                uint32_t* vb, uint32_t& scw) {
    const uint32_t tp = uint32_t(c & 1);
    const uint32_t L0[5] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w, r.l0e};
    const uint32_t L1[5] = {r.l1.x, r.l1.y, r.l1.z, r.l1.w, r.l1e};
    const uint32_t QH[5] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w, r.qhe};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      q6_code_words(L0[k], L0[k + 1], L1[k], L1[k + 1], QH[k], QH[k + 1], shift, tp, va[k], vb[k]);
    }
    scw = realign(r.s0, r.s1, shift);
  }
};

// ----------------------------------------------------- activation pre-pass --
// X f32 -> bf16 (round to nearest even), 8 elements per thread.
// X f32 -> bf16 (round to nearest even) in the order the bf16 kernel's
// consumer waves load their A fragments: piece i = ((T * nchunks + c) * 4 +
// s) * 64 + lane holds token 32 T + (lane & 31) (the last token repeated
// past m), elements c * 64 + 32 (lane >> 5) + 8 s .. + 8, so one wave load
// of a fragment is 1 KiB of contiguous bytes. One thread per piece.
__global__ void x_bf16_tiled_kernel(const float* __restrict__ x, u32x4* __restrict__ xt, int m, int cols,
                                    int64_t pieces) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= pieces) return;
  const int lane = int(i & 63), s = int((i >> 6) & 3);
  const int64_t rest = i >> 8;
  const int nchunks = cols / kMmKC;
  const int c = int(rest % nchunks);
  const int64_t T = rest / nchunks;
  const int64_t t = min(32 * T + (lane & 31), int64_t(m) - 1);
  const f32x4* src = reinterpret_cast<const f32x4*>(x + t * cols + c * kMmKC + 32 * (lane >> 5) + 8 * s);
  const f32x4 a = src[0], b = src[1];
  xt[i] = u32x4{pack_bf16(a.x, a.y), pack_bf16(a.z, a.w), pack_bf16(b.x, b.y), pack_bf16(b.z, b.w)};
}

// X f32 -> Q8 blocks of 32: s = max|x| / 127 (f32 division), q = rne(x / s)
// (0 where s == 0), plus u = s * sum(q) for the Q4_K min term. One thread
// per block; `blocks` = m * cols / 32, scales indexed [token][block].
__device__ __forceinline__ void q8_block(const float* __restrict__ x32, uint32_t* w, float& s_out, float& u_out) {
  const f32x4* xv = reinterpret_cast<const f32x4*>(x32);
  float v[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const f32x4 t = xv[k];
    v[4 * k] = t.x;
    v[4 * k + 1] = t.y;
    v[4 * k + 2] = t.z;
    v[4 * k + 3] = t.w;
  }
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(v[k]));
  const float s = __fdiv_rn(amax, 127.f);
  int sum = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = s > 0.f ? int(__builtin_rintf(__fdiv_rn(v[4 * k + e], s))) : 0;
      sum += c;
      word |= (uint32_t(c) & 0xFFu) << (8 * e);
    }
    w[k] = word;
  }
  s_out = s;
  u_out = s * float(sum);
}

__global__ void x_q8_kernel(const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ s_out,
                            float* __restrict__ u_out, int64_t blocks) {
  const int64_t b = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (b >= blocks) return;
  uint32_t w[8];
  float sv, uv;
  q8_block(x + 32 * b, w, sv, uv);
  u32x4* qv = reinterpret_cast<u32x4*>(q + 32 * b);
  qv[0] = u32x4{w[0], w[1], w[2], w[3]};
  qv[1] = u32x4{w[4], w[5], w[6], w[7]};
  s_out[b] = sv;
  u_out[b] = uv;
}

// The same blocks for the q8 matmul, in the order its waves load them
// (tokens padded with zero blocks to a multiple of 32; T = token / 32,
// l = token % 32, block j = 2c + s of chunk c, nsb = ceil(blocks / 8)):
//   codes: 16-byte piece ((T * nch + c) * 2 + s) * 64 + 32 h + l holds codes
//          [16h, 16h + 16) of the block (one 1 KiB wave load per fragment);
//   s:     float (T * nblk + j) * 32 + l (one 128-byte run per block);
//   u:     u = s * sum(codes) split into bf16 halves hi = bf16(u), lo =
//          bf16(u - hi) (u to about 2^-17), as the B operand of the min-term
//          MFMA: 16-byte piece (T * nsb + j / 8) * 64 + 32 ((j % 8) / 4) + l,
//          word j % 4 = hi | lo << 16.
__global__ void x_q8_tiled_kernel(const float* __restrict__ x, u32x4* __restrict__ qt, float* __restrict__ st,
                                  uint32_t* __restrict__ ut, int m, int cols, int64_t blocks) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;  // (T, j, l)
  if (i >= blocks) return;
  const int nblk = cols / 32, nch = cols / kMmKC, nsb = (nblk + 7) >> 3;
  const int l = int(i & 31);
  const int64_t tj = i >> 5;
  const int j = int(tj % nblk);
  const int64_t T = tj / nblk;
  const int64_t t = 32 * T + l;
  uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  float sv = 0.f, uv = 0.f;
  if (t < m) q8_block(x + t * cols + 32 * j, w, sv, uv);
  const int c = j >> 1, s = j & 1;
  u32x4* dst = qt + ((T * nch + c) * 2 + s) * 64 + l;
  dst[0] = u32x4{w[0], w[1], w[2], w[3]};
  dst[32] = u32x4{w[4], w[5], w[6], w[7]};
  st[i] = sv;
  const uint32_t hi = __builtin_bit_cast(unsigned short, __bf16(uv));
  const uint32_t lo = __builtin_bit_cast(unsigned short, __bf16(uv - float(__builtin_bit_cast(__bf16, (unsigned short)hi))));
  ut[((T * nsb + (j >> 3)) * 64 + 32 * ((j & 7) >> 2) + l) * 4 + (j & 3)] = hi | (lo << 16);
}

// X f32 -> Q8 blocks of 256 (the K-quant int8 path: one scale per weight
// super-block): s = max|x| / 127 over the 256 (f32 division), q = rne(x / s)
// (0 where s == 0), and the integer code sum of each 32-element sub-block.
// One wave per (token, super-block), lane L holding elements 4L .. 4L + 3;
// the lane's four codes, s (from every lane) and its sub-block's sum (from
// lanes 8j, zero elsewhere) are returned.
__device__ __forceinline__ void q8k_wave(const float* __restrict__ x256, bool live, int lane, uint32_t& codes,
                                         float& s_out, int& sum_out) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (live) v = reinterpret_cast<const f32x4*>(x256)[lane];
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  const float s = __fdiv_rn(amax, 127.f);
  const float e[4] = {v.x, v.y, v.z, v.w};
  uint32_t word = 0;
  int sum = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = s > 0.f ? int(__builtin_rintf(__fdiv_rn(e[k], s))) : 0;
    sum += c;
    word |= (uint32_t(c) & 0xFFu) << (8 * k);
  }
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  sum += __shfl_xor(sum, 4, 64);
  codes = word;
  s_out = s;
  sum_out = sum;
}

// Plain layout (sh_quantize_q8k_dev): codes [n], scales [n / 256], sums [n / 32].
__global__ void __launch_bounds__(256) x_q8k_kernel(const float* __restrict__ x, uint32_t* __restrict__ q,
                                                    float* __restrict__ s_out, int* __restrict__ sums,
                                                    int64_t supers) {
  const int64_t wv = (blockIdx.x * int64_t(blockDim.x) + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wv >= supers) return;  // whole waves
  uint32_t codes;
  float sv;
  int sum;
  q8k_wave(x + 256 * wv, true, lane, codes, sv, sum);
  q[64 * wv + lane] = codes;
  if (lane == 0) s_out[wv] = sv;
  if ((lane & 7) == 0) sums[8 * wv + (lane >> 3)] = sum;
}

// The same blocks for mm_q8k_kernel, in the order its waves load them
// (tokens padded with zero blocks to a multiple of 32; T = token / 16,
// j = token % 16, nch = cols / 64, nsb = cols / 256):
//   codes: 16-byte piece (T * nch + c) * 64 + 16 g + j holds chunk c's
//          elements [16 g, 16 g + 16) (one 1 KiB wave load per 16-token tile);
//   s:     float (T * nsb + sb) * 16 + j;
//   sums:  8-byte piece (T * nsb + sb) * 64 + 16 g + j, four f16: g = 0, 1
//          the high parts b >> 6 of sub-blocks 4g .. 4g + 3, g = 2, 3 the low
//          parts b & 63 of sub-blocks 4(g - 2) .. +3 (b = 64 hi + lo exactly;
//          both exact in f16): the B operand of the min-term MFMA.
__global__ void __launch_bounds__(256) x_q8k_tiled_kernel(const float* __restrict__ x, uint8_t* __restrict__ qt,
                                                          float* __restrict__ st, uint8_t* __restrict__ bt, int m,
                                                          int cols, int64_t waves) {
  const int64_t wv = (blockIdx.x * int64_t(blockDim.x) + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wv >= waves) return;  // whole waves
  const int nsb = cols >> 8, nch = cols / kMmKC;
  const int sb = int(wv % nsb);
  const int64_t t = wv / nsb;  // padded token
  const int64_t T = t >> 4;
  const int j = int(t & 15);
  uint32_t codes;
  float sv;
  int sum;
  q8k_wave(x + (t < m ? t : 0) * int64_t(cols) + 256 * sb, t < m, lane, codes, sv, sum);
  // element 4 lane of the super-block: chunk 4 sb + lane / 16, group
  // (lane / 4) & 3, bytes 4 (lane & 3) of the piece
  const int c = 4 * sb + (lane >> 4), g = (lane >> 2) & 3;
  const int64_t piece = (T * nch + c) * 64 + 16 * g + j;
  *reinterpret_cast<uint32_t*>(qt + piece * 16 + 4 * (lane & 3)) = codes;
  if (lane == 0) st[(T * nsb + sb) * 16 + j] = sv;
  if ((lane & 7) == 0) {
    const int sj = lane >> 3;  // sub-block
    _Float16* b = reinterpret_cast<_Float16*>(bt + ((T * nsb + sb) * 64 + j) * 8);
    b[16 * 4 * (sj >> 2) + (sj & 3)] = _Float16(float(sum >> 6));            // group sj / 4
    b[16 * 4 * (2 + (sj >> 2)) + (sj & 3)] = _Float16(float(sum & 63));      // group 2 + sj / 4
  }
}

// --------------------------------------------------------------- tile order --
__device__ __forceinline__ void tile_of(int n_tiles_m, int& r0, int& t0) {
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  r0 = (bid / n_tiles_m) * kMmBN;
  t0 = (bid % n_tiles_m) * kMmBM;
}

// Q6_K piece -> bf16 runs (scale bytes of the runs: hb and 2 + hb)
__device__ __forceinline__ void q6k_emit_bf16(const StQ6K::Raw& r, int c, int hb, uint32_t shift,
                                              uint32_t* run0, uint32_t* run1, int& o0, int& o1, int q6s) {
  uint32_t va[4], vb[4], scw;
  StQ6K::decode(r, c, shift, va, vb, scw);
  const uint32_t b0 = (scw >> (8 * hb)) & 0xFFu, b1 = (scw >> (8 * (2 + hb))) & 0xFFu;
  const float sc0 = q6s ? float(int8_t(b0)) : float(b0), sc1 = q6s ? float(int8_t(b1)) : float(b1);
  const float d = h2f(r.d);
  const float ds0 = d * sc0, ds1 = d * sc1;
  const float z0 = -32.f * ds0, z1 = -32.f * ds1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    run0[2 * k] = pack_bf16(__builtin_fmaf(ds0, ubyte<0>(va[k]), z0), __builtin_fmaf(ds0, ubyte<1>(va[k]), z0));
    run0[2 * k + 1] =
        pack_bf16(__builtin_fmaf(ds0, ubyte<2>(va[k]), z0), __builtin_fmaf(ds0, ubyte<3>(va[k]), z0));
    run1[2 * k] = pack_bf16(__builtin_fmaf(ds1, ubyte<0>(vb[k]), z1), __builtin_fmaf(ds1, ubyte<1>(vb[k]), z1));
    run1[2 * k + 1] =
        pack_bf16(__builtin_fmaf(ds1, ubyte<2>(vb[k]), z1), __builtin_fmaf(ds1, ubyte<3>(vb[k]), z1));
  }
  o0 = 16 * hb;
  o1 = 32 + 16 * hb;
}

template <class S>
struct Bf16Emit {
  __device__ static __forceinline__ void run(const typename S::Raw& r, int c, int hb, uint32_t,
                                             uint32_t* run0, uint32_t* run1, int& o0, int& o1, int q6s) {
    S::emit_bf16(r, c, hb, run0, run1, o0, o1, q6s);
  }
};
template <>
struct Bf16Emit<StQ6K> {
  __device__ static __forceinline__ void run(const StQ6K::Raw& r, int c, int hb, uint32_t shift,
                                             uint32_t* run0, uint32_t* run1, int& o0, int& o1, int q6s) {
    q6k_emit_bf16(r, c, hb, shift, run0, run1, o0, o1, q6s);
  }
};

// K-quants with 8 sub-block scales per 256-element super-block (4 chunks):
// the bf16 stagers decode them once per super-block (sb_scales).
template <class S>
struct SbScales {
  static constexpr bool value = false;
};
template <>
struct SbScales<StQ4K> {
  static constexpr bool value = true;
};
template <>
struct SbScales<StQ5K> {
  static constexpr bool value = true;
};

// Alignment shift of the block a Q6_K piece reads (0 for the other formats).
template <class S>
__device__ __forceinline__ uint32_t block_shift(const uint8_t*, int) {
  return 0;
}
template <>
__device__ __forceinline__ uint32_t block_shift<StQ6K>(const uint8_t* row, int c) {
  return uint32_t(reinterpret_cast<uintptr_t>(row + (c >> 2) * 210)) & 3u;
}

// ------------------------------------------------- bf16 kernel, 8 waves --
// The same tile (256 tokens x 96 weight rows, K in 64-element chunks) with
// the work split by role, so that each SIMD holds a wave that issues MFMAs
// next to one that stages (waves w and w + 4 share a SIMD; an MFMA wave
// slows the other wave's VALU issue by about a tenth, so the two overlap):
// waves 0-3 consume (tokens [64 w, 64 w + 64) x
// all 96 rows), waves 4-6 dequantize the weight chunks (one 32-element run
// of one row per lane, loads kBfDepth chunks ahead) into a double-buffered
// bf16 LDS tile, wave 7 only keeps the barrier count. A consumer's
// activation rows are its own, so it loads their fragments straight into
// registers two chunks ahead, from the fragment-ordered copy the pre-pass
// writes (every row tile re-reads them from L2, 1 KiB contiguous a wave
// load), and LDS carries only the weight tile the four consumers share. One barrier
// per chunk: during chunk c the consumers read B buffer c & 1 while B(c + 1)
// is staged into the other one.
constexpr int kMmWsThreads = 512;
constexpr size_t kMmLdsWs = 2 * kMmBN * kMmRowB;
constexpr int kBfDepth = 3;  // weight chunks a stager's loads run ahead (4: about 2% slower), Q8_0 / Q6_K

template <class S>
__global__ void __launch_bounds__(kMmWsThreads)
    mm_bf16_ws_kernel(const uint8_t* __restrict__ w, int n_rows, int cols, int64_t row_bytes,
                      const u32x4* __restrict__ xt, int m, float* __restrict__ y, int n_tiles_m, int q6s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t wlb[];  // [2][kMmBN * kMmRowB]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  int r0, t0;
  tile_of(n_tiles_m, r0, t0);
  const int nchunks = cols / kMmKC;
  const bool consumer = wave < 4, stager = wave >= 4 && wave < 7;

  // B staging: lane p = tid - 256 < 192 stages row p / 2, piece p % 2
  constexpr int kTasks = kMmBN * S::kPieces;
  static_assert(kTasks == 3 * kWave, "waves 4-6 stage one task a lane");
  const int task = max(tid - 4 * kWave, 0) % kTasks;
  const int srow = task / S::kPieces, piece = task % S::kPieces;
  const uint8_t* wrow = w + int64_t(min(r0 + srow, n_rows - 1)) * row_bytes;
  // K-quant stagers decode the 8 sub-block scales once per super-block into
  // sd / sm and run a ring of 4 aligned to super-blocks, so a chunk's
  // sub-block pair g is known at compile time; the other formats run a
  // ring of kBfDepth
  constexpr bool kSb = SbScales<S>::value;
  constexpr int kRingB = kSb ? 4 : kBfDepth;
  float sd[8], sm[8];
  auto stage = [&](const typename S::Raw& raw, int c, uint8_t* buf, int g) {
    uint32_t run0[8], run1[8];
    int o0, o1;
    if constexpr (kSb)
      S::emit_bf16_sc(raw, c, piece, sd[2 * g], sm[2 * g], sd[2 * g + 1], sm[2 * g + 1], run0, run1, o0, o1);
    else
      Bf16Emit<S>::run(raw, c, piece, block_shift<S>(wrow, c), run0, run1, o0, o1, q6s);
    uint8_t* dst = buf + srow * kMmRowB;
    *reinterpret_cast<u32x4*>(dst + 2 * o0) = u32x4{run0[0], run0[1], run0[2], run0[3]};
    *reinterpret_cast<u32x4*>(dst + 2 * o0 + 16) = u32x4{run0[4], run0[5], run0[6], run0[7]};
    *reinterpret_cast<u32x4*>(dst + 2 * o1) = u32x4{run1[0], run1[1], run1[2], run1[3]};
    *reinterpret_cast<u32x4*>(dst + 2 * o1 + 16) = u32x4{run1[4], run1[5], run1[6], run1[7]};
  };

  // consumer A fragments from the tiled pre-pass (x_bf16_tiled_kernel): lane
  // half h of k-step s holds chunk elements [32 h + 8 s, +8) of token 32 T +
  // l32, T the 32-token tile of M-subtile mi (clamped to the last tile)
  const int n_tt = (m + 31) >> 5;
  const uint8_t* xtile[2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int T = min((t0 + 64 * (wave & 3) + 32 * mi) >> 5, n_tt - 1);
    xtile[mi] = reinterpret_cast<const uint8_t*>(xt) + int64_t(T) * nchunks * 4096 + 16 * lane;
  }
  bf16x8 afr[2][2][4];  // [chunk parity][mi][s]
  auto load_a = [&](int c, bf16x8 (*dst)[4]) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        dst[mi][s] = *reinterpret_cast<const bf16x8*>(xtile[mi] + int64_t(c) * 4096 + 1024 * s);
  };
  f32x16 acc[2][3];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 3; ++ni) acc[mi][ni] = f32x16{};

  typename S::Raw raw[kRingB];
  if (consumer) {
    load_a(0, afr[0]);
    load_a(min(1, nchunks - 1), afr[1]);
  } else if (stager) {
#pragma unroll
    for (int k = 0; k < kRingB; ++k) raw[k] = S::load(wrow, min(k, nchunks - 1), piece);
    if constexpr (kSb) S::sb_scales(raw[0].h, sd, sm);
    stage(raw[0], 0, wlb, 0);
    raw[0] = S::load(wrow, min(kRingB, nchunks - 1), piece);
  }
  lds_barrier();

  // One loop per role, each with one barrier per chunk (the barrier counts
  // match): a loop whose every chunk branched on the role would merge both
  // roles' loads in flight at each join, and the compiler would then wait
  // for all of them before each chunk, undoing the prefetch distances. For
  // the same reason each role's main loop runs whole groups of chunks with
  // no exit inside (a group cut short at the last chunk would reach the loop
  // head with fewer loads in flight, and the head's waits would have to
  // assume that path); the chunks past the last whole group run after it.
  if (consumer) {
    auto consume = [&](int c, bf16x8 (*a)[4]) {
      const uint8_t* wb = wlb + (c & 1) * (kMmBN * kMmRowB);
      const int cnext = min(c + 2, nchunks - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 bfr[3];
#pragma unroll
        for (int ni = 0; ni < 3; ++ni)
          bfr[ni] = *reinterpret_cast<const bf16x8*>(wb + (32 * ni + l32) * kMmRowB + 2 * (32 * half + 8 * s));
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 3; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi][s], bfr[ni], acc[mi][ni], 0, 0, 0);
        // k-step s of chunk c + 2 into the registers this step used (past
        // the end: the last chunk again), spread over the chunk: the four
        // consumers' loads would otherwise reach the CU's memory pipe in one
        // burst at the chunk's end and stall at issue
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          a[mi][s] = *reinterpret_cast<const bf16x8*>(xtile[mi] + int64_t(cnext) * 4096 + 1024 * s);
        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);  // the step's 6 MFMAs,
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // then its 2 loads
      }
      lds_barrier();
    };
    int c0 = 0;
    for (; c0 + 2 <= nchunks; c0 += 2) {
      consume(c0, afr[0]);
      consume(c0 + 1, afr[1]);
    }
    if (c0 < nchunks) consume(c0, afr[0]);
  } else if (stager) {
    for (int c0 = 0; c0 < nchunks; c0 += kRingB) {
#pragma unroll
      for (int j = 0; j < kRingB; ++j) {
        const int c = c0 + j;
        if (c < nchunks) {  // uniform
          // B(c + 1) into the buffer chunk c - 1 used; past the last chunk
          // this re-stages the last one into the buffer nobody reads (for
          // the K-quants with the next super-block's scales: harmless)
          const int slot = (j + 1) % kRingB;
          // K-quants: c0 is a multiple of 4 (cols % 256 == 0), chunk c + 1
          // is pair (j + 1) & 3 of its super-block, and j = 3 starts the next
          if constexpr (kSb)
            if (j == kRingB - 1) S::sb_scales(raw[slot].h, sd, sm);
          stage(raw[slot], min(c + 1, nchunks - 1), wlb + ((c + 1) & 1) * (kMmBN * kMmRowB), (j + 1) & 3);
          raw[slot] = S::load(wrow, min(c + 1 + kRingB, nchunks - 1), piece);
          lds_barrier();
        }
      }
    }
  } else {
    for (int c = 0; c < nchunks; ++c) lds_barrier();
  }

  if (!consumer) return;
  // D layout of the 32x32 MFMA: lane l holds column l % 32 (a weight row)
  // and, in register i, row 8 * (i / 4) + 4 * (l / 32) + i % 4 (a token)
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 3; ++ni) {
      const int r = r0 + 32 * ni + l32;
      if (r >= n_rows) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = t0 + 64 * wave + 32 * mi + 8 * (i >> 2) + 4 * half + (i & 3);
        if (t < m) y[int64_t(t) * n_rows + r] = acc[mi][ni][i];
      }
    }
}

// ------------------------------------------------------- q8 kernel (int8) --
// Activations in Q8 blocks of 32 (scale s_tj = max|x| / 127, int8 codes c),
// weights Q8_0 / Q4_K / Q5_K, whose 32-element blocks carry one scale
// d_rj = d * sc_j (Q4_K / Q5_K also a min dmin * m_j). Per block j:
//   y_tr += d_rj * s_tj * I_trj - dmin_r * m_rj * u_tj,
// I_trj = sum_k q_rk c_tk (exact int32) and u_tj = s_tj * sum_k c_tk.
// Work per (tile of 32 rows x 32 tokens, block):
//   v_mfma_i32_32x32x32_i8      I (A = weight codes, B = activation codes);
//   v_mfma_f32_32x32x1_2b_f32   S = d_rj * s_tj, the outer products of the
//                               rows' and tokens' scales, both blocks of a
//                               64-element chunk in one instruction;
//   VALU                        acc += float(I) * S (a convert and an fma),
// so the per-output scale products run on the matrix pipe (which the int8
// dots leave idle most of the time) and the VALU keeps two instructions per
// output and block. The min term is one v_mfma_f32_32x32x16_bf16 per tile
// and super-block (K = 8 blocks x the high and low bf16 halves of u; the
// 6-bit m exact in bf16), scaled by -dmin_r on the VALU. I, S and the min
// sums share the D layout (lane l: token l % 32, rows 8 (i / 4) + 4 (l / 32)
// + i % 4), so the VALU works register by register.
//
// Workgroup tile 256 tokens x 96 rows, 8 waves: wave w owns tokens
// [32 w, +32) x all 96 rows (3 tiles), two waves per SIMD. A chunk's six
// (row tile, block) steps are software pipelined, across chunks too: step
// k's VALU runs while step k + 1's MFMAs execute and step k + 2's LDS
// operands load. The chunk tiles rotate through three LDS buffers, so the
// one barrier per chunk (before step 4) lets a wave read chunk c + 1 while
// others still finish chunk c. Waves 0-2 also stage: at the start of chunk c
// the codes of chunk c + 1 with d_rj per block, and per super-block
// (double-buffered) the rows' m_j as bf16 and dmin.
constexpr int kMiThreads = 512;
constexpr int kI8Depth = 4;  // chunks per unrolled loop body
constexpr int kI8Ring = 2;   // weight chunks in flight ahead of staging (register slots)
constexpr int kI8Bufs = 3;   // chunk tiles in LDS

template <class S>
__global__ void __launch_bounds__(kMiThreads)
    mm_i8_kernel(const uint8_t* __restrict__ w, int n_rows, int cols, int64_t row_bytes,
                 const int8_t* __restrict__ xq, const float* __restrict__ xs, const u32x4* __restrict__ xu,
                 int m, float* __restrict__ y, int n_tiles_m) {
  typedef float f32x32 __attribute__((ext_vector_type(32)));
  constexpr bool kMin = S::kMin;
  __shared__ __attribute__((aligned(16))) uint8_t wl[kI8Bufs][kMmBN * kMmRowQ];  // [chunk buf] codes
  __shared__ __attribute__((aligned(16))) float wsc[kI8Bufs][2][kMmBN];  // [chunk buf][block][row] d_rj
  __shared__ __attribute__((aligned(16))) u32x4 wm[2][kMmBN][2];                 // [sb buf][row][k half] m, bf16
  __shared__ __attribute__((aligned(16))) float wdm[2][kMmBN];                   // [sb buf][row] dmin
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  int r0, t0;
  tile_of(n_tiles_m, r0, t0);
  const int nchunks = cols / kMmKC;
  const int nblk = cols / 32, nsb = cols >> 8;

  constexpr int kTasks = kMmBN * S::kPieces;
  static_assert(kTasks % kWave == 0 && kTasks <= kMiThreads, "staging tasks fill whole waves");
  const bool stager = tid < kTasks;
  const int srow = stager ? tid / S::kPieces : 0, piece = tid % S::kPieces;
  const uint8_t* wrow = w + int64_t(min(r0 + srow, n_rows - 1)) * row_bytes;

  // the wave's token tile (clamped to the padded tokens; tokens past m are
  // computed on zero codes and not stored): codes of fragment (T, c, s) at
  // 16-byte piece ((T * nch + c) * 2 + s) * 64 + lane, scales of (T, j) at
  // float (T * nblk + j) * 32 + l32, the min operand of (T, sb) at 16-byte
  // piece (T * nsb + sb) * 64 + lane
  const int T = min((t0 >> 5) + wave, ((m + 31) >> 5) - 1);
  const int8_t* xr = xq + int64_t(T) * nchunks * 2048 + 16 * lane;
  const float* sr = xs + int64_t(T) * nblk * 32 + l32;
  const u32x4* ur = xu + int64_t(T) * nsb * 64 + lane;

  f32x16 acc[3];
#pragma unroll
  for (int ni = 0; ni < 3; ++ni) acc[ni] = f32x16{};

  // one piece of chunk c into chunk buffer buf (codes and block scales); a
  // K-quant row's m_j of the chunk's two blocks (and at the super-block's
  // first chunk its dmin) into super-block buffer (c / 4) % 2
  auto stage = [&](const typename S::Raw& raw, int c, int buf) {
    uint32_t run0[4], run1[4];
    int o0, o1, jb0, jb1;
    float dj[2], mj[2];
    S::emit_q8(raw, c, piece, run0, run1, o0, o1, jb0, jb1, dj, mj);
    uint8_t* dst = wl[buf] + srow * kMmRowQ;
    *reinterpret_cast<u32x4*>(dst + o0) = u32x4{run0[0], run0[1], run0[2], run0[3]};
    *reinterpret_cast<u32x4*>(dst + o1) = u32x4{run1[0], run1[1], run1[2], run1[3]};
    // (two pieces of a K-quant row write the same scales of both blocks)
    wsc[buf][jb0][srow] = dj[0];
    wsc[buf][jb1][srow] = dj[1];
    if constexpr (kMin) {
      if (piece == 0) {
        const int g = c & 3, sbuf = (c >> 2) & 1;
        uint32_t scp, mp;
        StQ4K::scale_bytes(raw.h, g, scp, mp);
        // k = 8 (j / 4) + 2 (j % 4) + p for block j of the super-block and
        // half p of u: blocks 2g and 2g + 1 are words 2 (g % 2), +1 of half g / 2
        const uint32_t b0 = __builtin_bit_cast(uint32_t, float(mp & 0xFFu)) >> 16;
        const uint32_t b1 = __builtin_bit_cast(uint32_t, float((mp >> 8) & 0xFFu)) >> 16;
        uint32_t* wd = reinterpret_cast<uint32_t*>(&wm[sbuf][srow][g >> 1]) + 2 * (g & 1);
        *reinterpret_cast<uint2*>(wd) = uint2{b0 | (b0 << 16), b1 | (b1 << 16)};
        if (g == 0) wdm[sbuf][srow] = h2f(raw.h.x >> 16);
      }
    }
  };

  static_assert(kI8Depth % kI8Ring == 0, "ring slots are constants of the unrolled loop");
  typename S::Raw raw[kI8Ring];
#pragma unroll
  for (int k = 0; k < kI8Ring; ++k) raw[k] = S::load(wrow, min(k, nchunks - 1), piece);
  if (stager) stage(raw[0], 0, 0);
  raw[0] = S::load(wrow, min(kI8Ring, nchunks - 1), piece);
  // chunk c's activation fragments and the lane's token scale of block
  // `half` (the B operand of the scale products), loaded a chunk ahead; the
  // min operand a super-block ahead
  i32x4 xc[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) xc[s] = *reinterpret_cast<const i32x4*>(xr + 1024 * s);
  float sxc = sr[32 * half];
  u32x4 uc = kMin ? ur[0] : u32x4{0u, 0u, 0u, 0u};
  lds_barrier();

  // step k of a chunk is (row tile k / 2, block k % 2); its weight
  // fragment, and a row tile's d_rj of block `half` (the A operand of the
  // scale products: lane half h supplies block h of the two-block MFMA)
  auto ld_a = [&](int buf, int k) {
    return *reinterpret_cast<const i32x4*>(wl[buf] + (32 * (k >> 1) + l32) * kMmRowQ + 32 * (k & 1) + 16 * half);
  };
  auto ld_d = [&](int buf, int ni) { return wsc[buf][half][32 * ni + l32]; };

  // The pipeline's products live in ping-pong pairs indexed by constants of
  // the unrolled loops, so that no register copy reads an MFMA result early:
  // step k's int8 sums in Ib[k % 2] (six steps a chunk), row tile g's scale
  // products (both blocks: registers 16 b + i) in Sb[g % 2] (g = 3 c + ni,
  // whose parity repeats every kI8Depth chunks). Entering a chunk: step 0's
  // int8 products and row tile 0's scale products issued, step 1's fragment
  // loaded.
  static_assert(kI8Depth % 4 == 0, "the super-block position repeats every kI8Depth chunks");
  i32x16 Ib[2];
  f32x32 Sb[2];
  i32x4 a_nn = ld_a(0, 1);
  float d_nn = 0.f;
  Ib[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ld_a(0, 0), xc[0], i32x16{}, 0, 0, 0);
  Sb[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(ld_d(0, 0), sxc, f32x32{}, 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);

  for (int c0 = 0; c0 < nchunks; c0 += kI8Depth) {
#pragma unroll
    for (int jj = 0; jj < kI8Depth; ++jj) {
      const int c = c0 + jj;
      if (c < nchunks) {  // uniform
        const bool more = c + 1 < nchunks;
        const int buf = c % kI8Bufs, nbuf = (c + 1) % kI8Bufs;
        {
          const int slot = (jj + 1) % kI8Ring;  // chunk c + 1 (a constant once unrolled)
          if (more && stager) stage(raw[slot], c + 1, nbuf);
          // every wave issues the weight loads (the other waves' lanes read
          // row r0, one cache line a wave): with loads on the stagers' path
          // only, the compiler's counted wait for the activation loads would
          // also wait for these, a whole memory latency each chunk
          raw[slot] = S::load(wrow, min(c + 1 + kI8Ring, nchunks - 1), piece);
        }
        const int cn = more ? c + 1 : c;
        i32x4 xn[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) xn[s] = *reinterpret_cast<const i32x4*>(xr + int64_t(cn) * 2048 + 1024 * s);
        const float sxn = sr[32 * (2 * cn + half)];
        // the super-block's min term runs in its last chunk (c % 4 == jj: c0 is
        // a multiple of kI8Depth)
        const bool min_chunk = kMin && jj % 4 == 3;
        const int sbuf = (c >> 2) & 1;
        const bf16x8 ub = __builtin_bit_cast(bf16x8, uc);
        f32x16 D_min = f32x16{};
#pragma unroll
        for (int k = 0; k < 6; ++k) {
          const int ni = k >> 1, s = k & 1;
          const int tp = (3 * jj + ni) & 1;  // this row tile's scale-product pair
          if (k == 4) lds_barrier();  // chunk c + 1 staged; nobody reads chunk c - 2's buffer any more
          // issue step k + 1's products (past the chunk: chunk c + 1's step 0;
          // after the last chunk they read an unstaged buffer and go unused)
          {
            const i32x4 xb = k < 5 ? xc[(k + 1) & 1] : xn[0];
            Ib[(k + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_nn, xb, i32x16{}, 0, 0, 0);
            if (s == 1)  // the next row tile's scale products
              Sb[tp ^ 1] = __builtin_amdgcn_mfma_f32_32x32x1f32(d_nn, k < 5 ? sxc : sxn, f32x32{}, 0, 0, 0);
          }
          // (LDS reads complete in order: issued before these MFMAs, step k + 2's
          // loads would make the MFMAs' wait for step k + 1's operands wait for them)
          __builtin_amdgcn_sched_barrier(0);
          // load step k + 2's operands (past the chunk: chunk c + 1's)
          {
            const int k2 = k + 2;
            const int b2 = k2 < 6 ? buf : nbuf, kk = k2 < 6 ? k2 : k2 - 6;
            a_nn = ld_a(b2, kk);
            if ((kk & 1) == 0) d_nn = ld_d(b2, kk >> 1);
          }
          if (min_chunk && s == 0) {  // this tile's min sums, used at its block 1 step
            const bf16x8 ma = __builtin_bit_cast(bf16x8, wm[sbuf][32 * ni + l32][half]);
            D_min = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ma, ub, f32x16{}, 0, 0, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          // step k's scaling
          const i32x16& I = Ib[k & 1];
          const f32x32& Sc = Sb[tp];
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[ni][i] = __builtin_fmaf(float(I[i]), Sc[16 * s + i], acc[ni][i]);
          if (min_chunk && s == 1) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 dm = *reinterpret_cast<const f32x4*>(&wdm[sbuf][32 * ni + 8 * q + 4 * half]);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                acc[ni][4 * q + e] = __builtin_fmaf(-dm[e], D_min[4 * q + e], acc[ni][4 * q + e]);
            }
          }
          // step k's sums are formed here: without this the compiler sinks the
          // scaling below later steps' MFMAs and holds all their products
          asm volatile("" : "+v"(acc[ni]));
          __builtin_amdgcn_sched_barrier(0);
        }
        if (min_chunk) uc = ur[64 * min((c >> 2) + 1, nsb - 1)];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          xc[s] = xn[s];
        }
        sxc = sxn;
      }
    }
  }

  // D: lane l holds column l % 32 (a token), register i the weight row
  // 8 * (i / 4) + 4 * (l / 32) + i % 4 -> four runs of 4 consecutive rows
  const int t = t0 + 32 * wave + l32;
  if (t < m) {
#pragma unroll
    for (int ni = 0; ni < 3; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = r0 + 32 * ni + 8 * q + 4 * half;
        float* dst = y + int64_t(t) * n_rows + r;
        if (r + 3 < n_rows && (n_rows & 3) == 0) {
          *reinterpret_cast<f32x4*>(dst) =
              f32x4{acc[ni][4 * q], acc[ni][4 * q + 1], acc[ni][4 * q + 2], acc[ni][4 * q + 3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (r + e < n_rows) dst[e] = acc[ni][4 * q + e];
        }
      }
  }
}

// ------------------------------------------------------- q8 kernel, Q6_K --
// Q6_K weights against the same 32-element Q8 activation blocks. Q6_K
// carries a scale per 16 elements (d * sc_j, values d * sc_j * (q - 32)), so
// each 32-element activation block j covers two weight sub-blocks and
//   y_tr += s_tj * sum_{h = 0, 1} d_r * sc_r,2j+h * I_tr,2j+h,
// I_tr,k = sum over sub-block k of (q - 32) c (exact int32). Per (tile of 32
// rows x 32 tokens, activation block):
//   v_mfma_i32_32x32x16_i8 twice    I of the two sub-blocks (K = 16; the
//                                   block's K = 32 activation fragment is
//                                   split into its two halves with one
//                                   exchange between the wave's lane halves);
//   v_mfma_f32_32x32x1_2b_f32       both sub-blocks' scale products d * sc *
//                                   s_t as the outer products of its two blocks;
//   VALU                            acc += float(I) * S, per sub-block.
// So against the 32-element K-quants it does twice the int8 MFMAs and twice
// the VALU per element. Tile 256 tokens x 96 rows, 8 waves (wave w owns
// tokens [32 w, +32) x all 96 rows); waves 0-2 stage chunk c + 1 (codes
// q - 32 as int8, d * sc per sub-block) while chunk c is computed, with a
// two-chunk ring of weight loads.
constexpr int kM6Threads = 512;

// Four 6-bit codes q (one per byte) -> the bytes q - 32 (int8, -32..31)
// without carries between bytes: q ^ 32 clears bit 5 of q >= 32 (giving
// q - 32) and sets it for q < 32 (giving q + 32, which bits 6 and 7 then
// turn into q - 32 + 256).
__device__ __forceinline__ uint32_t q6_centered(uint32_t q) {
  const uint32_t t = q ^ 0x20202020u, m = t & 0x20202020u;
  return t | (m << 1) | (m << 2);
}

__global__ void __launch_bounds__(kM6Threads)
    mm_i8q6_kernel(const uint8_t* __restrict__ w, int n_rows, int cols, int64_t row_bytes,
                   const int8_t* __restrict__ xq, const float* __restrict__ xs, int m, float* __restrict__ y,
                   int n_tiles_m, int q6s) {
  typedef float f32x32 __attribute__((ext_vector_type(32)));
  __shared__ __attribute__((aligned(16))) uint8_t wl[2][kMmBN * kMmRowQ];  // [chunk buf] codes q - 32
  __shared__ __attribute__((aligned(16))) float wsc[2][4][kMmBN];          // [chunk buf][sub-block][row] d * sc
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  int r0, t0;
  tile_of(n_tiles_m, r0, t0);
  const int nchunks = cols / kMmKC;
  const int nblk = cols / 32;

  constexpr int kTasks = kMmBN * StQ6K::kPieces;
  static_assert(kTasks % kWave == 0 && kTasks <= kM6Threads, "staging tasks fill whole waves");
  const bool stager = tid < kTasks;
  const int srow = stager ? tid / StQ6K::kPieces : 0, piece = tid % StQ6K::kPieces;
  const uint8_t* wrow = w + int64_t(min(r0 + srow, n_rows - 1)) * row_bytes;

  // the wave's token tile, as mm_i8_kernel: fragment (T, c, s) at 16-byte
  // piece ((T * nch + c) * 2 + s) * 64 + lane, scale of (T, j) at float
  // (T * nblk + j) * 32 + l32
  const int T = min((t0 >> 5) + wave, ((m + 31) >> 5) - 1);
  const int8_t* xr = xq + int64_t(T) * nchunks * 2048 + 16 * lane;
  const float* sr = xs + int64_t(T) * nblk * 32 + l32;

  f32x16 acc[3];
#pragma unroll
  for (int ni = 0; ni < 3; ++ni) acc[ni] = f32x16{};

  // piece hb of chunk c: elements [16 hb, +16) (sub-block hb) and
  // [32 + 16 hb, +16) (sub-block 2 + hb) of the row's chunk
  auto stage = [&](const StQ6K::Raw& raw, int c, int buf) {
    uint32_t va[4], vb[4], scw;
    StQ6K::decode(raw, c, block_shift<StQ6K>(wrow, c), va, vb, scw);
    uint8_t* dst = wl[buf] + srow * kMmRowQ;
    *reinterpret_cast<u32x4*>(dst + 16 * piece) =
        u32x4{q6_centered(va[0]), q6_centered(va[1]), q6_centered(va[2]), q6_centered(va[3])};
    *reinterpret_cast<u32x4*>(dst + 32 + 16 * piece) =
        u32x4{q6_centered(vb[0]), q6_centered(vb[1]), q6_centered(vb[2]), q6_centered(vb[3])};
    const uint32_t b0 = (scw >> (8 * piece)) & 0xFFu, b1 = (scw >> (8 * (2 + piece))) & 0xFFu;
    const float d = h2f(raw.d);
    wsc[buf][piece][srow] = d * (q6s ? float(int8_t(b0)) : float(b0));
    wsc[buf][2 + piece][srow] = d * (q6s ? float(int8_t(b1)) : float(b1));
  };

  // a two-chunk ring of weight loads (slots are constants: two chunks per
  // loop body); every wave issues them (other lanes read row r0), as in
  // mm_i8_kernel
  StQ6K::Raw raw[2];
  raw[0] = StQ6K::load(wrow, 0, piece);
  raw[1] = StQ6K::load(wrow, min(1, nchunks - 1), piece);
  if (stager) stage(raw[0], 0, 0);
  raw[0] = StQ6K::load(wrow, min(2, nchunks - 1), piece);
  i32x4 xc[2];
  float sxc[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    xc[s] = *reinterpret_cast<const i32x4*>(xr + 1024 * s);
    sxc[s] = sr[32 * s];
  }
  lds_barrier();

  for (int c0 = 0; c0 < nchunks; c0 += 2) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int c = c0 + jj;
      if (c < nchunks) {  // uniform
        const int buf = c & 1;
        const bool more = c + 1 < nchunks;
        // stage chunk c + 1 (slot (jj + 1) % 2) and refill the slot with c + 3
        if (more && stager) stage(raw[(jj + 1) & 1], c + 1, buf ^ 1);
        raw[(jj + 1) & 1] = StQ6K::load(wrow, min(c + 3, nchunks - 1), piece);
        // chunk c + 1's activations, a chunk ahead
        const int cn = more ? c + 1 : c;
        i32x4 xn[2];
        float sxn[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          xn[s] = *reinterpret_cast<const i32x4*>(xr + int64_t(cn) * 2048 + 1024 * s);
          sxn[s] = sr[32 * (2 * cn + s)];
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          // the block's K = 32 fragment (lane half h: bytes 16 h .. 16 h + 15
          // of the block) -> the K = 16 fragments of its two sub-blocks (lane
          // half h: bytes 8 h .. 8 h + 7 of the sub-block)
          const i32x4 f = xc[s];
          i32x4 pf;
#pragma unroll
          for (int q = 0; q < 4; ++q) pf[q] = __shfl_xor(f[q], 32, kWave);
          const long b_lo = half ? (long(uint32_t(pf[2])) | (long(uint32_t(pf[3])) << 32))
                                 : (long(uint32_t(f[0])) | (long(uint32_t(f[1])) << 32));
          const long b_hi = half ? (long(uint32_t(f[2])) | (long(uint32_t(f[3])) << 32))
                                 : (long(uint32_t(pf[0])) | (long(uint32_t(pf[1])) << 32));
#pragma unroll
          for (int ni = 0; ni < 3; ++ni) {
            const uint8_t* wa = wl[buf] + (32 * ni + l32) * kMmRowQ + 32 * s + 8 * half;
            const i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(*reinterpret_cast<const long*>(wa), b_lo,
                                                                    i32x16{}, 0, 0, 0);
            const i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(*reinterpret_cast<const long*>(wa + 16), b_hi,
                                                                    i32x16{}, 0, 0, 0);
            // A: lane half h supplies sub-block 2 s + h's d * sc of row l32;
            // B: the lane's token scale of block s (both halves)
            const f32x32 Sc = __builtin_amdgcn_mfma_f32_32x32x1f32(wsc[buf][2 * s + half][32 * ni + l32], sxc[s],
                                                                   f32x32{}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              acc[ni][i] = __builtin_fmaf(float(I0[i]), Sc[i], acc[ni][i]);
              acc[ni][i] = __builtin_fmaf(float(I1[i]), Sc[16 + i], acc[ni][i]);
            }
            // the step's sums are formed here: otherwise the compiler holds
            // every step's products at once (hundreds of registers)
            asm volatile("" : "+v"(acc[ni]));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          xc[s] = xn[s];
          sxc[s] = sxn[s];
        }
        lds_barrier();  // chunk c + 1 staged; nobody reads chunk c's buffer any more
      }
    }
  }

  // D layout as mm_i8_kernel's
  const int t = t0 + 32 * wave + l32;
  if (t < m) {
#pragma unroll
    for (int ni = 0; ni < 3; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = r0 + 32 * ni + 8 * q + 4 * half;
        float* dst = y + int64_t(t) * n_rows + r;
        if (r + 3 < n_rows && (n_rows & 3) == 0) {
          *reinterpret_cast<f32x4*>(dst) =
              f32x4{acc[ni][4 * q], acc[ni][4 * q + 1], acc[ni][4 * q + 2], acc[ni][4 * q + 3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (r + e < n_rows) dst[e] = acc[ni][4 * q + e];
        }
      }
  }
}

// ------------------------------------------------------ q8 kernel, K-quants --
// Q4_K / Q5_K weights against activations in 256-element Q8 blocks (one scale
// s_t per token and super-block, codes c, sub-block code sums b_tj). One
// super-block of row r holds values d * sc_j * q_k - dmin * m_j for element k
// of sub-block j; with q_k = z + p_k (z = 0 for Q4_K, 16 for Q5_K, so p fits
// a signed byte) and sc_j = 8 sh_j + sl_j:
//   sum_k value_k * x_k = s_t * (d * (8 H + L + z * sum_j sc_j b_tj)
//                                - dmin * sum_j m_j b_tj)
// H = sum_k sh_j p_k c_k and L = sum_k sl_j p_k c_k run on
// v_mfma_i32_16x16x64_i8 (weight operands sh * p and sl * p, int8; one
// instruction covers a 64-element chunk) with the int32 sums carried
// through the super-block's 4 chunks; the two sums over b_tj are exact
// integers on one v_mfma_f32_16x16x16_f16 each (b = 64 hi + lo, the weight
// side 64 m | m, every value exact in f16); the VALU rescales once per
// super-block and output (5 ops, 6 for Q5_K), not once per 32-element block.
//
// Workgroup tile 256 tokens x 96 rows (as the other prefill kernels), 8
// waves: wave w owns tokens [64 (w % 4), +64) x rows [48 (w / 4), +48), 4 x 3
// output tiles of 16 x 16 (144 accumulator registers, so two waves fit each
// SIMD and cover each other's LDS, load and barrier waits; the f32 sums live
// in LDS, which leaves the registers to the int32 sums and the load ring).
// Waves 0-2 also stage: the codes times both limbs into a double-buffered
// LDS tile, two chunks of weight loads in flight, and per super-block
// (double-buffered) the rows' f16 operands of the sum MFMAs and d, dmin.
constexpr int kMqThreads = 512;

template <class S>
__global__ void __launch_bounds__(kMqThreads)
    mm_q8k_kernel(const uint8_t* __restrict__ w, int n_rows, int cols, int64_t row_bytes,
                  const int8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ xb,
                  int m, float* __restrict__ y, int n_tiles_m) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  constexpr bool kZ = S::kCenter != 0;
  constexpr int kA = kZ ? 32 : 16;  // f16 per row and super-block: 64 m | m (| 1024 sc | 16 sc)
  __shared__ __attribute__((aligned(16))) uint8_t wl[2][2][kMmBN * kMmRowQ];  // [buf][sh * p | sl * p]
  __shared__ __attribute__((aligned(16))) _Float16 ma[2][kMmBN * kA];         // [super-block buf]
  __shared__ __attribute__((aligned(16))) float dsc[2][2][kMmBN];             // [super-block buf][d | dmin]
  // the f32 sums, touched once per super-block by the lane that owns them
  // (in LDS, the registers carry the int32 sums and a deeper load ring)
  __shared__ f32x4 accl[kMqThreads / kWave][12][kWave];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int tg = wave & 3, rg = wave >> 2;
  int r0, t0;
  tile_of(n_tiles_m, r0, t0);
  const int nchunks = cols / kMmKC;
  const int nsb = cols >> 8;

  constexpr int kTasks = kMmBN * S::kPieces;
  static_assert(kTasks % kWave == 0 && kTasks <= kMqThreads, "staging tasks fill whole waves");
  const bool stager = tid < kTasks;
  const int srow = stager ? tid / S::kPieces : 0, piece = tid % S::kPieces;
  const uint8_t* wrow = w + int64_t(min(r0 + srow, n_rows - 1)) * row_bytes;

  // the wave's 4 token tiles of 16 (clamped to the padded tokens; rows past m
  // are computed on zero codes and not stored): wave-uniform bases, so the
  // loads take a scalar base and the lane's 32-bit offset
  const int n_t16 = ((m + 31) >> 5) * 2;
  const int8_t* xr[4];
  const float* sr[4];
  const uint8_t* br[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int T = min((t0 + 64 * tg + 16 * mt) >> 4, n_t16 - 1);
    xr[mt] = xq + int64_t(T) * nchunks * 1024;
    sr[mt] = xs + int64_t(T) * nsb * 16;
    br[mt] = xb + int64_t(T) * nsb * 512;
  }
  const uint32_t xo = 16u * uint32_t(lane), so = uint32_t(l16), bo = 8u * uint32_t(lane);

  i32x4 ah[4][3], al[4][3];
  f32x4(&acc)[12][kWave] = accl[wave];
#pragma unroll
  for (int k = 0; k < 12; ++k) acc[k][lane] = f32x4{0.f, 0.f, 0.f, 0.f};

  // one piece of chunk c: its codes times both limbs into LDS buffer buf
  auto stage = [&](const typename S::Raw& raw, int c, int buf) {
    uint32_t h0[4], l0[4], h1[4], l1[4];
    S::emit_q8k(raw, c, h0, l0, h1, l1);
    const int o0 = srow * kMmRowQ + 16 * piece, o1 = o0 + 32;
    *reinterpret_cast<u32x4*>(wl[buf][0] + o0) = u32x4{h0[0], h0[1], h0[2], h0[3]};
    *reinterpret_cast<u32x4*>(wl[buf][1] + o0) = u32x4{l0[0], l0[1], l0[2], l0[3]};
    *reinterpret_cast<u32x4*>(wl[buf][0] + o1) = u32x4{h1[0], h1[1], h1[2], h1[3]};
    *reinterpret_cast<u32x4*>(wl[buf][1] + o1) = u32x4{l1[0], l1[1], l1[2], l1[3]};
  };
  // the row's super-block operands (piece 0 of the super-block's first chunk)
  auto header = [&](const typename S::Raw& raw, int sbuf) {
    uint32_t sc03, sc47, m03, m47;
    StQ4K::all_scale_bytes(raw.h, sc03, sc47, m03, m47);
    _Float16* dst = ma[sbuf] + srow * kA;
    f16x8 a0, a1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float mj = float(((j < 4 ? m03 : m47) >> (8 * (j & 3))) & 0xFFu);
      a0[j] = _Float16(64.f * mj);
      a1[j] = _Float16(mj);
    }
    *reinterpret_cast<f16x8*>(dst) = a0;
    *reinterpret_cast<f16x8*>(dst + 8) = a1;
    if constexpr (kZ) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sj = float(S::kCenter) * float(((j < 4 ? sc03 : sc47) >> (8 * (j & 3))) & 0xFFu);
        a0[j] = _Float16(64.f * sj);
        a1[j] = _Float16(sj);
      }
      *reinterpret_cast<f16x8*>(dst + 16) = a0;
      *reinterpret_cast<f16x8*>(dst + 24) = a1;
    }
    dsc[sbuf][0][srow] = h2f(raw.h.x);
    dsc[sbuf][1][srow] = h2f(raw.h.x >> 16);
  };

  constexpr int kRing = 2;  // weight chunks in flight ahead of staging
  static_assert(4 % kRing == 0, "ring slots are constants of the unrolled super-block loop");
  // Every wave issues the weight loads (the other waves' lanes read row r0,
  // one cache line a wave): with loads on one path only, the compiler's
  // wait for the next chunk's activation fragments would also wait for
  // these, a whole memory latency each chunk.
  typename S::Raw raw[kRing];
#pragma unroll
  for (int k = 0; k < kRing; ++k) raw[k] = S::load(wrow, min(k, nchunks - 1), piece);
  if (stager) {
    stage(raw[0], 0, 0);
    if (piece == 0) header(raw[0], 0);
  }
  // activation fragments, then the next weight loads: the order of the
  // chunk loop, so its waits count the same loads on entry as around it
  i32x4 xc[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) xc[mt] = *reinterpret_cast<const i32x4*>(xr[mt] + xo);
  raw[0] = S::load(wrow, min(kRing, nchunks - 1), piece);
  lds_barrier();

  for (int sb = 0; sb < nsb; ++sb) {
    const int sbuf = sb & 1;
    float sx[4];
    f16x4 bs[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {  // chunks of the super-block
      const int c = 4 * sb + cc;
      const bool more = c + 1 < nchunks;  // uniform
      const uint8_t* wh = wl[cc & 1][0];
      const uint8_t* wo = wl[cc & 1][1];
      i32x4 a_h[3], a_l[3];
#pragma unroll
      for (int nt = 0; nt < 3; ++nt) {
        const int ro = (48 * rg + 16 * nt + l16) * kMmRowQ + 16 * g;
        a_h[nt] = *reinterpret_cast<const i32x4*>(wh + ro);
        a_l[nt] = *reinterpret_cast<const i32x4*>(wo + ro);
      }
      // token tile mt's six MFMAs, then its fragments of the next chunk (past
      // the end: the last chunk again) into the registers they read: the
      // eight waves' loads spread over the chunk instead of reaching the
      // CU's memory pipe in one burst after all the MFMAs
      const int cx = min(c + 1, nchunks - 1);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 3; ++nt) {
          // a new super-block: the int32 sums start at zero
          ah[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_h[nt], xc[mt],
                                                             cc == 0 ? i32x4{0, 0, 0, 0} : ah[mt][nt], 0, 0, 0);
          al[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_l[nt], xc[mt],
                                                             cc == 0 ? i32x4{0, 0, 0, 0} : al[mt][nt], 0, 0, 0);
        }
        xc[mt] = *reinterpret_cast<const i32x4*>(xr[mt] + int64_t(cx) * 1024 + xo);
        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      if (more) {
        const int slot = (cc + 1) % kRing;  // where chunk c + 1 was loaded (c % 4 == cc)
        if (stager) {
          stage(raw[slot], c + 1, (cc + 1) & 1);
          if (cc == 3 && piece == 0) header(raw[slot], sbuf ^ 1);
        }
        raw[slot] = S::load(wrow, min(c + 1 + kRing, nchunks - 1), piece);
      }
      if (cc == 2) {
        // the tokens' scales and sums of this super-block, a chunk before the
        // rescale needs them (not held through the whole super-block)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          sx[mt] = (sr[mt] + 16 * sb)[so];
          bs[mt] = *reinterpret_cast<const f16x4*>(br[mt] + 512 * sb + bo);
        }
      }
      if (cc == 3) {
        // rescale: acc += s_t * (d * (8 H + L [+ z sc.b]) - dmin * m.b)
#pragma unroll
        for (int nt = 0; nt < 3; ++nt) {
          const int row = 48 * rg + 16 * nt;
          const _Float16* mrow = ma[sbuf] + (row + l16) * kA;
          const f16x4 am = *reinterpret_cast<const f16x4*>(mrow + 4 * g);
          f16x4 az;
          if constexpr (kZ) az = *reinterpret_cast<const f16x4*>(mrow + 16 + 4 * g);
          const f32x4 dv = *reinterpret_cast<const f32x4*>(&dsc[sbuf][0][row + 4 * g]);
          const f32x4 mv = *reinterpret_cast<const f32x4*>(&dsc[sbuf][1][row + 4 * g]);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            const f32x4 mb = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bs[mt], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            f32x4 zb = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (kZ) zb = __builtin_amdgcn_mfma_f32_16x16x16f16(az, bs[mt], zb, 0, 0, 0);
            f32x4 av = acc[3 * mt + nt][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float f = float((ah[mt][nt][i] << 3) + al[mt][nt][i]);
              if constexpr (kZ) f += zb[i];
              const float t = __builtin_fmaf(f, dv[i], -(mb[i] * mv[i]));
              av[i] = __builtin_fmaf(t, sx[mt], av[i]);
            }
            acc[3 * mt + nt][lane] = av;
          }
        }
      }
      lds_barrier();
    }
  }

  // D of a 16 x 16 tile: lane l holds column l % 16 (a token) and rows
  // 4 (l / 16) .. + 3
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int t = t0 + 64 * tg + 16 * mt + l16;
    if (t >= m) continue;
#pragma unroll
    for (int nt = 0; nt < 3; ++nt) {
      const int r = r0 + 48 * rg + 16 * nt + 4 * g;
      float* dst = y + int64_t(t) * n_rows + r;
      const f32x4 av = acc[3 * mt + nt][lane];
      if (r + 3 < n_rows && (n_rows & 3) == 0) {
        *reinterpret_cast<f32x4*>(dst) = av;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (r + e < n_rows) dst[e] = av[e];
      }
    }
  }
}

// -------------------------------------------------------------------- host --
static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Modes: 0 bf16; 1 q8 (activations in 32-element Q8 blocks, every int8
// format); 2 q8k (activations in 256-element blocks, one scale per weight
// super-block: Q4_K / Q5_K only; a coarser rounding than mode 1, kept as an
// opt-in alternative).
bool matmul_shape_ok(uint32_t quant, int64_t rows, int64_t cols, int64_t m, uint32_t mode) {
  if (!device_quant(quant) || rows <= 0 || cols <= 0 || m <= 0) return false;
  if (cols % kMmKC != 0 || cols % geometry(quant).block != 0) return false;
  if (rows > (int64_t(1) << 31) - 1 || cols > (int64_t(1) << 30) || m > (int64_t(1) << 24)) return false;
  if (mode == 2 && quant != kQ4_K && quant != kQ5_K) return false;
  if (mode > 2) return false;
  const int64_t tiles = ((rows + kMmBN - 1) / kMmBN) * ((m + kMmBM - 1) / kMmBM);
  return tiles <= (int64_t(1) << 31) - 1;
}

// Workspace carve-up of the 32-element int8 path: codes, scales (f32 per
// block), min-term operands (bf16 halves per block, whole super-blocks).
struct Q8Ws {
  int8_t* codes;
  float* scales;
  uint32_t* u;
  size_t bytes;
};
static Q8Ws q8_ws(uint8_t* ws, int64_t cols, int64_t m) {
  const size_t mp = size_t((m + 31) / 32 * 32);  // tokens padded to whole 32-token tiles
  const size_t nblk = size_t(cols / 32), nsb = (nblk + 7) / 8;
  Q8Ws r;
  const size_t o1 = align256(mp * size_t(cols)), o2 = o1 + align256(mp * nblk * sizeof(float));
  r.codes = reinterpret_cast<int8_t*>(ws);
  r.scales = reinterpret_cast<float*>(ws + o1);
  r.u = reinterpret_cast<uint32_t*>(ws + o2);
  r.bytes = o2 + align256(mp * nsb * 32);
  return r;
}

// Workspace carve-up of the 256-element int8 path: codes, scales, sums.
struct Q8kWs {
  uint8_t* codes;
  float* scales;
  uint8_t* sums;
  size_t bytes;
};
static Q8kWs q8k_ws(uint8_t* ws, int64_t cols, int64_t m) {
  const size_t mp = size_t((m + 31) / 32 * 32);
  const size_t nsb = size_t(cols / 256);
  Q8kWs r;
  const size_t o1 = align256(mp * size_t(cols)), o2 = o1 + align256(mp * nsb * sizeof(float));
  r.codes = ws;
  r.scales = reinterpret_cast<float*>(ws + o1);
  r.sums = ws + o2;
  r.bytes = o2 + align256(mp * nsb * 32);  // 512 bytes per 16 tokens and super-block
  return r;
}

size_t matmul_workspace_bytes(int64_t cols, int64_t m, uint32_t mode) {
  if (mode == 0) return align256(size_t((m + 31) / 32 * 32) * size_t(cols) * 2);  // whole 32-token tiles
  if (mode == 2) return q8k_ws(nullptr, cols, m).bytes;
  return q8_ws(nullptr, cols, m).bytes;
}

template <class S>
static void launch_mm(uint32_t mode, const uint8_t* w, int rows, int cols, int64_t rb, uint8_t* ws, int m,
                      float* y, int q6s, hipStream_t s) {
  const int ntm = (m + kMmBM - 1) / kMmBM, ntn = (rows + kMmBN - 1) / kMmBN;
  const dim3 grid(unsigned(ntm * ntn));
  if (mode == 0) {
    hipLaunchKernelGGL(mm_bf16_ws_kernel<S>, grid, dim3(kMmWsThreads), kMmLdsWs, s, w, rows, cols, rb,
                       reinterpret_cast<const u32x4*>(ws), m, y, ntm, q6s);
  } else if constexpr (std::is_same<S, StQ6K>::value) {
    if (mode == 1) {  // 16-element scales: the Q6_K int8 kernel
      const Q8Ws q = q8_ws(ws, cols, m);
      hipLaunchKernelGGL(mm_i8q6_kernel, grid, dim3(kM6Threads), 0, s, w, rows, cols, rb, q.codes, q.scales, m, y,
                         ntm, q6s);
    }
  } else if constexpr (S::kQ8) {
    if (mode == 2) {
      if constexpr (S::kQ8K) {
        const Q8kWs q = q8k_ws(ws, cols, m);
        hipLaunchKernelGGL(mm_q8k_kernel<S>, grid, dim3(kMqThreads), 0, s, w, rows, cols, rb,
                           reinterpret_cast<const int8_t*>(q.codes), q.scales, q.sums, m, y, ntm);
      }
    } else {
      const Q8Ws q = q8_ws(ws, cols, m);
      hipLaunchKernelGGL(mm_i8_kernel<S>, grid, dim3(kMiThreads), 0, s, w, rows, cols, rb, q.codes, q.scales,
                         reinterpret_cast<const u32x4*>(q.u), m, y, ntm);
    }
  }
}

hipError_t launch_quantize_q8(const float* x, int64_t n, int8_t* q, float* scales, float* usum,
                              hipStream_t s) {
  if (n <= 0 || n % 32 != 0) return hipErrorInvalidValue;
  const int64_t blocks = n / 32;
  hipLaunchKernelGGL(x_q8_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, s, x, q, scales,
                     usum, blocks);
  return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float* x, int64_t n, int8_t* q, float* scales, int32_t* sums,
                               hipStream_t s) {
  if (n <= 0 || n % 256 != 0) return hipErrorInvalidValue;
  const int64_t supers = n / 256;  // a wave each
  hipLaunchKernelGGL(x_q8k_kernel, dim3(unsigned((supers + 3) / 4)), dim3(256), 0, s, x,
                     reinterpret_cast<uint32_t*>(q), scales, sums, supers);
  return hipGetLastError();
}

hipError_t launch_matmul(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                         int64_t m, float* y, uint32_t mode, void* workspace, int q6_signed,
                         hipStream_t s) {
  if (!matmul_shape_ok(quant, rows, cols, m, mode)) return hipErrorInvalidValue;
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int64_t rb = byte_size(quant, cols);
  if (mode == 0) {
    const int64_t pieces = (m + 31) / 32 * 32 * cols / 8;  // 16-byte pieces of whole 32-token tiles
    hipLaunchKernelGGL(x_bf16_tiled_kernel, dim3(unsigned((pieces + 255) / 256)), dim3(256), 0, s, x,
                       reinterpret_cast<u32x4*>(ws), int(m), int(cols), pieces);
  } else if (mode == 2) {
    const Q8kWs q = q8k_ws(ws, cols, m);
    const int64_t waves = (m + 31) / 32 * 32 * (cols / 256);  // one per (padded token, super-block)
    hipLaunchKernelGGL(x_q8k_tiled_kernel, dim3(unsigned((waves + 3) / 4)), dim3(256), 0, s, x, q.codes,
                       q.scales, q.sums, int(m), int(cols), waves);
  } else {
    const Q8Ws q = q8_ws(ws, cols, m);
    const int64_t blocks = (m + 31) / 32 * 32 * (cols / 32);
    hipLaunchKernelGGL(x_q8_tiled_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, s, x,
                       reinterpret_cast<u32x4*>(q.codes), q.scales, q.u, int(m), int(cols), blocks);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (quant) {
    case kQ4_K: launch_mm<StQ4K>(mode, w, int(rows), int(cols), rb, ws, int(m), y, q6_signed, s); break;
    case kQ5_K: launch_mm<StQ5K>(mode, w, int(rows), int(cols), rb, ws, int(m), y, q6_signed, s); break;
    case kQ8_0: launch_mm<StQ8>(mode, w, int(rows), int(cols), rb, ws, int(m), y, q6_signed, s); break;
    case kQ6_K: launch_mm<StQ6K>(mode, w, int(rows), int(cols), rb, ws, int(m), y, q6_signed, s); break;
    case kIQ4_XS:  // the reading (reference or ggml qs bytes) is a template argument
      if (q6_signed) launch_mm<StIQ4XS<true>>(mode, w, int(rows), int(cols), rb, ws, int(m), y, 0, s);
      else launch_mm<StIQ4XS<false>>(mode, w, int(rows), int(cols), rb, ws, int(m), y, 0, s);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sh
