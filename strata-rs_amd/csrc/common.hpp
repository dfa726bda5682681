// Shared definitions for the CDNA4 (gfx950) quantized-weight kernels.
//
// Block layouts read directly from HBM, exactly as GGUF stores them
// (crates/strata-gguf/src/quant.rs:125-164):
//   Q8_0  32 elements /  34 B: [d: f16][q: i8 x 32]
//   Q4_K 256 elements / 144 B: [d: f16][dmin: f16][scales: 12 B][qs: 128 B]
//   Q5_K 256 elements / 176 B: [d: f16][dmin: f16][scales: 12 B][qh: 32 B][qs: 128 B]
//   Q6_K 256 elements / 210 B: [ql: 128 B][qh: 64 B][sc: 16 B][d: f16]
//   IQ4_XS 256 elements / 136 B: [d: f16][scales_h: u16][scales_l: 4 B][qs: 128 B]
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sh {

enum QuantId : uint32_t {
  kF32 = 0,
  kF16 = 1,
  kQ8_0 = 8,
  kQ4_K = 12,
  kQ5_K = 13,
  kQ6_K = 14,
  kIQ4_XS = 23,
  kBF16 = 30,
};

struct Geometry {
  int64_t block;  // elements per block
  int64_t bytes;  // bytes per block
};

// quant.rs:125-164 for the ids this path accepts; {0, 0} otherwise.
inline Geometry geometry(uint32_t q) {
  switch (q) {
    case kF32: return {1, 4};
    case kF16: return {1, 2};
    case kBF16: return {1, 2};
    case kQ8_0: return {32, 34};
    case kQ4_K: return {256, 144};
    case kQ5_K: return {256, 176};
    case kQ6_K: return {256, 210};
    case kIQ4_XS: return {256, 136};
    default: return {0, 0};
  }
}

// quant.rs:173-181: ceil(n / block) * bytes.
inline int64_t byte_size(uint32_t q, int64_t n) {
  Geometry g = geometry(q);
  if (g.block == 0 || n < 0) return -1;
  return (n + g.block - 1) / g.block * g.bytes;
}

// The quantized types every kernel family takes (matvec, expert, MoE, matmul).
inline bool device_quant(uint32_t q) {
  return q == kQ8_0 || q == kQ4_K || q == kQ5_K || q == kQ6_K || q == kIQ4_XS;
}
// Plain-float element types: matvec (f64 sums) and dequant only.
inline bool plain_quant(uint32_t q) { return q == kF32 || q == kF16 || q == kBF16; }
// Types the matvec (and dequant) kernels take: the quantized ones.
inline bool gemv_quant(uint32_t q) { return device_quant(q); }

// The IQ4_NL / IQ4_XS code book: 4-bit index -> int8 value (a format
// table: ggml's kvalues_iq4nl, crates/strata-gguf/src/tables.rs:2052-2054),
// packed little-endian four to a word.
constexpr uint32_t kIq4Tab[4] = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};

// Four nibble indices (one per byte) -> the four int8 code-book values.
__device__ __forceinline__ uint32_t iq4_lut(uint32_t idx) {
  const uint32_t i7 = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIq4Tab[1], kIq4Tab[0], i7);
  const uint32_t hi = __builtin_amdgcn_perm(kIq4Tab[3], kIq4Tab[2], i7);
  const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}

// IQ4_XS super-block header (bytes 0..7: d f16, scales_h u16, scales_l[4]):
// the 6-bit scale of sub-block ib is the nibble ib % 2 of scales_l[ib / 2]
// and bits 2 ib, 2 ib + 1 of scales_h (dequant.rs:189-206); h0 holds bytes
// 0..3, h1 bytes 4..7. Returns ls - 32.
__device__ __forceinline__ float iq4xs_scale(uint32_t h0, uint32_t h1, int ib) {
  const uint32_t lo = (h1 >> (4 * ib)) & 0x0Fu;  // nibble ib % 2 of byte ib / 2 = nibble ib of h1
  const uint32_t hi = (h0 >> (16 + 2 * ib)) & 3u;
  return float(lo | (hi << 4)) - 32.f;
}

constexpr int kWave = 64;

// bf16::from_f32(v).to_f32() (crates/strata-core/src/hyper.rs:22-24): round
// to nearest even with v_cvt_pk_bf16_f32 (a NaN stays a NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf16_rne(float v) {
  const bf16x2_t b = __builtin_convertvector((f32x2_t){v, 0.f}, bf16x2_t);
  return __builtin_bit_cast(float, uint32_t(__builtin_bit_cast(uint32_t, b) & 0xFFFFu) << 16);
}

// A 16-byte vector that only promises 4-byte alignment: GGUF blocks of 34 and
// 210 bytes start at 2-byte boundaries, so every wide load below goes through
// a dword-aligned address and a realignment.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// The same 16 bytes from an address known only to be 4-byte aligned (safe
// for LDS as well as global memory).
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ u32x4 ld16u(const uint8_t* p) {
  const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
  return u32x4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// Non-temporal 16-byte weight load: the packed weights are streamed exactly
// once per launch, so they should not displace x or the partial sums in L2.
__device__ __forceinline__ u32x4 ld16_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ uint32_t ld4_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// s_waitcnt vmcnt(N) (vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left at
// their maxima), with the scheduler kept from moving memory operations across.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  __builtin_amdgcn_sched_barrier(0);
}

// vmcnt(n) for a wave-uniform n: at most n of this wave's vector memory
// operations (loads, and global_load_lds copies, which complete in order)
// remain outstanding. n above 15 waits for 15 (stricter).
__device__ __forceinline__ void wait_vmem(int n) {
  switch (n) {
    case 0: wait_vmem<0>(); break;
    case 1: wait_vmem<1>(); break;
    case 2: wait_vmem<2>(); break;
    case 3: wait_vmem<3>(); break;
    case 4: wait_vmem<4>(); break;
    case 5: wait_vmem<5>(); break;
    case 6: wait_vmem<6>(); break;
    case 7: wait_vmem<7>(); break;
    case 8: wait_vmem<8>(); break;
    case 9: wait_vmem<9>(); break;
    case 10: wait_vmem<10>(); break;
    case 11: wait_vmem<11>(); break;
    case 12: wait_vmem<12>(); break;
    case 13: wait_vmem<13>(); break;
    case 14: wait_vmem<14>(); break;
    default: wait_vmem<15>();
  }
}

// Workgroup barrier after this wave's LDS writes have completed, without
// waiting for outstanding global loads or global_load_lds copies (which
// __syncthreads() drains): for pipelines that keep copies in flight across
// barriers and wait for them with wait_vmem().
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15 << 0) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// 16 bytes a lane from global `src` (per lane) to LDS at `dst` + 16 * lane,
// `dst` wave-uniform, without passing through registers (global_load_lds).
__device__ __forceinline__ void copy16_to_lds(const uint8_t* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// 4 int32 values -> bytes 0, 1 and 2 of each, packed v0..v3 low to high
// (p0 the byte-0s, p1 the byte-1s, p2 the byte-2s; one v_perm each)
__device__ __forceinline__ void transpose_bytes(uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                                uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  const uint32_t t01 = __builtin_amdgcn_perm(v1, v0, 0x05010400u);  // v0b0 v1b0 v0b1 v1b1
  const uint32_t t23 = __builtin_amdgcn_perm(v3, v2, 0x05010400u);
  const uint32_t u01 = __builtin_amdgcn_perm(v1, v0, 0x07030602u);  // v0b2 v1b2 v0b3 v1b3
  const uint32_t u23 = __builtin_amdgcn_perm(v3, v2, 0x07030602u);
  p0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u);  // byte 0 of v0..v3
  p1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u);  // byte 1
  p2 = __builtin_amdgcn_perm(u23, u01, 0x05040100u);  // byte 2
}

// Lane exchanges inside a quad of lanes as DPP moves (VALU, no LDS round
// trip): the value of lane i ^ 1, and of lane i ^ 2.
__device__ __forceinline__ uint32_t dpp_xor1(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ uint32_t dpp_xor2(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ float dpp_xor1(float v) { return __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(uint32_t, v))); }
__device__ __forceinline__ float dpp_xor2(float v) { return __builtin_bit_cast(float, dpp_xor2(__builtin_bit_cast(uint32_t, v))); }

// bytes [shift, shift + 4) of the 8-byte little-endian pair (lo, hi).
__device__ __forceinline__ uint32_t realign(uint32_t lo, uint32_t hi, uint32_t shift_bytes) {
  return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

// Q6_K 6-bit codes, four to a word, from a lane's ql and qh words loaded
// from the 4-byte boundary `s` (0..3) bytes below its bytes: va takes the
// low nibbles of the ql bytes (high nibbles when `tp`) of words la0:la1
// under bits 4-5 from bit pair 0 of the qh bytes (pair 2 when `tp`); vb
// the same of lb0:lb1 with pair 1 (3). The byte realignment and the nibble
// shift are one funnel shift (v_alignbit), and the pair moves to bits 4-5
// by one shift of lane-dependent width: 3 instructions fewer per pair of
// words than realigning, shifting and selecting.
__device__ __forceinline__ void q6_code_words(uint32_t la0, uint32_t la1, uint32_t lb0, uint32_t lb1, uint32_t h0,
                                              uint32_t h1, uint32_t s, uint32_t tp, uint32_t& va, uint32_t& vb) {
  const uint32_t qs = __builtin_amdgcn_alignbyte(h1, h0, s) << (4u - 4u * tp);
  const uint32_t sh = 8u * s + 4u * tp;
  va = (__builtin_amdgcn_alignbit(la1, la0, sh) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
  vb = (__builtin_amdgcn_alignbit(lb1, lb0, sh) & 0x0F0F0F0Fu) | ((qs >> 2) & 0x30303030u);
}

// IEEE binary16 bits -> f32 through the hardware conversion (exact, f16
// denormals preserved under the default FP16 denorm mode).
__device__ __forceinline__ float h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16 & 0xFFFFu));
  return static_cast<float>(h);
}

// Byte k of w as an exact float (v_cvt_f32_ubyte{0..3}).
template <int K>
__device__ __forceinline__ float ubyte(uint32_t w) {
  return static_cast<float>((w >> (8 * K)) & 0xFFu);
}

// Q5_K codes of group g (dequant.rs:285-297): four code bytes q and the
// four qh bytes of the same element positions l (l = element % 32); the low
// nibbles (sub-block 2g) take bit 2g of qh[l] as 16, the high nibbles
// (sub-block 2g + 1) bit 2g + 1, so codes run 0..31.
__device__ __forceinline__ void q5k_codes(uint32_t q, uint32_t qh, uint32_t g, uint32_t& lo, uint32_t& hi) {
  const uint32_t t = qh >> (2u * g);  // bit 2g of byte j at bit 8j, bit 2g+1 at 8j+1
  lo = (q & 0x0F0F0F0Fu) | ((t << 4) & 0x10101010u);
  hi = ((q >> 4) & 0x0F0F0F0Fu) | ((t << 3) & 0x10101010u);
}

// Q4_K / Q5_K (scale, min) of sub-blocks 2g and 2g+1 in the two low bytes of
// scp / mp, from the 12 packed bytes in words h.y, h.z, h.w of the header
// (get_scale_min_k4, dequant.rs:237-245).
__device__ __forceinline__ void k4_pair(u32x4 h, int g, uint32_t& scp, uint32_t& mp) {
  const uint32_t sh = (g & 1) << 4;
  const uint32_t t1 = h.y >> sh, t2 = h.z >> sh, t3 = h.w >> sh;
  scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
  mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
}

// Sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace sh
