// Bit-exact device dequantization: packed GGUF rows -> f32.
//
// Follows crates/strata-gguf/src/dequant.rs:123-128 (Q8_0), :189-206
// (IQ4_XS), :208-234 (Q6_K), :237-270 (Q4_K) and :272-302 (Q5_K) element for
// element, with the same rounding: every
// product and difference is a separate f32 operation (contraction is off for
// this file's arithmetic), f16 scales widen exactly.
//
// One thread per output element; the block header bytes it needs are re-read
// through L1. This kernel exists to pin the block layouts on the device; the
// matvec kernels never materialise dequantized weights.
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

__device__ __forceinline__ uint32_t rd16(const uint8_t* b) { return b[0] | (uint32_t(b[1]) << 8); }

__device__ __forceinline__ float dq_q8_0(const uint8_t* blk, int j) {
#pragma clang fp contract(off)
  float d = h2f(rd16(blk));
  return static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d;
}

// get_scale_min_k4 (dequant.rs:237-245) for sub-block j of the 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = (q[j + 4] & 0x0Fu) | ((uint32_t(q[j - 4]) >> 6) << 4);
    m = (uint32_t(q[j + 4]) >> 4) | ((uint32_t(q[j]) >> 6) << 4);
  }
}

__device__ __forceinline__ float dq_q4_k(const uint8_t* blk, int j) {
#pragma clang fp contract(off)
  float d = h2f(rd16(blk));
  float mn = h2f(rd16(blk + 2));
  int grp = j >> 6, k = j & 63;
  int sub = 2 * grp + (k >> 5);
  uint32_t sc, m;
  scale_min_k4(sub, blk + 4, sc, m);
  float d1 = d * static_cast<float>(sc);
  float m1 = mn * static_cast<float>(m);
  uint32_t byte = blk[16 + 32 * grp + (k & 31)];
  uint32_t q = (k < 32) ? (byte & 0x0Fu) : (byte >> 4);
  float p = d1 * static_cast<float>(q);
  return p - m1;
}

// Q5_K element j: Q4_K's nibble plus 16 when bit `sub` of qh[j % 32] is set
// (sub-block sub = j / 32 reads bit sub: 2*grp for the low nibbles, 2*grp + 1
// for the high ones, dequant.rs:285-297). q + 16 is exact; then one product
// and one difference, each rounded.
__device__ __forceinline__ float dq_q5_k(const uint8_t* blk, int j) {
#pragma clang fp contract(off)
  float d = h2f(rd16(blk));
  float mn = h2f(rd16(blk + 2));
  int grp = j >> 6, k = j & 63;
  int sub = 2 * grp + (k >> 5);
  uint32_t sc, m;
  scale_min_k4(sub, blk + 4, sc, m);
  float d1 = d * static_cast<float>(sc);
  float m1 = mn * static_cast<float>(m);
  uint32_t byte = blk[48 + 32 * grp + (k & 31)];
  uint32_t q = (k < 32) ? (byte & 0x0Fu) : (byte >> 4);
  uint32_t h = (uint32_t(blk[16 + (k & 31)]) >> sub) & 1u;
  float p = d1 * static_cast<float>(q + 16u * h);
  return p - m1;
}

// Q6_K element j: half h, quarter t, lane l of dequant.rs:217-229.
__device__ __forceinline__ float dq_q6_k(const uint8_t* blk, int j, int signed_scales) {
#pragma clang fp contract(off)
  int h = j >> 7, r = j & 127, t = r >> 5, l = r & 31;
  uint32_t qlb = blk[64 * h + l + 32 * (t & 1)];
  uint32_t low = (t < 2) ? (qlb & 0x0Fu) : (qlb >> 4);
  uint32_t high = (uint32_t(blk[128 + 32 * h + l]) >> (2 * t)) & 3u;
  int q = int(low | (high << 4)) - 32;
  uint8_t raw = blk[192 + 8 * h + (l >> 4) + 2 * t];
  float sc = signed_scales ? static_cast<float>(static_cast<int8_t>(raw)) : static_cast<float>(raw);
  float d = h2f(rd16(blk + 208));
  float a = d * sc;
  return a * static_cast<float>(q);
}

// IQ4_XS element j (dequant.rs:189-206): sub-block ib = j / 32 has the 6-bit
// scale ls from scales_l (nibble ib % 2 of byte ib / 2) and scales_h (bits
// 2 ib, 2 ib + 1), dl = d * (ls - 32) (the difference exact, one rounding
// for the product), and element 32 ib + i takes code-book entry
// kvalues_iq4nl[q & 15] of byte i % 16 of its 16 qs bytes (low nibble for
// i < 16, high for i >= 16), then one more rounding for dl * value. The
// reference reads the same 16 qs bytes, qs[0..16], for every sub-block (its
// qs slice is never advanced); `ggml` selects ggml's layout, qs[16 ib ..].
__device__ __forceinline__ float dq_iq4_xs(const uint8_t* blk, int j, int ggml) {
#pragma clang fp contract(off)
  const float d = h2f(rd16(blk));
  const uint32_t sh = rd16(blk + 2);
  const int ib = j >> 5, i = j & 31;
  const uint32_t ls = ((uint32_t(blk[4 + (ib >> 1)]) >> (4 * (ib & 1))) & 0x0Fu) | (((sh >> (2 * ib)) & 3u) << 4);
  const float dl = d * (static_cast<float>(ls) - 32.0f);
  const uint32_t byte = blk[8 + (ggml ? 16 * ib : 0) + (i & 15)];
  const uint32_t n = i < 16 ? (byte & 0x0Fu) : (byte >> 4);
  const int v = int8_t((kIq4Tab[n >> 2] >> (8 * (n & 3))) & 0xFFu);
  return dl * static_cast<float>(v);
}

__global__ void dequant_kernel(uint32_t quant, const uint8_t* __restrict__ w, int64_t rows,
                               int64_t cols, int64_t row_bytes, float* __restrict__ out,
                               int q6_signed) {  // the type's alternate reading (Q6_K i8 scales, IQ4_XS ggml qs)
  int64_t total = rows * cols;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t r = i / cols, c = i - r * cols;
    const uint8_t* row = w + r * row_bytes;
    float v;
    switch (quant) {
      case kQ8_0: v = dq_q8_0(row + (c >> 5) * 34, int(c & 31)); break;
      case kQ4_K: v = dq_q4_k(row + (c >> 8) * 144, int(c & 255)); break;
      case kQ5_K: v = dq_q5_k(row + (c >> 8) * 176, int(c & 255)); break;
      case kQ6_K: v = dq_q6_k(row + (c >> 8) * 210, int(c & 255), q6_signed); break;
      case kIQ4_XS: v = dq_iq4_xs(row + (c >> 8) * 136, int(c & 255), q6_signed); break;
      case kF16: v = h2f(rd16(row + 2 * c)); break;
      case kBF16: v = __builtin_bit_cast(float, rd16(row + 2 * c) << 16); break;
      default: v = __builtin_bit_cast(float, uint32_t(row[4 * c]) | (uint32_t(row[4 * c + 1]) << 8) |
                                                 (uint32_t(row[4 * c + 2]) << 16) |
                                                 (uint32_t(row[4 * c + 3]) << 24));
    }
    out[i] = v;
  }
}

hipError_t launch_dequant(uint32_t quant, const void* w, int64_t rows, int64_t cols, float* out,
                          int q6_signed, hipStream_t stream) {
  int64_t total = rows * cols;
  if (total == 0) return hipSuccess;
  int64_t row_bytes = byte_size(quant, cols);
  int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(dequant_kernel, dim3(unsigned(blocks)), dim3(threads), 0, stream, quant,
                     static_cast<const uint8_t*>(w), rows, cols, row_bytes, out, q6_signed);
  return hipGetLastError();
}

}  // namespace sh
