// Batched (2..8 vectors) Q4_K / Q5_K matvec on int8 MFMA with exact integer
// activations.
//
// Semantics: y[b][r] = sum_c W[r][c] * x[b][c] for every vector b, as
// `batch` calls of ops::gemv (crates/strata-core/src/ops.rs:14-28) with the
// Q4_K / Q5_K dequantization of crates/strata-gguf/src/dequant.rs:237-302.
//
// Per 256-element super-block of vector b a power-of-two scale 2^-k is
// chosen so that its largest |x| * 2^k < 2^22, and every element becomes the
// integer v = rne(x * 2^k) = a * 2^16 + b * 2^8 + c with balanced signed
// bytes a, b, c (so all three are int8; they are the bytes of
// v + 0x808080, each less 128). Q4_K codes q are 0..15 (Q5_K's 0..31: the
// nibble plus 16 times its bit of qh), so for a super-block
// with weights d * sc_j * q - dmin * m_j in sub-block j:
//   sum_e w_e x_e = d * 2^-k * (2^16 A + 2^8 B + C) - dmin * sum_j m_j * sx_j,
//   A = sum_j sc_j * sum_{e in j} q_e a_e   (B, C likewise)
// where each sub-block's integer sums are exact v_mfma_i32_16x16x32_i8
// products (K = 32) and the 6-bit scales sc_j are applied in integers
// (v_mad_i32_i24), so the f32 work is once per super-block; sx_j is the f32
// sum of x over sub-block j. x is represented to 2^-23 of its super-block's
// maximum.
//
// Mapping: a wave owns a tile of 16 weight rows (the MFMA's B columns) and a
// share of the super-blocks; the MFMA's 16 A rows are two limbs of the 8
// vectors (rows 0-7 one limb, rows 8-15 another), so a sub-block takes two
// MFMAs: (a | b) and (c | zero). A workgroup is T row tiles x S super-block
// shares (T * S waves), with the activations' limbs for every block and
// vector of one window of up to 4096 columns in LDS; wider rows take their
// windows in turn (restaging the limbs), the accumulators carried across.
// The S shares of a row tile are added through LDS at the end.
//
// With a workspace, the activations are converted once per call by
// mb_prep_kernel (a thread per vector and 32-element block) into the
// workspace, and each workgroup copies a window's limbs, scales and sums
// from there (L2) into LDS instead of converting them itself.
// Lane l of a wave holds, in D, weight row l % 16 for vectors
// 4 * ((l / 16) & 1) + i, i < 4: the a and c sums in lanes 0-31, the b sums
// in lanes 32-63.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

typedef int i32x4v __attribute__((ext_vector_type(4)));

constexpr int kMbMaxVec = 8;            // vectors per call
constexpr int kMbTokStride = 40;        // LDS bytes per (limb, block, vector): 32 codes + 8 pad
constexpr int kMbMaxCols = 4096;        // columns per window: their limbs fit LDS with the rest

__host__ __device__ inline int mb_limb_bytes(int nblk) { return 3 * nblk * kMbMaxVec * kMbTokStride; }

constexpr int kMbMaxWaves = 12;  // waves per workgroup (T * S)

// DPP lane exchanges inside 8 adjacent lanes (a super-block's 8 blocks):
// xor 1 and xor 2 as quad permutes; the other quad of the 8 through the
// half-row mirror (lane i <-> 7 - i), which for values already uniform over
// each quad is the same as xor 4.
__device__ __forceinline__ float max8_dpp(float m) {
  m = fmaxf(m, dpp_xor1(m));
  m = fmaxf(m, dpp_xor2(m));
  return fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x141, 0xF, 0xF,
                                                                          false)));  // row_half_mirror
}

// One 32-element block of one vector -> the three limb rows (32 bytes each),
// its 2^-k (per 256-element super-block: the 8 adjacent lanes of a
// super-block share their maximum) and its sum of x.
__device__ __forceinline__ void mb_convert_block(const float* src, uint32_t* wa, uint32_t* wb, uint32_t* wc,
                                                 float& down, float& sum) {
  float v[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const f32x4 t = reinterpret_cast<const f32x4*>(src)[k];
    v[4 * k] = t.x;
    v[4 * k + 1] = t.y;
    v[4 * k + 2] = t.z;
    v[4 * k + 3] = t.w;
  }
  float m = 0.f, s = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    m = fmaxf(m, fabsf(v[k]));
    s += v[k];
  }
  m = max8_dpp(m);
  int e = 0;
  (void)frexpf(m, &e);
  const int kk = m > 0.f ? min(22 - e, 126) : 0;
  const float up = ldexpf(1.f, kk);
  down = (m - m == 0.f) ? ldexpf(1.f, -kk) : __builtin_nanf("");
  sum = s;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    // rne(x * 2^k) through the 1.5 * 2^23 magic constant (|x * 2^k| < 2^22),
    // less 0x4B400000 plus 0x808080: u = v + 0x808080, whose bytes less 128
    // are the balanced digits c, b, a
    uint32_t u[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      u[q] = __builtin_bit_cast(uint32_t, __builtin_fmaf(v[4 * k + q], up, 12582912.0f)) - 0x4ABF7F80u;
    uint32_t pc, pb, pa;
    transpose_bytes(u[0], u[1], u[2], u[3], pc, pb, pa);
    wa[k] = pa ^ 0x80808080u;
    wb[k] = pb ^ 0x80808080u;
    wc[k] = pc ^ 0x80808080u;
  }
}

// Workspace layout, per window of nblk = min(cols, 4096) / 32 blocks (the
// last window may use fewer): limbs [3][nblk][8 vectors][32 bytes], then
// 2^-k [nblk / 8][8], then sums of x [nblk][8].
__host__ __device__ inline size_t mb_win_bytes(int nblk) {
  return size_t(3) * nblk * kMbMaxVec * 32 + size_t(nblk / 8) * kMbMaxVec * 4 + size_t(nblk) * kMbMaxVec * 4;
}

// The whole workspace: row-block counters of the split-K combine (zeroed
// by mb_prep_kernel on every call), the windows' partial sums
// [nwin][8][rows] (rows wider than one window), then the windows' images.
static size_t mb_align(size_t v) { return (v + 255) & ~size_t(255); }
static size_t mb_counters_bytes(int64_t rows) { return mb_align(size_t((rows + 15) / 16) * 4); }
static size_t mb_part_bytes(int64_t rows, int64_t cols) {
  const int64_t nwin = (cols + kMbMaxCols - 1) / kMbMaxCols;
  return nwin > 1 ? mb_align(size_t(nwin) * kMbMaxVec * size_t(rows) * 4) : 0;
}

size_t gemv_mfma_workspace_bytes(int64_t rows, int64_t cols) {
  const int nblk = int((cols < kMbMaxCols ? cols : kMbMaxCols) / 32);
  const int64_t nwin = (cols + kMbMaxCols - 1) / kMbMaxCols;
  return mb_counters_bytes(rows) + mb_part_bytes(rows, cols) + size_t(nwin) * mb_win_bytes(nblk);
}

// The activations of a call, converted once: thread p takes vector
// p / (cols / 32) and block p % (cols / 32); threads p < n_count also clear
// the split-K counters for the matvec launch that follows.
__global__ void __launch_bounds__(256) mb_prep_kernel(const float* __restrict__ x, int cols, int nb,
                                                      uint8_t* __restrict__ ws, uint32_t* __restrict__ count,
                                                      int n_count) {
  const int nblk_all = cols >> 5;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < n_count) count[p] = 0u;
  const int pc = min(p, nb * nblk_all - 1);  // past the end: a valid copy of the last block, not written
  const int b = pc / nblk_all, jg = pc - b * nblk_all;
  uint32_t wa[8], wb[8], wc[8];
  float down, sum;
  mb_convert_block(x + int64_t(b) * cols + 32 * jg, wa, wb, wc, down, sum);
  if (p >= nb * nblk_all) return;
  const int nblk = min(cols, kMbMaxCols) >> 5;
  const int win = jg / nblk, j = jg - win * nblk;
  uint8_t* img = ws + size_t(win) * mb_win_bytes(nblk);
  u32x4* da = reinterpret_cast<u32x4*>(img + ((size_t(0) * nblk + j) * kMbMaxVec + b) * 32);
  u32x4* db = reinterpret_cast<u32x4*>(img + ((size_t(1) * nblk + j) * kMbMaxVec + b) * 32);
  u32x4* dc = reinterpret_cast<u32x4*>(img + ((size_t(2) * nblk + j) * kMbMaxVec + b) * 32);
  da[0] = u32x4{wa[0], wa[1], wa[2], wa[3]};
  da[1] = u32x4{wa[4], wa[5], wa[6], wa[7]};
  db[0] = u32x4{wb[0], wb[1], wb[2], wb[3]};
  db[1] = u32x4{wb[4], wb[5], wb[6], wb[7]};
  dc[0] = u32x4{wc[0], wc[1], wc[2], wc[3]};
  dc[1] = u32x4{wc[4], wc[5], wc[6], wc[7]};
  float* pkw = reinterpret_cast<float*>(img + size_t(3) * nblk * kMbMaxVec * 32);
  float* sxw = pkw + (nblk / 8) * kMbMaxVec;
  if ((j & 7) == 0) pkw[(j >> 3) * kMbMaxVec + b] = down;
  sxw[j * kMbMaxVec + b] = sum;
}

// Q: kQ4_K (144-byte super-blocks, codes at byte 16) or kQ5_K (176 bytes:
// qh at 16, codes at 48). ONE: the row is a single window (cols <= 4096),
// which lets the compiler drop the window loop.
//
// SPLIT (with PREP, rows of two or more windows): workgroup b takes window
// b % nwin of row block b / nwin only, so it copies one window's limbs; the
// row block's sums per window go to part[win][vector][row] with
// device-scope (L2-bypassing) stores, the workgroup counts itself in on
// count[row block] once its stores are complete, and the last of the nwin
// workgroups adds the windows' sums in window order (deterministic) and
// writes y. No workgroup waits on another.
constexpr int kMbCopyRounds = 12;  // 16-byte chunks per thread of one window's copy (6144 / 512)

template <int Q, int PER, bool ONE, bool PREP, bool SPLIT>
__global__ void __launch_bounds__(64 * kMbMaxWaves)
    gemv_mfma_kq_kernel(const uint8_t* __restrict__ w, int rows, int cols, int64_t row_bytes,
                        const float* __restrict__ x, float* __restrict__ y, int nb, int T, int S,
                        const uint8_t* __restrict__ ws, float* part, uint32_t* count) {
  static_assert(!SPLIT || PREP, "the split-K combine needs the prepared workspace");
  constexpr int kSbBytes = Q == kQ5_K ? 176 : 144;
  constexpr int kCodes = Q == kQ5_K ? 48 : 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nthreads = blockDim.x;
  // LDS holds the limbs of one window of up to 4096 columns at a time
  const int nblk = min(cols, kMbMaxCols) >> 5;
  uint8_t* limbs = lds;                                                  // [3][nblk][8][40]
  float* pk = reinterpret_cast<float*>(lds + mb_limb_bytes(nblk));      // [nblk][8] (2^-k uses [nsb][8])
  float* sx = pk + nblk * kMbMaxVec;                                     // [nblk][8]: sum of x
  float* red = sx + nblk * kMbMaxVec;                                    // [T][S][64][4]

  // ---- this workgroup's row block (and window, SPLIT); this wave's row
  // tile and super-block share
  const int nwin = (cols + kMbMaxCols - 1) / kMbMaxCols;
  const int rtb = SPLIT ? blockIdx.x / nwin : blockIdx.x;
  const int win = SPLIT ? blockIdx.x - rtb * nwin : 0;
  const int rt = wave % T, sh_ = wave / T;
  const int r16 = lane & 15, kg = lane >> 4;  // B column (weight row) and k group
  const int row = min(rtb * (16 * T) + 16 * rt + r16, rows - 1);
  const uint8_t* wr = w + int64_t(row) * row_bytes;
  // A rows 0-7 carry one limb of vectors 0-7 and rows 8-15 another limb of
  // the same vectors: MFMA 1 takes limbs (a | b), MFMA 2 (c | zero). So lanes
  // of k groups 0, 1 hold a and c sums of vectors 4 kg + i in D, lanes of k
  // groups 2, 3 the b sums of the same vectors (kg - 2), exchanged once per
  // super-block.
  const int vec_a = r16 & 7;                  // the vector this lane feeds as an A row
  const bool a_real = vec_a < nb;
  const bool a_hi = r16 >= 8;                 // A rows 8-15: the second limb
  const int tok_d = 4 * (kg & 1);             // first vector of this lane's D values
  const bool d_out = kg < 2;                  // lanes whose D holds the a and c sums

  float acc[4] = {0.f, 0.f, 0.f, 0.f};

  // ---- column windows of up to 4096: stage the window's limbs, then each
  // wave accumulates its share of the window's super-blocks
  for (int c0 = SPLIT ? win * kMbMaxCols : 0; c0 < (ONE ? 1 : SPLIT ? win * kMbMaxCols + 1 : cols);
       c0 += kMbMaxCols) {
    const int nblk_w = ONE ? nblk : min(cols - c0, kMbMaxCols) >> 5, nsb_w = nblk_w >> 3;
    if (c0 > 0) __syncthreads();  // every wave is done with the previous window's limbs
    // ---- activations -> limbs: one (vector, block) pair per thread per round;
    // the 8 blocks of a super-block are 8 adjacent lanes (nblk_w and the
    // workgroup size are multiples of 8), which share its maximum
    float* pk8 = pk;  // [nsb_w][8]: 2^-k of (super-block, vector)
    if constexpr (PREP) {
      // copy the window's image from the workspace: 16-byte chunks (half a
      // limb row) to their 40-byte LDS slots, then the scales and sums; all
      // of a thread's loads are issued before its stores
      const uint8_t* img = ws + size_t(ONE ? 0 : c0 / kMbMaxCols) * mb_win_bytes(nblk);
      const int nchunk = 3 * nblk_w * nb * 2;
      u32x4 cv[kMbCopyRounds];
      size_t cdst[kMbCopyRounds];
#pragma unroll
      for (int k = 0; k < kMbCopyRounds; ++k) {
        const int q = min(tid + k * nthreads, nchunk - 1);
        const int half = q & 1, r = q >> 1;               // r: (limb, block, vector) record
        const int b = r % nb, lj = r / nb;                  // lj = limb * nblk_w + block
        const int l = lj / nblk_w, j = lj - l * nblk_w;
        const size_t rec = (size_t(l) * nblk + j) * kMbMaxVec + b;
        cv[k] = *reinterpret_cast<const u32x4*>(img + rec * 32 + 16 * half);
        cdst[k] = rec * kMbTokStride + 16 * half;
      }
#pragma unroll
      for (int k = 0; k < kMbCopyRounds; ++k) {
        if (tid + k * nthreads < nchunk) {
          uint64_t* d = reinterpret_cast<uint64_t*>(limbs + cdst[k]);
          d[0] = uint64_t(cv[k].x) | (uint64_t(cv[k].y) << 32);
          d[1] = uint64_t(cv[k].z) | (uint64_t(cv[k].w) << 32);
        }
      }
      for (int q = tid + kMbCopyRounds * nthreads; q < nchunk; q += nthreads) {  // larger workgroup shapes
        const int half = q & 1, r = q >> 1;
        const int b = r % nb, lj = r / nb;
        const int l = lj / nblk_w, j = lj - l * nblk_w;
        const size_t rec = (size_t(l) * nblk + j) * kMbMaxVec + b;
        const u32x4 v = *reinterpret_cast<const u32x4*>(img + rec * 32 + 16 * half);
        uint64_t* d = reinterpret_cast<uint64_t*>(limbs + rec * kMbTokStride + 16 * half);
        d[0] = uint64_t(v.x) | (uint64_t(v.y) << 32);
        d[1] = uint64_t(v.z) | (uint64_t(v.w) << 32);
      }
      const float* pkw = reinterpret_cast<const float*>(img + size_t(3) * nblk * kMbMaxVec * 32);
      const float* sxw = pkw + (nblk / 8) * kMbMaxVec;
      for (int q = tid; q < nblk_w * kMbMaxVec; q += nthreads) {
        sx[q] = sxw[q];
        if (q < (nblk_w / 8) * kMbMaxVec) pk8[q] = pkw[q];
      }
    } else {
      // ---- activations -> limbs: one (vector, block) pair per thread per
      // round; the 8 blocks of a super-block are 8 adjacent lanes (nblk_w and
      // the workgroup size are multiples of 8), which share its maximum
      for (int p = tid; p < nb * nblk_w; p += nthreads) {
        const int b = p / nblk_w, j = p - b * nblk_w;
        uint32_t wa[8], wb[8], wc[8];
        float down, sum;
        mb_convert_block(x + int64_t(b) * cols + c0 + 32 * j, wa, wb, wc, down, sum);
        if ((j & 7) == 0) pk8[(j >> 3) * kMbMaxVec + b] = down;
        sx[j * kMbMaxVec + b] = sum;
        uint8_t* da = limbs + (0 * nblk + j) * (kMbMaxVec * kMbTokStride) + b * kMbTokStride;
        uint8_t* db = limbs + (1 * nblk + j) * (kMbMaxVec * kMbTokStride) + b * kMbTokStride;
        uint8_t* dc = limbs + (2 * nblk + j) * (kMbMaxVec * kMbTokStride) + b * kMbTokStride;
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
          *reinterpret_cast<uint64_t*>(da + 4 * k) = uint64_t(wa[k]) | (uint64_t(wa[k + 1]) << 32);
          *reinterpret_cast<uint64_t*>(db + 4 * k) = uint64_t(wb[k]) | (uint64_t(wb[k + 1]) << 32);
          *reinterpret_cast<uint64_t*>(dc + 4 * k) = uint64_t(wc[k]) | (uint64_t(wc[k + 1]) << 32);
        }
      }
    }
    __syncthreads();

    const int sb0 = sh_ * PER, sb1 = min(nsb_w, sb0 + PER);
    const uint8_t* wr_w = wr + int64_t(c0 >> 8) * kSbBytes;
    u32x4 h_cur, h_nxt;
    uint64_t q_cur[4], q_nxt[4];
    uint64_t qh_cur = 0, qh_nxt = 0;  // Q5_K: qh bytes 8 kg .. 8 kg + 7 (this lane's elements)
    auto load_sb = [&](int sb, u32x4& h, uint64_t* q, uint64_t& qh) {
      const uint8_t* p = wr_w + int64_t(min(sb, nsb_w - 1)) * kSbBytes;
      h = ld16(p);
      if constexpr (Q == kQ5_K) qh = *reinterpret_cast<const uint64_t*>(p + 16 + 8 * kg);
#pragma unroll
      for (int g = 0; g < 4; ++g) q[g] = *reinterpret_cast<const uint64_t*>(p + kCodes + 32 * g + 8 * kg);
    };
    if (sb0 < sb1) load_sb(sb0, h_cur, q_cur, qh_cur);
    for (int sb = sb0; sb < sb1; ++sb) {
      load_sb(sb + 1, h_nxt, q_nxt, qh_nxt);  // the next super-block in flight (past the share: valid, unused)
      // per limb: sum over the sub-blocks of sc_j * (integer dot); and the
      // f32 min term sum_j m_j * sx_j
      int i1[4] = {0, 0, 0, 0}, i2[4] = {0, 0, 0, 0};  // (a | b) and (c | 0) sums
      float mn[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // scales and mins of sub-blocks 2g, 2g + 1 (get_scale_min_k4)
        const uint32_t shv = (g & 1) << 4;
        const uint32_t t1 = h_cur.y >> shv, t2 = h_cur.z >> shv, t3 = h_cur.w >> shv;
        const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
        const uint32_t mp = g < 2 ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int jb = 8 * sb + 2 * g + hh;  // 32-element block of this sub-block
          uint64_t codes = hh ? ((q_cur[g] >> 4) & 0x0F0F0F0F0F0F0F0Full) : (q_cur[g] & 0x0F0F0F0F0F0F0F0Full);
          // Q5_K: sub-block 2g + hh takes bit 2g + hh of each qh byte as 16
          if constexpr (Q == kQ5_K) codes |= ((qh_cur >> (2 * g + hh)) & 0x0101010101010101ull) << 4;
          // loads from in-range addresses whatever the lane, then a select
          // (no branches: the loads and MFMAs of neighbouring sub-blocks can
          // be scheduled together)
          const uint8_t* blk = limbs + jb * (kMbMaxVec * kMbTokStride) + vec_a * kMbTokStride + 8 * kg;
          const int limb_stride = nblk * (kMbMaxVec * kMbTokStride);
          const long v1 = *reinterpret_cast<const long*>(blk + (a_hi ? limb_stride : 0));  // a | b
          const long v2 = *reinterpret_cast<const long*>(blk + 2 * limb_stride);           // c
          const long A1 = a_real ? v1 : 0l;
          const long A2 = a_real && !a_hi ? v2 : 0l;
          const i32x4v I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A1, long(codes), i32x4v{}, 0, 0, 0);
          const i32x4v I2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A2, long(codes), i32x4v{}, 0, 0, 0);
          const int scj = int((hh ? (scp >> 8) : scp) & 0xFFu);
          const float mj = float((hh ? (mp >> 8) : mp) & 0xFFu);
          const f32x4 sx4 = *reinterpret_cast<const f32x4*>(sx + jb * kMbMaxVec + tok_d);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // |integer dot| <= 31 * 32 * 128 and sc <= 63: 24-bit operands
            i1[k] = __mul24(I1[k], scj) + i1[k];
            i2[k] = __mul24(I2[k], scj) + i2[k];
            mn[k] = __builtin_fmaf(mj, sx4[k], mn[k]);
          }
        }
      }
      // the b sums from the lanes 32 apart; |a|, |b|, |c| sums <= 8 * 63 * 126976
      // < 2^26: f32 conversions within an ulp
      int ib[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) ib[k] = __shfl_xor(i1[k], 32, kWave);
      const float d = h2f(h_cur.x), dm = h2f(h_cur.x >> 16);
      const f32x4 pk4 = *reinterpret_cast<const f32x4*>(pk8 + sb * kMbMaxVec + tok_d);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float f = __builtin_fmaf(float(i1[k]), 65536.f, __builtin_fmaf(float(ib[k]), 256.f, float(i2[k])));
        acc[k] = __builtin_fmaf(f, d * pk4[k], acc[k]);
        acc[k] = __builtin_fmaf(-dm, mn[k], acc[k]);
      }
      h_cur = h_nxt;
      qh_cur = qh_nxt;
#pragma unroll
      for (int g = 0; g < 4; ++g) q_cur[g] = q_nxt[g];
    }
  }

  // ---- add the S shares of each row tile, in share order
  float* mine = red + ((rt * S + sh_) * 64 + lane) * 4;
  *reinterpret_cast<f32x4*>(mine) = f32x4{acc[0], acc[1], acc[2], acc[3]};
  __syncthreads();
  if (sh_ == 0) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    for (int s2 = 0; s2 < S; ++s2) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(red + ((rt * S + s2) * 64 + lane) * 4);
      t = f32x4{t.x + v.x, t.y + v.y, t.z + v.z, t.w + v.w};
    }
    const int r = rtb * (16 * T) + 16 * rt + r16;
    if (r < rows) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (d_out && tok_d + i < nb) {
          if constexpr (SPLIT)
            __hip_atomic_store(part + (int64_t(win) * kMbMaxVec + tok_d + i) * rows + r, t[i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          else
            y[int64_t(tok_d + i) * rows + r] = t[i];
        }
      }
    }
  }
  if constexpr (SPLIT) {
    __shared__ uint32_t s_last;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial sums are in memory
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(count + rtb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_last != uint32_t(nwin - 1)) return;
    // the last workgroup of the row block: the windows' sums in window order
    const int r0 = rtb * (16 * T), nr = min(16 * T, rows - r0);
    for (int i = tid; i < nb * nr; i += nthreads) {
      const int b = i / nr, r = r0 + (i - b * nr);
      float v = __hip_atomic_load(part + int64_t(b) * rows + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int k = 1; k < nwin; ++k)
        v += __hip_atomic_load(part + (int64_t(k) * kMbMaxVec + b) * rows + r, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      y[int64_t(b) * rows + r] = v;
    }
  }
}

bool gemv_mfma_ok(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  return (quant == kQ4_K || quant == kQ5_K) && batch >= 2 && batch <= kMbMaxVec && cols > 0 && cols % 256 == 0 &&
         cols <= (int64_t(1) << 20) && rows > 0 && rows <= (int64_t(1) << 31) - 1;
}

template <int PER, bool PREP, bool SPLIT>
static void launch_mb(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x, float* y,
                      int batch, int T, int S, size_t lds, const uint8_t* ws, float* part, uint32_t* count,
                      hipStream_t s) {
  const int64_t nwin = (cols + kMbMaxCols - 1) / kMbMaxCols;
  const unsigned blocks = unsigned((rows + 16 * T - 1) / (16 * T) * (SPLIT ? nwin : 1));
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  const int64_t rb = byte_size(quant, cols);
  const bool one = cols <= kMbMaxCols;
  const dim3 grid = dim3(blocks), block = dim3(unsigned(64 * T * S));
  if (quant == kQ5_K) {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, true, PREP, false>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, ws, part, count);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, false, PREP, SPLIT>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, ws, part, count);
  } else {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, true, PREP, false>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, ws, part, count);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, false, PREP, SPLIT>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, ws, part, count);
  }
}

template <bool PREP, bool SPLIT>
static void launch_mb_per(int per, uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                          float* y, int batch, int T, int S, size_t lds, const uint8_t* ws, float* part,
                          uint32_t* count, hipStream_t s) {
  switch (per) {
    case 1: launch_mb<1, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 2: launch_mb<2, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 3: launch_mb<3, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 4: launch_mb<4, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 5: launch_mb<5, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 6: launch_mb<6, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    case 7: launch_mb<7, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
    default: launch_mb<8, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, lds, ws, part, count, s); break;
  }
}

hipError_t launch_gemv_mfma(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x, float* y,
                            int batch, int cu, hipStream_t s, void* ws) {
  if (!gemv_mfma_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  if (ws && (reinterpret_cast<uintptr_t>(ws) & 255u)) return hipErrorInvalidValue;
  const int64_t nwin = (cols + kMbMaxCols - 1) / kMbMaxCols;
  const bool split = ws && nwin > 1;
  // T row tiles per workgroup so the tiles cover the CUs about once (with
  // the split, the row blocks times the windows); the workgroup's waves (12
  // for 3 or 4 tiles, 8 otherwise: one workgroup per CU, the activations'
  // LDS allowing no more) split the super-blocks into shares of PER <= 8
  const int64_t slots = split ? (cu / nwin > 0 ? cu / nwin : 1) : cu;
  int T = int((rows + 16LL * slots - 1) / (16LL * slots));
  if (T < 1) T = 1;
  if (T > 4) T = 4;
  const int S = T >= 3 ? kMbMaxWaves / T : 8 / T;
  const int64_t wcols = cols < kMbMaxCols ? cols : kMbMaxCols;  // one window of columns
  const int nsb = int(wcols / 256);
  const int per = (nsb + S - 1) / S;  // <= 8: a window is <= 4096 columns and S >= 2
  const int nblk = int(wcols / 32);
  const size_t lds = size_t(mb_limb_bytes(nblk)) + 2 * sizeof(float) * nblk * kMbMaxVec +
                     sizeof(float) * T * S * 64 * 4;
  if (ws) {
    // the activations converted once for every workgroup (and the split-K
    // counters cleared)
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    uint32_t* count = reinterpret_cast<uint32_t*>(wsb);
    float* part = reinterpret_cast<float*>(wsb + mb_counters_bytes(rows));
    const uint8_t* img = wsb + mb_counters_bytes(rows) + mb_part_bytes(rows, cols);
    const int n_count = int((rows + 16 * T - 1) / (16 * T));
    const int64_t n = std::max<int64_t>(int64_t(batch) * (cols / 32), n_count);
    hipLaunchKernelGGL(mb_prep_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, int(cols), batch,
                       const_cast<uint8_t*>(img), count, n_count);
    if (split)
      launch_mb_per<true, true>(per, quant, wv, rows, cols, x, y, batch, T, S, lds, img, part, count, s);
    else
      launch_mb_per<true, false>(per, quant, wv, rows, cols, x, y, batch, T, S, lds, img, nullptr, nullptr, s);
  } else {
    launch_mb_per<false, false>(per, quant, wv, rows, cols, x, y, batch, T, S, lds, nullptr, nullptr, nullptr, s);
  }
  return hipGetLastError();
}

}  // namespace sh
