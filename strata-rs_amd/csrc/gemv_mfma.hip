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
// mb_prep_kernel (a wave per vector and 256-element super-block) into the
// workspace, and each workgroup copies a window's limbs, scales and sums
// from there (L2) into LDS instead of converting them itself.
// Lane l of a wave holds, in D, weight row l % 16 for vectors
// 4 * ((l / 16) & 1) + i, i < 4: the a and c sums in lanes 0-31, the b sums
// in lanes 32-63.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace sh {

typedef int i32x4v __attribute__((ext_vector_type(4)));

constexpr int kMbMaxVec = 8;            // vectors per call
constexpr int kMbTokStride = 32;        // bytes per (limb, block, vector): the 32 limb bytes
constexpr int kMbMaxCols = 4096;        // columns per window at most: their limbs fit LDS with the rest

// Limb layout (in LDS, and in the workspace image, which is copied to LDS
// as is): plane l (limb a, b, c) at l * mb_plane(nblk), block j of a plane
// at j * kMbBlkStride, vector b's 32 bytes at b * 32 in the block. The 16
// spare bytes per block move block j + 1 four banks on from block j (the
// conversion's stores of adjacent blocks, and paired reads of adjacent
// sub-blocks, fall in different banks), and the 16 spare bytes per plane do
// the same for the a and b limbs read by one instruction.
constexpr int kMbBlkStride = kMbMaxVec * kMbTokStride + 16;
__host__ __device__ inline int mb_plane(int nblk) { return nblk * kMbBlkStride + 16; }
__host__ __device__ inline int mb_limb_bytes(int nblk) { return 3 * mb_plane(nblk); }

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

// One 32-element block of one vector: its 8 x 16-byte loads (issued apart
// from the conversion, so that other loads can be queued behind them).
__device__ __forceinline__ void mb_load_block(const float* src, float (&v)[32]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const f32x4 t = reinterpret_cast<const f32x4*>(src)[k];
    v[4 * k] = t.x;
    v[4 * k + 1] = t.y;
    v[4 * k + 2] = t.z;
    v[4 * k + 3] = t.w;
  }
}

// Four elements with the super-block's 2^k -> their bytes of limbs a, b, c.
// rne(x * 2^k) through the 1.5 * 2^23 magic constant (|x * 2^k| < 2^22),
// less 0x4B400000 plus 0x808080: u = v + 0x808080, whose bytes less 128 are
// the balanced digits c, b, a.
__device__ __forceinline__ void mb_limb_word(float v0, float v1, float v2, float v3, float up, uint32_t& wa,
                                             uint32_t& wb, uint32_t& wc) {
  const uint32_t u0 = __builtin_bit_cast(uint32_t, __builtin_fmaf(v0, up, 12582912.0f)) - 0x4ABF7F80u;
  const uint32_t u1 = __builtin_bit_cast(uint32_t, __builtin_fmaf(v1, up, 12582912.0f)) - 0x4ABF7F80u;
  const uint32_t u2 = __builtin_bit_cast(uint32_t, __builtin_fmaf(v2, up, 12582912.0f)) - 0x4ABF7F80u;
  const uint32_t u3 = __builtin_bit_cast(uint32_t, __builtin_fmaf(v3, up, 12582912.0f)) - 0x4ABF7F80u;
  uint32_t pc, pb, pa;
  transpose_bytes(u0, u1, u2, u3, pc, pb, pa);
  wa = pa ^ 0x80808080u;
  wb = pb ^ 0x80808080u;
  wc = pc ^ 0x80808080u;
}

// 2^k of a super-block from its largest |x| (k = min(22 - e, 126), so the
// scaled maximum is below 2^22), and 2^-k (NaN when the maximum is not finite).
__device__ __forceinline__ void mb_scales(float m, float& up, float& down) {
  int e = 0;
  (void)frexpf(m, &e);
  const int kk = m > 0.f ? min(22 - e, 126) : 0;
  up = ldexpf(1.f, kk);
  down = (m - m == 0.f) ? ldexpf(1.f, -kk) : __builtin_nanf("");
}

// A loaded 32-element block of one vector -> the three limb rows (32 bytes
// each), its 2^-k (per 256-element super-block: the 8 adjacent lanes of a
// super-block share their maximum) and its sum of x.
__device__ __forceinline__ void mb_convert_block(const float (&v)[32], uint32_t* wa, uint32_t* wb, uint32_t* wc,
                                                 float& down, float& sum) {
  float m = 0.f, s = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    m = fmaxf(m, fabsf(v[k]));
    s += v[k];
  }
  m = max8_dpp(m);
  float up;
  mb_scales(m, up, down);
  sum = s;
#pragma unroll
  for (int k = 0; k < 8; ++k) mb_limb_word(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3], up, wa[k], wb[k], wc[k]);
}

// Workspace image, per window of nblk = min(cols, 4096) / 32 blocks (the
// last window may use fewer): the limb planes (mb_plane), then 2^-k
// [nblk / 8][8], then sums of x [nblk][8]; LDS holds the same layout.
__host__ __device__ inline size_t mb_win_bytes(int nblk) {
  return size_t(mb_limb_bytes(nblk)) + size_t(nblk / 8) * kMbMaxVec * 4 + size_t(nblk) * kMbMaxVec * 4;
}
// The window image rounded up to whole KiB: what the copies move, and the
// LDS it takes.
__host__ __device__ inline int mb_win_alloc(int nblk) { return int((mb_win_bytes(nblk) + 1023) & ~size_t(1023)); }

// The whole workspace: row-block counters of the split-K combine (zeroed
// by mb_prep_kernel on every call), the windows' partial sums
// [nwin][8][rows] (rows wider than one window), then the windows' images.
static size_t mb_align(size_t v) { return (v + 255) & ~size_t(255); }
static size_t mb_counters_bytes(int64_t rows) { return mb_align(size_t((rows + 15) / 16) * 4); }
static size_t mb_part_bytes(int64_t rows, int64_t cols, int wc) {
  const int64_t nwin = (cols + wc - 1) / wc;
  return nwin > 1 ? mb_align(size_t(nwin) * kMbMaxVec * size_t(rows) * 4) : 0;
}
static size_t mb_images_bytes(int64_t cols, int wc) {
  const int nblk = int((cols < wc ? cols : wc) / 32);
  // + 1 KiB: the last window's copy, rounded up to whole KiB, reads past its image
  return size_t((cols + wc - 1) / wc) * mb_win_bytes(nblk) + 1024;
}

// Window widths the launcher chooses from (columns; multiples of 256).
constexpr int kMbWindows[3] = {4096, 3072, 2048};

size_t gemv_mfma_workspace_bytes(int64_t rows, int64_t cols) {
  size_t most = 0;
  for (int wc : kMbWindows) most = std::max(most, mb_part_bytes(rows, cols, wc) + mb_images_bytes(cols, wc));
  return mb_counters_bytes(rows) + most;
}

// The activations of a call, converted once: a wave per (vector, 256-element
// super-block), lane l taking elements 4l .. 4l + 3 (lanes 8i .. 8i + 7 hold
// block i of the super-block); threads below n_count also clear the split-K
// counters for the matvec launch that follows. Block sums are added as
// (lane sums of 4, in order) over the 8 lanes pairwise.
__global__ void __launch_bounds__(256) mb_prep_kernel(const float* __restrict__ x, int cols, int wcols, int nb,
                                                      uint8_t* __restrict__ ws, uint32_t* __restrict__ count,
                                                      int n_count) {
  const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gtid < n_count) count[gtid] = 0u;
  const int nsb_all = cols >> 8;
  const int wv = gtid >> 6, lane = threadIdx.x & 63;
  if (wv >= nb * nsb_all) return;  // whole waves
  const int b = wv / nsb_all, sbg = wv - b * nsb_all;
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + int64_t(b) * cols + 256 * sbg + 4 * lane);
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  m = max8_dpp(m);
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x140, 0xF, 0xF,
                                                                   false)));  // row_mirror: 16 lanes
  m = fmaxf(m, __shfl_xor(m, 16, kWave));
  m = fmaxf(m, __shfl_xor(m, 32, kWave));
  float s = ((v.x + v.y) + v.z) + v.w;
  s += dpp_xor1(s);
  s += dpp_xor2(s);
  s += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s), 0x141, 0xF, 0xF,
                                                           false));  // row_half_mirror: the other quad
  float up, down;
  mb_scales(m, up, down);
  uint32_t wa, wb, wc;
  mb_limb_word(v.x, v.y, v.z, v.w, up, wa, wb, wc);
  const int nblk = min(cols, wcols) >> 5;
  const int jg = 8 * sbg + (lane >> 3);
  const int win = jg / nblk, j = jg - win * nblk;
  uint8_t* img = ws + size_t(win) * mb_win_bytes(nblk);
  const size_t word = 4 * (lane & 7);
  uint8_t* rec = img + size_t(j) * kMbBlkStride + b * kMbTokStride + word;
  *reinterpret_cast<uint32_t*>(rec) = wa;
  *reinterpret_cast<uint32_t*>(rec + mb_plane(nblk)) = wb;
  *reinterpret_cast<uint32_t*>(rec + 2 * mb_plane(nblk)) = wc;
  float* pkw = reinterpret_cast<float*>(img + mb_limb_bytes(nblk));
  float* sxw = pkw + (nblk / 8) * kMbMaxVec;
  if (lane == 0) pkw[(j >> 3) * kMbMaxVec + b] = down;
  if ((lane & 7) == 0) sxw[j * kMbMaxVec + b] = s;
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
template <int Q, int PER, bool ONE, bool PREP, bool SPLIT>
__global__ void __launch_bounds__(64 * kMbMaxWaves)
    gemv_mfma_kq_kernel(const uint8_t* __restrict__ w, int rows, int cols, int64_t row_bytes,
                        const float* __restrict__ x, float* __restrict__ y, int nb, int T, int S, int wc,
                        const uint8_t* __restrict__ ws, float* part, uint32_t* count) {
  static_assert(!SPLIT || PREP, "the split-K combine needs the prepared workspace");
  constexpr int kSbBytes = Q == kQ5_K ? 176 : 144;
  constexpr int kCodes = Q == kQ5_K ? 48 : 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // the wave index as a scalar, so that per-wave conditions are uniform
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nthreads = blockDim.x;
  // LDS holds the limbs of one window of wc <= 4096 columns at a time
  const int nblk = min(cols, wc) >> 5;
  // the workspace image's layout: limbs, 2^-k, sums of x
  uint8_t* limbs = lds;                                                  // 3 planes, see mb_plane
  float* pk = reinterpret_cast<float*>(lds + mb_limb_bytes(nblk));      // [nblk / 8][8]: 2^-k
  float* sx = pk + (nblk / 8) * kMbMaxVec;                               // [nblk][8]: sum of x
  float* red = reinterpret_cast<float*>(lds + mb_win_alloc(nblk));     // [T][S][64][4]

  // ---- this workgroup's row block (and window, SPLIT); this wave's row
  // tile and super-block share
  const int nwin = (cols + wc - 1) / wc;
  const int rtb = SPLIT ? blockIdx.x / nwin : blockIdx.x;
  const int win = SPLIT ? blockIdx.x - rtb * nwin : 0;
  const int rt = wave % T, sh_ = wave / T;
  const int r16 = lane & 15, kg = lane >> 4;  // B column (weight row) and k group
  const int row = min(rtb * (16 * T) + 16 * rt + r16, rows - 1);
  const uint8_t* wr = w + int64_t(row) * row_bytes;
  // A rows 0-7 carry one limb of vectors 0-7 and rows 8-15 another limb of
  // the same vectors: MFMA 1 takes limbs (a | b), MFMA 2 (c | c). So lanes
  // of k groups 0, 1 hold a and c sums of vectors 4 kg + i in D, lanes of k
  // groups 2, 3 the b sums of the same vectors (kg - 2), exchanged once per
  // super-block; their second D (c again) is not used. A rows of vectors at
  // or past nb read LDS slots nothing has written: the MFMA keeps rows
  // apart, so they reach only D rows that are never stored.
  const int vec_a = r16 & 7;                  // the vector this lane feeds as an A row
  const bool a_hi = r16 >= 8;                 // A rows 8-15: the second limb
  const int tok_d = 4 * (kg & 1);             // first vector of this lane's D values
  const bool d_out = kg < 2;                  // lanes whose D holds the a and c sums

  float acc[4] = {0.f, 0.f, 0.f, 0.f};

  // ---- column windows of up to 4096: stage the window's limbs, then each
  // wave accumulates its share of the window's super-blocks
  for (int c0 = SPLIT ? win * wc : 0; c0 < (ONE ? 1 : SPLIT ? win * wc + 1 : cols); c0 += wc) {
    const int nblk_w = ONE ? nblk : min(cols - c0, wc) >> 5, nsb_w = nblk_w >> 3;
    float* pk8 = pk;  // [nsb_w][8]: 2^-k of (super-block, vector)
    auto sb_of = [&](int i) { return sh_ * PER + i; };  // this wave's share of the window's super-blocks
    const uint8_t* wr_w = wr + int64_t(c0 >> 8) * kSbBytes;

    // ---- 1. the staging loads, issued first: the workspace image copied as
    // is straight into LDS (global_load_lds, whole 1 KiB wave instructions,
    // no registers; the LDS area is the image rounded up to whole KiB and
    // the workspace ends in 1 KiB of slack for the last window's overrun),
    // or x for the conversion. No LDS store of this wave follows the copies
    // before the barrier (that would make the compiler wait for every load).
    if constexpr (PREP) {
      const uint8_t* img = ws + size_t(ONE ? 0 : c0 / wc) * mb_win_bytes(nblk);
      const int nwaves = nthreads >> 6;
      for (int c = wave; c < (mb_win_alloc(nblk) >> 10); c += nwaves)
        copy16_to_lds(img + (c << 10) + 16 * lane, limbs + (c << 10));
      __builtin_amdgcn_sched_barrier(0);  // the weight loads stay behind the copies
    }
    const int npairs = nb * nblk_w;  // conversion: (vector, block) pairs, at most two per thread
    float xv0[PREP ? 1 : 32], xv1[PREP ? 1 : 32];
    auto pair_src = [&](int p) {
      const int pc = min(p, npairs - 1);  // past the end: a valid copy of the last block, not stored
      const int b = pc / nblk_w, j = pc - b * nblk_w;
      return x + int64_t(b) * cols + c0 + 32 * j;
    };
    if constexpr (!PREP) {
      // both rounds unconditionally (a second round past the pairs reads the
      // last block again: an L1 hit), so that no branch lets the weight loads
      // below be placed ahead of these
      mb_load_block(pair_src(tid), xv0);
      mb_load_block(pair_src(tid + nthreads), xv1);
    }
    // the weight loads go behind the staging's (a compiler barrier for
    // memory operations; it waits on nothing), and behind every other
    // wave's: a CU returns loads about in issue order, so one wave's weight
    // loads ahead of another's staging loads would hold that staging up. An
    // issue-only barrier orders them (batch 8: Q4_K 12288x4096 16.1 -> 15.3
    // us, Q5_K 17.8 -> 16.7 and 19.4 -> 18.8)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's weights, a ring kRing super-blocks deep:
    // super-block i + kRing is issued when super-block i is computed. The
    // first kRing go out beside the conversion (their latency overlaps it),
    // or, after a copy, once the copy has landed: more weight loads in
    // flight only stall the wave at issue (the CU's memory queue is full)
    // and hold the staging up behind them. Addresses past the share or the
    // window: valid, unused.
    constexpr int kRing = PER < 2 ? PER : 2;
    u32x4 hq[PER];
    uint64_t qq[PER][4], qhq[PER];
    auto issue_sb = [&](int i) {
      const uint8_t* p = wr_w + int64_t(min(sb_of(i), nsb_w - 1)) * kSbBytes;
      hq[i] = ld16(p);
      qhq[i] = 0;
      if constexpr (Q == kQ5_K) qhq[i] = *reinterpret_cast<const uint64_t*>(p + 16 + 8 * kg);
#pragma unroll
      for (int g = 0; g < 4; ++g) qq[i][g] = *reinterpret_cast<const uint64_t*>(p + kCodes + 32 * g + 8 * kg);
    };
    // issued before the staging completes; with the image copy, the first
    // super-block's loads go behind the copies (in-order completion: waiting
    // until only they are outstanding means the copies have landed)
    constexpr int kPre = PREP ? 1 : kRing;
    // vector loads of issue_sb: the 16-byte header, the lane's 8 qh bytes
    // (Q5_K) and its four 8-byte code runs, at lane-dependent offsets that
    // the compiler cannot merge (the ISA shows exactly these, then the wait)
    constexpr int kSbLoads = Q == kQ5_K ? 6 : 5;
#pragma unroll
    for (int i = 0; i < kPre; ++i) issue_sb(i);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. the staging's completion: the copies landed (nothing else is
    // outstanding), or the conversion's LDS stores
    if (!SPLIT && c0 > 0) lds_barrier();  // every wave is done with the previous window's limbs
    if constexpr (PREP) {
      wait_vmem<kSbLoads * kPre>();
    } else {
      // one (vector, block) pair per thread per round; the 8 blocks of a
      // super-block are 8 adjacent lanes (nblk_w and the workgroup size are
      // multiples of 8), which share its maximum
#pragma unroll
      for (int rnd = 0; rnd < 2; ++rnd) {
        const int p = tid + rnd * nthreads;
        if (rnd == 1 && npairs <= nthreads) break;
        uint32_t wa[8], wb[8], wc[8];
        float down, sum;
        mb_convert_block(rnd ? xv1 : xv0, wa, wb, wc, down, sum);
        if (p < npairs) {
          const int b = p / nblk_w, j = p - b * nblk_w;
          if ((j & 7) == 0) pk8[(j >> 3) * kMbMaxVec + b] = down;
          sx[j * kMbMaxVec + b] = sum;
          uint8_t* da = limbs + j * kMbBlkStride + b * kMbTokStride;
          uint8_t* db = da + mb_plane(nblk);
          uint8_t* dc = da + 2 * mb_plane(nblk);
#pragma unroll
          for (int k = 0; k < 8; k += 4) {
            *reinterpret_cast<u32x4*>(da + 4 * k) = u32x4{wa[k], wa[k + 1], wa[k + 2], wa[k + 3]};
            *reinterpret_cast<u32x4*>(db + 4 * k) = u32x4{wb[k], wb[k + 1], wb[k + 2], wb[k + 3]};
            *reinterpret_cast<u32x4*>(dc + 4 * k) = u32x4{wc[k], wc[k + 1], wc[k + 2], wc[k + 3]};
          }
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int i = kPre; i < kRing; ++i) issue_sb(i);

    // ---- 4. the share's super-blocks. Per sub-block: two int8 MFMAs and
    // the 6-bit scale applied in integers; per super-block the min term
    // sum_j m_j * sx_j on two f32 MFMAs (K = 4: A = sx of sub-blocks kg and
    // 4 + kg for vector r16 & 7, B = m of the same sub-blocks for row r16),
    // whose D has the int8 MFMAs' layout
    const int off_a = vec_a * kMbTokStride + 8 * kg + (a_hi ? mb_plane(nblk) : 0);  // limb a or b
    const int off_c = vec_a * kMbTokStride + 8 * kg + 2 * mb_plane(nblk);           // limb c
    // Branch-free over the PER slots (a slot past the share computes on its
    // clamped copy and is not added): the loads above then stay where they
    // are issued rather than sinking into a conditional block.
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (i + kRing < PER) issue_sb(i + kRing);
      asm volatile("" ::: "memory");  // the next loads go out before this super-block's work
      const bool live = sb_of(i) < nsb_w;  // a share past the window's end (narrow last windows)
      const int sb = min(sb_of(i), nsb_w - 1);
      const u32x4 h = hq[i];
      const uint8_t* la = limbs + (8 * sb) * kMbBlkStride + off_a;
      const uint8_t* lc = limbs + (8 * sb) * kMbBlkStride + off_c;
      int i1[4] = {0, 0, 0, 0}, i2[4] = {0, 0, 0, 0};  // (a | b) and (c | c) sums
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // scales of sub-blocks 2g, 2g + 1 (get_scale_min_k4)
        const uint32_t shv = (g & 1) << 4;
        const uint32_t t1 = h.y >> shv, t3 = h.w >> shv;
        const uint32_t scp = g < 2 ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          uint64_t codes = hh ? ((qq[i][g] >> 4) & 0x0F0F0F0F0F0F0F0Full) : (qq[i][g] & 0x0F0F0F0F0F0F0F0Full);
          // Q5_K: sub-block 2g + hh takes bit 2g + hh of each qh byte as 16
          if constexpr (Q == kQ5_K) codes |= ((qhq[i] >> (2 * g + hh)) & 0x0101010101010101ull) << 4;
          const long A1 = *reinterpret_cast<const long*>(la + (2 * g + hh) * kMbBlkStride);
          const long A2 = *reinterpret_cast<const long*>(lc + (2 * g + hh) * kMbBlkStride);
          const i32x4v I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A1, long(codes), i32x4v{}, 0, 0, 0);
          const i32x4v I2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A2, long(codes), i32x4v{}, 0, 0, 0);
          const int scj = int((hh ? (scp >> 8) : scp) & 0xFFu);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // |integer dot| <= 31 * 32 * 128 and sc <= 63: 24-bit operands
            i1[k] = __mul24(I1[k], scj) + i1[k];
            i2[k] = __mul24(I2[k], scj) + i2[k];
          }
        }
      }
      // min term: m_j of sub-blocks kg (scale byte 4 + kg, low 6 bits) and
      // 4 + kg (high nibble of byte 8 + kg, top bits of byte 4 + kg)
      const uint32_t zb = h.z >> (8 * kg), wb = h.w >> (8 * kg);
      const float m_lo = float(zb & 0x3Fu);
      const float m_hi = float(((wb >> 4) & 0x0Fu) | (((zb >> 6) & 0x3u) << 4));
      const float sx_lo = sx[(8 * sb + kg) * kMbMaxVec + vec_a];
      const float sx_hi = sx[(8 * sb + 4 + kg) * kMbMaxVec + vec_a];
      f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_lo, m_lo, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      mn = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_hi, m_hi, mn, 0, 0, 0);
      // the b sums from the lanes 32 apart; |a|, |b|, |c| sums <= 8 * 63 * 126976
      // < 2^26: f32 conversions within an ulp
      int ib[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) ib[k] = __shfl_xor(i1[k], 32, kWave);
      const float d = h2f(h.x), dm = h2f(h.x >> 16);
      const f32x4 pk4 = *reinterpret_cast<const f32x4*>(pk8 + sb * kMbMaxVec + tok_d);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float f = __builtin_fmaf(float(i1[k]), 65536.f, __builtin_fmaf(float(ib[k]), 256.f, float(i2[k])));
        const float t = __builtin_fmaf(-dm, mn[k], __builtin_fmaf(f, d * pk4[k], acc[k]));
        acc[k] = live ? t : acc[k];
      }
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
    // The partial sums are agent-scope atomic stores, which complete at the
    // device's coherence point; the wait makes every wave's stores complete
    // before the barrier, so they are visible device-wide before the count.
    // (A release on the count, which the memory model would ask for instead,
    // writes back the whole L2 on gfx950: measured 18 -> 30 us per launch at
    // 4096x12288, batch 8.)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(count + rtb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_last != uint32_t(nwin - 1)) return;
    // The last workgroup of the row block: the windows' sums in window
    // order. Its loads are agent-scope atomic loads (global_load sc1, which
    // read at the device's coherence point rather than from a possibly
    // stale line of this XCD's L2) and are issued only after the count's
    // value has come back, i.e. after every other window's stores have
    // completed. An acquire fence (buffer_inv sc1) would invalidate the
    // XCD's L2 under the other workgroups still streaming there: measured
    // 18 -> 30 us per launch at 4096x12288, batch 8.
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
                      int batch, int T, int S, int wc, size_t lds, const uint8_t* ws, float* part, uint32_t* count,
                      hipStream_t s) {
  const int64_t nwin = (cols + wc - 1) / wc;
  const unsigned blocks = unsigned((rows + 16 * T - 1) / (16 * T) * (SPLIT ? nwin : 1));
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  const int64_t rb = byte_size(quant, cols);
  const bool one = cols <= wc;
  const dim3 grid = dim3(blocks), block = dim3(unsigned(64 * T * S));
  if (quant == kQ5_K) {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, true, PREP, false>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, wc, ws, part, count);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, false, PREP, SPLIT>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, wc, ws, part, count);
  } else {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, true, PREP, false>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, wc, ws, part, count);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, false, PREP, SPLIT>), grid, block, lds, s, w, int(rows),
                         int(cols), rb, x, y, batch, T, S, wc, ws, part, count);
  }
}

template <bool PREP, bool SPLIT>
static void launch_mb_per(int per, uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x,
                          float* y, int batch, int T, int S, int wc, size_t lds, const uint8_t* ws, float* part,
                          uint32_t* count, hipStream_t s) {
  switch (per) {
    case 1: launch_mb<1, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
    case 2: launch_mb<2, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
    case 3: launch_mb<3, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
    case 4: launch_mb<4, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
    case 5: launch_mb<5, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
    default: launch_mb<6, PREP, SPLIT>(quant, wv, rows, cols, x, y, batch, T, S, wc, lds, ws, part, count, s); break;
  }
}

// The launch shape: window width wc, T row tiles and S super-block shares
// per workgroup (12 waves for 3 or 4 tiles, 8 otherwise: one workgroup per
// CU, the activations' LDS allowing no more), PER super-blocks a wave. Of
// the window widths, the one whose waves run the fewest super-blocks one
// after another (rounds of workgroups over the CUs times PER) wins; the
// first listed on a tie. Without a workspace the windows are the widest
// and taken in turn by each workgroup.
struct MbShape {
  int wc, T, S, per;
  bool split;
};
static MbShape mb_shape(int64_t rows, int64_t cols, int cu, bool ws) {
  MbShape best{};
  int64_t best_score = -1;
  for (int wc : kMbWindows) {
    if (!ws && wc != kMbMaxCols) continue;
    const int64_t w = cols < wc ? cols : wc;
    const int64_t nwin = (cols + w - 1) / w;
    const bool split = ws && nwin > 1;
    const int64_t slots = split ? (cu / nwin > 0 ? cu / nwin : 1) : cu;
    int T = int((rows + 16LL * slots - 1) / (16LL * slots));
    if (T < 1) T = 1;
    if (T > 4) T = 4;
    if (!ws && T > 3) T = 3;  // the conversion's x in registers beside the weights: at most 4 super-blocks a wave
    const int S = T >= 3 ? kMbMaxWaves / T : 8 / T;
    const int per = int((w / 256 + S - 1) / S);  // <= 6: a window is <= 4096 columns and S >= 3
    const int64_t nwg = (rows + 16 * T - 1) / (16 * T) * (split ? nwin : 1);
    const int64_t score = (nwg + cu - 1) / cu * per * (split ? 1 : nwin);
    if (best_score < 0 || score < best_score) {
      best = {int(w), T, S, per, split};
      best_score = score;
    }
  }
  return best;
}

hipError_t launch_gemv_mfma(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x, float* y,
                            int batch, int cu, hipStream_t s, void* ws) {
  if (!gemv_mfma_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  if (ws && (reinterpret_cast<uintptr_t>(ws) & 255u)) return hipErrorInvalidValue;
  const MbShape sh = mb_shape(rows, cols, cu, ws != nullptr);
  const int T = sh.T, S = sh.S, wc = sh.wc;
  const int nblk = wc / 32;
  const size_t lds = size_t(mb_win_alloc(nblk)) + sizeof(float) * T * S * 64 * 4;
  if (ws) {
    // the activations converted once for every workgroup (and the split-K
    // counters cleared)
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    uint32_t* count = reinterpret_cast<uint32_t*>(wsb);
    float* part = reinterpret_cast<float*>(wsb + mb_counters_bytes(rows));
    const uint8_t* img = wsb + mb_counters_bytes(rows) + mb_part_bytes(rows, cols, wc);
    const int n_count = int((rows + 16 * T - 1) / (16 * T));
    const int64_t n = std::max<int64_t>(int64_t(batch) * (cols / 256) * 64, n_count);  // a wave per super-block
    hipLaunchKernelGGL(mb_prep_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, int(cols), wc, batch,
                       const_cast<uint8_t*>(img), count, n_count);
    if (sh.split)
      launch_mb_per<true, true>(sh.per, quant, wv, rows, cols, x, y, batch, T, S, wc, lds, img, part, count, s);
    else
      launch_mb_per<true, false>(sh.per, quant, wv, rows, cols, x, y, batch, T, S, wc, lds, img, nullptr, nullptr, s);
  } else {
    launch_mb_per<false, false>(sh.per, quant, wv, rows, cols, x, y, batch, T, S, wc, lds, nullptr, nullptr, nullptr,
                                s);
  }
  return hipGetLastError();
}

}  // namespace sh
