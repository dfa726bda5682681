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
// Lane l of a wave holds, in D, weight row l % 16 for vectors
// 4 * ((l / 16) & 1) + i, i < 4: the a and c sums in lanes 0-31, the b sums
// in lanes 32-63.
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

typedef int i32x4v __attribute__((ext_vector_type(4)));

constexpr int kMbMaxVec = 8;            // vectors per call
constexpr int kMbTokStride = 40;        // LDS bytes per (limb, block, vector): 32 codes + 8 pad
constexpr int kMbMaxCols = 4096;        // columns per window: their limbs fit LDS with the rest

__host__ __device__ inline int mb_limb_bytes(int nblk) { return 3 * nblk * kMbMaxVec * kMbTokStride; }

constexpr int kMbMaxWaves = 12;  // waves per workgroup (T * S)

// Q: kQ4_K (144-byte super-blocks, codes at byte 16) or kQ5_K (176 bytes:
// qh at 16, codes at 48). ONE: the row is a single window (cols <= 4096),
// which lets the compiler drop the window loop.
template <int Q, int PER, bool ONE>
__global__ void __launch_bounds__(64 * kMbMaxWaves)
    gemv_mfma_kq_kernel(const uint8_t* __restrict__ w, int rows, int cols, int64_t row_bytes,
                        const float* __restrict__ x, float* __restrict__ y, int nb, int T, int S) {
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

  // ---- this wave's row tile and super-block share
  const int rt = wave % T, sh_ = wave / T;
  const int r16 = lane & 15, kg = lane >> 4;  // B column (weight row) and k group
  const int row = min(blockIdx.x * (16 * T) + 16 * rt + r16, rows - 1);
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
  for (int c0 = 0; c0 < (ONE ? 1 : cols); c0 += kMbMaxCols) {
    const int nblk_w = ONE ? nblk : min(cols - c0, kMbMaxCols) >> 5, nsb_w = nblk_w >> 3;
    if (c0 > 0) __syncthreads();  // every wave is done with the previous window's limbs
    // ---- activations -> limbs: one (vector, block) pair per thread per round;
    // the 8 blocks of a super-block are 8 adjacent lanes (nblk_w and the
    // workgroup size are multiples of 8), which share its maximum
    float* pk8 = pk;  // [nsb_w][8]: 2^-k of (super-block, vector)
    for (int p = tid; p < nb * nblk_w; p += nthreads) {
      const int b = p / nblk_w, j = p - b * nblk_w;
      const f32x4* src = reinterpret_cast<const f32x4*>(x + int64_t(b) * cols + c0 + 32 * j);
      float v[32];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const f32x4 t = src[k];
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
      m = fmaxf(m, __shfl_xor(m, 1, kWave));
      m = fmaxf(m, __shfl_xor(m, 2, kWave));
      m = fmaxf(m, __shfl_xor(m, 4, kWave));
      int e = 0;
      (void)frexpf(m, &e);
      const int kk = m > 0.f ? min(22 - e, 126) : 0;
      const float up = ldexpf(1.f, kk);
      if ((j & 7) == 0) pk8[(j >> 3) * kMbMaxVec + b] = (m - m == 0.f) ? ldexpf(1.f, -kk) : __builtin_nanf("");
      sx[j * kMbMaxVec + b] = s;
      uint32_t wa[8], wb[8], wc[8];
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
    const int r = blockIdx.x * (16 * T) + 16 * rt + r16;
    if (r < rows) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (d_out && tok_d + i < nb) y[int64_t(tok_d + i) * rows + r] = t[i];
    }
  }
}

bool gemv_mfma_ok(uint32_t quant, int64_t rows, int64_t cols, int batch) {
  return (quant == kQ4_K || quant == kQ5_K) && batch >= 2 && batch <= kMbMaxVec && cols > 0 && cols % 256 == 0 &&
         cols <= (int64_t(1) << 20) && rows > 0 && rows <= (int64_t(1) << 31) - 1;
}

template <int PER>
static void launch_mb(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x, float* y,
                      int batch, int T, int S, size_t lds, hipStream_t s) {
  const unsigned blocks = unsigned((rows + 16 * T - 1) / (16 * T));
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  const int64_t rb = byte_size(quant, cols);
  const bool one = cols <= kMbMaxCols;
  if (quant == kQ5_K) {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, true>), dim3(blocks), dim3(64 * T * S), lds, s, w,
                         int(rows), int(cols), rb, x, y, batch, T, S);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ5_K, PER, false>), dim3(blocks), dim3(64 * T * S), lds, s, w,
                         int(rows), int(cols), rb, x, y, batch, T, S);
  } else {
    if (one)
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, true>), dim3(blocks), dim3(64 * T * S), lds, s, w,
                         int(rows), int(cols), rb, x, y, batch, T, S);
    else
      hipLaunchKernelGGL((gemv_mfma_kq_kernel<kQ4_K, PER, false>), dim3(blocks), dim3(64 * T * S), lds, s, w,
                         int(rows), int(cols), rb, x, y, batch, T, S);
  }
}

hipError_t launch_gemv_mfma(uint32_t quant, const void* wv, int64_t rows, int64_t cols, const float* x, float* y,
                            int batch, int cu, hipStream_t s) {
  if (!gemv_mfma_ok(quant, rows, cols, batch)) return hipErrorInvalidValue;
  // T row tiles per workgroup so the tiles cover the CUs about once; the
  // workgroup's waves (12 for 3 or 4 tiles, 8 otherwise: one workgroup per
  // CU, the activations' LDS allowing no more) split the super-blocks into
  // shares of PER <= 8
  int T = int((rows + 16LL * cu - 1) / (16LL * cu));
  if (T < 1) T = 1;
  if (T > 4) T = 4;
  const int S = T >= 3 ? kMbMaxWaves / T : 8 / T;
  const int64_t wcols = cols < kMbMaxCols ? cols : kMbMaxCols;  // one window of columns
  const int nsb = int(wcols / 256);
  const int per = (nsb + S - 1) / S;  // <= 8: a window is <= 4096 columns and S >= 2
  const int nblk = int(wcols / 32);
  const size_t lds = size_t(mb_limb_bytes(nblk)) + 2 * sizeof(float) * nblk * kMbMaxVec +
                     sizeof(float) * T * S * 64 * 4;
  switch (per) {
    case 1: launch_mb<1>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 2: launch_mb<2>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 3: launch_mb<3>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 4: launch_mb<4>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 5: launch_mb<5>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 6: launch_mb<6>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    case 7: launch_mb<7>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
    default: launch_mb<8>(quant, wv, rows, cols, x, y, batch, T, S, lds, s); break;
  }
  return hipGetLastError();
}

}  // namespace sh
