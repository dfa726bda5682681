/*
 * CPU oracle: plain-C restatement of the reference's scalar quantized
 * matvec path. TEST INFRASTRUCTURE ONLY -- see oracle.h. Build with
 * -O2 -ffp-contract=off (oracle/Makefile); never with -ffast-math.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- f16 <-> f32 -------------------------------------------------------
 * The reference converts with the `half` crate 2.7.1 (dequant.rs:34-36,
 * Cargo.lock:764-766): the exact IEEE binary16 -> binary32 widening; NaNs
 * come out quiet with the payload kept in the top mantissa bits.
 * Written here from the binary16 definition:
 *   normal    (-1)^s * 2^(e-15) * (1 + m/1024)
 *   subnormal (-1)^s * m * 2^-24                                        */
float sho_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
  uint32_t m = (uint32_t)h & 0x3FFu;
  float v;
  if (e == 0x1F) {
    uint32_t bits;
    if (m == 0) {
      bits = 0x7F800000u;
    } else {
      bits = 0x7FC00000u | (m << 13);
    }
    bits |= sign << 31;
    memcpy(&v, &bits, 4);
    return v;
  }
  if (e == 0) {
    v = ldexpf((float)m, -24); /* exact: m < 2^10 */
  } else {
    v = ldexpf((float)(1024u + m), (int)e - 25); /* exact */
  }
  return sign ? -v : v;
}

/* binary32 -> binary16, round to nearest even (half::f16::from_f32). Used
 * only by the synthetic block generators and the known-answer tests. */
uint16_t sho_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf or NaN */
    if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
  }
  float a;
  memcpy(&a, &ax, 4);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
  if (a < ldexpf(1.0f, -14)) {
    /* subnormal (or zero): value = k * 2^-24, k = rne(a * 2^24). The
     * scaling by 2^24 is exact; nearbyintf rounds half to even. */
    float k = nearbyintf(ldexpf(a, 24));
    return (uint16_t)(sign | (uint16_t)k); /* k == 1024 is the min normal */
  }
  int e;
  float fr = frexpf(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  /* significand with 11 bits: rne(fr * 2^11) in [1024, 2048] */
  float s = nearbyintf(ldexpf(fr, 11));
  int be = e - 1 + 15; /* biased exponent of 2^(e-1) */
  uint32_t si = (uint32_t)s;
  if (si == 2048u) {
    si = 1024u;
    be += 1;
  }
  if (be >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | (uint16_t)(be << 10) | (uint16_t)(si - 1024u));
}

/* bf16 round trip, round to nearest even (half::bf16::from_f32; used by the
 * router input rounding, hyper.rs:22-24). */
float sho_bf16_round(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) {
    x = (x | 0x00400000u) & 0xFFFF0000u;
  } else {
    uint32_t lsb = (x >> 16) & 1u;
    x = (x + 0x7FFFu + lsb) & 0xFFFF0000u;
  }
  float r;
  memcpy(&r, &x, 4);
  return r;
}

/* ---- geometry (quant.rs:125-181), for the types this path handles ------ */
int64_t sho_block_size(uint32_t quant) {
  switch (quant) {
    case SHO_F32:
    case SHO_F16:
    case SHO_BF16:
      return 1;
    case SHO_Q8_0:
      return 32;
    case SHO_Q4_K:
    case SHO_Q5_K:
    case SHO_Q6_K:
    case SHO_IQ4_XS:
      return 256;
    default:
      return -1;
  }
}

int64_t sho_type_size(uint32_t quant) {
  switch (quant) {
    case SHO_F32:
      return 4;
    case SHO_F16:
    case SHO_BF16:
      return 2;
    case SHO_Q8_0:
      return 34;
    case SHO_Q4_K:
      return 144;
    case SHO_Q5_K:
      return 176;
    case SHO_Q6_K:
      return 210;
    case SHO_IQ4_XS:
      return 136;
    default:
      return -1;
  }
}

/* n_blocks = ceil(n / block_size); byte_size = n_blocks * type_size. */
int64_t sho_byte_size(uint32_t quant, int64_t n_elements) {
  int64_t bs = sho_block_size(quant), ts = sho_type_size(quant);
  if (bs <= 0 || ts <= 0 || n_elements < 0) return -1;
  return ((n_elements + bs - 1) / bs) * ts;
}

static uint16_t rd16(const uint8_t* b) { return (uint16_t)(b[0] | (b[1] << 8)); }

/* ---- block decoders ----------------------------------------------------- */

/* dequant.rs:123-128: out[j] = (i8)q[j] as f32 * d. */
static void dq_q8_0(const uint8_t* b, float* out) {
  float d = sho_f16_to_f32(rd16(b));
  for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)b[2 + j] * d;
}

/* dequant.rs:237-245: the packed 6-bit (scale, min) of sub-block j. */
void sho_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* dequant.rs:247-270. d1 = d*sc and m1 = dmin*m are rounded to f32 first;
 * each output is (d1*q) - m1 with two roundings (no fused multiply-add). */
static void dq_q4_k(const uint8_t* b, float* out) {
  float d = sho_f16_to_f32(rd16(b));
  float mn = sho_f16_to_f32(rd16(b + 2));
  const uint8_t* scales = b + 4;
  const uint8_t* q = b + 16;
  for (int grp = 0; grp < 4; ++grp) {
    uint8_t sc, m;
    sho_get_scale_min_k4(2 * grp, scales, &sc, &m);
    float d1 = d * (float)sc;
    float m1 = mn * (float)m;
    sho_get_scale_min_k4(2 * grp + 1, scales, &sc, &m);
    float d2 = d * (float)sc;
    float m2 = mn * (float)m;
    const uint8_t* qq = q + 32 * grp;
    float* o = out + 64 * grp;
    for (int l = 0; l < 32; ++l) {
      float p1 = d1 * (float)(qq[l] & 0x0F);
      o[l] = p1 - m1;
      float p2 = d2 * (float)(qq[l] >> 4);
      o[32 + l] = p2 - m2;
    }
  }
}

/* dequant.rs:272-302. As Q4_K with a fifth bit: group g's low-nibble half
 * takes bit 2g of qh[l], its high-nibble half bit 2g + 1; the code q + 16h
 * (exact in f32) is scaled by d1 and m1 subtracted, two roundings. */
static void dq_q5_k(const uint8_t* b, float* out) {
  float d = sho_f16_to_f32(rd16(b));
  float mn = sho_f16_to_f32(rd16(b + 2));
  const uint8_t* scales = b + 4;
  const uint8_t* qh = b + 16;
  const uint8_t* ql = b + 48;
  for (int grp = 0; grp < 4; ++grp) {
    uint8_t sc, m;
    sho_get_scale_min_k4(2 * grp, scales, &sc, &m);
    float d1 = d * (float)sc;
    float m1 = mn * (float)m;
    sho_get_scale_min_k4(2 * grp + 1, scales, &sc, &m);
    float d2 = d * (float)sc;
    float m2 = mn * (float)m;
    const uint8_t u1 = (uint8_t)(1u << (2 * grp)), u2 = (uint8_t)(2u << (2 * grp));
    const uint8_t* qq = ql + 32 * grp;
    float* o = out + 64 * grp;
    for (int l = 0; l < 32; ++l) {
      float c1 = (float)(qq[l] & 0x0F) + ((qh[l] & u1) ? 16.0f : 0.0f);
      float p1 = d1 * c1;
      o[l] = p1 - m1;
      float c2 = (float)(qq[l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f);
      float p2 = d2 * c2;
      o[32 + l] = p2 - m2;
    }
  }
}

/* dequant.rs:208-234. Two halves of 128 elements; q = 6-bit code - 32 and
 * out = (d * sc) * q. The reference reads sc as u8 (F4); SHO_Q6K_SCALE_I8
 * gives ggml's int8_t reading for comparison. */
static void dq_q6_k(const uint8_t* b, float* out, int scale_mode) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const uint8_t* sc = b + 192;
  float d = sho_f16_to_f32(rd16(b + 208));
  for (int half = 0; half < 2; ++half) {
    const uint8_t* l0 = ql + 64 * half;
    const uint8_t* h0 = qh + 32 * half;
    const uint8_t* s0 = sc + 8 * half;
    float* o = out + 128 * half;
    for (int l = 0; l < 32; ++l) {
      int is = l / 16;
      int q1 = ((l0[l] & 0x0F) | ((h0[l] & 3) << 4)) - 32;
      int q2 = ((l0[l + 32] & 0x0F) | (((h0[l] >> 2) & 3) << 4)) - 32;
      int q3 = ((l0[l] >> 4) | (((h0[l] >> 4) & 3) << 4)) - 32;
      int q4 = ((l0[l + 32] >> 4) | (((h0[l] >> 6) & 3) << 4)) - 32;
      float s[4];
      for (int t = 0; t < 4; ++t) {
        uint8_t raw = s0[is + 2 * t];
        s[t] = scale_mode == SHO_Q6K_SCALE_I8 ? (float)(int8_t)raw : (float)raw;
      }
      float a;
      a = d * s[0];
      o[l] = a * (float)q1;
      a = d * s[1];
      o[l + 32] = a * (float)q2;
      a = d * s[2];
      o[l + 64] = a * (float)q3;
      a = d * s[3];
      o[l + 96] = a * (float)q4;
    }
  }
}

/* The IQ4_NL / IQ4_XS code book (a format table: ggml's kvalues_iq4nl,
 * crates/strata-gguf/src/tables.rs:2052-2054). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

/* dequant.rs:189-206. [d: f16][scales_h: u16][scales_l: 4 B][qs: 128 B];
 * sub-block ib (32 elements) has the 6-bit scale ls = low nibble ib % 2 of
 * scales_l[ib / 2] | bits 2ib..2ib+1 of scales_h << 4, dl = d * (ls - 32)
 * rounded once, and out = dl * code for the code book's value of each
 * nibble (low nibbles first, then high). Code bytes: the first 16 for every
 * sub-block (SHO_IQ4XS_REFERENCE) or bytes 16ib.. (SHO_IQ4XS_GGML). */
static void dq_iq4_xs(const uint8_t* b, float* out, int mode) {
  float d = sho_f16_to_f32(rd16(b));
  uint32_t sh = rd16(b + 2);
  const uint8_t* sl = b + 4;
  const uint8_t* qs = b + 8;
  for (int ib = 0; ib < 8; ++ib) {
    uint32_t ls = ((uint32_t)(sl[ib / 2] >> (4 * (ib % 2))) & 0x0Fu) | (((sh >> (2 * ib)) & 3u) << 4);
    float dl = d * ((float)ls - 32.0f);
    const uint8_t* q = mode == SHO_IQ4XS_GGML ? qs + 16 * ib : qs;
    for (int j = 0; j < 16; ++j) {
      out[32 * ib + j] = dl * (float)kIq4nl[q[j] & 0x0F];
      out[32 * ib + j + 16] = dl * (float)kIq4nl[q[j] >> 4];
    }
  }
}

static int dq_block(uint32_t quant, const uint8_t* b, float* out, int mode) {  /* mode: the Q6_K or IQ4_XS reading */
  switch (quant) {
    case SHO_F32:
      memcpy(out, b, 4);
      return SHO_OK;
    case SHO_F16:
      out[0] = sho_f16_to_f32(rd16(b));
      return SHO_OK;
    case SHO_BF16: {
      uint32_t bits = (uint32_t)rd16(b) << 16;
      memcpy(out, &bits, 4);
      return SHO_OK;
    }
    case SHO_Q8_0:
      dq_q8_0(b, out);
      return SHO_OK;
    case SHO_Q4_K:
      dq_q4_k(b, out);
      return SHO_OK;
    case SHO_Q5_K:
      dq_q5_k(b, out);
      return SHO_OK;
    case SHO_Q6_K:
      dq_q6_k(b, out, mode);
      return SHO_OK;
    case SHO_IQ4_XS:
      dq_iq4_xs(b, out, mode);
      return SHO_OK;
    default:
      return SHO_UNSUPPORTED;
  }
}

/* dequant.rs:45-61: Truncated when n is not a whole number of blocks or the
 * buffer is short; otherwise block by block. */
static int dequant_row_mode(uint32_t quant, const uint8_t* block, size_t nbytes,
                            float* out, size_t n, int mode) {
  int64_t bs = sho_block_size(quant), ts = sho_type_size(quant);
  if (bs <= 0) return SHO_UNSUPPORTED;
  size_t n_blocks = (n + (size_t)bs - 1) / (size_t)bs;
  if (n % (size_t)bs != 0 || nbytes < n_blocks * (size_t)ts) return SHO_TRUNCATED;
  for (size_t i = 0; i < n_blocks; ++i) {
    int rc = dq_block(quant, block + i * (size_t)ts, out + i * (size_t)bs, mode);
    if (rc) return rc;
  }
  return SHO_OK;
}

int sho_dequantize_row(uint32_t quant, const uint8_t* block, size_t nbytes,
                       float* out, size_t n) {
  return dequant_row_mode(quant, block, nbytes, out, n, SHO_Q6K_SCALE_U8);
}

int sho_dequantize_row_q6k_mode(const uint8_t* block, size_t nbytes, float* out,
                                size_t n, int scale_mode) {
  return dequant_row_mode(SHO_Q6_K, block, nbytes, out, n, scale_mode);
}

int sho_dequantize_row_mode(uint32_t quant, const uint8_t* block, size_t nbytes,
                            float* out, size_t n, int mode) {
  return dequant_row_mode(quant, block, nbytes, out, n, mode);
}

/* ---- gemv (ops.rs:14-28) -----------------------------------------------
 * For each row: dequantize into scratch, then a sequential f64 dot, cast to
 * f32 at the end. Rows [r0, r1) only, so the threaded variant reuses it. */
static int gemv_rows(uint32_t quant, int64_t r0, int64_t r1, int64_t cols,
                     const uint8_t* data, size_t nbytes, const float* x,
                     float* y, int mode) {
  int64_t rb = sho_byte_size(quant, cols);
  if (rb < 0) return SHO_UNSUPPORTED;
  float* row = (float*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(float));
  if (!row) return SHO_UNSUPPORTED;
  int rc = SHO_OK;
  for (int64_t r = r0; r < r1; ++r) {
    size_t off = (size_t)(r * rb);
    if (off + (size_t)rb > nbytes) {
      rc = SHO_TRUNCATED;
      break;
    }
    rc = dequant_row_mode(quant, data + off, (size_t)rb, row, (size_t)cols, mode);
    if (rc) break;
    double acc = 0.0;
    for (int64_t c = 0; c < cols; ++c) acc += (double)row[c] * (double)x[c];
    y[r] = (float)acc;
  }
  free(row);
  return rc;
}

int sho_gemv(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
             size_t nbytes, const float* x, float* y) {
  return gemv_rows(quant, 0, rows, cols, data, nbytes, x, y, SHO_Q6K_SCALE_U8);
}

int sho_gemv_mode(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
                  size_t nbytes, const float* x, float* y, int mode) {
  return gemv_rows(quant, 0, rows, cols, data, nbytes, x, y, mode);
}

int sho_gemv_q6k_mode(int64_t rows, int64_t cols, const uint8_t* data,
                      size_t nbytes, const float* x, float* y, int scale_mode) {
  return gemv_rows(SHO_Q6_K, 0, rows, cols, data, nbytes, x, y, scale_mode);
}

/* Row-parallel gemv: the same per-row arithmetic on n_threads threads, so
 * its output is bit-identical to sho_gemv. This is the all-cores CPU
 * baseline the reference's backend description promises
 * (crates/strata-backend-cpu/Cargo.toml:3) but never runs. */
typedef struct {
  uint32_t quant;
  int64_t r0, r1, cols;
  const uint8_t* data;
  size_t nbytes;
  const float* x;
  float* y;
  int mode;
  int rc;
} gemv_job;

static void* gemv_worker(void* p) {
  gemv_job* j = (gemv_job*)p;
  j->rc = gemv_rows(j->quant, j->r0, j->r1, j->cols, j->data, j->nbytes, j->x,
                    j->y, j->mode);
  return NULL;
}

static int gemv_threads_mode(uint32_t quant, int64_t rows, int64_t cols,
                             const uint8_t* data, size_t nbytes, const float* x,
                             float* y, int n_threads, int mode) {
  if (n_threads <= 1 || rows < 2) return gemv_rows(quant, 0, rows, cols, data, nbytes, x, y, mode);
  if (n_threads > 256) n_threads = 256;
  pthread_t th[256];
  int started[256];
  gemv_job jobs[256];
  int64_t per = (rows + n_threads - 1) / n_threads;
  int n_jobs = 0;
  for (int t = 0; t < n_threads; ++t) {
    int64_t r0 = t * per;
    if (r0 >= rows) break;
    int64_t r1 = r0 + per < rows ? r0 + per : rows;
    jobs[t] = (gemv_job){quant, r0, r1, cols, data, nbytes, x, y, mode, 0};
    started[t] = pthread_create(&th[t], NULL, gemv_worker, &jobs[t]) == 0;
    if (!started[t]) gemv_worker(&jobs[t]); /* could not start: run inline */
    ++n_jobs;
  }
  int rc = SHO_OK;
  for (int t = 0; t < n_jobs; ++t) {
    if (started[t]) pthread_join(th[t], NULL);
    if (jobs[t].rc) rc = jobs[t].rc;
  }
  return rc;
}

int sho_gemv_threads(uint32_t quant, int64_t rows, int64_t cols,
                     const uint8_t* data, size_t nbytes, const float* x,
                     float* y, int n_threads) {
  return gemv_threads_mode(quant, rows, cols, data, nbytes, x, y, n_threads, SHO_Q6K_SCALE_U8);
}

/* ---- expert_gemv (ops.rs:169-195) --------------------------------------
 * Expert-major [n_expert][rows = in][cols = out] (weights.rs:14-34):
 * acc[c] += x[i] * W_e[i][c] in f64 over input rows i, skipping x[i] == 0,
 * then cast to f32. */
int sho_expert_gemv_mode(uint32_t quant, int64_t n_expert, int64_t rows,
                         int64_t cols, const uint8_t* data, size_t nbytes,
                         int64_t e, const float* x, float* y, int mode) {
  int64_t rb = sho_byte_size(quant, cols);
  if (rb < 0) return SHO_UNSUPPORTED;
  if (e < 0 || e >= n_expert) return SHO_TRUNCATED;
  double* acc = (double*)calloc((size_t)(cols > 0 ? cols : 1), sizeof(double));
  float* row = (float*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(float));
  if (!acc || !row) {
    free(acc);
    free(row);
    return SHO_UNSUPPORTED;
  }
  int rc = SHO_OK;
  size_t base = (size_t)(e * rows * rb);
  for (int64_t i = 0; i < rows; ++i) {
    double xi = (double)x[i];
    if (xi == 0.0) continue;
    size_t off = base + (size_t)(i * rb);
    if (off + (size_t)rb > nbytes) {
      rc = SHO_TRUNCATED;
      break;
    }
    rc = sho_dequantize_row_mode(quant, data + off, (size_t)rb, row, (size_t)cols, mode);
    if (rc) break;
    for (int64_t c = 0; c < cols; ++c) acc[c] += xi * (double)row[c];
  }
  if (rc == SHO_OK)
    for (int64_t c = 0; c < cols; ++c) y[c] = (float)acc[c];
  free(acc);
  free(row);
  return rc;
}

int sho_expert_gemv(uint32_t quant, int64_t n_expert, int64_t rows,
                    int64_t cols, const uint8_t* data, size_t nbytes,
                    int64_t e, const float* x, float* y) {
  return sho_expert_gemv_mode(quant, n_expert, rows, cols, data, nbytes, e, x, y, 0);
}

/* ops.rs:85-87 */
float sho_silu(float x) { return x / (1.0f + expf(-x)); }

/* ---- MoE routing (moe.rs:58-90), from the router logits ---------------
 * softmax: max-shift, f32 exp, f64 sum, inv = (f32)(1/sum), p *= inv;
 * top-k by descending p, ties by ascending id; ids returned ascending;
 * weights renormalised as (f32)((f64)p / max(sum_f64, 2^-14)).
 * Returns k = min(top_k, n_expert). */
static const float* g_rank_p;
static int rank_cmp(const void* a, const void* b) {
  int64_t ia = *(const int64_t*)a, ib = *(const int64_t*)b;
  float pa = g_rank_p[ia], pb = g_rank_p[ib];
  if (pa > pb) return -1;
  if (pa < pb) return 1;
  return ia < ib ? -1 : (ia > ib ? 1 : 0);
}
static int id_cmp(const void* a, const void* b) {
  int64_t ia = *(const int64_t*)a, ib = *(const int64_t*)b;
  return ia < ib ? -1 : (ia > ib ? 1 : 0);
}

int sho_moe_route(const float* logits, int64_t n_expert, int64_t top_k,
                  int64_t* ids, float* weights) {
  if (n_expert <= 0 || top_k <= 0) return 0;
  float* p = (float*)malloc((size_t)n_expert * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)n_expert * sizeof(int64_t));
  float mx = -INFINITY;
  for (int64_t i = 0; i < n_expert; ++i) mx = fmaxf(mx, logits[i]);
  double sum = 0.0;
  for (int64_t i = 0; i < n_expert; ++i) {
    p[i] = expf(logits[i] - mx);
    sum += (double)p[i];
  }
  float inv = (float)(1.0 / sum);
  for (int64_t i = 0; i < n_expert; ++i) p[i] *= inv;
  for (int64_t i = 0; i < n_expert; ++i) idx[i] = i;
  int64_t k = top_k < n_expert ? top_k : n_expert;
  g_rank_p = p; /* the comparator is a total order: the k-set is unique */
  qsort(idx, (size_t)n_expert, sizeof(int64_t), rank_cmp);
  qsort(idx, (size_t)k, sizeof(int64_t), id_cmp);
  double ws = 0.0;
  for (int64_t j = 0; j < k; ++j) {
    ids[j] = idx[j];
    weights[j] = p[idx[j]];
    ws += (double)weights[j];
  }
  double s = ws > ldexp(1.0, -14) ? ws : ldexp(1.0, -14);
  for (int64_t j = 0; j < k; ++j) weights[j] = (float)((double)weights[j] / s);
  free(p);
  free(idx);
  return (int)k;
}

/* ---- routed combine (moe.rs:108-127) -----------------------------------
 * For each selected expert in the given (ascending) order with w != 0:
 *   h = gate_e . x, p = up_e . x, h = silu(h) * p, d = down_e . h,
 *   out += w * d   (f32, product then sum).
 * gate/up: [n_expert][n_embd][n_ff]; down: [n_expert][n_ff][n_embd].
 * out (n_embd) is overwritten. The shared expert (moe.rs:129-143) is not
 * part of this op. */
/* One expert's matvec in either orientation: in-major [n_expert][in][out]
 * through ops::expert_gemv (the reference's), or out-major
 * [n_expert][out][in] (llama.cpp's expert stacks) as ops::gemv of the
 * expert's [out][in] slice. */
static int expert_apply(uint32_t quant, int64_t n_expert, int64_t n_in, int64_t n_out, const uint8_t* data,
                        size_t nbytes, int64_t e, const float* x, float* y, int out_major, int mode) {
  if (!out_major) return sho_expert_gemv_mode(quant, n_expert, n_in, n_out, data, nbytes, e, x, y, mode);
  int64_t rb = sho_byte_size(quant, n_in);
  if (rb < 0) return SHO_UNSUPPORTED;
  if (e < 0 || e >= n_expert) return SHO_TRUNCATED;
  size_t off = (size_t)(e * n_out * rb);
  if (off > nbytes) return SHO_TRUNCATED;
  return gemv_rows(quant, 0, n_out, n_in, data + off, nbytes - off, x, y, mode);
}

/* moe.rs:108-127 for one token: for each selected expert j with w != 0 (in
 * the order given, ascending id): h = gate_e . x, p = up_e . x,
 * h = silu(h) * p, d = down_e . h, out += w * d (f32 product, then sum). */
int sho_moe_routed_m(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                     int64_t n_expert, int64_t n_embd, int64_t n_ff,
                     const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                     size_t up_bytes, const uint8_t* down, size_t down_bytes,
                     const int64_t* ids, const float* weights, int64_t k,
                     const float* x, float* out, int out_major, const int* modes) {
  const int mg = modes ? modes[0] : 0, mu = modes ? modes[1] : 0, md = modes ? modes[2] : 0;
  float* h = (float*)malloc((size_t)n_ff * sizeof(float));
  float* part = (float*)malloc((size_t)n_ff * sizeof(float));
  float* d = (float*)malloc((size_t)n_embd * sizeof(float));
  int rc = SHO_OK;
  for (int64_t i = 0; i < n_embd; ++i) out[i] = 0.0f;
  for (int64_t j = 0; j < k && rc == SHO_OK; ++j) {
    float w = weights[j];
    if (w == 0.0f) continue;
    int64_t e = ids[j];
    rc = expert_apply(gate_quant, n_expert, n_embd, n_ff, gate, gate_bytes, e, x, h, out_major, mg);
    if (rc) break;
    rc = expert_apply(up_quant, n_expert, n_embd, n_ff, up, up_bytes, e, x, part, out_major, mu);
    if (rc) break;
    for (int64_t i = 0; i < n_ff; ++i) h[i] = sho_silu(h[i]) * part[i];
    rc = expert_apply(down_quant, n_expert, n_ff, n_embd, down, down_bytes, e, h, d, out_major, md);
    if (rc) break;
    for (int64_t i = 0; i < n_embd; ++i) {
      float t = w * d[i];
      out[i] = out[i] + t;
    }
  }
  free(h);
  free(part);
  free(d);
  return rc;
}

int sho_moe_routed_o(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                     int64_t n_expert, int64_t n_embd, int64_t n_ff,
                     const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                     size_t up_bytes, const uint8_t* down, size_t down_bytes,
                     const int64_t* ids, const float* weights, int64_t k,
                     const float* x, float* out, int out_major) {
  return sho_moe_routed_m(gate_quant, up_quant, down_quant, n_expert, n_embd, n_ff, gate, gate_bytes, up,
                          up_bytes, down, down_bytes, ids, weights, k, x, out, out_major, NULL);
}

int sho_moe_routed(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                   int64_t n_expert, int64_t n_embd, int64_t n_ff,
                   const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                   size_t up_bytes, const uint8_t* down, size_t down_bytes,
                   const int64_t* ids, const float* weights, int64_t k,
                   const float* x, float* out) {
  return sho_moe_routed_o(gate_quant, up_quant, down_quant, n_expert, n_embd, n_ff, gate, gate_bytes, up,
                          up_bytes, down, down_bytes, ids, weights, k, x, out, 0);
}

/* ops.rs:90-92 */
float sho_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ---- the whole MoE layer for one token (moe.rs:48-143) -----------------
 * route:   x_bf = bf16(x) (hyper.rs:22-24), logits = router . x_bf
 *          (ops::gemv), then sho_moe_route;
 * combine: the routed experts (sho_moe_routed), then the shared expert
 *          g = gate_sh . x, p = up_sh . x, h = silu(g) * p, d = down_sh . h,
 *          s = gate_inp . x, out += sigmoid(s) * d (f32, product then sum).
 * router [n_expert][n_embd], gate_sh / up_sh [n_ff_sh][n_embd], down_sh
 * [n_embd][n_ff_sh], gate_inp [1][n_embd] (ops::gemv orientation).
 * q[8]: the types of router, gate, up, down, gate_sh, up_sh, down_sh,
 * gate_inp; t[8] / nb[8] their bytes. out (n_embd) is overwritten. */
int sho_moe_layer_m(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                    int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                    float* out, int out_major, const int* modes) {
  int md[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (modes)
    for (int i = 0; i < 8; ++i) md[i] = modes[i];
  float* xb = (float*)malloc((size_t)n_embd * sizeof(float));
  float* logits = (float*)malloc((size_t)n_expert * sizeof(float));
  int64_t* ids = (int64_t*)malloc((size_t)top_k * sizeof(int64_t));
  float* w = (float*)malloc((size_t)top_k * sizeof(float));
  float* g = (float*)malloc((size_t)n_ff_sh * sizeof(float));
  float* part = (float*)malloc((size_t)n_ff_sh * sizeof(float));
  float* d = (float*)malloc((size_t)n_embd * sizeof(float));
  float s = 0.0f;
  int rc = SHO_OK;
  for (int64_t i = 0; i < n_embd; ++i) xb[i] = sho_bf16_round(x[i]);
  rc = sho_gemv_mode(q[0], n_expert, n_embd, t[0], nb[0], xb, logits, md[0]);
  int64_t k = 0;
  if (rc == SHO_OK) {
    k = sho_moe_route(logits, n_expert, top_k, ids, w);
    rc = sho_moe_routed_m(q[1], q[2], q[3], n_expert, n_embd, n_ff, t[1], nb[1], t[2], nb[2], t[3], nb[3],
                          ids, w, k, x, out, out_major, md + 1);
  }
  if (rc == SHO_OK) rc = sho_gemv_mode(q[4], n_ff_sh, n_embd, t[4], nb[4], x, g, md[4]);
  if (rc == SHO_OK) rc = sho_gemv_mode(q[5], n_ff_sh, n_embd, t[5], nb[5], x, part, md[5]);
  if (rc == SHO_OK) {
    for (int64_t i = 0; i < n_ff_sh; ++i) g[i] = sho_silu(g[i]) * part[i];
    rc = sho_gemv_mode(q[6], n_embd, n_ff_sh, t[6], nb[6], g, d, md[6]);
  }
  if (rc == SHO_OK) rc = sho_gemv_mode(q[7], 1, n_embd, t[7], nb[7], x, &s, md[7]);
  if (rc == SHO_OK) {
    const float gate = sho_sigmoid(s);
    for (int64_t i = 0; i < n_embd; ++i) {
      float v = gate * d[i];
      out[i] = out[i] + v;
    }
  }
  free(xb);
  free(logits);
  free(ids);
  free(w);
  free(g);
  free(part);
  free(d);
  return rc;
}

int sho_moe_layer_o(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                    int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                    float* out, int out_major) {
  return sho_moe_layer_m(q, t, nb, n_expert, n_embd, n_ff, n_ff_sh, top_k, x, out, out_major, NULL);
}

int sho_moe_layer(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                  int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                  float* out) {
  return sho_moe_layer_o(q, t, nb, n_expert, n_embd, n_ff, n_ff_sh, top_k, x, out, 0);
}

int sho_matmul_mode(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
                    size_t nbytes, const float* x, int64_t m, float* y, int n_threads, int mode) {
  if (m < 0) return SHO_UNSUPPORTED;
  for (int64_t t = 0; t < m; ++t) {
    int rc = gemv_threads_mode(quant, rows, cols, data, nbytes, x + t * cols, y + t * rows, n_threads, mode);
    if (rc != SHO_OK) return rc;
  }
  return SHO_OK;
}

int sho_matmul(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
               size_t nbytes, const float* x, int64_t m, float* y, int n_threads) {
  return sho_matmul_mode(quant, rows, cols, data, nbytes, x, m, y, n_threads, SHO_Q6K_SCALE_U8);
}

int sho_quantize_q8(const float* x, size_t n, int8_t* q, float* scales,
                    float* sums) {
  if (n % 32 != 0) return SHO_TRUNCATED;
  for (size_t b = 0; b < n / 32; ++b) {
    const float* v = x + 32 * b;
    float amax = 0.0f;
    for (int k = 0; k < 32; ++k) {
      const float a = fabsf(v[k]);
      if (a > amax) amax = a;
    }
    const float s = amax / 127.0f;
    int sum = 0;
    for (int k = 0; k < 32; ++k) {
      const int c = s > 0.0f ? (int)rintf(v[k] / s) : 0;
      q[32 * b + k] = (int8_t)c;
      sum += c;
    }
    scales[b] = s;
    sums[b] = s * (float)sum;
  }
  return SHO_OK;
}

int sho_quantize_q8k(const float* x, size_t n, int8_t* q, float* scales,
                     int32_t* sums) {
  if (n % 256 != 0) return SHO_TRUNCATED;
  for (size_t b = 0; b < n / 256; ++b) {
    const float* v = x + 256 * b;
    float amax = 0.0f;
    for (int k = 0; k < 256; ++k) {
      const float a = fabsf(v[k]);
      if (a > amax) amax = a;
    }
    const float s = amax / 127.0f;
    for (int j = 0; j < 8; ++j) {
      int sum = 0;
      for (int k = 32 * j; k < 32 * j + 32; ++k) {
        const int c = s > 0.0f ? (int)rintf(v[k] / s) : 0;
        q[256 * b + k] = (int8_t)c;
        sum += c;
      }
      sums[8 * b + j] = sum;
    }
    scales[b] = s;
  }
  return SHO_OK;
}

/* ---- the trait's elementwise methods (backend.rs:38-50, ops.rs:46-165) --
 * f64 where the reference works in f64; the sums run in its sequential
 * order. pow / sin / cos are the C library's, as Rust's f64::powf and
 * f64::sin_cos call the platform libm. */

/* ops.rs:46-69 (rms_norm, rms_norm_into): ss = sum v*v (f64) / n,
 * scale = 1 / sqrt(ss + eps), out[i] = (f32)((f64)x[i] * scale * (f64)w[i]).
 * out may equal x. */
void sho_rms_norm(const float* x, const float* w, size_t n, double eps, float* out) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  ss /= (double)n;
  const double scale = 1.0 / sqrt(ss + eps);
  for (size_t i = 0; i < n; ++i) out[i] = (float)((double)x[i] * scale * (double)w[i]);
}

/* ops.rs:73-82: inv = 1 / sqrt(sum v*v + eps); v = (f32)((f64)v * inv). */
void sho_l2_norm(float* head, size_t n, double eps) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)head[i] * (double)head[i];
  const double inv = 1.0 / sqrt(ss + eps);
  for (size_t i = 0; i < n; ++i) head[i] = (float)((double)head[i] * inv);
}

/* ops.rs:105-116: mx = max (f32, from -inf), v = expf(v - mx) in f32,
 * sum in f64, inv = 1 / sum, v = (f32)((f64)v * inv). */
void sho_softmax(float* xs, size_t n) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, xs[i]);
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    xs[i] = expf(xs[i] - mx);
    sum += (double)xs[i];
  }
  const double inv = 1.0 / sum;
  for (size_t i = 0; i < n; ++i) xs[i] = (float)((double)xs[i] * inv);
}

/* ops.rs:120-135: r = min(n_rot, head_dim, len) & ~1, half = r / 2; pair
 * (i, i + half): theta = freq_base^(-2i / r), angle = theta * pos,
 * a' = (f32)(a cos - b sin), b' = (f32)(a sin + b cos), all f64; dims from
 * r on pass through. */
void sho_rope_neox(float* head, size_t len, uint64_t pos, size_t n_rot, size_t head_dim,
                   double freq_base) {
  size_t r = n_rot < head_dim ? n_rot : head_dim;
  if (len < r) r = len;
  r &= ~(size_t)1;
  const size_t half = r / 2;
  const double p = (double)pos;
  for (size_t i = 0; i < half; ++i) {
    const double theta = pow(freq_base, -2.0 * (double)i / (double)r);
    const double angle = theta * p;
    const double s = sin(angle), c = cos(angle);
    const double a = head[i], b = head[i + half];
    head[i] = (float)(a * c - b * s);
    head[i + half] = (float)(a * s + b * c);
  }
}

/* ops.rs:161-165 (add_into): a[i] += b[i] in f32. */
void sho_add(float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) a[i] = a[i] + b[i];
}

/* ---- the dense FFN half of a layer (qwen35.rs:112-129), one token ----------
 * mixed = rms_norm_into(x, post_norm, eps); g = gate . mixed; u = up . mixed;
 * h[i] = g[i] / (1 + expf(-g[i])) * u[i] (f32); m = down . h; out = x + m
 * (f32). gate / up [n_ff][n_embd], down [n_embd][n_ff]. out may equal x. */
int sho_dense_ffn(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_embd, int64_t n_ff,
                  const float* x, const float* post_norm, double eps, float* out) {
  float* mixed = malloc(sizeof(float) * (size_t)n_embd);
  float* g = malloc(sizeof(float) * (size_t)n_ff);
  float* u = malloc(sizeof(float) * (size_t)n_ff);
  float* m = malloc(sizeof(float) * (size_t)n_embd);
  int rc = (mixed && g && u && m) ? SHO_OK : SHO_TRUNCATED;
  if (rc == SHO_OK) {
    sho_rms_norm(x, post_norm, (size_t)n_embd, eps, mixed);
    rc = sho_gemv(q[0], n_ff, n_embd, t[0], nb[0], mixed, g);
  }
  if (rc == SHO_OK) rc = sho_gemv(q[1], n_ff, n_embd, t[1], nb[1], mixed, u);
  if (rc == SHO_OK) {
    for (int64_t i = 0; i < n_ff; ++i) {
      const float gv = g[i];
      g[i] = gv / (1.0f + expf(-gv)) * u[i];
    }
    rc = sho_gemv(q[2], n_embd, n_ff, t[2], nb[2], g, m);
  }
  if (rc == SHO_OK)
    for (int64_t i = 0; i < n_embd; ++i) out[i] = x[i] + m[i];
  free(mixed);
  free(g);
  free(u);
  free(m);
  return rc;
}
