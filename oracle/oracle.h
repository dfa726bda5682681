/*
 * CPU oracle for the quantized-weight matvec/matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links this file;
 * only the tests, the smoke check and the CPU-baseline leg of the benchmark
 * load it, and only as the checker / the timed CPU reference.
 *
 * It restates, in plain C, the reference's scalar CPU path:
 *   - block geometry          crates/strata-gguf/src/quant.rs:125-181
 *   - f16 -> f32, row dequant crates/strata-gguf/src/dequant.rs:28-61,123-128,189-206,208-302
 *   - gemv / expert_gemv      crates/strata-core/src/ops.rs:14-28,169-195
 *   - silu                    crates/strata-core/src/ops.rs:85-87
 *   - MoE route / combine     crates/strata-core/src/moe.rs:48-127
 *   - the whole MoE layer     crates/strata-core/src/moe.rs:48-143 (router
 *                             matvec on bf16(x), shared expert, sigmoid gate)
 *   - dense FFN half      crates/strata-core/src/qwen35.rs:112-129
 *   - rms_norm, l2_norm, softmax, rope_neox, add
 *                             crates/strata-core/src/ops.rs:46-165 (the
 *                             trait's elementwise methods, backend.rs:38-50)
 *   - prefill matmul          no reference op: m independent ops::gemv calls
 *                             (crates/strata-core/src/generate.rs:116-117)
 *   - Q8 activation blocks    the quantization the int8 prefill mode applies
 *                             to activations (32 elements, scale max|x|/127,
 *                             codes rounded to nearest even)
 * Compiled with -ffp-contract=off and no fast-math so every f32 product and
 * difference rounds exactly as the Rust source (which never fuses), and the
 * f64 dot products are summed in the same sequential order.
 */
#ifndef STRATA_ORACLE_H
#define STRATA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Strata QuantType ids (crates/strata-gguf/src/quant.rs:15-43). */
enum {
  SHO_F32 = 0,
  SHO_F16 = 1,
  SHO_Q8_0 = 8,
  SHO_Q4_K = 12,
  SHO_Q5_K = 13,
  SHO_Q6_K = 14,
  SHO_IQ4_XS = 23,
  SHO_BF16 = 30,
};

/* Status codes. */
enum {
  SHO_OK = 0,
  SHO_TRUNCATED = -1,   /* dequant.rs:50-55 Error::Truncated */
  SHO_UNSUPPORTED = -2, /* quant.rs:47-80 Error::UnsupportedQuant */
};

/* Q6_K sub-block scale semantics: the reference reads the 16 scale bytes as
 * u8 (dequant.rs:211,224-227); ggml declares them int8_t. */
enum { SHO_Q6K_SCALE_U8 = 0, SHO_Q6K_SCALE_I8 = 1 };

/* IQ4_XS code bytes: the reference reads the first 16 qs bytes for every
 * 32-element sub-block (dequant.rs:194-204, `qs` is never advanced); ggml's
 * dequantize_row_iq4_xs advances 16 bytes per sub-block. */
enum { SHO_IQ4XS_REFERENCE = 0, SHO_IQ4XS_GGML = 1 };

float sho_f16_to_f32(uint16_t h);
uint16_t sho_f32_to_f16(float f);
float sho_bf16_round(float f);

int64_t sho_block_size(uint32_t quant);
int64_t sho_type_size(uint32_t quant);
int64_t sho_byte_size(uint32_t quant, int64_t n_elements);

void sho_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);

int sho_dequantize_row(uint32_t quant, const uint8_t* block, size_t nbytes,
                       float* out, size_t n);
int sho_dequantize_row_q6k_mode(const uint8_t* block, size_t nbytes, float* out,
                                size_t n, int scale_mode);

/* Either reading where the format has two (mode: the Q6_K scale reading
 * for Q6_K, the IQ4_XS code-byte reading for IQ4_XS; ignored otherwise). */
int sho_dequantize_row_mode(uint32_t quant, const uint8_t* block, size_t nbytes,
                            float* out, size_t n, int mode);
int sho_gemv_mode(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
                  size_t nbytes, const float* x, float* y, int mode);

int sho_gemv(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
             size_t nbytes, const float* x, float* y);
int sho_gemv_q6k_mode(int64_t rows, int64_t cols, const uint8_t* data,
                      size_t nbytes, const float* x, float* y, int scale_mode);
int sho_gemv_threads(uint32_t quant, int64_t rows, int64_t cols,
                     const uint8_t* data, size_t nbytes, const float* x,
                     float* y, int n_threads);

int sho_expert_gemv(uint32_t quant, int64_t n_expert, int64_t rows,
                    int64_t cols, const uint8_t* data, size_t nbytes,
                    int64_t e, const float* x, float* y);
/* The same under either reading of a two-reading format (as
 * sho_dequantize_row_mode). */
int sho_expert_gemv_mode(uint32_t quant, int64_t n_expert, int64_t rows,
                         int64_t cols, const uint8_t* data, size_t nbytes,
                         int64_t e, const float* x, float* y, int mode);

float sho_silu(float x);
float sho_sigmoid(float x);

/* the trait's elementwise methods, one row / head each */
void sho_rms_norm(const float* x, const float* w, size_t n, double eps, float* out);
void sho_l2_norm(float* head, size_t n, double eps);
void sho_softmax(float* xs, size_t n);
void sho_rope_neox(float* head, size_t len, uint64_t pos, size_t n_rot, size_t head_dim,
                   double freq_base);
void sho_add(float* a, const float* b, size_t n);

/* the dense FFN half of a layer, one token (qwen35.rs:112-129): q, t, nb
 * for gate, up, down */
int sho_dense_ffn(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_embd, int64_t n_ff,
                  const float* x, const float* post_norm, double eps, float* out);

int sho_moe_route(const float* logits, int64_t n_expert, int64_t top_k,
                  int64_t* ids, float* weights);

int sho_moe_routed(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                   int64_t n_expert, int64_t n_embd, int64_t n_ff,
                   const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                   size_t up_bytes, const uint8_t* down, size_t down_bytes,
                   const int64_t* ids, const float* weights, int64_t k,
                   const float* x, float* out);
int sho_moe_layer(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                  int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                  float* out);
/* The same with the routed expert stacks in llama.cpp's out-major
 * orientation when out_major is set: gate / up [n_expert][n_ff][n_embd],
 * down [n_expert][n_embd][n_ff], each expert an ops::gemv of its slice. */
int sho_moe_routed_o(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                     int64_t n_expert, int64_t n_embd, int64_t n_ff,
                     const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                     size_t up_bytes, const uint8_t* down, size_t down_bytes,
                     const int64_t* ids, const float* weights, int64_t k,
                     const float* x, float* out, int out_major);
int sho_moe_layer_o(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                    int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                    float* out, int out_major);
/* The same with each tensor's reading (modes[3] for gate, up, down; modes[8]
 * in the order of q for the layer; NULL: all 0). */
int sho_moe_routed_m(uint32_t gate_quant, uint32_t up_quant, uint32_t down_quant,
                     int64_t n_expert, int64_t n_embd, int64_t n_ff,
                     const uint8_t* gate, size_t gate_bytes, const uint8_t* up,
                     size_t up_bytes, const uint8_t* down, size_t down_bytes,
                     const int64_t* ids, const float* weights, int64_t k,
                     const float* x, float* out, int out_major, const int* modes);
int sho_moe_layer_m(const uint32_t* q, const uint8_t* const* t, const size_t* nb, int64_t n_expert,
                    int64_t n_embd, int64_t n_ff, int64_t n_ff_sh, int64_t top_k, const float* x,
                    float* out, int out_major, const int* modes);

/* y[t][r] = gemv(W, x[t]) for t < m: m independent sho_gemv calls, each
 * row-parallel over n_threads (bit-identical to the sequential loop). */
int sho_matmul(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
               size_t nbytes, const float* x, int64_t m, float* y, int n_threads);
int sho_matmul_mode(uint32_t quant, int64_t rows, int64_t cols, const uint8_t* data,
                    size_t nbytes, const float* x, int64_t m, float* y, int n_threads, int mode);

/* Activation blocks of 32 (n % 32 == 0): s = max|x| / 127 (f32 division),
 * q = rint(x / s) (round to nearest even; 0 when s == 0), sums[b] =
 * s * (float)sum(q). */
int sho_quantize_q8(const float* x, size_t n, int8_t* q, float* scales,
                    float* sums);

/* Activation blocks of 256 (n % 256 == 0), the rounding the q8 matmul
 * mode applies for Q4_K / Q5_K weights (one scale per weight super-block):
 * s = max|x| / 127 over the 256 (f32 division), q = rint(x / s) (nearest
 * even; 0 when s == 0), sums[8b + j] = sum of the codes of elements
 * [32j, 32j + 32) of block b (exact integers). */
int sho_quantize_q8k(const float* x, size_t n, int8_t* q, float* scales,
                     int32_t* sums);

#ifdef __cplusplus
}
#endif

#endif
