/*
 * strata_hip.h -- C ABI of libstrata_hip.so, the MI355X (gfx950) quantized
 * weight compute path for strata-rs.
 *
 * The library replaces the matvec/matmul half of strata-core's
 * `trait ComputeBackend` (crates/strata-core/src/backend.rs:20-51) for the
 * GGUF types Q8_0, Q4_K, Q5_K, Q6_K and IQ4_XS (and, for the matvec and
 * dequant only, F32 / F16 / BF16, the types router and gate tensors use).
 * Weights stay packed in device memory in their GGUF block layout; kernels
 * dequantize in registers.
 *
 * Conventions
 *  - Every function returns int: SH_OK (0) or a negative SH_ERR_* code, and
 *    never aborts the process. sh_last_error() gives a message for the last
 *    failure on the calling thread.
 *  - Host-slice entry points (sh_gemv, sh_expert_gemv, ...) are synchronous:
 *    on return the output slice is written. A context serialises its calls
 *    with an internal lock, so one context may be shared by many threads
 *    (the trait is `Send + Sync`, backend.rs:20).
 *  - Weights are identified by a caller-chosen 64-bit key (the Rust shim
 *    hashes the tensor name, as the wgpu backend keys its cache by name,
 *    crates/strata-backend-wgpu/src/gpu.rs:271,287). The first call with a
 *    key copies the packed bytes to the device; later calls reuse them. The
 *    resident set is bounded by the context's byte budget and evicted
 *    least-recently-used (gpu.rs:61-113). Host pointers are not retained
 *    after a call returns (weights are borrowed mmap slices, engine.rs:77-79).
 *  - *_dev entry points take device pointers and a hipStream_t (as void*),
 *    enqueue work and return without synchronising.
 *  - No CPU fallback exists inside the library: without a usable device,
 *    sh_create fails with SH_ERR_NO_DEVICE and the caller keeps its CPU
 *    backend, as strata_backend_wgpu::select does
 *    (crates/strata-backend-wgpu/src/lib.rs:36-43).
 */
#ifndef STRATA_HIP_H
#define STRATA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SH_ABI_VERSION 1

/* ---- status codes ------------------------------------------------------ */
#define SH_OK 0
#define SH_ERR_INVALID_ARGUMENT (-1) /* null pointer, zero batch, bad mode   */
#define SH_ERR_SHAPE (-2)            /* length mismatch: ops.rs:15-17 asserts */
#define SH_ERR_TRUNCATED (-3)        /* dequant.rs:50-55 Error::Truncated     */
#define SH_ERR_UNSUPPORTED_QUANT (-4) /* type the device path does not read   */
#define SH_ERR_UNSUPPORTED_SHAPE (-5) /* a shape the kernels do not take      */
#define SH_ERR_NO_DEVICE (-6)        /* no usable HIP device                  */
#define SH_ERR_DEVICE (-7)           /* HIP runtime failure                   */
#define SH_ERR_OUT_OF_MEMORY (-8)    /* device or pinned allocation failed    */
#define SH_ERR_FORMAT (-9)           /* malformed GGUF: reader.rs's BadMagic,
                                        UnsupportedVersion, BadKeyLength,
                                        StringNotUtf8, BadValueType,
                                        WrongTensorDims, duplicate tensor     */
#define SH_ERR_IO (-10)              /* the file cannot be opened or mapped   */
#define SH_ERR_NOT_FOUND (-11)       /* no such tensor / key (or not of the
                                        asked type): the reference's None     */

/* ---- quant type ids (Strata's scheme, crates/strata-gguf/src/quant.rs:15-43) */
#define SH_QUANT_F32 0u
#define SH_QUANT_F16 1u
#define SH_QUANT_Q8_0 8u
#define SH_QUANT_Q4_K 12u
#define SH_QUANT_Q5_K 13u
#define SH_QUANT_Q6_K 14u
#define SH_QUANT_IQ4_XS 23u
#define SH_QUANT_BF16 30u

/* ---- tensor flags ------------------------------------------------------ */
/* Q6_K sub-block scales as ggml's int8_t instead of strata-gguf's u8 reading
 * (crates/strata-gguf/src/dequant.rs:211,224-227 reads them as u8). */
#define SH_FLAG_Q6K_SIGNED_SCALES 1u
/* Expert stacks in ggml's orientation, as llama.cpp GGUF files store them:
 * [n_expert][rows = out][cols = in] with blocks along the input.
 * sh_expert_gemv then computes y[r] = sum_c W_e[r][c] x[c] (x_len = cols,
 * y_len = rows) with the matvec kernels; the fused MoE entry points
 * (sh_moe_ffn, sh_moe_layer and their _dev forms) take gate / up
 * [n_expert][n_ff][n_embd] and down [n_expert][n_embd][n_ff], each expert
 * an ops::gemv of its slice, when all three stacks carry the flag (mixed
 * orientations are refused). The reference's in-major orientation
 * (weights.rs:14-34) is the default. */
#define SH_FLAG_EXPERT_OUT_MAJOR 2u
/* IQ4_XS in ggml's layout, sub-block ib reading qs[16 ib .. 16 ib + 16).
 * strata-gguf reads qs[0..16] for every sub-block (its qs slice is never
 * advanced, crates/strata-gguf/src/dequant.rs:189-206); that reading is the
 * default. */
#define SH_FLAG_IQ4XS_GGML 4u

/* ---- matmul modes ------------------------------------------------------ */
#define SH_MATMUL_BF16 0u /* bf16 activations, dequant-to-bf16 LDS tiles, bf16 MFMA */
#define SH_MATMUL_Q8 1u   /* activations in 32-element Q8 blocks, int8 MFMA */
#define SH_MATMUL_Q8K 2u  /* activations in 256-element Q8 blocks, int8 MFMA (K-quants) */

typedef struct sh_context sh_context;

/* A quantized matrix: QuantTensor (crates/strata-core/src/backend.rs:117-153).
 * `rows` rows of `cols` elements, row-major packed blocks of `quant`; a row
 * is ceil(cols / block) * block_bytes long (backend.rs:139-152). */
typedef struct sh_quant_tensor {
  uint64_t key;
  uint32_t quant;
  uint32_t flags;
  uint64_t rows;
  uint64_t cols;
  const uint8_t* data;
  uint64_t nbytes;
} sh_quant_tensor;

/* A 3-D expert tensor: ExpertView (crates/strata-core/src/weights.rs:14-34).
 * Expert-major [n_expert][rows = in][cols = out]; quant blocks run along the
 * output axis. */
typedef struct sh_expert_view {
  uint64_t key;
  uint32_t quant;
  uint32_t flags;
  uint64_t n_expert;
  uint64_t rows;
  uint64_t cols;
  const uint8_t* data;
  uint64_t nbytes;
} sh_expert_view;

/* RopeCfg (crates/strata-core/src/backend.rs:158-167). */
typedef struct sh_rope_cfg {
  uint64_t pos;      /* token position */
  uint64_t n_rot;    /* leading head dims rotated (NEOX pairs) */
  uint64_t head_dim; /* stride between heads */
  double freq_base;  /* theta */
} sh_rope_cfg;

/* An open GGUF file: GgufFile (crates/strata-gguf/src/reader.rs:200-445). */
typedef struct sh_gguf sh_gguf;

/* TensorInfo (reader.rs:179-197) plus its payload size. */
typedef struct sh_gguf_tensor_info {
  const char* name; /* valid until sh_gguf_close */
  uint32_t n_dims;  /* 1..4 */
  uint32_t type;    /* quant type id */
  uint64_t shape[4]; /* GGUF order, dim 0 fastest; 1 past n_dims */
  uint64_t offset;  /* from the start of the data section */
  uint64_t nbytes;  /* tensor_payload_bytes (reader.rs:399-423); 0 for an unknown type */
} sh_gguf_tensor_info;

/* ---- library and context ----------------------------------------------- */
int sh_abi_version(void);
/* Message for the last failure on this thread ("" if none). */
const char* sh_last_error(void);
/* Number of visible HIP devices (0 is not an error). */
int sh_device_count(int* count);
/* Block geometry of a quant id: quant.rs:125-164 (block_size, type_size). */
int sh_quant_geometry(uint32_t quant, uint32_t* block_size, uint32_t* type_size);

/* Opens `device` with a resident-weight budget in bytes; 0 means 4 GiB, the
 * wgpu backend's default (crates/strata-backend-wgpu/src/gpu.rs:227-230). */
int sh_create(int device, uint64_t weight_budget_bytes, sh_context** out);
int sh_destroy(sh_context* ctx);
/* ComputeBackend::name (backend.rs:22): "hip". */
const char* sh_name(const sh_context* ctx);
/* Bytes of resident weights (WgpuBackend::resident_bytes, gpu.rs:238-241). */
int sh_resident_bytes(sh_context* ctx, uint64_t* bytes);
/* Drops one resident weight (no-op when absent). */
int sh_evict(sh_context* ctx, uint64_t key);

/* ---- the trait's quantized primitives (host slices, synchronous) ------- */

/* ComputeBackend::gemv (backend.rs:25), semantics of ops::gemv
 * (crates/strata-core/src/ops.rs:14-28): y[r] = sum_c W[r][c] * x[c].
 * x_len must equal cols and y_len rows. Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_XS,
 * and F32 / F16 / BF16 (products and sums in f64, as ops::gemv does). */
int sh_gemv(sh_context* ctx, const sh_quant_tensor* w, const float* x, uint64_t x_len, float* y,
            uint64_t y_len);

/* `batch` independent gemvs against one weight read: x is [batch][cols],
 * y is [batch][rows]; batch 1..8. No reference counterpart; equal to
 * `batch` calls of ops::gemv. */
int sh_gemv_batch(sh_context* ctx, const sh_quant_tensor* w, const float* x, float* y,
                  uint32_t batch);

/* ComputeBackend::expert_gemv (backend.rs:28-35), semantics of
 * ops::expert_gemv (ops.rs:169-195): y[c] = sum_i x[i] * W_e[i][c].
 * x_len must equal rows and y_len cols; e < n_expert. */
int sh_expert_gemv(sh_context* ctx, const sh_expert_view* w, uint64_t e, const float* x,
                   uint64_t x_len, float* y, uint64_t y_len);

/* Admits a packed tensor into the resident store under `key` ahead of use
 * (what the first matvec call with that key would do): idempotent, a key
 * already resident with the same type and shape is left as it is, one with
 * another is replaced; LRU under the budget. Layout as sh_expert_view /
 * sh_quant_tensor (n_expert = 1 for a matrix). src_row_pitch: bytes from one
 * row start to the next in `data` (0 = packed rows of byte_size(quant,
 * cols)); rows are stored packed on the device. Later calls with the key
 * may pass data = NULL. Types with a device kernel only. */
int sh_weight_upload(sh_context* ctx, uint64_t key, uint32_t quant, uint64_t n_expert, uint64_t rows,
                     uint64_t cols, const uint8_t* data, uint64_t src_row_pitch);

/* ---- the trait's elementwise methods (host slices, synchronous) -------
 * ComputeBackend::{rms_norm, rope_neox, softmax, l2_norm, add}
 * (backend.rs:38-50) with the CPU bodies' arithmetic (ops.rs:46-165): f64
 * sums and scales, one rounding to f32 per output as the Rust source. The
 * sums run in a different order and expf / pow / sin / cos are the device
 * library's, so outputs agree with the CPU backend to within an ulp. */

/* ops::rms_norm (ops.rs:46-56): x = x * w / sqrt(mean(x^2) + eps), in place. */
int sh_rms_norm(sh_context* ctx, float* x, const float* w, uint64_t n, double eps);
/* ops::rope_neox (ops.rs:120-135) on one head of n floats, in place. */
int sh_rope_neox(sh_context* ctx, float* head, uint64_t n, const sh_rope_cfg* cfg);
/* ops::softmax (ops.rs:105-116), in place. */
int sh_softmax(sh_context* ctx, float* xs, uint64_t n);
/* ops::l2_norm (ops.rs:73-82), in place. */
int sh_l2_norm(sh_context* ctx, float* head, uint64_t n, double eps);
/* ops::add_into (ops.rs:161-165): a += b. */
int sh_add(sh_context* ctx, float* a, const float* b, uint64_t n);

/* dequantize_row (crates/strata-gguf/src/dequant.rs:45-61) on the device:
 * `n` f32 values from `nbytes` packed bytes, bit-exact. SH_ERR_TRUNCATED
 * when n is not a whole number of blocks or the buffer is short. */
int sh_dequantize_row(sh_context* ctx, uint32_t quant, uint32_t flags, const uint8_t* block,
                      uint64_t nbytes, float* out, uint64_t n);

/* MoeLayer::route from router logits (crates/strata-core/src/moe.rs:58-90):
 * softmax over all experts, top-k by descending probability (ties to the
 * lower id), ids ascending, weights renormalised by max(sum, 2^-14).
 * logits [n_tok][n_expert]; ids/weights [n_tok][top_k]. n_expert <= 1024,
 * top_k <= min(32, n_expert), n_tok <= 256. */
int sh_moe_route(sh_context* ctx, const float* logits, uint32_t n_tok, uint32_t n_expert,
                 uint32_t top_k, int32_t* ids, float* weights);

/* The routed half of MoeLayer::combine (moe.rs:108-127) for n_tok tokens,
 * from router logits: out[t] = sum over t's top_k experts (ascending id) of
 * w * down_e(silu(gate_e x_t) * up_e x_t). gate/up are [n_expert][n_embd]
 * [n_ff], down [n_expert][n_ff][n_embd] (reference orientation), or with
 * SH_FLAG_EXPERT_OUT_MAJOR on all three [n_expert][n_ff][n_embd] and
 * [n_expert][n_embd][n_ff]; x and out are [n_tok][n_embd]. The shared expert (moe.rs:129-143) is not included.
 * gate and up must have the same quant type. */
int sh_moe_ffn(sh_context* ctx, const sh_expert_view* gate, const sh_expert_view* up,
               const sh_expert_view* down, const float* logits, uint32_t n_tok, uint32_t top_k,
               const float* x, float* out);

/* The whole MoE layer, MoeLayer::route + MoeLayer::combine
 * (crates/strata-core/src/moe.rs:48-143), for n_tok tokens of x [n_tok]
 * [n_embd]: logits = router . bf16(x) (route, moe.rs:55-56), the routed
 * experts as sh_moe_ffn, then the always-on shared expert added plain:
 * out += sigmoid(gate_inp_shexp . x) * down_shexp . (silu(gate_shexp . x) *
 * (up_shexp . x)) (moe.rs:129-142). router [n_expert][n_embd], gate/up_shexp
 * [n_ff_shexp][n_embd], down_shexp [n_embd][n_ff_shexp], gate_inp_shexp
 * [1][n_embd] are ops::gemv matrices of any matvec type (IQ4_XS and F32 /
 * F16 / BF16 included); the expert views as in sh_moe_ffn. n_ff_shexp must be a
 * multiple of 4. The weight budget must hold the eight tensors at once. */
int sh_moe_layer(sh_context* ctx, const sh_quant_tensor* router, const sh_expert_view* gate,
                 const sh_expert_view* up, const sh_expert_view* down, const sh_quant_tensor* gate_shexp,
                 const sh_quant_tensor* up_shexp, const sh_quant_tensor* down_shexp,
                 const sh_quant_tensor* gate_inp_shexp, const float* x, uint32_t n_tok, uint32_t top_k,
                 float* out);

/* Batched prefill matmul: y[t][r] = sum_c W[r][c] * x[t][c] for t < m, x
 * [m][cols] and y [m][rows] row-major f32. The reference has no matmul
 * (prefill is one forward per token, crates/strata-core/src/generate.rs:
 * 116-117); the result equals m calls of ops::gemv (ops.rs:14-28) up to the
 * activation rounding of `mode`:
 *   SH_MATMUL_BF16  x rounded to bf16, weights dequantized to bf16, f32
 *                   accumulation (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS);
 *   SH_MATMUL_Q8    x quantized to Q8 blocks of 32 elements (f32 scale
 *                   max|x| / 127 per block, int8 codes rounded to nearest
 *                   even), int8 products (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS);
 *   SH_MATMUL_Q8K   x quantized to blocks of 256 elements, one scale per
 *                   weight super-block (Q4_K, Q5_K): a coarser activation
 *                   rounding than SH_MATMUL_Q8 (the step is max|x| over 256
 *                   elements), an opt-in alternative.
 * cols must be a multiple of 64. */
int sh_matmul(sh_context* ctx, const sh_quant_tensor* w, const float* x, uint32_t m, float* y,
              uint32_t mode);

/* ---- device-pointer variants (asynchronous on `stream`) ---------------- */

/* Bytes of device workspace sh_matmul_dev needs. */
int sh_matmul_workspace_bytes(uint32_t quant, uint64_t rows, uint64_t cols, uint32_t m, uint32_t mode,
                              uint64_t* bytes);

/* sh_matmul on device pointers: w (4-byte aligned), x [m][cols], y
 * [m][rows], workspace at least sh_matmul_workspace_bytes() long and
 * 256-byte aligned. Calls sharing one workspace must not overlap in time. */
int sh_matmul_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                  const float* x, uint32_t m, float* y, uint32_t mode, void* workspace,
                  uint64_t workspace_bytes, void* stream);

/* The activation quantization of SH_MATMUL_Q8 on its own: n f32 (n a
 * multiple of 32, x 16-byte aligned) -> n int8 codes, n / 32 scales
 * (max|x| / 127 per block) and n / 32 values scale * sum(codes). */
int sh_quantize_q8_dev(const float* x, uint64_t n, int8_t* codes, float* scales, float* code_sums,
                       void* stream);

/* The activation rounding of SH_MATMUL_Q8K (Q4_K / Q5_K weights) on its
 * own: n f32 (n a multiple of 256, x 16-byte aligned) -> n int8 codes, n /
 * 256 scales (max|x| / 127 per 256 elements, one per weight super-block) and
 * n / 32 integer code sums (one per 32-element sub-block). No counterpart in
 * the reference (it has no matmul). */
int sh_quantize_q8k_dev(const float* x, uint64_t n, int8_t* codes, float* scales, int32_t* sub_sums,
                        void* stream);

/* One expert tensor already in device memory. */
typedef struct sh_expert_dev {
  uint32_t quant;
  uint32_t flags;
  const void* data; /* [n_expert][rows][cols] packed, as in sh_expert_view */
} sh_expert_dev;

/* Bytes of device workspace sh_moe_ffn_dev needs for these shapes, in
 * either orientation of the expert stacks. */
int sh_moe_workspace_bytes(uint32_t n_tok, uint32_t top_k, uint64_t n_expert, uint64_t n_embd,
                           uint64_t n_ff, uint32_t quant_gate_up, uint32_t quant_down,
                           uint64_t* bytes);

/* sh_moe_ffn on device pointers; logits, x, out and workspace are device
 * buffers, workspace at least sh_moe_workspace_bytes() long and 256-byte
 * aligned. Calls sharing one workspace must not overlap in time. */
int sh_moe_ffn_dev(const sh_expert_dev* gate, const sh_expert_dev* up, const sh_expert_dev* down,
                   uint64_t n_expert, uint64_t n_embd, uint64_t n_ff, const float* logits,
                   uint32_t n_tok, uint32_t top_k, const float* x, float* out, void* workspace,
                   uint64_t workspace_bytes, void* stream);

/* Bytes of device workspace sh_moe_layer_dev needs (either orientation of
 * the expert stacks); quants[8] are the types of router, gate, up, down,
 * gate_shexp, up_shexp, down_shexp, gate_inp_shexp. */
int sh_moe_layer_workspace_bytes(uint32_t n_tok, uint32_t top_k, uint64_t n_expert, uint64_t n_embd,
                                 uint64_t n_ff, uint64_t n_ff_shexp, const uint32_t* quants, uint64_t* bytes);

/* sh_moe_layer on device pointers: tensors[8] in the order router, gate,
 * up, down (expert tensors, as in sh_moe_ffn_dev), gate_shexp, up_shexp,
 * down_shexp, gate_inp_shexp (row-major matrices); x (16-byte aligned) and
 * out [n_tok][n_embd]; workspace at least sh_moe_layer_workspace_bytes()
 * long and 256-byte aligned. Calls sharing one workspace must not overlap
 * in time. */
int sh_moe_layer_dev(const sh_expert_dev* tensors, uint64_t n_expert, uint64_t n_embd, uint64_t n_ff,
                     uint64_t n_ff_shexp, uint32_t n_tok, uint32_t top_k, const float* x, float* out,
                     void* workspace, uint64_t workspace_bytes, void* stream);

/* rows x cols of packed blocks at `w` -> out[rows][cols] f32, bit-exact. */
int sh_dequant_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                   float* out, void* stream);

/* y[b][r] = sum_c W[r][c] x[b][c], b < batch (1..8); w at least 2-byte
 * aligned (4 for Q8_0 and F32), x 16-byte aligned. Q6_K rows of whole
 * 4096-column windows read fastest from a 16-byte aligned w. */
int sh_gemv_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                const float* x, float* y, uint32_t batch, void* stream);

/* Bytes of device workspace sh_gemv_dev_ws uses for this shape and batch:
 * nonzero for batches of 2..8 of the types with a batched int8-MFMA kernel
 * (Q4_K, Q5_K), else 0. No reference counterpart. */
int sh_gemv_workspace_bytes(uint32_t quant, uint64_t rows, uint64_t cols, uint32_t batch, uint64_t* bytes);

/* sh_gemv_dev with a workspace (256-byte aligned, at least
 * sh_gemv_workspace_bytes() long, no initialisation needed; unused, and may
 * be NULL, when that is 0): batches of 2..8 convert their activations once
 * per call into it (one small extra launch), and every workgroup copies the
 * window of them it needs instead of converting it; rows wider than one
 * window (2048 to 4096 columns, chosen per shape) run split-K over the
 * windows, and the last workgroup of a row block adds the windows' sums in
 * window order, so results do not depend on timing (they differ from
 * sh_gemv_dev's by the order of a few f32 additions). Calls sharing one
 * workspace must not overlap in time. No reference counterpart. */
int sh_gemv_dev_ws(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols, const float* x,
                   float* y, uint32_t batch, void* workspace, uint64_t workspace_bytes, void* stream);

/* A plain streaming read of `nbytes` at `data` (16-byte aligned, a multiple
 * of 16 bytes), the read-bandwidth ceiling the matvecs are measured against:
 * 2048 workgroups of 256 threads, one 16-byte load per lane per step;
 * out[2048] receives per-workgroup XOR folds of the 32-bit words read (their
 * XOR is the XOR of all words). No reference counterpart. */
int sh_stream_read_dev(const void* data, uint64_t nbytes, uint32_t* out, void* stream);

/* ---- GGUF weight source (host code; no device needed except the upload) */
/* GgufFile::open (reader.rs:231-353): maps `path` read-only and parses the
 * header, metadata and tensor directory with the reference's checks and
 * limits; data_start is the directory's end rounded up to the alignment
 * (general.alignment when an integer type and positive, else 32). */
int sh_gguf_open(const char* path, sh_gguf** out);
int sh_gguf_close(sh_gguf* gguf);
int sh_gguf_header(const sh_gguf* gguf, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv,
                   uint64_t* alignment, uint64_t* data_start, uint64_t* file_size);
/* The index-th directory entry (file order). */
int sh_gguf_tensor(const sh_gguf* gguf, uint64_t index, sh_gguf_tensor_info* out);
/* GgufFile::find (reader.rs:387-389). */
int sh_gguf_find(const sh_gguf* gguf, const char* name, uint64_t* index);
/* GgufFile::tensor_data (reader.rs:425-445): the payload inside the mapping,
 * bounds-checked (SH_ERR_TRUNCATED past the end of the file). */
int sh_gguf_tensor_data(const sh_gguf* gguf, uint64_t index, const uint8_t** data, uint64_t* nbytes);
/* Metadata (metadata.rs): the value's type tag, array element type and
 * count; MetaValue::as_int (integer types; a u64 value reads as 0, as in
 * the reference), as_float (numbers), as_str (strings, valid until close). */
int sh_gguf_meta_type(const sh_gguf* gguf, const char* key, uint32_t* type, uint32_t* elem, uint64_t* count);
int sh_gguf_meta_int(const sh_gguf* gguf, const char* key, int64_t* value);
int sh_gguf_meta_float(const sh_gguf* gguf, const char* key, double* value);
int sh_gguf_meta_str(const sh_gguf* gguf, const char* key, const char** s, uint64_t* len);
/* A whole model: GgufModel (reader.rs:450-522). `any_shard` of a split
 * model `<name>-NNNNN-of-MMMMM.gguf` opens every shard (split_paths,
 * reader.rs:524-572; a missing one is SH_ERR_IO naming it); any other path
 * is a single shard. Metadata lives in shard 0. The shard handles are
 * borrowed: valid until sh_gguf_model_close (sh_gguf_close on them is a
 * no-op). A tensor name in two shards is SH_ERR_FORMAT. */
typedef struct sh_gguf_model sh_gguf_model;
int sh_gguf_model_open(const char* any_shard, sh_gguf_model** out);
int sh_gguf_model_close(sh_gguf_model* model);
int sh_gguf_model_shards(const sh_gguf_model* model, uint64_t* n_shards);
int sh_gguf_model_shard(sh_gguf_model* model, uint64_t i, sh_gguf** shard);
/* GgufModel::find (reader.rs:496-501): the shard and its tensor index. */
int sh_gguf_model_find(const sh_gguf_model* model, const char* name, uint64_t* shard, uint64_t* index);

/* Admits tensor `index` into ctx's resident store under `key`, packed as
 * stored, copied from the mapping through pinned staging chunks. Dims map
 * as [cols, rows, n_expert] (weights.rs:14-34), so a later sh_gemv /
 * sh_expert_gemv / sh_moe_* call with the same key and shape finds it
 * resident. Types with a device kernel only; 1 to 3 dims. */
int sh_upload_gguf_tensor(sh_context* ctx, const sh_gguf* gguf, uint64_t index, uint64_t key);

/* The dense FFN half of a decoder layer (crates/strata-core/src/qwen35.rs:
 * 112-129) for n_tok tokens on device pointers: mixed = rms_norm(x,
 * post_norm, eps) (ops.rs:59-69); g = gate . mixed; u = up . mixed;
 * h = g / (1 + exp(-g)) * u (f32); out = x + down . h (f32). tensors[3]:
 * gate, up [n_ff][n_embd] and down [n_embd][n_ff], any matvec types; x, out
 * [n_tok][n_embd] (out may equal x: the residual add in place); post_norm
 * [n_embd]; workspace >= sh_ffn_workspace_bytes, 256-byte aligned. One token
 * with one quantized type runs in three launches (rms_norm; gate and up
 * together; down with silu(g) * u staged and the residual added). No
 * reference counterpart as one call: it replaces the six steps above. */
int sh_ffn_workspace_bytes(uint32_t n_tok, uint64_t n_embd, uint64_t n_ff, uint64_t* bytes);
/* The same on host slices, in place as the reference's `*x += *m`: x
 * [n_tok][n_embd] holds the layer input and receives the output; gate / up
 * [n_ff][n_embd] and down [n_embd][n_ff] are resident weights (admitted on
 * first use; the budget must hold all three). Synchronous. */
int sh_ffn(sh_context* ctx, const sh_quant_tensor* gate, const sh_quant_tensor* up, const sh_quant_tensor* down,
           const float* post_norm, double eps, uint32_t n_tok, float* x);
int sh_ffn_dev(const sh_expert_dev* tensors, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok, const float* x,
               const float* post_norm, double eps, float* out, void* workspace, uint64_t workspace_bytes,
               void* stream);
/* sh_ffn_dev without a workspace argument, and without allocating anything:
 * its intermediates live in a fixed 4 MiB device array inside the library
 * (one per GPU, held until the process ends). No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Shapes whose sh_ffn_workspace_bytes exceed 4 MiB are refused with
 * SH_ERR_UNSUPPORTED_SHAPE (at n_embd 4096, n_ff 12288: up to 23 tokens).
 * WARNING: every call on one GPU shares that array. Calls that overlap in
 * time on one GPU (on other streams, from other threads or processes, or
 * graphs holding this call replayed concurrently) race on it and corrupt each
 * other's results without an error; the caller must serialise them (one
 * stream, or an event between them). Same results as sh_ffn_dev, bit for
 * bit. */
int sh_ffn_dev_noalloc(const sh_expert_dev* tensors, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok,
                       const float* x, const float* post_norm, double eps, float* out, void* stream);

/* The elementwise methods batched over rows, on device pointers: the same
 * arithmetic per row as the host-slice forms; enqueued on `stream`.
 * rms_norm: x, out [rows][n] (out may equal x), w [n]. */
int sh_rms_norm_dev(const float* x, const float* w, float* out, uint64_t rows, uint64_t n, double eps,
                    void* stream);
/* l2_norm and softmax of each row of x [rows][n], in place. */
int sh_l2_norm_dev(float* x, uint64_t rows, uint64_t n, double eps, void* stream);
int sh_softmax_dev(float* x, uint64_t rows, uint64_t n, void* stream);
/* rope_neox of `rows` heads of cfg->head_dim floats (x [rows][head_dim]);
 * head r is at position cfg->pos + r / heads_per_pos (heads_per_pos = the
 * heads of one token, so a prefill batch of consecutive tokens is one call). */
int sh_rope_neox_dev(float* x, uint64_t rows, uint64_t heads_per_pos, const sh_rope_cfg* cfg, void* stream);
/* a[i] += b[i], i < n. */
int sh_add_dev(float* a, const float* b, uint64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATA_HIP_H */
