// Host-side launchers of the device kernels (internal to libstrata_hip).
// Every launcher validates shapes on the host before any launch, so a kernel
// never sees a grid or a buffer size it was not written for.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sh {

// Bit-exact dequantization of rows x cols (row-major packed rows) into f32.
hipError_t launch_dequant(uint32_t quant, const void* w, int64_t rows, int64_t cols, float* out,
                          int q6_signed, hipStream_t stream);

// y[b][r] = sum_c W[r][c] * x[b][c] for b < batch (1..8). Returns
// hipErrorInvalidValue for shapes the kernels do not take (checked by
// gemv_shape_ok first).
bool gemv_shape_ok(uint32_t quant, int64_t rows, int64_t cols, int batch);
// `ws`: optional workspace of gemv_workspace_bytes() for batches of 2..8
// (the activations are then converted once per call); null: none.
hipError_t launch_gemv(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x,
                       float* y, int batch, int q6_signed, hipStream_t stream, void* ws = nullptr);
size_t gemv_workspace_bytes(uint32_t quant, int64_t rows, int64_t cols, int batch);
// One token of the dense FFN (qwen35.rs:112-129) after its rms_norm, in two
// matvec launches: gu = [gate . x; up . x] (2 * n_ff floats), then
// out = xres + down . (silu(g) * u). All three matrices of type `quant`
// (Q8_0 / Q4_K / Q5_K / Q6_K); ffn_fused_ok checks the shapes.
bool ffn_fused_ok(uint32_t quant, int64_t n_embd, int64_t n_ff);
hipError_t launch_ffn_one(uint32_t quant, const void* gate, const void* up, const void* down, int64_t n_embd,
                          int64_t n_ff, const float* x, float* gu, const float* xres, float* out, int q6s,
                          hipStream_t stream);
// h = silu(g) * u elementwise (ops.rs:85-87, f32).
hipError_t launch_silu_mul(const float* g, const float* u, float* h, int64_t n, hipStream_t stream);

// The dense FFN half of a layer for n_tok tokens (rms_norm, gate, up, silu,
// down, residual); workspace of ffn_workspace_bytes.
size_t ffn_workspace_bytes(int64_t n_tok, int64_t n_embd, int64_t n_ff);
hipError_t launch_ffn(uint32_t q_gate, uint32_t q_up, uint32_t q_down, const void* gate, const void* up,
                      const void* down, int q6g, int q6u, int q6d, int64_t n_embd, int64_t n_ff, int n_tok,
                      const float* x, const float* post_norm, double eps, float* out, void* workspace,
                      hipStream_t stream);
// The same for F32 / F16 / BF16 rows against bf16(x) (rounded as loaded).
hipError_t launch_gemv_plain_bf16x(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x,
                                   float* y, int batch, hipStream_t stream);
// Both in one launch: y1 = W1 . bf16(x) (rows1 rows) and y2 = W2 . x (rows2
// rows of the same type and width), e.g. a MoE layer's router and gate input.
hipError_t launch_gemv_plain_pair(uint32_t quant, const void* w1, int64_t rows1, const void* w2, int64_t rows2,
                                  int64_t cols, const float* x, float* y1, float* y2, int batch, hipStream_t stream);
// A MoE layer's shared expert for one token in two limb launches: gu = [gate;
// up] . x (2 n_ff floats, g then u), d = down . (silu(g) * u).
bool shexp_fused_ok(uint32_t q_gu, uint32_t q_d, int64_t n_embd, int64_t n_ff);
hipError_t launch_shexp_one(uint32_t q_gu, uint32_t q_d, const void* gate, const void* up, const void* down,
                            int64_t n_embd, int64_t n_ff, const float* x, float* gu, float* d, int q6gu, int q6d,
                            hipStream_t s);

// Batch 2..8 of Q4_K or Q5_K rows on int8 MFMA (exact integer
// activations, staged in LDS 4096 columns at a time); `cu` is the device's
// CU count.
// With `ws` (gemv_mfma_workspace_bytes(rows, cols), 256-byte aligned, no
// initialisation needed) the activations are converted once per call into
// it (one extra launch) instead of by every workgroup, and rows wider than
// one 4096-column window run split-K over the windows.
bool gemv_mfma_ok(uint32_t quant, int64_t rows, int64_t cols, int batch);
size_t gemv_mfma_workspace_bytes(int64_t rows, int64_t cols);
hipError_t launch_gemv_mfma(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x, float* y,
                            int batch, int cu, hipStream_t stream, void* ws = nullptr);

// y[c] = sum_i x[i] * W[i][c] for one expert matrix W[rows = in][cols = out]
// (reference orientation). `workspace` holds expert_workspace_bytes().
bool expert_shape_ok(uint32_t quant, int64_t rows, int64_t cols);
size_t expert_workspace_bytes(int64_t rows, int64_t cols);
hipError_t launch_expert_gemv(uint32_t quant, const void* w, int64_t rows, int64_t cols,
                              const float* x, float* y, float* workspace, int q6_signed,
                              hipStream_t stream);

// Routed MoE FFN (router logits -> top-k -> gate/up -> silu*up -> down ->
// weighted combine). A plan fixes the launch shapes and the workspace layout
// (byte offsets into one device buffer of `bytes` bytes).
constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopK = 32;
constexpr int kMoeMaxTokens = 256;
constexpr int kMoeMaxChunks = 32;  // down chunk sums a combine adds per column (in one load round)

struct MoePlan {
  int n_tok, top_k, n_expert, n_embd, n_ff;
  int s_max;                     // most unique experts a call can route to
  int z_max;                     // most work items: (expert, one or two of its pairs)
  int64_t rb_a, rb_b;            // row bytes of gate/up and of down
  int ca, nch_a;                 // gate/up: rows per chunk, chunks (over n_embd)
  int cb, nch_b;                 // down: rows per chunk, chunks (over n_ff)
  int sr_a, sr_b;                // rows per LDS sub-tile
  int nbuf_a, nbuf_b;            // LDS sub-tile buffers (1 when one sub-tile holds the chunk)
  int reg_a, reg_b;              // LDS bytes of the sub-tiles, reused for the row-slot reduction
  size_t o_ids, o_wts, o_meta, o_tokpair;
  size_t o_item_e, o_item_off, o_item_cnt;  // per work item: expert, first pair, pairs (1 or 2)
  size_t o_item_tok;             // per work item: the tokens of its pairs
  size_t o_part_a;               // [pair][2][nch_a][n_ff]: chunk sums of gate . x, up . x
  size_t o_part_b;               // [pair][nch_b][n_embd]: chunk sums of down . a
  size_t route_lds, lds_a, lds_b;  // dynamic LDS per kernel
  bool staged;                   // row bytes allow 16-byte tile copies
  bool out_major;                // expert stacks [n_expert][out][in] (moe_om.hip)
  int om_rows_a, om_rows_b;      // out-major: rows per workgroup of gate/up and of down
  // one token over in-major stacks (moe_one.hip): per phase the 64-column
  // units of a column block, column blocks, row slots, rows per chunk,
  // chunks, and threads per column in the row-slot reduction
  bool one;
  int a1_cbu, a1_ncb, a1_rs, a1_rc, a1_nrc, a1_tpc;
  int b1_cbu, b1_ncb, b1_rs, b1_rc, b1_nrc, b1_tpc;
  size_t o_p1a;                  // [item][2][a1_nrc][n_ff]: gate/up chunk sums
  size_t o_p1b;                  // [item][b1_nrc][n_embd]: down chunk sums
  size_t lds1_a, lds1_b;
  size_t bytes;
};

// out_major: gate / up [n_expert][n_ff][n_embd] and down [n_expert][n_embd]
// [n_ff] (llama.cpp's stacks) instead of [n_expert][in][out].
bool moe_plan(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, uint32_t q_gateup,
              uint32_t q_down, MoePlan* plan, bool out_major = false);
bool moe_plan_out_major(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, uint32_t q_gateup,
                        uint32_t q_down, MoePlan* plan);
// The gate/up and down launches of an out-major plan (route and combine as
// launch_moe's).
void launch_moe_out_major(const MoePlan& p, uint32_t qg, uint32_t qd, const void* gate, const void* up,
                          const void* down, int q6g, int q6u, int q6d, const float* logits, const float* x,
                          void* workspace, bool fused_route, hipStream_t s);
// The shared expert's part of the layer's combine: out[t] += sigmoid(s[t])
// * d[t] after the routed sum, once `join` (if any) has completed.
struct MoeShared {
  const float* d;
  const float* s;
  hipEvent_t join;
};
hipError_t launch_moe(const MoePlan& p, uint32_t qg, uint32_t qu, uint32_t qd, const void* gate,
                      const void* up, const void* down, int q6g, int q6u, int q6d,
                      const float* logits, const float* x, float* out, void* workspace,
                      hipStream_t s, const MoeShared* shared = nullptr);
hipError_t launch_moe_route(const MoePlan& p, const float* logits, void* workspace, hipStream_t s);
// out[t] = sum over t's experts in ascending id with w != 0 of w * (the
// sum of the pair's nch_b down chunk sums at o_part_b), plus the shared
// expert's gated output when `shared` is given. `pairs_in_order`: token t's
// a-th expert is pair t * top_k + a (one token routed inside gate/up), so
// the pair table is not read.
hipError_t launch_moe_combine(const MoePlan& p, const uint8_t* ws, float* out, const MoeShared* shared,
                              hipStream_t s, bool pairs_in_order = false);
// The one-token in-major path (moe_one.hip): fills p's one-token fields
// and sets p.one when the shape allows it; the launches (gate/up, down,
// then launch_moe_combine over its sums).
bool moe_one_plan(MoePlan& p, uint32_t q_gateup, uint32_t q_down);
hipError_t launch_moe_one(const MoePlan& p, uint32_t qg, uint32_t qd, const void* gate, const void* up,
                          const void* down, int q6g, int q6u, int q6d, const float* logits, const float* x,
                          float* out, void* workspace, bool fused_route, hipStream_t s, const MoeShared* shared);

// The whole MoE layer (router matvec on bf16-rounded x, routed experts,
// shared expert with its sigmoid gate): the routed plan plus the layer's
// intermediate buffers after it in the same workspace.
struct MoeLayerTypes {
  uint32_t router, gate, up, down, gate_sh, up_sh, down_sh, gate_inp;
};
struct MoeLayerTensors {
  const void *router, *gate, *up, *down, *gate_sh, *up_sh, *down_sh, *gate_inp;
  int q6_router, q6_gate, q6_up, q6_down, q6_gate_sh, q6_up_sh, q6_down_sh, q6_gate_inp;
};
struct MoeLayerPlan {
  MoePlan moe;
  int n_ff_sh;
  size_t o_logits, o_xb, o_g, o_u, o_h, o_d, o_s;  // [n_tok][...] f32 each
  size_t bytes;
};
bool moe_layer_plan(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, int n_ff_sh,
                    const MoeLayerTypes& q, MoeLayerPlan* plan, bool out_major = false);
hipError_t launch_moe_layer(const MoeLayerPlan& p, const MoeLayerTypes& q, const MoeLayerTensors& w,
                            const float* x, float* out, void* workspace, hipStream_t s);

// Prefill matmul Y[t][r] = sum_c W[r][c] X[t][c], t < m. mode 0: bf16
// activations on bf16 MFMA; mode 1: Q8-quantized activations on int8 MFMA
// (Q4_K and Q8_0 weights). `workspace` holds matmul_workspace_bytes().
bool matmul_shape_ok(uint32_t quant, int64_t rows, int64_t cols, int64_t m, uint32_t mode);
size_t matmul_workspace_bytes(int64_t cols, int64_t m, uint32_t mode);
hipError_t launch_matmul(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x,
                         int64_t m, float* y, uint32_t mode, void* workspace, int q6_signed,
                         hipStream_t stream);
// Activation quantization of the int8 mode: n f32 (n % 32 == 0) -> int8
// codes, per-32 scales and per-32 scale * sum of codes.
hipError_t launch_quantize_q8(const float* x, int64_t n, int8_t* q, float* scales, float* usum,
                              hipStream_t stream);
// The int8 mode's rounding for Q4_K / Q5_K weights: n f32 (n % 256 == 0)
// -> int8 codes, one scale per 256 and the integer code sum per 32.
hipError_t launch_quantize_q8k(const float* x, int64_t n, int8_t* q, float* scales, int32_t* sums,
                               hipStream_t stream);

// The trait's elementwise methods over `rows` rows of n floats (rope:
// head_dim floats per row, row r at position pos0 + r / heads_per_pos).
// rowops_shape_ok bounds rows and n for the grids.
bool rowops_shape_ok(int64_t rows, int64_t n);
hipError_t launch_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t n, double eps,
                           hipStream_t stream);
hipError_t launch_l2_norm(float* x, int64_t rows, int64_t n, double eps, hipStream_t stream);
hipError_t launch_softmax(float* x, int64_t rows, int64_t n, hipStream_t stream);
hipError_t launch_rope_neox(float* x, int64_t rows, int64_t head_dim, int64_t n_rot, uint64_t pos0,
                            int64_t heads_per_pos, double freq_base, hipStream_t stream);
hipError_t launch_add(float* a, const float* b, int64_t n, hipStream_t stream);
hipError_t launch_add_out(float* out, const float* a, const float* b, int64_t n, hipStream_t stream);

// A plain streaming read of n bytes (16-byte aligned, a multiple of 16):
// workgroup b of kStreamBlocks writes the XOR of the 32-bit words it read to
// out[b]; the XOR of out[] is the XOR of all words.
constexpr int kStreamBlocks = 2048;
hipError_t launch_stream_read(const void* data, uint64_t nbytes, uint32_t* out, hipStream_t stream);
// n bytes from src to dst (device memory or mapped pinned host memory).
hipError_t launch_copy_bytes(const void* src, void* dst, uint64_t n, hipStream_t stream);

}  // namespace sh
