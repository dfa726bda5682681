// The dense FFN half of a decoder layer (crates/strata-core/src/qwen35.rs:
// 112-129) on the device, for n_tok tokens:
//   mixed = rms_norm_into(x, post_norm, eps)            (ops.rs:59-69)
//   g = gate . mixed, u = up . mixed                     (ops::gemv)
//   h = g / (1 + exp(-g)) * u                            (qwen35.rs:120-124, f32)
//   out = x + down . h                                   (qwen35.rs:127-129, f32)
// One token with the three matrices of one quantized type takes three
// launches: rms_norm, gate and up in one matvec launch (x staged once), and
// down with silu(g) * u formed while its x is staged and the residual added
// as its sums are written. Otherwise each step is its own launch (matvecs 8
// tokens at a time).
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// [mixed: n_tok x n_embd][gu: n_tok x 2 n_ff][h: n_tok x n_ff][m: n_tok x n_embd]
size_t ffn_workspace_bytes(int64_t n_tok, int64_t n_embd, int64_t n_ff) {
  const size_t T = size_t(n_tok);
  return align256(sizeof(float) * T * n_embd) + align256(sizeof(float) * T * 2 * n_ff) +
         align256(sizeof(float) * T * n_ff) + align256(sizeof(float) * T * n_embd);
}

static hipError_t gemv_rows(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x, float* y,
                            int n_tok, int q6s, hipStream_t s) {
  for (int t0 = 0; t0 < n_tok; t0 += 8) {
    const int nb = n_tok - t0 < 8 ? n_tok - t0 : 8;
    const hipError_t e = launch_gemv(quant, w, rows, cols, x + int64_t(t0) * cols, y + int64_t(t0) * rows, nb,
                                     q6s, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_ffn(uint32_t q_gate, uint32_t q_up, uint32_t q_down, const void* gate, const void* up,
                      const void* down, int q6g, int q6u, int q6d, int64_t n_embd, int64_t n_ff, int n_tok,
                      const float* x, const float* post_norm, double eps, float* out, void* workspace,
                      hipStream_t s) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const size_t T = size_t(n_tok);
  float* mixed = reinterpret_cast<float*>(ws);
  float* gu = reinterpret_cast<float*>(ws + align256(sizeof(float) * T * n_embd));
  float* h = gu + align256(sizeof(float) * T * 2 * n_ff) / sizeof(float);
  float* m = h + align256(sizeof(float) * T * n_ff) / sizeof(float);
  hipError_t e = launch_rms_norm(x, post_norm, mixed, n_tok, n_embd, eps, s);
  if (e != hipSuccess) return e;
  const bool same = q_gate == q_up && q_up == q_down && q6g == q6u && q6u == q6d;
  if (n_tok == 1 && same && ffn_fused_ok(q_gate, n_embd, n_ff))
    return launch_ffn_one(q_gate, gate, up, down, n_embd, n_ff, mixed, gu, x, out, q6g, s);
  // general path: g in gu[t][0, n_ff), u in gu[t][n_ff, 2 n_ff) as [2][T][n_ff]
  float* g = gu;
  float* u = gu + T * n_ff;
  if ((e = gemv_rows(q_gate, gate, n_ff, n_embd, mixed, g, n_tok, q6g, s)) != hipSuccess) return e;
  if ((e = gemv_rows(q_up, up, n_ff, n_embd, mixed, u, n_tok, q6u, s)) != hipSuccess) return e;
  if ((e = launch_silu_mul(g, u, h, int64_t(T) * n_ff, s)) != hipSuccess) return e;
  if ((e = gemv_rows(q_down, down, n_embd, n_ff, h, m, n_tok, q6d, s)) != hipSuccess) return e;
  return launch_add_out(out, x, m, int64_t(T) * n_embd, s);
}

}  // namespace sh
