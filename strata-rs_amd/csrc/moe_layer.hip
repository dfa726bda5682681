// The whole MoE layer on the device: MoeLayer::route and MoeLayer::combine
// (crates/strata-core/src/moe.rs:48-143) for n_tok tokens.
//
//   route    x_bf = bf16(x), rounded to nearest even (hyper.rs:22-24), and
//            logits = router . x_bf (ops::gemv, moe.rs:55-56); then the
//            routed FFN of moe.hip: softmax, top-k, the experts, and
//            out = sum over the token's experts (ascending id) of w * d;
//   shared   g = gate_shexp . x, u = up_shexp . x, h = silu(g) * u,
//            d = down_shexp . h, s = gate_inp_shexp . x (ops::gemv each,
//            moe.rs:129-138);
//   combine  out += sigmoid(s) * d, after the routed sum (moe.rs:139-142),
//            inside the routed combine kernel.
// For several tokens the shared expert runs on a second stream, forked from
// and joined back to the caller's (just before the combine), beside the route
// and the routed experts; for one token it is two launches on the caller's
// stream (gate and up as one matvec, silu(g) * u formed inside the down
// launch). A plain-float router rounds x to bf16 as its matvec loads it, and
// a gate-input row of the same plain type shares its launch. The matvecs are
// the library's gemv kernels (F32 / F16 / BF16 rows sum in f64 as ops::gemv
// does; Q8_0 / Q4_K / Q6_K on the integer-limb path), up to 8 tokens per
// launch.
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// bf16(x) for a quantized router (a plain-float router rounds x as it loads
// it, inside the matvec).
__global__ void bf16_round_kernel(const float* __restrict__ x, float* __restrict__ xb, int64_t n) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  xb[i] = bf16_rne(x[i]);
}

// h = silu(g) * u with silu(v) = v / (1 + exp(-v)) in f32 (ops.rs:85-87).
__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ h,
                                int64_t n) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  const float v = g[i];
  h[i] = v / (1.f + expf(-v)) * u[i];
}

hipError_t launch_silu_mul(const float* g, const float* u, float* h, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
  return hipGetLastError();
}

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

bool moe_layer_plan(int n_tok, int top_k, int n_expert, int n_embd, int n_ff, int n_ff_sh,
                    const MoeLayerTypes& q, MoeLayerPlan* plan, bool out_major) {
  MoeLayerPlan p{};
  if (!moe_plan(n_tok, top_k, n_expert, n_embd, n_ff, q.gate, q.down, &p.moe, out_major)) return false;
  if (q.up != q.gate || n_ff_sh <= 0) return false;
  // the matvecs of the layer, at the shapes the gemv kernels take
  if (!gemv_shape_ok(q.router, n_expert, n_embd, 1) || !gemv_shape_ok(q.gate_sh, n_ff_sh, n_embd, 1) ||
      !gemv_shape_ok(q.up_sh, n_ff_sh, n_embd, 1) || !gemv_shape_ok(q.down_sh, n_embd, n_ff_sh, 1) ||
      !gemv_shape_ok(q.gate_inp, 1, n_embd, 1))
    return false;
  if (n_ff_sh % 4 != 0) return false;  // h rows stay 16-byte aligned as gemv inputs
  size_t o = align256(p.moe.bytes);
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  const size_t T = size_t(n_tok);
  p.o_logits = take(sizeof(float) * T * n_expert);
  p.o_xb = take(sizeof(float) * T * n_embd);
  p.o_g = take(sizeof(float) * 2 * T * n_ff_sh);  // g, or [g | u] from one two-matrix launch
  p.o_u = take(sizeof(float) * T * n_ff_sh);
  p.o_h = take(sizeof(float) * T * n_ff_sh);
  p.o_d = take(sizeof(float) * T * n_embd);
  p.o_s = take(sizeof(float) * T);
  p.bytes = o;
  p.n_ff_sh = n_ff_sh;
  *plan = p;
  return true;
}

// y[t] = W . x[t] for t < n_tok, 8 tokens per launch; `xbf16`: W . bf16(x[t])
// (plain-float W only).
static hipError_t gemv_tokens(uint32_t quant, const void* w, int rows, int cols, const float* x, float* y,
                              int n_tok, int q6s, hipStream_t s, bool xbf16 = false) {
  for (int t0 = 0; t0 < n_tok; t0 += 8) {
    const int nb = n_tok - t0 < 8 ? n_tok - t0 : 8;
    const float* xt = x + int64_t(t0) * cols;
    float* yt = y + int64_t(t0) * rows;
    const hipError_t e = xbf16 ? launch_gemv_plain_bf16x(quant, w, rows, cols, xt, yt, nb, s)
                               : launch_gemv(quant, w, rows, cols, xt, yt, nb, q6s, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// A second stream per (thread, device) for the shared expert: forked from
// the caller's stream with an event and joined back before the final add,
// so the shared expert runs beside the routed experts (under stream capture
// the two become parallel branches of the graph). Thread-local, so
// concurrent callers (and concurrent captures) never share it; default
// priority, like every stream here. The streams live until the process
// ends (no destructor: at exit the runtime may already be gone).
namespace {
struct SideStreams {
  int dev[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
  hipStream_t s[8] = {};
};
thread_local SideStreams g_side;

hipError_t side_stream(hipStream_t* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  for (int i = 0; i < 8; ++i) {
    if (g_side.dev[i] == dev) {
      *out = g_side.s[i];
      return hipSuccess;
    }
    if (g_side.dev[i] < 0) {
      e = hipStreamCreateWithFlags(&g_side.s[i], hipStreamNonBlocking);
      if (e != hipSuccess) return e;
      g_side.dev[i] = dev;
      *out = g_side.s[i];
      return hipSuccess;
    }
  }
  *out = nullptr;  // more than 8 devices on one thread: no side stream
  return hipSuccess;
}
}  // namespace

hipError_t launch_moe_layer(const MoeLayerPlan& p, const MoeLayerTypes& q, const MoeLayerTensors& w,
                            const float* x, float* out, void* workspace, hipStream_t s) {
  const MoePlan& m = p.moe;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* logits = reinterpret_cast<float*>(ws + p.o_logits);
  float* xb = reinterpret_cast<float*>(ws + p.o_xb);
  float* g = reinterpret_cast<float*>(ws + p.o_g);
  float* u = reinterpret_cast<float*>(ws + p.o_u);
  float* h = reinterpret_cast<float*>(ws + p.o_h);
  float* d = reinterpret_cast<float*>(ws + p.o_d);
  float* sg = reinterpret_cast<float*>(ws + p.o_s);
  const int T = m.n_tok, E = m.n_expert, n_embd = m.n_embd, n_sh = p.n_ff_sh;
  const int64_t nx = int64_t(T) * n_embd, nh = int64_t(T) * n_sh;
  auto blocks = [](int64_t n) { return dim3(unsigned((n + 255) / 256)); };
  hipError_t e;
  // fewer launches where the types allow: one token's shared expert in two
  // launches, the router and the gate-input row in one
  const bool fuse_sh = T == 1 && q.gate_sh == q.up_sh && w.q6_gate_sh == w.q6_up_sh &&
                       shexp_fused_ok(q.gate_sh, q.down_sh, n_embd, n_sh);
  const bool pair_rg = plain_quant(q.router) && q.gate_inp == q.router;
  // the shared expert on the side stream (on `s` itself without one); its
  // two-launch form costs less on `s` than a fork and join (one token, in a
  // captured graph: 41.8 against 47.0 us), the many-token form runs faster
  // beside the routed experts (16 tokens: 155 against 182 us)
  hipStream_t side = nullptr;
  if (!fuse_sh && (e = side_stream(&side)) != hipSuccess) return e;
  hipEvent_t fork = nullptr, join = nullptr;
  if (side) {
    if ((e = hipEventCreateWithFlags(&fork, hipEventDisableTiming)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&join, hipEventDisableTiming)) != hipSuccess) {
      (void)hipEventDestroy(fork);
      return e;
    }
  }
  auto run = [&]() -> hipError_t {
    hipError_t r;
    hipStream_t ss = s;
    if (side) {
      if ((r = hipEventRecord(fork, s)) != hipSuccess) return r;
      if ((r = hipStreamWaitEvent(side, fork, 0)) != hipSuccess) return r;
      ss = side;
    }
    if (fuse_sh) {
      // one token: [g | u] in one launch, then down with silu(g) * u staged
      if ((r = launch_shexp_one(q.gate_sh, q.down_sh, w.gate_sh, w.up_sh, w.down_sh, n_embd, n_sh, x, g, d,
                                w.q6_gate_sh, w.q6_down_sh, ss)) != hipSuccess)
        return r;
    } else {
      if ((r = gemv_tokens(q.gate_sh, w.gate_sh, n_sh, n_embd, x, g, T, w.q6_gate_sh, ss)) != hipSuccess) return r;
      if ((r = gemv_tokens(q.up_sh, w.up_sh, n_sh, n_embd, x, u, T, w.q6_up_sh, ss)) != hipSuccess) return r;
      hipLaunchKernelGGL(silu_mul_kernel, blocks(nh), dim3(256), 0, ss, g, u, h, nh);
      if ((r = gemv_tokens(q.down_sh, w.down_sh, n_embd, n_sh, h, d, T, w.q6_down_sh, ss)) != hipSuccess) return r;
    }
    if (!pair_rg &&
        (r = gemv_tokens(q.gate_inp, w.gate_inp, 1, n_embd, x, sg, T, w.q6_gate_inp, ss)) != hipSuccess)
      return r;
    if (side && (r = hipEventRecord(join, side)) != hipSuccess) return r;
    // route: router . bf16(x), then the routed experts into out; the combine
    // waits for the shared expert and adds sigmoid(s) * d after the routed sum
    if (pair_rg) {
      // the router on bf16(x) and the gate-input row on x in one launch
      for (int t0 = 0; t0 < T; t0 += 8) {
        const int nb = T - t0 < 8 ? T - t0 : 8;
        if ((r = launch_gemv_plain_pair(q.router, w.router, E, w.gate_inp, 1, n_embd, x + int64_t(t0) * n_embd,
                                        logits + int64_t(t0) * E, sg + t0, nb, s)) != hipSuccess)
          return r;
      }
    } else if (plain_quant(q.router)) {
      if ((r = gemv_tokens(q.router, w.router, E, n_embd, x, logits, T, 0, s, true)) != hipSuccess) return r;
    } else {
      hipLaunchKernelGGL(bf16_round_kernel, blocks(nx), dim3(256), 0, s, x, xb, nx);
      if ((r = gemv_tokens(q.router, w.router, E, n_embd, xb, logits, T, w.q6_router, s)) != hipSuccess) return r;
    }
    const MoeShared shared{d, sg, side ? join : nullptr};
    if ((r = launch_moe(m, q.gate, q.up, q.down, w.gate, w.up, w.down, w.q6_gate, w.q6_up, w.q6_down, logits, x,
                        out, workspace, s, &shared)) != hipSuccess)
      return r;
    return hipGetLastError();
  };
  e = run();
  if (side) {
    (void)hipEventDestroy(fork);
    (void)hipEventDestroy(join);
  }
  return e;
}

}  // namespace sh
