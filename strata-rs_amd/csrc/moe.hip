// Routed mixture-of-experts FFN on the device.
//
// Semantics: crates/strata-core/src/moe.rs:48-127, routed part, from router
// logits:
//   route   softmax over all experts (max-shifted, f32 exp, f64 sum,
//           inv = f32(1/sum)), top-k by descending probability with ties to
//           the lower id, ids ascending, weights w / max(sum_f64, 2^-14);
//   combine for each selected expert in ascending id order with w != 0:
//           h = gate_e . x, p = up_e . x, h = silu(h) * p, d = down_e . h,
//           out += w * d.
// Expert tensors are in the reference orientation [n_expert][in][out]
// (crates/strata-core/src/weights.rs:14-34). The shared expert
// (moe.rs:129-143) is not part of this op.
//
// Four launches:
//   K0 route: one workgroup routes every token and groups the (token, expert)
//      pairs by expert: unique experts in ascending id order ("slots"), each
//      with its tokens in ascending order ("pairs").
//   KA gate+up: workgroup (slot, matrix, row chunk) streams that expert's rows
//      once and applies them to all of the slot's tokens (two at a time, the
//      repeats of a chunk hit in L2); partial sums per chunk.
//   KB down: workgroup (slot, row chunk) first forms a = silu(h) * p for the
//      slot's tokens from the KA partials, then streams the down rows.
//   KC combine: out[t] = sum over t's experts in ascending id of w * d.
// Weight bytes cross HBM once per unique expert, however many tokens chose it.
#include "common.hpp"
#include "kernels.hpp"

namespace sh {

// Device axpy units shared with the expert matvec (same 64-column units).
struct AxQ4K;
struct AxQ6K;
struct AxQ8;

}  // namespace sh
