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
hipError_t launch_gemv(uint32_t quant, const void* w, int64_t rows, int64_t cols, const float* x,
                       float* y, int batch, int q6_signed, hipStream_t stream);

// y[c] = sum_i x[i] * W[i][c] for one expert matrix W[rows = in][cols = out]
// (reference orientation). `workspace` holds expert_workspace_bytes().
bool expert_shape_ok(uint32_t quant, int64_t rows, int64_t cols);
size_t expert_workspace_bytes(int64_t rows, int64_t cols);
hipError_t launch_expert_gemv(uint32_t quant, const void* w, int64_t rows, int64_t cols,
                              const float* x, float* y, float* workspace, int q6_signed,
                              hipStream_t stream);

}  // namespace sh
