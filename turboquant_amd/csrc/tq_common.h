// tq_common.h -- shared constants and small helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/turboquant_amd.h"

namespace tq {

constexpr int kEinval = -22;
constexpr int kTile = 16;  // tokens per decode tile (one MFMA M/K block)

// 16-level Lloyd-Max centroids for N(0,1) (reference page_turbo.cuh:18-23).
// The table is symmetric: c[15-i] == -c[i].
__host__ __device__ constexpr float codebook(int i) {
  constexpr float c[16] = {
      -2.7326368f, -2.0693470f, -1.6180345f, -1.2562491f,
      -0.9423684f, -0.6567591f, -0.3880823f, -0.1284154f,
      0.1284154f,  0.3880823f,  0.6567591f,  0.9423684f,
      1.2562491f,  1.6180345f,  2.0693470f,  2.7326368f};
  return c[i];
}

// Positive half of the 15 midpoint boundaries as fp32 literals (reference
// quantize_write_kernel.cuh:22-28); boundary 7 is 0 and the negative half
// mirrors these, so b[7+k] == -b[7-k].
__host__ __device__ constexpr float boundary_pos(int k) {  // k = 1..7 -> b[7+k]
  constexpr float b[8] = {0.0f,
                          0.2582488430577470f, 0.5224207238480534f,
                          0.7995637494657970f, 1.0993087223329937f,
                          1.4371417912897455f, 1.8436907609368955f,
                          2.4009919259139040f};
  return b[k];
}

// Thread-local error message for the C ABI.
void set_error(const char* fmt, ...);

// Compute units of the current device, queried once per device (0 if unknown).
int device_cus();

}  // namespace tq
