// Dispatch of the tuned gfx950 kernels (kernels_q4k_mfma.hip,
// kernels_q6k_mfma.hip): which matrix-core kernel takes a quantized matvec of
// a given type and batch.  A shape none of them takes returns false, and the
// caller runs the exact generic kernels (kernels_generic.hip).
#include "kquant_device.h"
#include "si_hip_tuned.h"

#include <cstdlib>

namespace sihip {
namespace {

int env_flag(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

}  // namespace

bool launch_matvec_tuned(uint32_t type, const uint8_t* w, const float* x, float* y, uint32_t rows,
                         uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                         hipError_t* err) {
  if (batch == 0) return false;
  const bool q4_mfma = type == kTypeQ4K;
  static const int tokens_per_pass = env_flag("SI_HIP_Q4K_BATCH_PASS", 1);
  if (q4_mfma && batch > 1 && tokens_per_pass &&
      launch_q4k_matmul_mfma(w, x, y, rows, cols, batch, ws, s, err))
    return true;
  if (type == kTypeQ5K)
    return batch == 1 ? launch_q5k_matvec_mfma(w, x, y, rows, cols, ws, s, err)
                      : launch_q5k_matmul_mfma(w, x, y, rows, cols, batch, ws, s, err);
  if (type == kTypeQ6K && batch > 1 &&
      launch_q6k_matmul_mfma(w, x, y, rows, cols, batch, ws, s, err))
    return true;
  if (type == kTypeQ6K || (q4_mfma && batch > 1)) {
    // several candidates (batch-major x and y, metal.rs:1104-1126): one
    // matrix-core matvec per candidate, each bit-identical to its M = 1 call
    for (uint32_t b = 0; b < batch; ++b) {
      const float* xb = x + (size_t)b * cols;
      float* yb = y + (size_t)b * rows;
      const bool ok = type == kTypeQ6K ? launch_q6k_matvec_mfma(w, xb, yb, rows, cols, ws, s, err)
                                       : launch_q4k_matvec_mfma(w, xb, yb, rows, cols, ws, s, err);
      if (!ok) return b == 0 ? false : (*err = hipErrorInvalidValue, true);
      if (*err != hipSuccess) return true;
    }
    return true;
  }
  if (type != kTypeQ4K || batch != 1) return false;
  return launch_q4k_matvec_mfma(w, x, y, rows, cols, ws, s, err);
}

bool launch_fused_gate_up_tuned(const uint8_t* gate, const uint8_t* up, const float* x, float* h,
                                uint32_t rows, uint32_t cols, const Workspace& ws, hipStream_t s,
                                hipError_t* err) {
  return launch_q4k_gate_up_mfma(gate, up, x, h, rows, cols, ws, s, err);
}

}  // namespace sihip
