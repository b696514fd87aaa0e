// Tuned gfx950 K-quant kernels (placeholder until the streaming kernels land).
#include "si_hip_tuned.h"

namespace sihip {

bool launch_matvec_tuned(uint32_t, const uint8_t*, const float*, float*, uint32_t, uint32_t,
                         uint32_t, hipStream_t, hipError_t*) {
  return false;
}

bool launch_fused_gate_up_tuned(const uint8_t*, const uint8_t*, const float*, float*, uint32_t,
                                uint32_t, hipStream_t, hipError_t*) {
  return false;
}

}  // namespace sihip
