// Internal launch interface between the C ABI (api.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sihip {

// Device memory a context lends to the kernels that combine partial sums
// across workgroups: kWorkspaceCounterBytes of zeroed counters, then entries
// that hold kWorkspaceEmpty when unused (kWorkspaceBytes in all; the kernels
// leave it in that state), then kWorkspaceScratchBytes of scratch that a
// launch overwrites before it reads (partial sums handed from one kernel to
// the next in the same stream).
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  float* scratch = nullptr;
  size_t scratch_bytes = 0;
};
constexpr size_t kWorkspaceBytes = size_t(2) << 20;
constexpr size_t kWorkspaceScratchBytes = size_t(8) << 20;
constexpr size_t kWorkspaceCounterBytes = size_t(1) << 20;
// a signalling-NaN pattern: no arithmetic result has it (results of
// operations are quiet NaNs)
constexpr uint32_t kWorkspaceEmpty = 0x7fbadbadu;
// the argmax reduction's counter (the last counter word) and its 256 u64
// entries (the last 4 KB)
constexpr size_t kWorkspaceArgmaxCounter = kWorkspaceCounterBytes - 4;
constexpr size_t kWorkspaceArgmaxEntries = kWorkspaceBytes - 4096;

// silu(g) * u exactly as src/runtime.rs:4296-4298 / metal.rs:585 write it.
__host__ __device__ __forceinline__ float silu_times(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

// Greedy-argmax tie rules.
enum ArgmaxRule : uint32_t {
  kArgmaxLastFinite = 0,     // runtime.rs:4301-4309 (finite, total order, last max)
  kArgmaxFirstGreater = 1,   // qwen35_runtime.rs:2237-2244 (strict '>', first max)
};

// Packed (order key, index) candidate: larger is better; 0 = no candidate.
__host__ __device__ __forceinline__ uint64_t argmax_candidate(float v, uint32_t index,
                                                              uint32_t rule) {
  uint32_t bits;
  if (rule == kArgmaxFirstGreater) {
    if (v != v || v == -__builtin_huge_valf()) return 0;  // never beats -inf
    v = v + 0.0f;                                         // -0 == +0 under '>'
  } else {
    if (!__builtin_isfinite(v)) return 0;
  }
  __builtin_memcpy(&bits, &v, 4);
  const int32_t key = (int32_t)bits ^ (int32_t)((uint32_t)((int32_t)bits >> 31) >> 1);
  const uint32_t ukey = (uint32_t)key ^ 0x80000000u;
  const uint32_t tie = rule == kArgmaxFirstGreater ? 0xffffffffu - index : index;
  return ((uint64_t)ukey << 32) | tie;
}

__host__ __device__ __forceinline__ uint32_t argmax_candidate_index(uint64_t c, uint32_t rule) {
  const uint32_t lo = (uint32_t)c;
  return rule == kArgmaxFirstGreater ? 0xffffffffu - lo : lo;
}

// noalloc.hip: sets up the current device's workspace of
// si_hip_quant_matvec_noalloc (once per device; `stream` not under capture).
int noalloc_setup(hipStream_t stream);

// kernels_generic.hip
hipError_t launch_matvec_generic(uint32_t type, const uint8_t* w, const float* x, float* y,
                                 uint32_t rows, uint32_t cols, uint32_t batch, hipStream_t s);
hipError_t launch_fused_gate_up_generic(const uint8_t* gate, const uint8_t* up, const float* x,
                                        float* h, uint32_t rows, uint32_t cols, hipStream_t s);
hipError_t launch_dequant(uint32_t type, const uint8_t* w, const uint32_t* row_index, float* out,
                          uint32_t out_rows, uint32_t cols, hipStream_t s);

// kernels_f32.hip: y = W x for a row-major F32 matrix; RMSNorm of `heads`
// vectors of head_dim values, mode 0 (x * inv * w), 1 (x * inv * (1 + w)) or
// 2 (x * inv * w * silu(gate)).
hipError_t launch_f32_matvec(const float* w, const float* x, float* y, uint32_t rows,
                             uint32_t cols, hipStream_t s);
hipError_t launch_rms_norm(uint32_t mode, const float* x, const float* gate, const float* w,
                           float* y, uint32_t heads, uint32_t head_dim, float eps, hipStream_t s);

// kernels_argmax.hip: max-loc over n < 2^31 logits in one launch, using the
// context workspace's argmax area; the winner lands in *result (packed
// candidate, 0 when there is none).
hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t rule, const Workspace& ws,
                         uint64_t* result, hipStream_t s);

}  // namespace sihip
