// Greedy argmax over a logits vector in HBM (src/runtime.rs:4301-4309 and the
// first-wins variant at src/qwen35_runtime.rs:2237-2244).  Each candidate is
// packed into one u64 whose unsigned order is the tie rule's order, so the
// reduction is a plain max and the result does not depend on timing.
#include "argmax_device.h"

namespace sihip {
namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kMaxBlocks = 256;

// One launch: every block reduces a grid-strided share of the logits, then
// its first wave publishes the block's best candidate (argmax_publish_wave),
// and the block that counts last stores the result.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ logits,
                                                          uint32_t n, uint32_t rule, void* ws,
                                                          uint64_t* __restrict__ result) {
  __shared__ uint64_t wave_best[kThreads / 64];
  uint64_t best = 0;
  for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
    best = umax64(best, argmax_candidate(logits[i], i, rule));
  best = wave_max_u64(best);
  const uint32_t wave = threadIdx.x / 64u, lane = threadIdx.x & 63u;
  if (lane == 0u) wave_best[wave] = best;
  __syncthreads();
  if (wave != 0u) return;
  uint64_t m = lane < kThreads / 64u ? wave_best[lane] : 0u;
  argmax_publish_wave(wave_max_u64(m), ws, result, lane);
}

}  // namespace

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t rule, const Workspace& ws,
                         uint64_t* result, hipStream_t s) {
  if (ws.bytes < kWorkspaceBytes || n == 0 || n >= kArgmaxMaxRows) return hipErrorInvalidValue;
  static_assert(kMaxBlocks <= kArgmaxMaxGroups, "an entry per block");
  const uint32_t blocks = min(kMaxBlocks, (n + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kThreads), 0, s, logits, n, rule, ws.ptr,
                     result);
  return hipGetLastError();
}

}  // namespace sihip
