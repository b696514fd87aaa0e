// Greedy argmax over a logits vector in HBM (src/runtime.rs:4301-4309 and the
// first-wins variant at src/qwen35_runtime.rs:2237-2244).  Each candidate is
// packed into one u64 whose unsigned order is the tie rule's order, so both
// stages are a plain max-reduction and the result is deterministic.
#include "si_hip_internal.h"

namespace sihip {
namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kPerThread = 16;
constexpr uint32_t kPerBlock = kThreads * kPerThread;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t block_max(uint64_t v, uint64_t* smem) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, 64);
    v = umax64(v, o);
  }
  const uint32_t wave = threadIdx.x / 64u;
  if ((threadIdx.x & 63u) == 0) smem[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = smem[0];
    for (uint32_t w = 1; w < blockDim.x / 64u; ++w) m = umax64(m, smem[w]);
    smem[0] = m;
  }
  __syncthreads();
  return smem[0];
}

__global__ __launch_bounds__(kThreads) void argmax_stage1(const float* __restrict__ logits,
                                                          uint32_t n, uint32_t rule,
                                                          uint64_t* __restrict__ partials) {
  __shared__ uint64_t smem[kThreads / 64];
  uint64_t best = 0;
  const uint32_t base = blockIdx.x * kPerBlock;
#pragma unroll 4
  for (uint32_t k = 0; k < kPerThread; ++k) {
    const uint32_t i = base + k * kThreads + threadIdx.x;
    if (i < n) best = umax64(best, argmax_candidate(logits[i], i, rule));
  }
  best = block_max(best, smem);
  if (threadIdx.x == 0) partials[blockIdx.x] = best;
}

__global__ __launch_bounds__(kThreads) void argmax_stage2(const uint64_t* __restrict__ partials,
                                                          uint32_t count,
                                                          uint64_t* __restrict__ result) {
  __shared__ uint64_t smem[kThreads / 64];
  uint64_t best = 0;
  for (uint32_t i = threadIdx.x; i < count; i += kThreads) best = umax64(best, partials[i]);
  best = block_max(best, smem);
  if (threadIdx.x == 0) *result = best;
}

}  // namespace

uint32_t argmax_partials(uint32_t n) { return (n + kPerBlock - 1) / kPerBlock; }

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t rule, uint64_t* partials,
                         uint64_t* result, hipStream_t s) {
  const uint32_t blocks = argmax_partials(n);
  hipLaunchKernelGGL(argmax_stage1, dim3(blocks), dim3(kThreads), 0, s, logits, n, rule, partials);
  hipLaunchKernelGGL(argmax_stage2, dim3(1), dim3(kThreads), 0, s, partials, blocks, result);
  return hipGetLastError();
}

}  // namespace sihip
