// Greedy argmax over a logits vector in HBM (src/runtime.rs:4301-4309 and the
// first-wins variant at src/qwen35_runtime.rs:2237-2244).  Each candidate is
// packed into one u64 whose unsigned order is the tie rule's order, so the
// reduction is a plain max and the result does not depend on timing.
#include "si_hip_internal.h"

namespace sihip {
namespace {

constexpr uint32_t kThreads = 256;

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

// 64-bit entry of the workspace's argmax area that holds no candidate: the
// area is filled with the 32-bit empty pattern.  No candidate has this value:
// it would need a row index of at least 2^31.
constexpr uint64_t kNoPartial = ((uint64_t)kWorkspaceEmpty << 32) | kWorkspaceEmpty;
constexpr uint32_t kMaxBlocks = 256;

__device__ __forceinline__ void store_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_u64(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One launch: every block reduces a grid-strided share of the logits and
// publishes its best candidate; the block that arrives last (counted on a
// device-scope counter) waits for every published candidate -- entries hold
// kNoPartial until their store lands -- reduces them, stores the result and
// puts the area back (entries empty, counter zero).
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ logits,
                                                          uint32_t n, uint32_t rule,
                                                          uint64_t* __restrict__ parts,
                                                          uint32_t* __restrict__ counter,
                                                          uint64_t* __restrict__ result) {
  __shared__ uint64_t smem[kThreads / 64];
  __shared__ uint32_t last;
  uint64_t best = 0;
  for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
    best = umax64(best, argmax_candidate(logits[i], i, rule));
  best = block_max(best, smem);
  if (threadIdx.x == 0) {
    store_u64(parts + blockIdx.x, best);
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           gridDim.x - 1u;
  }
  __syncthreads();
  if (!last) return;
  uint64_t m = 0;
  for (uint32_t b = threadIdx.x; b < gridDim.x; b += kThreads) {
    uint64_t v = load_u64(parts + b);
    for (uint32_t spin = 0; v == kNoPartial && spin < (1u << 22); ++spin) {
      __builtin_amdgcn_s_sleep(1);
      v = load_u64(parts + b);
    }
    m = umax64(m, v);
    store_u64(parts + b, kNoPartial);
  }
  m = block_max(m, smem);
  if (threadIdx.x == 0) {
    *result = m;
    (void)__hip_atomic_exchange(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t rule, const Workspace& ws,
                         uint64_t* result, hipStream_t s) {
  if (ws.bytes < kWorkspaceBytes || n == 0 || n >= 0x80000000u) return hipErrorInvalidValue;
  uint8_t* base = static_cast<uint8_t*>(ws.ptr);
  uint64_t* parts = reinterpret_cast<uint64_t*>(base + kWorkspaceArgmaxEntries);
  uint32_t* counter = reinterpret_cast<uint32_t*>(base + kWorkspaceArgmaxCounter);
  const uint32_t blocks = min(kMaxBlocks, (n + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kThreads), 0, s, logits, n, rule, parts,
                     counter, result);
  return hipGetLastError();
}

}  // namespace sihip
