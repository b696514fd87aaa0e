// Device side of the greedy argmax's cross-workgroup reduction, shared by the
// standalone argmax kernel and the Q6_K output-head kernel that fuses it.
//
// Every workgroup publishes its best packed candidate (argmax_candidate: one
// u64 whose unsigned order is the tie rule's order) as its entry of the
// workspace's argmax area and counts it on the area's counter; the workgroup
// that counts last reduces all entries into the result and puts the area
// back (entries empty, counter zero).  No fence orders an entry's store
// before its count: the last workgroup waits, bounded, for each entry to
// leave the empty state.
#pragma once

#include "si_hip_internal.h"

namespace sihip {

// 64-bit entry that holds no candidate: the area is filled with the 32-bit
// empty pattern.  A candidate with this value would index row 0x7fbadbad or
// beyond (kArgmaxMaxRows keeps launches below).
constexpr uint64_t kArgmaxNoEntry = ((uint64_t)kWorkspaceEmpty << 32) | kWorkspaceEmpty;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = umax64(v, __shfl_xor(v, off, 64));
  return v;
}

// Called by one whole wave of each workgroup, with the workgroup's best
// candidate `best` (the same in every lane; 0 = none).  In the workgroup
// that completes the count, the wave stores the grid's best candidate (0 when
// there is none) to *result.  The wait for entries is bounded (about 2^22
// polls, or the workspace's test-hook count): on giving up the wave reports
// kDevErrArgmaxWait and reduces the entries that did land.
__device__ inline void argmax_publish_wave(uint64_t best, void* ws, uint64_t* result,
                                           uint32_t lane) {
  uint8_t* const base = static_cast<uint8_t*>(ws);
  uint64_t* const parts = reinterpret_cast<uint64_t*>(base + kWorkspaceArgmaxEntries);
  uint32_t* const counter = reinterpret_cast<uint32_t*>(base + kWorkspaceArgmaxCounter);
  uint32_t before = 0u;
  if (lane == 0u) {
    __hip_atomic_store(parts + blockIdx.x, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  before = __builtin_amdgcn_readlane(before, 0);
  if (before != gridDim.x - 1u) return;
  const uint32_t force = __builtin_amdgcn_readfirstlane(give_up_polls(ws));
  const uint32_t cap = force != 0u ? force : (1u << 22);
  uint64_t m = 0u;
  for (uint32_t b0 = 0; b0 < gridDim.x; b0 += 64u) {
    const uint32_t b = b0 + lane;
    const bool mine = b < gridDim.x;
    uint64_t v = mine ? __hip_atomic_load(parts + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0u;
    for (uint32_t spin = 0;; ++spin) {
      const bool missing = mine && (force != 0u || v == kArgmaxNoEntry);
      if (!__builtin_amdgcn_ballot_w64(missing)) break;
      if (spin == cap) {
        report_device_error(ws, kDevErrArgmaxWait);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if (missing) v = __hip_atomic_load(parts + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (mine) {
      m = umax64(m, v == kArgmaxNoEntry ? 0u : v);
      __hip_atomic_store(parts + b, kArgmaxNoEntry, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  m = wave_max_u64(m);
  if (lane == 0u) {
    *result = m;
    (void)__hip_atomic_exchange(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace sihip
