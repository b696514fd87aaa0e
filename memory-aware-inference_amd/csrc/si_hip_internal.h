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
constexpr size_t kWorkspaceScratchBytes = size_t(64) << 20;
constexpr size_t kWorkspaceCounterBytes = size_t(1) << 20;
// a signalling-NaN pattern: no arithmetic result has it (results of
// operations are quiet NaNs)
constexpr uint32_t kWorkspaceEmpty = 0x7fbadbadu;
// Reserved words at the end of the counter region (the tile counters stop
// 64 bytes before its end):
//   kWorkspaceArgmaxCounter  the argmax reduction's counter
//   kWorkspaceGiveUpWord     a test hook, zero otherwise: while it holds
//                            n > 0, the bounded waits of the split-tile
//                            combine and of the argmax reduction take every
//                            entry for missing and give up after n polls
//   kWorkspaceReportSlot     the device address (u64) of the owner's
//                            host-visible error word, or 0 (no owner reads it)
// and the argmax reduction's 512 u64 entries (the last 4 KB).
constexpr size_t kWorkspaceArgmaxCounter = kWorkspaceCounterBytes - 4;
constexpr size_t kWorkspaceGiveUpWord = kWorkspaceCounterBytes - 8;
constexpr size_t kWorkspaceReportSlot = kWorkspaceCounterBytes - 16;
constexpr size_t kWorkspaceArgmaxEntries = kWorkspaceBytes - 4096;
constexpr uint32_t kArgmaxMaxGroups = 512;
// Candidates index fewer rows than this, so that no candidate equals an entry
// that holds none (both halves kWorkspaceEmpty).
constexpr uint32_t kArgmaxMaxRows = 0x7fb00000u;

// What a kernel reports through the error word when it cannot finish its work
// correctly (it still ends normally).
enum DeviceError : uint32_t {
  kDevErrNone = 0,
  kDevErrSlotWait = 1,     // a wave gave up waiting for its tile's LDS slot
  kDevErrCombineWait = 2,  // a split tile's partial sums did not arrive
  kDevErrArgmaxWait = 3,   // a workgroup's argmax candidate did not arrive
  kDevErrTokenId = 4,      // an embedding token id beyond the table
};

// Stores `code` into the workspace owner's error word (a system-scope store
// into host memory; the last report wins).  Taken only on failure paths.
__device__ inline void report_device_error(void* ws, uint32_t code) {
  uint64_t* slot = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(ws) + kWorkspaceReportSlot);
  const uint64_t a = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a != 0u)
    __hip_atomic_store(reinterpret_cast<uint32_t*>(a), code, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
// The test hook's poll count (0: the waits run their normal course).
__device__ inline uint32_t give_up_polls(void* ws) {
  uint32_t* w = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + kWorkspaceGiveUpWord);
  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

// The index a packed best candidate names.  With no candidate (c == 0, no
// logit beat -inf or none was finite): 0 under kArgmaxFirstGreater, the id
// the reference's strict '>' scan keeps when nothing beats its starting -inf
// (qwen35_runtime.rs:2237-2244); kArgmaxNone under kArgmaxLastFinite, where
// the reference returns "logits contain no finite values" (runtime.rs:4301-4309).
constexpr uint32_t kArgmaxNone = 0xffffffffu;
__host__ __device__ __forceinline__ uint32_t argmax_candidate_index(uint64_t c, uint32_t rule) {
  if (c == 0u) return rule == kArgmaxFirstGreater ? 0u : kArgmaxNone;
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
// y[0] = the dot of one row (w: its nb = cols / 256 blocks) with x, by one
// workgroup.
hipError_t launch_row_dot(uint32_t type, const uint8_t* w, const float* x, float* y,
                          uint32_t cols, hipStream_t s);
// Dequantises out_rows rows; with row_index, output row r is table row
// row_index[r], and an index of table_rows or more gives a row of NaNs and
// reports kDevErrTokenId through the workspace `ws` (when not null).
hipError_t launch_dequant(uint32_t type, const uint8_t* w, const uint32_t* row_index, float* out,
                          uint32_t out_rows, uint32_t cols, hipStream_t s,
                          uint32_t table_rows = 0xffffffffu, void* ws = nullptr);

// kernels_f32.hip: y = W x for a row-major F32 matrix; RMSNorm of `heads`
// vectors of head_dim values, mode 0 (x * inv * w), 1 (x * inv * (1 + w)) or
// 2 (x * inv * w * silu(gate)).
hipError_t launch_f32_matvec(const float* w, const float* x, float* y, uint32_t rows,
                             uint32_t cols, hipStream_t s);
hipError_t launch_rms_norm(uint32_t mode, const float* x, const float* gate, const float* w,
                           float* y, uint32_t heads, uint32_t head_dim, float eps, hipStream_t s);

// kernels_probe.hip: one launch of the matrix-core kernels' weight stream
// alone (Q4_K / Q5_K blocks of block_bytes, a grid of min(tiles, cus)).
enum ProbeMode : uint32_t {
  kProbeDefault = 0,      // the kernels' copies, default cache policy
  kProbeNontemporal = 1,  // the same with the nontemporal bit
  kProbeEmpty = 2,        // the launch shape with no work
  kProbeWide = 3,         // the same stages as 4-row x 256-byte copies
  kProbeLines = 4,        // Q4_K: whole 128-byte lines (the one-vector kernel's copies)
  kProbeRegisters = 5,    // Q4_K: 16-byte loads into registers, two stages in flight
  kProbeRegistersNontemporal = 6,  // the same with the nontemporal bit
};
hipError_t launch_stream_probe(uint32_t mode, const uint8_t* w, uint32_t rows, uint32_t cols,
                               uint32_t block_bytes, uint32_t cus, hipStream_t s);

// kernels_argmax.hip: max-loc over n < kArgmaxMaxRows logits in one launch, using the
// context workspace's argmax area; the winner lands in *result (packed
// candidate, 0 when there is none).
hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t rule, const Workspace& ws,
                         uint64_t* result, hipStream_t s);

}  // namespace sihip
