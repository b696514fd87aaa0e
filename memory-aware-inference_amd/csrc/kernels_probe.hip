// Measurement probe: the weight stream of the Q4_K / Q5_K matrix-core
// kernels without their arithmetic.
//
// The launch has the shape of the one-vector kernel (one workgroup of twelve
// waves per CU, 16-row tiles of 4-block stages dealt to the workgroups, a
// workgroup's (tile, stage) pairs dealt to its waves round-robin) and every
// wave copies its stages into its own LDS buffer with the same 16-byte
// buffer->LDS instructions (16 rows x 64 bytes each), one stage in flight,
// then reads nothing.  Mode kProbeNontemporal sets the nontemporal bit on
// the copies; mode kProbeEmpty launches the same grid with no work.  The
// time of back-to-back launches bounds what the matvec kernels can reach on
// this copy path.
//
// Mode kProbeWide times another copy form of the same stages: each copy
// instruction reads 4 rows x 256 contiguous bytes (lane l: row 4 g + l / 16
// of the copy's row group g, the 16-byte piece (l - row) mod 16 of the copy's
// 256-byte column, so that a later 16-lane read of one piece of 16 rows would
// still meet 16 different LDS bank groups), and the pieces past the last
// whole 256-byte column go as 16 rows x 64 bytes.
#include "si_hip_internal.h"

#include <algorithm>

namespace sihip {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kWaves = 12;

template <int AUX, bool EMPTY, bool WIDE = false>
__global__ __launch_bounds__(kWaves * 64) void stream_probe(const uint8_t* __restrict__ w,
                                                            uint32_t rows, uint32_t nb,
                                                            uint32_t block_bytes,
                                                            uint32_t* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  if constexpr (EMPTY) {
    if (threadIdx.x == 0xffffu) sink[0] = 0u;  // never: keeps the launch
    return;
  }
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t row_bytes = nb * block_bytes;
  const uint32_t nstages = (nb + 3u) / 4u;
  const uint32_t stage_bytes = 4u * block_bytes;        // per row
  const uint32_t pieces = (stage_bytes + 63u) / 64u;    // copy instructions per stage
  const uint32_t row_pieces = (stage_bytes + 15u) / 16u;
  const uint32_t ncol = row_pieces / 16u;              // WIDE: whole 256-byte columns
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t my_tiles = blockIdx.x < ntiles ? (ntiles - 1u - blockIdx.x) / gridDim.x + 1u : 0u;
  const uint32_t npairs = my_tiles * nstages;
  uint8_t* const buf = smem + wave * 1024u * pieces;
  for (uint32_t k = wave; k < npairs; k += kWaves) {
    const uint32_t lt = k / nstages, st = k - lt * nstages;
    const uint32_t tile = blockIdx.x + gridDim.x * lt;
    const uint32_t row0 = tile * 16u, nrows = min(16u, rows - row0);
    const uint8_t* sb = w + (size_t)row0 * row_bytes + stage_bytes * st;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - stage_bytes * st), kBufferWord3);
    if constexpr (WIDE) {
      uint32_t i = 0;
      for (; i < 4u * ncol; ++i) {
        const uint32_t row = 4u * (i & 3u) + grp;
        const uint32_t piece = 16u * (i >> 2) + ((n - row) & 15u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(buf + 1024u * i), 16,
                                                  row * row_bytes + 16u * piece, 0, 0, AUX);
      }
      for (uint32_t t = 0; 16u * ncol + 4u * t < row_pieces; ++t, ++i) {
        const uint32_t piece = min(16u * ncol + 4u * t + grp, row_pieces - 1u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(buf + 1024u * i), 16,
                                                  n * row_bytes + 16u * piece, 0, 0, AUX);
      }
    } else {
      for (uint32_t i = 0; i < pieces; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(buf + 1024u * i), 16,
                                                  n * row_bytes + 16u * grp + 64u * i, 0, 0, AUX);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stage has landed
  }
}

}  // namespace

hipError_t launch_stream_probe(uint32_t mode, const uint8_t* w, uint32_t rows, uint32_t cols,
                               uint32_t block_bytes, uint32_t cus, hipStream_t s) {
  const uint32_t nb = cols / 256u;
  const uint32_t ntiles = (rows + 15u) / 16u;
  if (nb == 0 || rows == 0 || (uint64_t)nb * block_bytes * 16u > 0x7fffffffu) return hipErrorInvalidValue;
  const uint32_t rp = (4u * block_bytes + 15u) / 16u;  // 16-byte pieces of a row's stage
  const uint32_t lds = kWaves * 1024u * std::max((4u * block_bytes + 63u) / 64u,
                                                 4u * (rp / 16u) + (rp % 16u + 3u) / 4u);
  if (lds > 163840u) return hipErrorInvalidValue;
  const dim3 grid(min(ntiles, cus)), block(kWaves * 64);
#define SIHIP_PROBE(AUX, EMPTY, WIDE)                                                         \
  do {                                                                                       \
    static const hipError_t attr = hipFuncSetAttribute(                                     \
        reinterpret_cast<const void*>(&stream_probe<AUX, EMPTY, WIDE>),                    \
        hipFuncAttributeMaxDynamicSharedMemorySize, 163840);                                \
    if (attr != hipSuccess) return attr;                                                     \
    hipLaunchKernelGGL((stream_probe<AUX, EMPTY, WIDE>), grid, block, lds, s, w, rows, nb,    \
                       block_bytes, nullptr);                                                \
  } while (0)
  switch (mode) {
    case kProbeDefault: SIHIP_PROBE(0, false, false); break;
    case kProbeNontemporal: SIHIP_PROBE(2, false, false); break;
    case kProbeEmpty: SIHIP_PROBE(0, true, false); break;
    case kProbeWide: SIHIP_PROBE(0, false, true); break;
    default: return hipErrorInvalidValue;
  }
#undef SIHIP_PROBE
  return hipGetLastError();
}

}  // namespace sihip
