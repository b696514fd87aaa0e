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
//
// Modes kProbeLines and kProbeRegisters deal the (tile, stage) pairs of the
// whole matrix evenly to the workgroups, as the one-vector kernel's split
// schedule does (workgroup g of G: pairs [g P / G, (g + 1) P / G)), then
// round-robin to its waves.  kProbeLines copies each Q4_K stage as the five
// whole 128-byte lines of each of its 16 rows (ten 64-lane buffer->LDS
// copies, nontemporal, one stage in flight per wave; nb = 4 mod 8 blocks per
// row).  kProbeRegisters loads each lane's operands of the matrix-core
// layout straight into registers -- per block the header and qs pieces
// 1 + 2 g and 2 + 2 g of row n (lane 16 g + n), twelve 16-byte loads per
// stage -- with two stages in flight per wave of eight;
// kProbeRegistersNontemporal does the same with the nontemporal bit.
#include "si_hip_internal.h"

#include <algorithm>

namespace sihip {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kQ4Bytes = 144;
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

// Workgroup g's share [lo, hi) of the matrix's P (tile, stage) pairs.
__device__ __forceinline__ void balanced_share(uint32_t pairs, uint32_t& lo, uint32_t& hi) {
  lo = (uint32_t)((uint64_t)pairs * blockIdx.x / gridDim.x);
  hi = (uint32_t)((uint64_t)pairs * (blockIdx.x + 1u) / gridDim.x);
}

__global__ __launch_bounds__(kWaves * 64) void stream_probe_lines(const uint8_t* __restrict__ w,
                                                                  uint32_t rows, uint32_t nb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr uint32_t kStage = 10240u;  // ten copies of 1 KB
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t row_bytes = nb * 144u;
  const uint32_t nstages = nb / 4u;  // nb = 4 mod 8: whole four-block stages
  const uint32_t ntiles = (rows + 15u) / 16u;
  uint32_t lo, hi;
  balanced_share(ntiles * nstages, lo, hi);
  // lane: line slot k of rows 2 i (copy class 0) and 2 i + 1 (class 1)
  const uint32_t li = lane >> 3, k = ((lane & 7u) - (li >> 1)) & 7u;
  const uint32_t l0 = 2u * li * row_bytes + 16u * k, l1 = l0 + row_bytes;
  uint8_t* const dst = smem + wave * kStage;
  for (uint32_t p = lo + wave; p < hi; p += kWaves) {
    const uint32_t tile = p / nstages, st = p - tile * nstages;
    const uint32_t row0 = tile * 16u, nrows = min(16u, rows - row0);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w + (size_t)row0 * row_bytes), 0, (int)(nrows * row_bytes),
        kBufferWord3);
    const uint32_t odd = st & 1u;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint32_t vo = (c ? l1 : l0) + (576u * st - 64u * ((uint32_t)c ^ odd));
      uint8_t* const region = dst + 1024u * ((uint32_t)c ^ odd);
#pragma unroll
      for (int j = 0; j < 5; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(region + 2048 * j), 16,
                                                  vo + 128u * j, 0, 0, 2);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stage has landed
  }
}

// The lane's twelve 16-byte pieces of pair p (tile p / nstages, stage
// p % nstages), loaded by inline asm: the compiler neither counts these loads
// nor waits for them, so a wave keeps exactly the stages it asks for in
// flight and waits with wait_stage.  Past the wave's share the descriptor
// holds no bytes, and the loads read zeros without touching memory.
struct RegStage {
  u32x4 v[12];
};
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ void load_stage_regs(const uint8_t* __restrict__ w, uint32_t rows,
                                                uint32_t row_bytes, uint32_t nstages, uint32_t p,
                                                uint32_t hi, uint32_t n, uint32_t grp,
                                                RegStage& r) {
  const bool live = p < hi;
  const uint32_t tile = live ? p / nstages : 0u, st = live ? p - tile * nstages : 0u;
  const uint32_t row0 = tile * 16u, nrows = live ? min(16u, rows - row0) : 0u;
  const uint64_t base = reinterpret_cast<uint64_t>(w + (size_t)row0 * row_bytes);
  const i32x4 rsrc = {(int32_t)(uint32_t)base, (int32_t)(uint32_t)(base >> 32) & 0xffff,
                      (int32_t)(nrows * row_bytes), kBufferWord3};
  const uint32_t o = n * row_bytes + 576u * st;  // the lane's row, block 0 of the stage
  const uint32_t oa = o + 16u + 32u * grp;        // qs piece 1 + 2 grp
  if constexpr (NT) {
    asm volatile(
        "buffer_load_dwordx4 %0, %12, %14, 0 offen nt\n"
        "buffer_load_dwordx4 %1, %13, %14, 0 offen nt\n"
        "buffer_load_dwordx4 %2, %13, %14, 0 offen offset:16 nt\n"
        "buffer_load_dwordx4 %3, %12, %14, 0 offen offset:144 nt\n"
        "buffer_load_dwordx4 %4, %13, %14, 0 offen offset:144 nt\n"
        "buffer_load_dwordx4 %5, %13, %14, 0 offen offset:160 nt\n"
        "buffer_load_dwordx4 %6, %12, %14, 0 offen offset:288 nt\n"
        "buffer_load_dwordx4 %7, %13, %14, 0 offen offset:288 nt\n"
        "buffer_load_dwordx4 %8, %13, %14, 0 offen offset:304 nt\n"
        "buffer_load_dwordx4 %9, %12, %14, 0 offen offset:432 nt\n"
        "buffer_load_dwordx4 %10, %13, %14, 0 offen offset:432 nt\n"
        "buffer_load_dwordx4 %11, %13, %14, 0 offen offset:448 nt"
        : "=&v"(r.v[0]), "=&v"(r.v[1]), "=&v"(r.v[2]), "=&v"(r.v[3]), "=&v"(r.v[4]),
          "=&v"(r.v[5]), "=&v"(r.v[6]), "=&v"(r.v[7]), "=&v"(r.v[8]), "=&v"(r.v[9]),
          "=&v"(r.v[10]), "=&v"(r.v[11])
        : "v"(o), "v"(oa), "s"(rsrc)
        : "memory");
  } else {
    asm volatile(
        "buffer_load_dwordx4 %0, %12, %14, 0 offen\n"
        "buffer_load_dwordx4 %1, %13, %14, 0 offen\n"
        "buffer_load_dwordx4 %2, %13, %14, 0 offen offset:16\n"
        "buffer_load_dwordx4 %3, %12, %14, 0 offen offset:144\n"
        "buffer_load_dwordx4 %4, %13, %14, 0 offen offset:144\n"
        "buffer_load_dwordx4 %5, %13, %14, 0 offen offset:160\n"
        "buffer_load_dwordx4 %6, %12, %14, 0 offen offset:288\n"
        "buffer_load_dwordx4 %7, %13, %14, 0 offen offset:288\n"
        "buffer_load_dwordx4 %8, %13, %14, 0 offen offset:304\n"
        "buffer_load_dwordx4 %9, %12, %14, 0 offen offset:432\n"
        "buffer_load_dwordx4 %10, %13, %14, 0 offen offset:432\n"
        "buffer_load_dwordx4 %11, %13, %14, 0 offen offset:448"
        : "=&v"(r.v[0]), "=&v"(r.v[1]), "=&v"(r.v[2]), "=&v"(r.v[3]), "=&v"(r.v[4]),
          "=&v"(r.v[5]), "=&v"(r.v[6]), "=&v"(r.v[7]), "=&v"(r.v[8]), "=&v"(r.v[9]),
          "=&v"(r.v[10]), "=&v"(r.v[11])
        : "v"(o), "v"(oa), "s"(rsrc)
        : "memory");
  }
}
// Waits until at most N of the wave's loads are in flight; `r` is tied to the
// wait, so no use of it moves above.
template <int N>
__device__ __forceinline__ void wait_stage(RegStage& r) {
  asm volatile("s_waitcnt vmcnt(%12)"
               : "+v"(r.v[0]), "+v"(r.v[1]), "+v"(r.v[2]), "+v"(r.v[3]), "+v"(r.v[4]),
                 "+v"(r.v[5]), "+v"(r.v[6]), "+v"(r.v[7]), "+v"(r.v[8]), "+v"(r.v[9]),
                 "+v"(r.v[10]), "+v"(r.v[11])
               : "i"(N));
}
__device__ __forceinline__ uint32_t fold_stage(const RegStage& r, uint32_t acc) {
#pragma unroll
  for (int i = 0; i < 12; ++i) acc ^= (r.v[i][0] ^ r.v[i][1]) ^ (r.v[i][2] ^ r.v[i][3]);
  return acc;
}

// NT: the nontemporal bit on the loads; kRegWaves waves per workgroup.
template <bool NT, uint32_t kRegWaves>
__global__ __launch_bounds__(kRegWaves * 64) void stream_probe_regs(const uint8_t* __restrict__ w,
                                                                    uint32_t rows, uint32_t nb,
                                                                    uint32_t* __restrict__ sink) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t row_bytes = nb * 144u;
  const uint32_t nstages = (nb + 3u) / 4u;
  const uint32_t ntiles = (rows + 15u) / 16u;
  uint32_t lo, hi;
  balanced_share(ntiles * nstages, lo, hi);
  RegStage a, b;
  uint32_t acc = 0u;
  uint32_t p = lo + wave;
  load_stage_regs<NT>(w, rows, row_bytes, nstages, p, hi, n, grp, a);
  load_stage_regs<NT>(w, rows, row_bytes, nstages, p + kRegWaves, hi, n, grp, b);
  while (p < hi) {
    wait_stage<12>(a);  // b's twelve loads may still be in flight
    acc = fold_stage(a, acc);
    load_stage_regs<NT>(w, rows, row_bytes, nstages, p + 2u * kRegWaves, hi, n, grp, a);
    if (p + kRegWaves >= hi) break;
    wait_stage<12>(b);
    acc = fold_stage(b, acc);
    load_stage_regs<NT>(w, rows, row_bytes, nstages, p + 3u * kRegWaves, hi, n, grp, b);
    p += 2u * kRegWaves;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // nothing in flight at the end
  // (the launch passes no sink: the store, which the compiler cannot rule
  // out, keeps the loads)
  if (sink != nullptr) sink[blockIdx.x * (kRegWaves * 64u) + threadIdx.x] = acc;
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
  if (mode >= kProbeLines) {
    if (block_bytes != kQ4Bytes || (mode == kProbeLines && nb % 8u != 4u) ||
        (reinterpret_cast<uintptr_t>(w) & 127u) != 0u)
      return hipErrorInvalidValue;
    const uint32_t pairs = ntiles * ((nb + 3u) / 4u);
    const dim3 g(min(pairs, cus));
    if (mode == kProbeLines) {
      static const hipError_t attr = hipFuncSetAttribute(
          reinterpret_cast<const void*>(&stream_probe_lines),
          hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      if (attr != hipSuccess) return attr;
      hipLaunchKernelGGL(stream_probe_lines, g, dim3(kWaves * 64), kWaves * 10240u, s, w, rows, nb);
    } else {
      if (mode == kProbeRegisters)
        hipLaunchKernelGGL((stream_probe_regs<false, 8>), g, dim3(512), 0, s, w, rows, nb, nullptr);
      else
        hipLaunchKernelGGL((stream_probe_regs<true, 8>), g, dim3(512), 0, s, w, rows, nb, nullptr);
    }
    return hipGetLastError();
  }
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
