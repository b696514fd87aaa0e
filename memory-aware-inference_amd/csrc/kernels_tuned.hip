// Tuned gfx950 K-quant matvec kernels.
//
// Q4_K, one input vector (replaces si_q4_k_matvec*, src/metal.rs:310-494).
//
// Work unit: a 16-row tile x 4 consecutive super-blocks (a "stage": 16 rows
// x 576 bytes).  Lane l of a wavefront is (p, n) = (l / 16, l % 16): it owns
// row n of the tile and decodes the whole 144-byte block p of the stage, so
// the 6-bit scale/min unpack (get_scale_min, quant.rs:176-185) is paid once
// per 256 weights.  Each 16-lane row p of the wavefront works on one block,
// i.e. on one set of 256 activations: the activations are held 16 per VGPR
// (lane i of row p holds columns 64g + 4i + c of its block) and fed into the
// FMAs with DPP row_newbcast, which broadcasts one lane of each 16-lane row
// to that row, so the broadcast costs no instruction.
//
// Data path: the 16 rows of a stage are 16 separate 576-byte runs; they are
// copied with 16-byte global->LDS loads in which consecutive lanes read
// consecutive 16-byte pieces of each run, then each lane reads its own block
// back from LDS (LDS is only the transposition buffer).  While a wave
// computes on a block in registers, the next stage's copy is in flight.
//
// Arithmetic: q (0..15) becomes f32 two at a time through the FP8 (e4m3)
// converter: a byte 0..15 is the e4m3 encoding of q * 2^-9 (subnormal for
// q < 8, exponent 1 for 8..15), exact.  Per 32-weight unit j the kernel
// accumulates A_j = sum q*x, then y += d*sum_j sc_j*A_j - dmin*sum_j m_j*X_j
// with X_j = sum of the unit's activations: the exact weight d*sc*q - dmin*m
// factored per unit (rounding differs from the per-weight form; the tests
// bound the result by 2e-5 * sum|w*x|).
//
// The waves of a workgroup split K (stage s goes to wave s % WAVES) and
// reduce through LDS in a fixed order, so results are deterministic.
#include "kquant_device.h"
#include "si_hip_tuned.h"

#include <cstdlib>

namespace sihip {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef float float2v __attribute__((ext_vector_type(2)));

// value of one e4m3 step for the nibble conversion: byte q decodes to q*2^-9
constexpr float kFp8Unit = 1.0f / 512.0f;

// buffer descriptor word 3 for raw (untyped, unswizzled) dword access on CDNA
constexpr int kBufferWord3 = 0x00020000;

constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ float byte_f(uint32_t v, int i) {
  return (float)((v >> (8 * i)) & 0xffu);
}

// DPP through the builtin (the combiner folds it into the consuming add).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114;
constexpr int kRowBcast7 = 0x157, kRowBcast15 = 0x15f;

// Read one lane's staged 144-byte block (nine 16-byte pieces) from LDS.  One
// asm block: the compiler cannot see which LDS bytes a global->LDS load
// writes and would otherwise drain every outstanding load first; the caller
// waits for exactly the copy it reads.
__device__ __forceinline__ void lds_read_block9(uint32_t addr, uint4 (&v)[9]) {
  asm volatile(
      "ds_read_b128 %0, %9\n"
      "ds_read_b128 %1, %9 offset:16\n"
      "ds_read_b128 %2, %9 offset:32\n"
      "ds_read_b128 %3, %9 offset:48\n"
      "ds_read_b128 %4, %9 offset:64\n"
      "ds_read_b128 %5, %9 offset:80\n"
      "ds_read_b128 %6, %9 offset:96\n"
      "ds_read_b128 %7, %9 offset:112\n"
      "ds_read_b128 %8, %9 offset:128\n"
      "s_waitcnt lgkmcnt(0)"
      // early-clobber: a returning read must not land on the address register
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8])
      : "v"(addr)
      : "memory");
}

#define SIHIP_FMAC_BCAST(ACC, X, Q, LANE)                                          \
  "v_fmac_f32_dpp %[" ACC "], %[" X "], %[" Q "] row_newbcast:%[" LANE "]"           \
  " row_mask:0xf bank_mask:0xf\n"

// Eight FMAs of one qs word: a_lo += x[4K+i] * qlo[i], a_hi += x[32+4K+i] * qhi[i]
// (i = 0..3), the activations broadcast from lanes K and 8+K of each 16-lane
// row.  The compiler does not fold DPP into v_fmac, hence asm; the leading
// s_nop 1 gives a DPP read its two wait states after a VALU write of its
// source, whatever the compiler scheduled just before the block.
template <int K>
__device__ __forceinline__ void q4_word_fma(float& a_lo, float& a_hi, float x0, float x1,
                                            float x2, float x3, float2v lo01, float2v lo23,
                                            float2v hi01, float2v hi23) {
  asm("s_nop 1\n"
      SIHIP_FMAC_BCAST("alo", "x0", "l0", "kl")
      SIHIP_FMAC_BCAST("ahi", "x0", "h0", "kh")
      SIHIP_FMAC_BCAST("alo", "x1", "l1", "kl")
      SIHIP_FMAC_BCAST("ahi", "x1", "h1", "kh")
      SIHIP_FMAC_BCAST("alo", "x2", "l2", "kl")
      SIHIP_FMAC_BCAST("ahi", "x2", "h2", "kh")
      SIHIP_FMAC_BCAST("alo", "x3", "l3", "kl")
      SIHIP_FMAC_BCAST("ahi", "x3", "h3", "kh")
      : [alo] "+v"(a_lo), [ahi] "+v"(a_hi)
      : [x0] "v"(x0), [x1] "v"(x1), [x2] "v"(x2), [x3] "v"(x3), [l0] "v"(lo01.x),
        [l1] "v"(lo01.y), [l2] "v"(lo23.x), [l3] "v"(lo23.y), [h0] "v"(hi01.x),
        [h1] "v"(hi01.y), [h2] "v"(hi23.x), [h3] "v"(hi23.y), [kl] "i"(K), [kh] "i"(8 + K));
}

template <int K>
__device__ __forceinline__ void q4_word(uint32_t q, float& a_lo, float& a_hi, const float4& xg) {
  const uint32_t lo = q & 0x0f0f0f0fu;
  const uint32_t hi = (q >> 4) & 0x0f0f0f0fu;
  const float2v lo01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
  const float2v lo23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
  const float2v hi01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
  const float2v hi23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
  q4_word_fma<K>(a_lo, a_hi, xg.x, xg.y, xg.z, xg.w, lo01, lo23, hi01, hi23);
}

// Activations of one block in the broadcast layout plus its unit sums.
struct Q4kBlockX {
  float4 xg[4];  // lane i of the 16-lane row: x[64g + 4i + c], c = 0..3
  float xs[8];   // X_j = sum of unit j's 32 activations (same in every lane)
};

__device__ __forceinline__ void load_block_x(const float* __restrict__ xb, uint32_t i,
                                             Q4kBlockX& bx) {
  const float4* xq = reinterpret_cast<const float4*>(xb) + i;
#pragma unroll
  for (int g = 0; g < 4; ++g) bx.xg[g] = xq[16 * g];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    // X_2g sums lanes 0..7 of the row, X_2g+1 lanes 8..15
    float s = (bx.xg[g].x + bx.xg[g].y) + (bx.xg[g].z + bx.xg[g].w);
    s += dpp<kRowShr1>(s);
    s += dpp<kRowShr2>(s);
    s += dpp<kRowShr4>(s);
    bx.xs[2 * g] = dpp<kRowBcast7>(s);
    bx.xs[2 * g + 1] = dpp<kRowBcast15>(s);
  }
}

// Dot of one Q4_K block (nine 16-byte words v) with its 256 activations.
__device__ __forceinline__ float q4k_block_dot(const uint4 (&v)[9], const Q4kBlockX& bx) {
  const uint32_t dm = v[0].x;
  const float d = half_bits_to_float(dm & 0xffffu) * (1.0f / kFp8Unit);
  const float dmin = half_bits_to_float(dm >> 16);
  const uint32_t s0 = v[0].y, s1 = v[0].z, s2 = v[0].w;
  const uint32_t sc03 = s0 & 0x3f3f3f3fu;
  const uint32_t mn03 = s1 & 0x3f3f3f3fu;
  const uint32_t sc47 = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mn47 = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);

  float t = 0.0f, u = 0.0f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float a_lo = 0.0f, a_hi = 0.0f;
    const uint4 qa = v[1 + 2 * g], qb = v[2 + 2 * g];
    const float4 xg = bx.xg[g];
    q4_word<0>(qa.x, a_lo, a_hi, xg);
    q4_word<1>(qa.y, a_lo, a_hi, xg);
    q4_word<2>(qa.z, a_lo, a_hi, xg);
    q4_word<3>(qa.w, a_lo, a_hi, xg);
    q4_word<4>(qb.x, a_lo, a_hi, xg);
    q4_word<5>(qb.y, a_lo, a_hi, xg);
    q4_word<6>(qb.z, a_lo, a_hi, xg);
    q4_word<7>(qb.w, a_lo, a_hi, xg);
    const uint32_t scw = g < 2 ? sc03 : sc47;
    const uint32_t mnw = g < 2 ? mn03 : mn47;
    const int j0 = (2 * g) & 3;
    t = fmaf(byte_f(scw, j0), a_lo, t);
    t = fmaf(byte_f(scw, j0 + 1), a_hi, t);
    u = fmaf(byte_f(mnw, j0), bx.xs[2 * g], u);
    u = fmaf(byte_f(mnw, j0 + 1), bx.xs[2 * g + 1], u);
  }
  return fmaf(d, t, -dmin * u);
}

// Persistent kernel.  Workgroup G processes the 16-row tiles G, G +
// gridDim.x, ...; K is cut into stages of 4 blocks and wave v of the
// WAVES waves owns stages v, v + WAVES, ... (at most SPW of them), so it
// loads the activations of its stages once and keeps them in registers for
// every tile.  Each wave has one LDS stage buffer: it waits for the copy of
// its current stage, reads its block into registers, starts the copy of its
// next stage (same tile, or its first stage of the next tile) into the same
// buffer and computes while that copy is in flight.
template <int WAVES, int SPW>
__global__ __launch_bounds__(WAVES * 64) void q4k_matvec_persistent(
    const uint8_t* __restrict__ w, const float* __restrict__ x, float* __restrict__ y,
    uint32_t rows, uint32_t nb) {
  __shared__ uint4 stage[WAVES][64 * 9];
  __shared__ float red[WAVES][64];

  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t p = lane >> 4, n = lane & 15u;
  const uint32_t row_bytes = nb * kQ4Bytes;
  const uint32_t ntiles = (rows + 15) / 16;
  const uint32_t nstages = (nb + 3) / 4;

  Q4kBlockX bx[SPW];
  bool live[SPW];
#pragma unroll
  for (int k = 0; k < SPW; ++k) {
    const uint32_t blk = 4u * (wave + k * WAVES) + p;
    live[k] = blk < nb;
    load_block_x(x + 256u * (live[k] ? blk : nb - 1u), n, bx[k]);
  }

  // piece c = 64i + lane of a stage: 16 bytes at byte (c % 36) * 16 of row
  // c / 36's 576-byte run of the stage.  The copies are buffer loads whose
  // descriptor covers exactly the tile's rows, so a piece past the matrix
  // (rows of the last tile, blocks of a short last stage) reads zero: those
  // lanes' results are discarded.
  uint32_t off[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const uint32_t c = (uint32_t)i * 64u + lane;
    const uint32_t r = c / 36u;
    off[i] = r * row_bytes + (c - r * 36u) * 16u;
  }
  uint4* st = stage[wave];
  auto issue = [&](uint32_t tile, uint32_t s) {
    const uint32_t row0 = tile * 16u;
    const uint32_t nrows = min(16u, rows - row0);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w) + (size_t)row0 * row_bytes, 0, (int)(nrows * row_bytes),
        kBufferWord3);
#pragma unroll
    for (int i = 0; i < 9; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(st + i * 64), 16, off[i],
                                                576u * s, 0, 0);
  };
  const uint32_t lds_addr = (uint32_t)(uintptr_t)(st + 36u * n + 9u * p);

  uint32_t tile = blockIdx.x;
  if (tile < ntiles) issue(tile, wave);
  while (tile < ntiles) {
    const uint32_t next = tile + gridDim.x;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const uint32_t s = wave + k * WAVES;
      if (k == 0 || s < nstages) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        uint4 v[9];
        lds_read_block9(lds_addr, v);
        // the buffer is free again: start the wave's next copy
        if (k + 1 < SPW && s + WAVES < nstages)
          issue(tile, s + WAVES);
        else if (next < ntiles)
          issue(next, wave);
        const float dot = q4k_block_dot(v, bx[k]);
        acc += live[k] ? dot : 0.0f;
      }
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (threadIdx.x < 16) {
      float sum = 0.0f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv)
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += red[wv][16 * q + threadIdx.x];
      const uint32_t row = tile * 16u + threadIdx.x;
      if (row < rows) y[row] = sum;
    }
    __syncthreads();
    tile = next;
  }
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

int device_cu_count() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    return n;
  }();
  return cus;
}

}  // namespace

bool launch_matvec_tuned(uint32_t type, const uint8_t* w, const float* x, float* y, uint32_t rows,
                         uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                         hipError_t* err) {
  if (batch == 0) return false;
  static const int mode = env_int("SI_HIP_Q4K_MODE", 0);
  const bool q4_mfma = type == kTypeQ4K && mode == 0;
  static const int tokens_per_pass = env_int("SI_HIP_Q4K_BATCH_PASS", 1);
  if (q4_mfma && batch > 1 && tokens_per_pass &&
      launch_q4k_matmul_mfma(w, x, y, rows, cols, batch, ws, s, err))
    return true;
  if (type == kTypeQ5K && mode == 0)
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
  // The VALU kernel below forms sums of x, so a non-finite activation turns
  // every row into NaN where the reference's per-weight products give +-inf:
  // it runs only when asked for (SI_HIP_Q4K_MODE=1).  By default a shape the
  // matrix-core kernel does not take goes to the exact generic kernel.
  if (mode == 0) return launch_q4k_matvec_mfma(w, x, y, rows, cols, ws, s, err);
  const uint32_t nb = cols / kBlockElems;
  const uint32_t nstages = (nb + 3) / 4;
  // offsets inside one 16-row tile are 32-bit
  if (nb == 0 || (uint64_t)nb * kQ4Bytes * 16u > 0xffffffffu) return false;
  const uint32_t spw = (nstages + 7) / 8;
  if (spw > 4) return false;
  const uint32_t waves = (nstages + spw - 1) / spw;
  const uint32_t ntiles = (rows + 15) / 16;
  // workgroups resident per CU, bounded by LDS (9 KB stage + 256 B per wave)
  static const int forced = env_int("SI_HIP_Q4K_WG_PER_CU", 0);
  const uint32_t lds_per_wg = waves * (9216u + 256u);
  uint32_t per_cu = forced > 0 ? (uint32_t)forced : (160u * 1024u) / lds_per_wg;
  if (per_cu == 0) per_cu = 1;
  const uint32_t grid = min(ntiles, (uint32_t)device_cu_count() * per_cu);
  const uint32_t key = spw * 16u + waves;
  switch (key) {
#define SIHIP_CASE(SPW, W)                                                                  \
  case SPW * 16 + W:                                                                        \
    hipLaunchKernelGGL((q4k_matvec_persistent<W, SPW>), dim3(grid), dim3(W * 64), 0, s, w,   \
                       x, y, rows, nb);                                                     \
    break;
    SIHIP_CASE(1, 1) SIHIP_CASE(1, 2) SIHIP_CASE(1, 3) SIHIP_CASE(1, 4)
    SIHIP_CASE(1, 5) SIHIP_CASE(1, 6) SIHIP_CASE(1, 7) SIHIP_CASE(1, 8)
    SIHIP_CASE(2, 5) SIHIP_CASE(2, 6) SIHIP_CASE(2, 7) SIHIP_CASE(2, 8)
    SIHIP_CASE(3, 6) SIHIP_CASE(3, 7) SIHIP_CASE(3, 8)
    SIHIP_CASE(4, 7) SIHIP_CASE(4, 8)
#undef SIHIP_CASE
    default:
      return false;
  }
  *err = hipGetLastError();
  return true;
}

bool launch_fused_gate_up_tuned(const uint8_t* gate, const uint8_t* up, const float* x, float* h,
                                uint32_t rows, uint32_t cols, const Workspace& ws, hipStream_t s,
                                hipError_t* err) {
  return launch_q4k_gate_up_mfma(gate, up, x, h, rows, cols, ws, s, err);
}

}  // namespace sihip
