// Tuned gfx950 K-quant matvec kernels.
//
// Q4_K, one input vector (si_q4_k_matvec*, src/metal.rs:310-494, re-designed):
//   * one lane owns one output row, so a wavefront covers 64 rows and every
//     lane needs the same activations at the same time: x is read with
//     wave-uniform (scalar) loads and used straight from SGPRs;
//   * each lane decodes whole 144-byte super-blocks, so the 6-bit
//     scale/min unpack (get_scale_min, quant.rs:176-185) is paid once per
//     256 weights;
//   * the blocks of 64 rows are not contiguous (row stride = K/256*144), so
//     they are staged through LDS with 16-byte global->LDS loads in which
//     consecutive lanes read consecutive 16-byte pieces of each row's
//     block, then each lane reads its own block back from LDS;
//   * DEPTH stages per wave keep several blocks in flight (software
//     pipeline); the waves of a workgroup split K and reduce through LDS;
//   * dot: per 32-weight unit j the kernel accumulates A_j = sum q*x in
//     f32 and forms y += d*sum_j sc_j*A_j - dmin*sum_j m_j*X_j with
//     X_j = sum x over the unit, i.e. the exact weight d*sc*q - dmin*m
//     factored per unit (f32 rounding differs from the per-weight form; the
//     tests bound it by 2e-5 * sum|w*x|).
#include "kquant_device.h"
#include "si_hip_tuned.h"

#include <cstdlib>

namespace sihip {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediates for gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8.
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
constexpr int kWaitLgkm0 = 0xf | (0x3 << 14) | (0x7 << 4);

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Read one lane's staged 144-byte block (nine 16-byte pieces) from LDS and
// wait for it.  Written as one asm block so that the compiler, which cannot
// see which stage a global->LDS load targets, does not add a full vmcnt(0)
// drain before the read; the caller waits for exactly the stage it reads.
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
      : "=v"(v[0]), "=v"(v[1]), "=v"(v[2]), "=v"(v[3]), "=v"(v[4]), "=v"(v[5]), "=v"(v[6]),
        "=v"(v[7]), "=v"(v[8])
      : "v"(addr)
      : "memory");
}

// v & mask, opaque to the combiner so that the byte conversions below stay
// single v_cvt_f32_ubyte{0..3} instead of being merged into bit-field
// extracts of the unmasked word.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t mask) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(mask), "v"(v));
  return r;
}

__device__ __forceinline__ float byte_f(uint32_t v, int i) {
  return (float)((v >> (8 * i)) & 0xffu);
}

#define SIHIP_STR2(x) #x
#define SIHIP_STR(x) SIHIP_STR2(x)

// Eight weights of one qs word into the two unit accumulators:
//   a_lo += q_lo[i] * x[4K + i],  a_hi += (16 * q_hi[i]) * x[32 + 4K + i]
// x0..x3 hold, in lane i of every 16-lane row, x[4i + c] (c = 0..3) of the
// 64-column group; v_fmac_f32_dpp with row_newbcast:n feeds lane n of each
// row to the whole row, so the activation broadcast costs no extra
// instruction.  The compiler cannot fold DPP into v_fmac, hence the asm.
// s_nop 1 gives the two wait states a DPP read needs after a VALU write of
// its source, whatever the compiler scheduled just before the block.
#define SIHIP_Q4_DWORD_ASM(K, KH)                                                            \
  asm("s_nop 1\n"                                                                            \
      "v_and_b32 %[lo], 0x0f0f0f0f, %[q]\n"                                                  \
      "v_and_b32 %[hi], 0xf0f0f0f0, %[q]\n"                                                  \
      "v_cvt_f32_ubyte0 %[t0], %[lo]\n"                                                      \
      "v_cvt_f32_ubyte0 %[t1], %[hi]\n"                                                      \
      "v_fmac_f32_dpp %[alo], %[x0], %[t0] row_newbcast:" SIHIP_STR(K) " row_mask:0xf bank_mask:0xf\n" \
      "v_fmac_f32_dpp %[ahi], %[x0], %[t1] row_newbcast:" SIHIP_STR(KH) " row_mask:0xf bank_mask:0xf\n" \
      "v_cvt_f32_ubyte1 %[t0], %[lo]\n"                                                      \
      "v_cvt_f32_ubyte1 %[t1], %[hi]\n"                                                      \
      "v_fmac_f32_dpp %[alo], %[x1], %[t0] row_newbcast:" SIHIP_STR(K) " row_mask:0xf bank_mask:0xf\n" \
      "v_fmac_f32_dpp %[ahi], %[x1], %[t1] row_newbcast:" SIHIP_STR(KH) " row_mask:0xf bank_mask:0xf\n" \
      "v_cvt_f32_ubyte2 %[t0], %[lo]\n"                                                      \
      "v_cvt_f32_ubyte2 %[t1], %[hi]\n"                                                      \
      "v_fmac_f32_dpp %[alo], %[x2], %[t0] row_newbcast:" SIHIP_STR(K) " row_mask:0xf bank_mask:0xf\n" \
      "v_fmac_f32_dpp %[ahi], %[x2], %[t1] row_newbcast:" SIHIP_STR(KH) " row_mask:0xf bank_mask:0xf\n" \
      "v_cvt_f32_ubyte3 %[t0], %[lo]\n"                                                      \
      "v_cvt_f32_ubyte3 %[t1], %[hi]\n"                                                      \
      "v_fmac_f32_dpp %[alo], %[x3], %[t0] row_newbcast:" SIHIP_STR(K) " row_mask:0xf bank_mask:0xf\n" \
      "v_fmac_f32_dpp %[ahi], %[x3], %[t1] row_newbcast:" SIHIP_STR(KH) " row_mask:0xf bank_mask:0xf" \
      : [alo] "+v"(a_lo), [ahi] "+v"(a_hi), [lo] "=&v"(lo_t), [hi] "=&v"(hi_t),              \
        [t0] "=&v"(t0_t), [t1] "=&v"(t1_t)                                                   \
      : [q] "v"(qw), [x0] "v"(xc0), [x1] "v"(xc1), [x2] "v"(xc2), [x3] "v"(xc3))

// Decode one staged Q4_K block held as 9 x 16 bytes.
// xg[g][c] (g = 64-column group, c = 0..3) holds, in lane i of every 16-lane
// row, activation 64*g + 4*i + c of the block.  xs: the 8 unit sums.
__device__ __forceinline__ float q4k_block_dot(const uint4 (&v)[9], const float4 (&xg)[4],
                                               const float* xs) {
  const uint32_t dm = v[0].x;
  const float d = half_bits_to_float(dm & 0xffffu);
  const float dmin = half_bits_to_float(dm >> 16);
  const uint32_t s0 = v[0].y, s1 = v[0].z, s2 = v[0].w;
  const uint32_t sc03 = s0 & 0x3f3f3f3fu;
  const uint32_t mn03 = s1 & 0x3f3f3f3fu;
  const uint32_t sc47 = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mn47 = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);

  float t_lo = 0.0f, t_hi = 0.0f, u = 0.0f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float xc0 = xg[g].x, xc1 = xg[g].y, xc2 = xg[g].z, xc3 = xg[g].w;
    float a_lo = 0.0f, a_hi = 0.0f;
    uint32_t lo_t, hi_t;
    float t0_t, t1_t;
#define SIHIP_Q4_DWORD(K, KH)                                                              \
    {                                                                                      \
      const uint4 q4 = v[1 + 2 * g + ((K) >> 2)];                                          \
      const uint32_t qw = ((K) & 3) == 0 ? q4.x : ((K) & 3) == 1 ? q4.y                     \
                        : ((K) & 3) == 2 ? q4.z : q4.w;                                     \
      SIHIP_Q4_DWORD_ASM(K, KH);                                                           \
    }
    SIHIP_Q4_DWORD(0, 8) SIHIP_Q4_DWORD(1, 9) SIHIP_Q4_DWORD(2, 10) SIHIP_Q4_DWORD(3, 11)
    SIHIP_Q4_DWORD(4, 12) SIHIP_Q4_DWORD(5, 13) SIHIP_Q4_DWORD(6, 14) SIHIP_Q4_DWORD(7, 15)
#undef SIHIP_Q4_DWORD
    const uint32_t scw = g < 2 ? sc03 : sc47;
    const uint32_t mnw = g < 2 ? mn03 : mn47;
    const int j0 = (2 * g) & 3;
    t_lo = fmaf(byte_f(scw, j0), a_lo, t_lo);
    t_hi = fmaf(byte_f(scw, j0 + 1), a_hi, t_hi);
    u = fmaf(byte_f(mnw, j0), xs[2 * g], u);
    u = fmaf(byte_f(mnw, j0 + 1), xs[2 * g + 1], u);
  }
  const float t = fmaf(t_hi, 0.0625f, t_lo);
  return fmaf(d, t, -dmin * u);
}

// Stage buffers are separate LDS objects so that the compiler's waitcnt
// insertion can tell the DMA writes into one stage from reads of another.
template <int WAVES>
struct Q4kStages {
  uint4 (*s[3])[64 * 9];
};

template <int WAVES, int DEPTH>
__global__ __launch_bounds__(WAVES * 64) void q4k_matvec_rowgroup(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x,
                                                                  float* __restrict__ y,
                                                                  uint32_t rows, uint32_t nb) {
  static_assert(DEPTH >= 2 && DEPTH <= 3, "two or three stages");
  __shared__ uint4 stage0[WAVES][64 * 9];
  __shared__ uint4 stage1[WAVES][64 * 9];
  __shared__ uint4 stage2[DEPTH > 2 ? WAVES : 1][64 * 9];
  extern __shared__ float xsum[];  // nb * 8 unit sums
  __shared__ float red[WAVES][64];

  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t row0 = blockIdx.x * 64u;
  const uint32_t nrows = min(64u, rows - row0);
  const size_t row_bytes = (size_t)nb * kQ4Bytes;

  for (uint32_t j = threadIdx.x; j < nb * 8u; j += blockDim.x) {
    const float4* xp = reinterpret_cast<const float4*>(x + 32u * j);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 a = xp[i];
      s += (a.x + a.y) + (a.z + a.w);
    }
    xsum[j] = s;
  }
  __syncthreads();

  // chunk c of the staged tile is byte (c % 9) * 16 of row c / 9's block
  uint32_t src_off[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const uint32_t c = (uint32_t)i * 64u + lane;
    uint32_t r = c / 9u;
    const uint32_t part = c - r * 9u;
    if (r >= nrows) r = nrows - 1u;  // keep loads in bounds for a short group
    src_off[i] = r * (uint32_t)row_bytes + part * 16u;
  }
  const uint8_t* base = w + (size_t)row0 * row_bytes;
  const uint32_t nblk = nb > wave ? (nb - wave + WAVES - 1) / WAVES : 0u;

  auto issue = [&](uint32_t k, uint4* dst) {
    const uint8_t* bp = base + (size_t)(wave + k * WAVES) * kQ4Bytes;
#pragma unroll
    for (int i = 0; i < 9; ++i)
      __builtin_amdgcn_global_load_lds(bp + src_off[i], (lds_void*)(dst + i * 64), 16, 0, 0);
  };
  auto consume = [&](uint32_t k, const uint4* src, uint4* refill_dst, bool last_group) -> float {
    if (!last_group) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(9 * (DEPTH - 1)));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    uint4 v[9];
    lds_read_block9((uint32_t)(uintptr_t)(src + lane * 9), v);
    if (k + DEPTH < nblk) issue(k + DEPTH, refill_dst);
    const uint32_t b = wave + k * WAVES;
    const float4* xq = reinterpret_cast<const float4*>(x + 256u * b) + (lane & 15u);
    const float4 xg[4] = {xq[0], xq[16], xq[32], xq[48]};
    return q4k_block_dot(v, xg, xsum + 8u * b);
  };

  uint4* stages[3] = {stage0[wave], stage1[wave], stage2[DEPTH > 2 ? wave : 0]};
#pragma unroll
  for (int k = 0; k < DEPTH; ++k)
    if ((uint32_t)k < nblk) issue((uint32_t)k, stages[k]);

  float acc = 0.0f;
  int slot = 0;
#pragma unroll 1
  for (uint32_t k = 0; k < nblk; ++k) {
    uint4* st = slot == 0 ? stages[0] : slot == 1 ? stages[1] : stages[2];
    acc += consume(k, st, st, k + DEPTH > nblk);
    slot = slot + 1 == DEPTH ? 0 : slot + 1;
  }

  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float s = red[0][lane];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) s += red[i][lane];
    if (lane < nrows) y[row0 + lane] = s;
  }
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

}  // namespace

bool launch_matvec_tuned(uint32_t type, const uint8_t* w, const float* x, float* y, uint32_t rows,
                         uint32_t cols, uint32_t batch, hipStream_t s, hipError_t* err) {
  if (type != kTypeQ4K || batch != 1) return false;
  const uint32_t nb = cols / kBlockElems;
  if (nb == 0 || nb > 4096) return false;
  static const int variant = env_int("SI_HIP_Q4K_VARIANT", 0);
  const dim3 grid((rows + 63) / 64);
  const size_t shmem = (size_t)nb * 8 * sizeof(float);
  switch (variant) {
    case 1:
      hipLaunchKernelGGL((q4k_matvec_rowgroup<4, 3>), grid, dim3(256), shmem, s, w, x, y, rows, nb);
      break;
    case 2:
      hipLaunchKernelGGL((q4k_matvec_rowgroup<8, 2>), grid, dim3(512), shmem, s, w, x, y, rows, nb);
      break;
    default:
      hipLaunchKernelGGL((q4k_matvec_rowgroup<4, 2>), grid, dim3(256), shmem, s, w, x, y, rows, nb);
      break;
  }
  *err = hipGetLastError();
  return true;
}

bool launch_fused_gate_up_tuned(const uint8_t*, const uint8_t*, const float*, float*, uint32_t,
                                uint32_t, hipStream_t, hipError_t*) {
  return false;
}

}  // namespace sihip
