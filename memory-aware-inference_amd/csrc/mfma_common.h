// Building blocks shared by the K-quant matvec kernels that run on the gfx950
// int8 matrix cores (kernels_q4k_mfma.hip, kernels_q6k_mfma.hip).
//
// Activations.  Each 256-element block b of x is written in fixed point,
// x_i = X_i * 2^(e_b - 30) with |X_i| <= 2^30 (e_b from the block's largest
// |x|, which is below 2^e_b), and X_i = sum_d D_d * 256^d in four signed byte
// digits.  Rounding costs at most 2^(e_b - 31), so an element of at least
// 2^(e_b - 14) keeps a relative error of at most 2^-17 whatever its weight.
// A block with smaller non-zero elements ("side" elements) is a "rounded"
// block (side count kSideRounded), so that the dot stays within its bar of
// 2e-5 * sum|w x| for any weights: the side elements stay in the fixed point,
// rounded like the rest, and the block keeps, per 16-element chunk, the sum
// of their rounding errors |x_i - X_i 2^(e_b - 30)|.  The kernel bounds a
// row's error from those blocks by (largest |w| the block header allows) x
// (that sum), and compares it with the sum of |partial dot| over the row's
// stage, which is at most sum|w x| over the stage.  A row whose bound exceeds
// kRoundedTol of it recomputes its rounded blocks exactly.  (The
// vectors-in-rows kernel, q4k_tokens_mfma, builds its own images and lists
// up to kSideMax side elements of a block as (index, x) entries instead,
// adding w_i * x_i for them with the exact per-weight decode: a rounded
// block there holds back the next stage's copy until its rows are checked.)
//
// A block with an activation that is not finite or reaches 2^100 takes the
// exact per-weight path whole.  For every
// 16-element chunk of a block the workgroup keeps an A-operand "image" of
// v_mfma_i32_16x16x64_i8 in LDS: A rows 4 p + d hold digit d of the chunk
// that meets lane group p's weights and every other row is zero, so the
// product with a B operand whose lane (p, n) holds 16 int8 weights of tile row
// n returns, in lane (p, n), the four digit sums of that lane's own chunk.
// Which chunk goes to which (MFMA, lane group) slot depends on how a format
// lays its weights out; build_images takes that map as a template argument.
//
// Workgroup protocol.  One persistent workgroup per CU walks a contiguous
// range of (tile, stage) pairs; a wave leaves each stage's 16 row partials in
// an LDS slot of its tile and counts them with an LDS atomic; the wave that
// completes the workgroup's share of a tile sums the partials in stage order
// (results do not depend on timing).  LDS is
// touched only through inline asm and the one barrier is a bare s_barrier:
// the compiler neither counts nor orders buffer->LDS copies, and a fence
// would drain them.
#pragma once

#include "kquant_device.h"
#include "si_hip_internal.h"

#include <cstdlib>
#include <type_traits>

namespace sihip {
namespace mfma {

typedef __attribute__((address_space(3))) void lds_void;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBufferWord3 = 0x00020000;  // raw dword access (CDNA buffer descriptor)
constexpr int kFixBits = 30;
constexpr uint32_t kLdsBytes = 163840u;
constexpr int kBadBlock = 0x40000000;  // exponent slot of a block taking the exact path
// Side elements: non-zero |x| below 2^(e_b - kSideShift).  Each block and
// activation vector has kSideBytes of LDS: for a rounded block, 16 f32 error
// sums, the one of chunk c at position 4 p + t for the chunk in MFMA t of
// lane group p (the four of a lane group side by side); in q4k_tokens_mfma,
// up to kSideMax 8-byte entries (element index, x bits) instead.
constexpr int kSideShift = 14;
constexpr uint32_t kSideMax = 8;
constexpr uint32_t kSideEntryBytes = 8;
constexpr uint32_t kSideBytes = kSideMax * kSideEntryBytes;  // 64
constexpr uint32_t kSideRounded = 0xffu;  // side count of a rounded block
// A row's stage passes when (error bound) * 1.01 <= kRoundedTol *
// (sum |partial| - error bound); 1.01 covers the f32 rounding of both sums.
constexpr float kRoundedTol = 4e-6f;
// The Q4_K / Q5_K kernels check every stage (stage_ok): the bound of the f32
// rounding of their factored dots plus that of their rounded blocks against
// kStageTol of the row's sum |partial|.  With the fixed point's 2^-17 on kept
// elements and the f32 accumulation of the partials (under 3e-6) the dot stays
// within 2e-5 * sum|w x|.
constexpr float kStageTol = 8e-6f;
// A stage partial the vectors-in-rows kernel leaves for its reduce kernel to
// recompute exactly (its lane failed the stage check): a signalling-NaN
// pattern, which no arithmetic result has.
constexpr uint32_t kPartRedo = 0x7f8c0de5u;

constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

// LDS map of one workgroup (byte offsets): per-wave stage buffers; for each
// of ntok activation vectors the digit images of all its blocks (a further
// 4 KB after the last one, which dead blocks of a short last stage may
// read), its unit sums [block][unit] (formats that need them) and its block
// metadata; then a ring of `slots` tile slots: [slot][partial][token][16 rows]
// f32 partials, and per slot a completion count and the tile index it
// currently belongs to.
//
// Block metadata of a vector (at expo + t expo_stride): the exponents
// [block] (4 bytes each, at most kMaxMetaBlocks blocks), at +kCountOff the
// side counts, one byte per block, and at +side_off the side areas
// [block][kSideBytes].  The counts of the bps blocks of a stage sit at
// kCountOff + 4 bps s, exactly kCountOff past the stage's exponents, so a
// kernel reads both from one address register (bytes of blocks past the
// matrix are not written; readers mask them).
constexpr uint32_t kCountOff = 512;
constexpr uint32_t kMaxMetaBlocks = kCountOff / 4u;
struct Layout {
  uint32_t img, xsum, expo, part, cnt, owner, ready, total;
  // per activation vector
  uint32_t img_stride, xsum_stride, expo_stride;
  uint32_t side_off, bps;  // side areas in the metadata; blocks per stage
};
__host__ __device__ constexpr Layout make_layout(uint32_t stage_bytes, uint32_t stage_blocks,
                                                 uint32_t xsum_per_block, uint32_t waves,
                                                 uint32_t depth, uint32_t nb, uint32_t slots,
                                                 uint32_t mats, uint32_t ntok = 1u) {
  Layout l{};
  const uint32_t nstages = (nb + stage_blocks - 1u) / stage_blocks;
  const uint32_t partials = nstages * mats;  // per tile
  l.bps = stage_blocks;
  l.img_stride = nb * 1024u;
  l.xsum_stride = nb * xsum_per_block;
  l.side_off = kCountOff + ((4u * stage_blocks * nstages + 15u) & ~15u);
  l.expo_stride = l.side_off + nb * kSideBytes;
  l.img = waves * depth * stage_bytes;
  l.xsum = l.img + ntok * l.img_stride + 4096u;
  l.expo = l.xsum + (xsum_per_block ? ntok * l.xsum_stride + 128u : 0u);
  l.part = l.expo + ntok * l.expo_stride + 16u;
  l.cnt = l.part + slots * partials * 64u * ntok;
  l.owner = l.cnt + slots * 4u;
  l.ready = l.owner + slots * 4u;  // count of image builders done (16 bytes)
  l.total = l.ready + 16u;
  return l;
}
// Offset of block b's side count in its vector's metadata.
__host__ __device__ constexpr uint32_t count_pos(const Layout& L, uint32_t b) {
  return kCountOff + 4u * L.bps * (b / L.bps) + b % L.bps;
}

// Lanes whose A rows carry digits: lane 16 g + n with n / 4 == g.
constexpr uint64_t kActiveLanes = 0xF0000F0000F0000Full;

__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// a * b + c with a, b signed 24-bit, as one v_mad_i32_i24: the empty asm
// keeps the compiler from pairing two products of a sum into v_add3_u32
// (three instructions for two products).  The product itself stays compiler
// code, which orders the MFMA result reads that feed it.
__device__ __forceinline__ int mad_i24(int a, int b, int c) {
  int d = __mul24(a, b) + c;
  asm("" : "+v"(d));
  return d;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kQuadSwap = 0xb1;  // quad_perm [1, 0, 3, 2]: lanes 2 k and 2 k + 1 trade
constexpr int kRowBcast15 = 0x15f;

// Word k (uniform, 0..3) of a 16-byte piece.
__device__ __forceinline__ uint32_t word_of(const u32x4& p, uint32_t k) {
  return k == 0u ? p[0] : k == 1u ? p[1] : k == 2u ? p[2] : p[3];
}
// Byte k (uniform, 0..15) of a 16-byte piece.
__device__ __forceinline__ uint32_t byte_of(const u32x4& p, uint32_t k) {
  return (word_of(p, k >> 2) >> (8u * (k & 3u))) & 0xffu;
}

// The stage's side counts, one byte per block, with the bytes of blocks at
// or past `nlive` cleared.
__device__ __forceinline__ uint32_t live_counts(uint32_t word, uint32_t nlive) {
  return nlive >= 4u ? word : word & ((1u << (8u * nlive)) - 1u);
}

__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void lds_write_b128(uint32_t addr, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b64(uint32_t addr, u32x2 v) {
  asm volatile("ds_write_b64 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b32(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b8(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b8 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// LDS atomic add; returns the previous value.
__device__ __forceinline__ uint32_t lds_add_rtn(uint32_t addr, uint32_t v) {
  uint32_t old;
  asm volatile("ds_add_rtn_u32 %0, %1, %2\ns_waitcnt lgkmcnt(0)" : "=&v"(old) : "v"(addr), "v"(v) : "memory");
  return old;
}
// The wave's claim on an LDS counter: one atomic add of 1 by lane 0 (the
// exec mask narrowed inside the asm), the old value returned in a scalar
// register so that loop conditions on it stay uniform.
__device__ __forceinline__ uint32_t lds_claim(uint32_t addr) {
  uint32_t v, s;
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %[sv], exec\n"
      "s_mov_b64 exec, 1\n"
      "ds_add_rtn_u32 %[v], %[a], %[one]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "s_mov_b64 exec, %[sv]\n"
      "v_readlane_b32 %[s], %[v], 0"
      : [v] "=&v"(v), [sv] "=&s"(saved), [s] "=s"(s)
      : [a] "v"(addr), [one] "v"(1u)
      : "memory");
  return s;
}
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_u16 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ u32x2 lds_read_b64(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
  return v;
}

// Four 16-byte reads at addr + STRIDE * t, t = 0..3.
template <int STRIDE, typename V>
__device__ __forceinline__ void lds_read4(uint32_t addr, V (&a)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n"
      "ds_read_b128 %1, %4 offset:%5\n"
      "ds_read_b128 %2, %4 offset:%6\n"
      "ds_read_b128 %3, %4 offset:%7\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3])
      : "v"(addr), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE)
      : "memory");
}

// Byte digits of four elements' biased values (X + 0x80808080): byte d of
// each element gathered into one word, then flipped to signed (b - 128).
__device__ __forceinline__ void transpose_digits(uint32_t u0, uint32_t u1, uint32_t u2,
                                                 uint32_t u3, uint32_t (&out)[4]) {
  // v_perm_b32 selector bytes 0..3 pick from the second source, 4..7 the first
  const uint32_t lo01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u);  // u0.b0 u1.b0 u0.b1 u1.b1
  const uint32_t hi01 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);  // u0.b2 u1.b2 u0.b3 u1.b3
  const uint32_t lo23 = __builtin_amdgcn_perm(u3, u2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(u3, u2, 0x07030602u);
  out[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
  out[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
  out[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
  out[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u) ^ 0x80808080u;
}

// Sum over the four 16-lane groups, ((g0 + g1) + (g2 + g3)), in every lane.
__device__ __forceinline__ float sum_lane_groups(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Copy of x (nb blocks of 256 f32) into the image area in natural order
// (block b at img + 1024 b): pass j of wave v copies blocks 4 (v + WAVES j)
// .. +3, one 64-lane 16-byte copy each -- the blocks build_images has the
// same wave convert, so that a wave's own wait covers what it converts.
// src_nb != 0: the image holds blocks first .. first + nb - 1 of x twice
// over (first + nb <= 2 src_nb), image block b being x block
// (first + b) mod src_nb.
template <int WAVES>
__device__ __forceinline__ void copy_x(uint8_t* smem, uint32_t img, const float* x, uint32_t nb,
                                       uint32_t wave, uint32_t lane, uint32_t src_nb = 0u,
                                       uint32_t first = 0u) {
  const uint32_t xn = src_nb != 0u ? src_nb : nb;
  const uint32_t npass = (nb + 4u * WAVES - 1u) / (4u * WAVES);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x), 0, (int)(xn * 1024u), kBufferWord3);
  for (uint32_t j = 0; j < npass; ++j) {
    const uint32_t b0 = 4u * (wave + WAVES * j);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t b = b0 + i, v = first + b;
      const uint32_t sb = v >= xn ? v - xn : v;
      if (b < nb)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(smem + img + 1024u * b), 16,
                                                  1024u * sb + 16u * lane, 0, 0, 0);
    }
  }
}

// The fixed-point split of one lane's 16 activations (a 16-element chunk of a
// block whose 16 lanes form one DPP row): the row's exponent e (largest |x|
// below 2^e), the fixed-point values X (two's complement), the mask of side
// elements, the f32 sum of all 16 and that of the side elements, the sum of
// the side elements' rounding errors, and whether the chunk alone forces the
// exact path.
struct ChunkSplit {
  int e;
  uint32_t fx[16];
  uint32_t smask;
  float xsum, xsum_side, err_side;
  bool bad;
};
__device__ __forceinline__ ChunkSplit split_chunk(const float (&xv)[16]) {
  ChunkSplit r;
  float amax = 0.0f, amin = __builtin_huge_valf();
  r.xsum = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    amax = fmaxf(amax, fabsf(xv[k]));
    amin = fminf(amin, fabsf(xv[k]));
    r.xsum += xv[k];
  }
  // not finite or huge: a NaN shows in the sum (which cannot overflow below
  // 2^100), an infinity in the maximum
  r.bad = !(amax < 0x1p100f) || r.xsum != r.xsum;
  amax = fmaxf(amax, dpp<kRowShr1>(amax));
  amax = fmaxf(amax, dpp<kRowShr2>(amax));
  amax = fmaxf(amax, dpp<kRowShr4>(amax));
  amax = fmaxf(amax, dpp<kRowShr8>(amax));
  amax = dpp<kRowBcast15>(amax);
  r.e = __builtin_amdgcn_frexp_expf(amax);  // amax < 2^e; 0 for amax == 0
  const float thr = __builtin_amdgcn_ldexpf(1.0f, r.e - kSideShift);
#pragma unroll
  for (int k = 0; k < 16; ++k)
    r.fx[k] = (uint32_t)__float2int_rn(__builtin_amdgcn_ldexpf(xv[k], kFixBits - r.e));
  r.smask = 0u;
  r.xsum_side = r.err_side = 0.0f;
  // (rare for dense activations: some |x| below the threshold, or a zero).
  // The empty asm keeps the compiler from hoisting this work above the
  // branch, into every block's build.
  if (__builtin_amdgcn_ballot_w64(amin < thr) != 0u) {
    float xs[16];
    uint32_t fs[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      xs[k] = xv[k];
      fs[k] = r.fx[k];
      asm volatile("" : "+v"(xs[k]), "+v"(fs[k]));
    }
    // side: 0 < |x| < thr, as integers: bits(|x|) - 1 below bits(thr) - 1
    const uint32_t tb = __float_as_uint(thr) - 1u;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool side = ((__float_as_uint(xs[k]) & 0x7fffffffu) - 1u) < tb;
      r.smask |= (uint32_t)side << k;
      r.xsum_side += side ? xs[k] : 0.0f;
      // |X| < 2^16 for a side element, so (float)X and the difference are exact
      const float err =
          fabsf(xs[k] - __builtin_amdgcn_ldexpf((float)(int)fs[k], r.e - kFixBits));
      r.err_side += side ? err : 0.0f;
    }
  }
  return r;
}

// Side list of one block from its 16 lanes (one DPP row, lane n holding
// elements 16 n .. 16 n + 15 in `xv`): returns the block's side count (the
// same in every lane of the row); when it is at most kSideMax and `write`,
// the lanes store their entries (element index, x bits) in element order at
// `list` (8 bytes each).
__device__ __forceinline__ uint32_t side_list(const float (&xv)[16], uint32_t smask, uint32_t n,
                                              uint32_t list, bool write) {
  const uint32_t own = __builtin_popcount(smask);
  uint32_t incl = own;  // inclusive prefix count over the row
  incl += dpp_u<kRowShr1>(incl);
  incl += dpp_u<kRowShr2>(incl);
  incl += dpp_u<kRowShr4>(incl);
  incl += dpp_u<kRowShr8>(incl);
  const uint32_t total = dpp_u<kRowBcast15>(incl);
  if (write && smask != 0u && total <= kSideMax) {
    uint32_t pos = incl - own;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if ((smask >> k) & 1u) {
        lds_write_b64(list + kSideEntryBytes * pos, u32x2{16u * n + (uint32_t)k,
                                                           __float_as_uint(xv[k])});
        ++pos;
      }
    }
  }
  return total;
}

// The biased digit words of a chunk: X + 0x80808080, with X = 0 for side
// elements that go to the block's side list (`listed`).
__device__ __forceinline__ void biased_values(const ChunkSplit& cs, bool listed, uint32_t (&u)[16]) {
#pragma unroll
  for (int k = 0; k < 16; ++k)
    u[k] = ((listed && ((cs.smask >> k) & 1u)) ? 0u : cs.fx[k]) + 0x80808080u;
}

// Sum of the fixed-point values X of a 32-element unit whose two 16-element
// halves are held by this lane (biased digit words u = X + 0x80808080) and the
// lane before it in its DPP row; the result is valid in the odd lanes.  The
// sum is exact (X = hi 2^15 + lo with both parts summed as integers below
// 2^20) and rounded to f32 once, so the min term d_min * m * sum X of a unit
// sees the activations rounded exactly as the MFMA digit sums do.
__device__ __forceinline__ float unit_fixed_sum(const uint32_t (&u)[16]) {
  uint32_t hi = 0u, lo = 0u;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int32_t X = (int32_t)(u[k] - 0x80808080u);
    hi += (uint32_t)(X >> 15);
    lo += (uint32_t)X & 0x7fffu;
  }
  hi += dpp_u<kRowShr1>(hi);
  lo += dpp_u<kRowShr1>(lo);
  return fmaf((float)(int32_t)hi, 32768.0f, (float)lo);
}

// Turns the copied blocks of activation vector `tok` into digit images in
// place, plus exponents, the error sums of rounded blocks, side counts
// (kSideRounded or 0) and, when the layout keeps them, the sums of each
// 32-element unit's fixed-point values (unit_fixed_sum, in units of
// 2^(e_b - 30)).  The caller has waited for the copies.  CHUNK_SLOT(c)
// gives the byte offset, inside the block's 1 KB, of the A row 4 p (digit 0)
// of MFMA t that holds chunk c (elements 16 c .. 16 c + 15): 256 t + 64 p.  A
// block with an activation that is not finite or reaches 2^100 gets exponent
// kBadBlock and side count 0.
template <int WAVES, typename ChunkSlot>
__device__ __forceinline__ void build_images(uint32_t sbase, const Layout& L, uint32_t nb,
                                             uint32_t wave, uint32_t grp, uint32_t n,
                                             ChunkSlot chunk_slot, uint32_t tok = 0u) {
  const uint32_t npass = (nb + 4u * WAVES - 1u) / (4u * WAVES);
  const bool want_sums = L.xsum_stride != 0u;
  const uint32_t img = L.img + tok * L.img_stride;
  const uint32_t xsb = L.xsum + tok * L.xsum_stride;
  const uint32_t exb = L.expo + tok * L.expo_stride;
  const uint32_t sdb = exb + L.side_off;
  for (uint32_t j = 0; j < npass; ++j) {
    if (4u * (wave + WAVES * j) >= nb) break;
    // lane (grp, n): elements 16n..16n+15 of block pb
    const uint32_t pb = 4u * (wave + WAVES * j) + grp;
    const uint32_t pbc = pb < nb ? pb : nb - 1u;  // lanes past K redo the last block, unstored
    u32x4 xq[4];
    lds_read4<16>(sbase + img + 1024u * pbc + 64u * n, xq);
    float xv[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int c = 0; c < 4; ++c) xv[4 * k + c] = __uint_as_float(xq[k][c]);
    const ChunkSplit cs = split_chunk(xv);
    const bool store = pb < nb;
    const bool bad_blk = (__builtin_amdgcn_ballot_w64(cs.bad) >> (16u * grp)) & 0xffffull;
    const uint32_t list = sbase + sdb + kSideBytes * pb;
    const bool rounded =
        !bad_blk && ((__builtin_amdgcn_ballot_w64(cs.smask != 0u) >> (16u * grp)) & 0xffffull);
    uint32_t u[16];
    biased_values(cs, false, u);
    uint32_t dg[4][4];  // [element quad][digit]
#pragma unroll
    for (int k = 0; k < 4; ++k) transpose_digits(u[4 * k], u[4 * k + 1], u[4 * k + 2], u[4 * k + 3], dg[k]);
    // all lanes of the group have read the block before any lane writes it
    const uint32_t slot = chunk_slot(n);
    const uint32_t ib = sbase + img + 1024u * pbc + slot;
    if (store) {
#pragma unroll
      for (int d = 0; d < 4; ++d)
        lds_write_b128(ib + 16u * d, u32x4{dg[0][d], dg[1][d], dg[2][d], dg[3][d]});
      if (rounded)  // position 4 p + t
        lds_write_b32(list + 4u * (4u * ((slot >> 6) & 3u) + (slot >> 8)),
                      __float_as_uint(cs.err_side));
    }
    if (want_sums) {
      const float xsum = unit_fixed_sum(u);  // odd lanes: unit n / 2
      if (store && (n & 1u))
        lds_write_b32(sbase + xsb + 32u * pb + 4u * (n >> 1), __float_as_uint(xsum));
    }
    if (store && n == 0u) {
      lds_write_b32(sbase + exb + 4u * pb, (uint32_t)(bad_blk ? kBadBlock : cs.e - kFixBits));
      lds_write_b8(sbase + exb + count_pos(L, pb), rounded ? kSideRounded : 0u);
    }
  }
}

// Whether the row of this lane passes the rounded-block check of a stage:
// `err` the lane's error bound from its rounded blocks, `abs_part` its sum of
// |partial dot| over all blocks of the stage (both summed over the four lane
// groups of the row here).  sum |partial| - err is at most the row's
// sum |w x| over the stage.
__device__ __forceinline__ bool rounded_ok(float err, float abs_part) {
  const float e = sum_lane_groups(err), a = sum_lane_groups(abs_part);
  return e * 1.01f <= kRoundedTol * (a - e);
}
// Sum of a rounded block's error sums over the four chunks of lane group p.
__device__ __forceinline__ float rounded_err(uint32_t list, uint32_t p) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(list + 16u * p) : "memory");
  return (__uint_as_float(v[0]) + __uint_as_float(v[1])) +
         (__uint_as_float(v[2]) + __uint_as_float(v[3]));
}

// f(integral_constant<int, I>) for I = 0 .. N-1, so that register arrays are
// indexed with constants.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Rounded blocks of a stage of NB blocks for one activation vector, in a
// kernel whose lane group `grp` holds a 64-element share of every block
// (part[b]: the lane's partial dot of block b).  `list`: the side area of the
// stage's first block; `counts`: the blocks' side counts, one byte each (0
// for blocks on the exact path or past the matrix).
// Bit b of the result: byte b of the counts marks a rounded block.
__device__ __forceinline__ uint32_t rounded_mask(uint32_t counts) {
  const uint32_t r = counts & (counts >> 1) & (counts >> 2) & (counts >> 3) & (counts >> 4) &
                     (counts >> 5) & (counts >> 6) & (counts >> 7) & 0x01010101u;
  return (r & 1u) | ((r >> 7) & 2u) | ((r >> 14) & 4u) | ((r >> 21) & 8u);
}

// The rounded blocks this lane must recompute exactly: all of the stage's
// rounded blocks when its row fails the check (rounded_ok), else none.
// bound(b): the largest |w| the lane's share of block b can hold.
template <int NB, typename Bound>
__device__ __forceinline__ uint32_t rounded_redo(uint32_t list, uint32_t counts, uint32_t grp,
                                                 const float (&part)[NB], Bound bound) {
  const uint32_t rmask = rounded_mask(counts);
  if (rmask == 0u) return 0u;
  float err = 0.0f, a = 0.0f;
  static_for<NB>([&](auto bc) {
    constexpr int b = decltype(bc)::value;
    if ((rmask >> b) & 1u) err = fmaf(bound(bc), rounded_err(list + kSideBytes * b, grp), err);
    a += fabsf(part[b]);
  });
  return rounded_ok(err, a) ? 0u : rmask;
}

// The lane's error bound from the rounded blocks of a stage (rmask: bit b
// for a rounded block b): the largest |w| of its share of the block times
// that share's rounding-error sum.
template <int NB, typename Bound>
__device__ __forceinline__ float rounded_bound(uint32_t list, uint32_t rmask, uint32_t grp,
                                               Bound bound) {
  float err = 0.0f;
  static_for<NB>([&](auto bc) {
    constexpr int b = decltype(bc)::value;
    if ((rmask >> b) & 1u) err = fmaf(bound(bc), rounded_err(list + kSideBytes * b, grp), err);
  });
  return err;
}

// The stage check of the Q4_K / Q5_K kernels: whether the row of this lane
// passes with `err`, the lane's bound on the error of its fast-path partials
// (their f32 rounding plus its rounded blocks), and `abs_part`, its sum of
// |partial| (both summed over the row's four lane groups here).  A row that
// fails recomputes the stage on the exact per-weight path.
__device__ __forceinline__ bool stage_ok(float err, float abs_part) {
  const float e = sum_lane_groups(err), a = sum_lane_groups(abs_part);
  return e * 1.01f <= kStageTol * (a - e);
}

// Slot ring set-up: every slot empty and owned by local tile == its index;
// no image builder done; the next pair to claim (L.ready + 4, for kernels
// whose waves claim their pairs after the first, pair `wave`) is WAVES.
template <int WAVES>
__device__ __forceinline__ void init_slots(uint32_t sbase, const Layout& L, uint32_t slots) {
  for (uint32_t k = threadIdx.x; k < slots; k += WAVES * 64u) {
    lds_write_b32(sbase + L.cnt + 4u * k, 0u);
    lds_write_b32(sbase + L.owner + 4u * k, k);
  }
  if (threadIdx.x == 0u) {
    lds_write_b32(sbase + L.ready, 0u);
    lds_write_b32(sbase + L.ready + 4u, (uint32_t)WAVES);
  }
}

// Waits until `builders` waves have counted their images done at L.ready.
// Bounded like wait_slot: a wave that gives up sets `fail`.
__device__ __forceinline__ void wait_images(uint32_t sbase, const Layout& L, uint32_t builders,
                                            uint32_t& fail) {
  uint32_t spin = 0;
  for (; lds_read_b32(sbase + L.ready) < builders && spin < (1u << 24); ++spin)
    __builtin_amdgcn_s_sleep(1);
  if (__builtin_amdgcn_readfirstlane(spin) == (1u << 24)) fail = kDevErrSlotWait;
}

// Division by a launch constant d as a multiply-high: m = ceil(2^32 / d) (0
// for d = 1) gives floor(x / d) exactly whenever x * d < 2^32, which the host
// guarantees for every quotient taken this way (pair, tile and range
// indices).  The constants come from the host: the GPU has no integer divide,
// and the dozen dependent instructions of each software division cost a
// workgroup a noticeable part of a microsecond before its first weight copy.
struct FastDiv {
  uint32_t d, m;
};
__host__ __device__ constexpr uint32_t div_magic(uint32_t d) {
  return d > 1u ? 0xffffffffu / d + 1u : 0u;
}
__device__ __forceinline__ uint32_t quo(uint32_t x, const FastDiv& f) {
  return f.m ? __umulhi(x, f.m) : x;
}

// The launch constants of the work split below, one kernel argument: the ring
// slot count (bits 0-7), the split flag (bit 8) and the workgroup count G
// (bits 16-31), then the division constants of G, the partials per tile and
// the slot count.  Kept to 16 bytes so a kernel's arguments stay within the
// first 64-byte line of its argument block (one memory round trip).
struct SchedArgs {
  uint32_t packed;
  uint32_t m_groups, m_parts, m_slots;
};

// Several matrices of one K in one launch (grouped matvec): matrix k's packed
// rows, the running count of 16-row tiles up to and including it (past the
// group's last matrix, UINT32_MAX, which no tile reaches) and its row count.
// After SchedArgs, so kernels that do not read it keep their first 64 bytes
// of arguments as they were; its 128 bytes are the next two 64-byte lines,
// which the grouped kernels load beside the first.
constexpr uint32_t kMaxGroup = 8;
struct GroupArgs {
  const uint8_t* w[kMaxGroup];
  uint32_t tile_end[kMaxGroup];
  uint32_t rows[kMaxGroup];
};
static_assert(sizeof(GroupArgs) == 128, "two argument lines");

// A grouped kernel's first statement: the matrix table's loads go out with
// those of the first argument line (the compiler would issue them once the
// schedule is worked out, and their latency would then come before the
// first weight copy).
__device__ __forceinline__ void load_group_args_early(const GroupArgs& ga) {
#pragma unroll
  for (uint32_t k = 0; k < kMaxGroup; ++k)
    asm volatile("" ::"s"(ga.w[k]), "s"(ga.rows[k]), "s"(ga.tile_end[k]));
}

// Work split.  With G workgroups and T tiles of S partials each, workgroup g
// owns the whole tiles g, g + G, ...  When that leaves some workgroups a
// round of pairs more than others (rounds = pairs / waves, rounded up), the
// launch "splits": workgroup g keeps q = T / G whole tiles g, g + G, ...,
// g + (q - 1) G, and the L = (T - q G) S pairs of the leftover tiles are cut
// into G contiguous ranges, so every workgroup gets the same number of pairs
// to within one.  A leftover tile whose pairs fall into two or more ranges is
// "split": each of its workgroups sums its own partials, publishes them in a
// small global workspace and counts them on the tile's global counter; the
// workgroup that completes the count adds the published sums in workgroup
// order and stores the rows (deterministic for a given grid).  That exchange
// costs a wave a few microseconds of waiting, so the leftover pairs go to the
// last waves of the first round -- waves with a pair less than the others --
// when the ring has a slot for every tile of the workgroup (tiles are then
// not taken in slot order), and first otherwise.
struct Sched {
  uint32_t a, b;        // [a, b): this workgroup's leftover pairs
  uint32_t lpairs;      // L
  uint32_t split_base;  // first leftover tile, q G
  uint32_t nsplit;      // leftover tiles this workgroup touches
  uint32_t nwhole;      // whole tiles g + G t, t < nwhole (g = blockIdx.x)
  uint32_t groups;      // G
  uint32_t npairs;      // this workgroup's pairs
  uint32_t slack0;      // > 0: leftover pairs at positions slack0 .. slack0 + nl - 1
  FastDiv by_parts, by_slots;
  uint32_t t_a;         // first leftover tile index (a / parts)
};
// First leftover pair of workgroup g: floor(g L / G).
__device__ __forceinline__ uint32_t range_start(uint32_t g, uint32_t lpairs,
                                                const FastDiv& by_groups) {
  return quo(g * lpairs, by_groups);
}
// (the division constant of G is taken from the kernel argument where it is
// needed rather than kept in the schedule, which would hold a scalar register
// through the whole kernel)
__device__ __forceinline__ uint32_t range_start(const Sched& s, const SchedArgs& sa, uint32_t g) {
  return range_start(g, s.lpairs, FastDiv{s.groups, sa.m_groups});
}
// The workgroup whose range holds leftover pair p (p < L), i.e. the g with
// range_start(g) <= p < range_start(g + 1): p G / L in floating point (with
// the approximate reciprocal) is within one or two of it, and the loops
// settle the rest.
__device__ __forceinline__ uint32_t range_of(const Sched& s, const SchedArgs& sa, uint32_t p) {
  const uint32_t G = s.groups;
  uint32_t g = min((uint32_t)((float)p * (float)G * __builtin_amdgcn_rcpf((float)s.lpairs)), G - 1u);
  while (g > 0u && range_start(s, sa, g) > p) --g;
  while (g + 1u < G && range_start(s, sa, g + 1u) <= p) ++g;
  return g;
}
__device__ __forceinline__ Sched make_sched(uint32_t ntiles, uint32_t tparts, uint32_t waves,
                                            const SchedArgs& sa) {
  Sched s;
  const uint32_t G = sa.packed >> 16, g = blockIdx.x, slots = sa.packed & 0xffu;
  const bool split = (sa.packed & 0x100u) != 0u;
  const FastDiv by_parts{tparts, sa.m_parts}, by_groups{G, sa.m_groups};
  // (plain locals first: the struct is filled in once at the end)
  const uint32_t nwhole = split ? quo(ntiles, by_groups)
                                : (g < ntiles ? quo(ntiles - 1u - g, by_groups) + 1u : 0u);
  const uint32_t split_base = split ? nwhole * G : ntiles;
  const uint32_t lpairs = split ? (ntiles - split_base) * tparts : 0u;
  const uint32_t a = split ? range_start(g, lpairs, by_groups) : 0u;
  const uint32_t b = split ? range_start(g + 1u, lpairs, by_groups) : 0u;
  const uint32_t t_a = quo(a, by_parts);
  s.by_parts = by_parts;
  s.by_slots = FastDiv{slots, sa.m_slots};
  s.groups = G;
  s.slack0 = 0u;
  s.nwhole = nwhole;
  s.split_base = split_base;
  s.lpairs = lpairs;
  s.a = a;
  s.b = b;
  s.t_a = t_a;
  s.nsplit = b > a ? quo(b - 1u, by_parts) - t_a + 1u : 0u;
  s.npairs = (s.b - s.a) + s.nwhole * tparts;
  const uint32_t nl = s.b - s.a, last = s.npairs % waves;
  if (nl > 0u && nl < waves && s.npairs > waves && last != 0u && last <= waves - nl &&
      s.nsplit + s.nwhole <= slots)
    s.slack0 = waves - nl;
  return s;
}
// The workgroup's pair k: tile, partial r, local tile index lt (its ring
// slot is lt % slots) and the workgroup's share [lo, hi) of that tile's
// partials.
struct Pair {
  uint32_t tile, r, lt, lo, hi;
};
__device__ __forceinline__ Pair pair_at(const Sched& s, uint32_t k, uint32_t tparts) {
  Pair p;
  const uint32_t nl = s.b - s.a;
  bool split;
  uint32_t ks;  // index among the leftover pairs, or nl + index among the whole-tile pairs
  if (s.slack0) {
    split = k >= s.slack0 && k < s.slack0 + nl;
    ks = split ? k - s.slack0 : (k < s.slack0 ? k + nl : k);
  } else {
    split = k < nl;
    ks = k;
  }
  if (split) {
    const uint32_t lp = s.a + ks, t = quo(lp, s.by_parts);
    p.tile = s.split_base + t;
    p.r = lp - t * tparts;
    p.lt = t - s.t_a;
    p.lo = max(s.a, t * tparts) - t * tparts;
    p.hi = min(s.b, (t + 1u) * tparts) - t * tparts;
  } else {
    const uint32_t kk = ks - nl, t = quo(kk, s.by_parts);
    p.tile = blockIdx.x + s.groups * t;
    p.r = kk - t * tparts;
    p.lt = s.nsplit + t;
    p.lo = 0u;
    p.hi = tparts;
  }
  return p;
}

// Global workspace of split tiles: one counter per tile at the start (a fixed
// region, so launches of any grid size find their counters at zero), then per
// workgroup two entries (its first and its last tile) of MATS x 16 row sums.
// An entry that holds no sum holds kPartEmpty, a signalling-NaN pattern that
// no arithmetic result can have (results of operations are quiet NaNs).
struct SplitWs {
  float* part;
  uint32_t* cnt;
};
constexpr size_t kCounterBytes = kWorkspaceCounterBytes;
constexpr uint32_t kPartEmpty = kWorkspaceEmpty;
__host__ __device__ constexpr bool split_ws_fits(size_t ws_bytes, uint32_t ngroups,
                                                 uint32_t ntiles, uint32_t mats) {
  return (size_t)ntiles * 4u + 64u <= kCounterBytes &&  // the last words are the argmax's
         kCounterBytes + (size_t)ngroups * 2u * mats * 64u <= ws_bytes;
}
__host__ __device__ inline SplitWs split_ws(void* base) {
  SplitWs w;
  w.cnt = static_cast<uint32_t*>(base);
  w.part = reinterpret_cast<float*>(static_cast<uint8_t*>(base) + kCounterBytes);
  return w;
}

// Device-coherent (sc1) word accesses: each XCD has its own L2, and these
// bypass it for the few words workgroups exchange.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until ring slot word `owner_at` names local tile lt.  The wait is
// bounded (about 2^24 polls, seconds): a wave that gives up sets `fail` to
// kDevErrSlotWait and goes on, its results then invalid.  (Kernels report a
// set `fail` once, at their end: report_device_error.)
__device__ __forceinline__ void wait_slot(uint32_t owner_at, uint32_t lt, uint32_t& fail) {
  uint32_t spin = 0;
  for (; lds_read_b32(owner_at) != lt && spin < (1u << 24); ++spin) __builtin_amdgcn_s_sleep(1);
  if (__builtin_amdgcn_readfirstlane(spin) == (1u << 24)) fail = kDevErrSlotWait;
}

// Hands partial pr.r (of tparts = MATS * nparts per tile) of tile pr.tile to
// the tile's LDS slot, waiting while an earlier tile still holds it.  The wave
// that completes the workgroup's share of the tile sums that share in partial
// order and stores the rows -- y[row] = sum, or with MATS == 2 silu(sum of
// partials < nparts) * (sum of the rest) -- or, for a split tile, publishes
// the sums and, if it completes the tile, combines all shares.  ARGMAX: every
// row also enters *best (argmax_candidate under `rule`), and y may be null.
//
// PAIRED (one matrix whose rows are taken in pairs, row r of the launch being
// rows 2 r and 2 r + 1 of y): each of the tile's nparts pairs hands two
// partials, rowsum for row 2 r at slot partial pr.r and rowsum2 for row
// 2 r + 1 at partial nparts + pr.r; the two sums are added and stored apart.
template <int MATS, bool ARGMAX = false, bool PAIRED = false>
__device__ __forceinline__ void hand_off(uint32_t sbase, const Layout& L, uint32_t slots,
                                         const Sched& sc, const SchedArgs& sa, const Pair& pr,
                                         uint32_t nparts,
                                         float rowsum, uint32_t lane, uint32_t rows,
                                         float* __restrict__ y, SplitWs ws, uint32_t& fail,
                                         uint64_t* best = nullptr, uint32_t rule = 0u,
                                         float rowsum2 = 0.0f) {
  static_assert(!PAIRED || MATS == 1, "paired rows of one matrix");
  constexpr bool kTwo = MATS > 1 || PAIRED;  // two sums per row of the tile
  constexpr uint32_t kSums = kTwo ? 2u : 1u;
  auto store_row = [&](uint32_t row, float v) {
    if constexpr (ARGMAX) {
      if (y) y[row] = v;  // a head whose logits are not wanted stores none
      const uint64_t c = argmax_candidate(v, row, rule);
      *best = c > *best ? c : *best;
    } else {
      y[row] = v;
    }
  };
  // the finished rows: y[row] = sum (MATS 1), silu(sum) * sum2 (MATS 2), or
  // y[2 row] = sum and y[2 row + 1] = sum2 (PAIRED)
  auto store_sums = [&](uint32_t row, float a, float b) {
    if constexpr (PAIRED) {
      store_row(2u * row, a);
      store_row(2u * row + 1u, b);
    } else {
      store_row(row, MATS > 1 ? silu_times(a, b) : a);
    }
  };
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t tparts = PAIRED ? nparts : MATS * nparts;  // pairs per tile
  const uint32_t sstride = kTwo ? 2u * nparts : nparts;      // LDS partials per slot
  const uint32_t slot = pr.lt - quo(pr.lt, sc.by_slots) * slots;
  wait_slot(sbase + L.owner + 4u * slot, pr.lt, fail);
  if (grp == 0u) {
    lds_write_b32(sbase + L.part + 64u * (slot * sstride + pr.r) + 4u * n, __float_as_uint(rowsum));
    if constexpr (PAIRED)
      lds_write_b32(sbase + L.part + 64u * (slot * sstride + nparts + pr.r) + 4u * n,
                    __float_as_uint(rowsum2));
  }
  uint32_t old = 0u;
  if (lane == 0u) old = lds_add_rtn(sbase + L.cnt + 4u * slot, 1u);  // one lane: no serialised atomics
  const uint32_t done = __builtin_amdgcn_readlane(old, 0);
  if (done != pr.hi - pr.lo - 1u) return;
  float sum = 0.0f, sum2 = 0.0f;
  for (uint32_t st = pr.lo; st < pr.hi; ++st) {
    const float v =
        __uint_as_float(lds_read_b32(sbase + L.part + 64u * (slot * sstride + st) + 4u * n));
    if constexpr (PAIRED) {
      sum += v;
      sum2 += __uint_as_float(
          lds_read_b32(sbase + L.part + 64u * (slot * sstride + nparts + st) + 4u * n));
    } else if (MATS == 1 || st < nparts) {
      sum += v;
    } else {
      sum2 += v;
    }
  }
  const uint32_t row = pr.tile * 16u + n;
  if (pr.lo == 0u && pr.hi == tparts) {
    if (grp == 0u && row < rows) store_sums(row, sum, sum2);
  } else {
    // Publish the share's sums, then count the share; no fence orders the
    // two: the workgroup that completes the count waits for each entry to
    // leave the empty state.  Only read-modify-write atomics touch the counter.
    // The tile's shares belong to workgroups g0..g1 (those with pairs of it);
    // lane group k reads the entry of share g0 + k of each batch of four, the
    // first batch before the count goes out, so the workgroup that completes
    // it waits about one memory round trip for the other shares.
    // (The lane's indices are taken afresh here, behind a compiler barrier,
    // so that no address of this rare path is kept live through the caller's
    // main loop.)
    uint32_t ln = lane;
    asm volatile("" : "+v"(ln));
    const uint32_t grp = ln >> 4, n = ln & 15u;
    const uint32_t t = pr.tile - sc.split_base;  // leftover tile index
    const uint32_t e = 2u * blockIdx.x + (t == sc.t_a ? 0u : 1u);
    if (grp == 0u) {
      store_coherent(ws.part + (e * kSums) * 16u + n, sum);
      if (kTwo) store_coherent(ws.part + (e * kSums + 1u) * 16u + n, sum2);
    }
    const uint32_t g0 = range_of(sc, sa, t * tparts);
    const uint32_t g1 = range_of(sc, sa, t * tparts + tparts - 1u);
    // float offset of share wg's entry for this tile in ws.part, or kNoEntry
    // when wg holds none of its pairs
    constexpr uint32_t kNoEntry = 0xffffffffu;
    auto entry = [&](uint32_t wg) -> uint32_t {
      if (wg > g1) return kNoEntry;
      const uint32_t wa = range_start(sc, sa, wg);
      if (wa == range_start(sc, sa, wg + 1u)) return kNoEntry;  // no leftover pairs
      const uint32_t t0 = quo(wa, sc.by_parts);
      return (2u * wg + (t == t0 ? 0u : 1u)) * kSums * 16u + n;
    };
    // this workgroup's own share is taken from registers, not read back
    auto fetch = [&](uint32_t off, uint32_t wg, float& v, float& v2) {
      if (wg == blockIdx.x) {
        v = sum;
        if (kTwo) v2 = sum2;
      } else if (off != kNoEntry) {
        v = load_coherent(ws.part + off);
        if (kTwo) v2 = load_coherent(ws.part + off + 16u);
      }
    };
    uint32_t off = entry(g0 + grp);
    float v = 0.0f, v2 = 0.0f;
    fetch(off, g0 + grp, v, v2);
    const uint32_t force = __builtin_amdgcn_readfirstlane(give_up_polls(ws.cnt));
    // (the count goes out after those reads, so waiting for it -- and for
    // every older memory operation of the wave -- takes one round trip)
    uint32_t before = 0u;
    if (lane == 0u)
      before = __hip_atomic_fetch_add(ws.cnt + t, pr.hi - pr.lo, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    before = __builtin_amdgcn_readlane(before, 0);
    if (before + (pr.hi - pr.lo) == tparts) {
      float g = 0.0f, u = 0.0f;
      for (uint32_t base = g0; base <= g1; base += 4u) {
        const uint32_t wg = base + grp;
        if (base != g0) {
          off = entry(wg);
          fetch(off, wg, v, v2);
        }
        // wait (bounded: about 2^22 polls, or the test hook's count) until
        // every entry of the batch has landed; on giving up, set `fail` and
        // add what is there
        for (uint32_t spin = 0;; ++spin) {
          const bool missing = off != kNoEntry && wg != blockIdx.x &&
                               (force != 0u || __float_as_uint(v) == kPartEmpty ||
                                (kTwo && __float_as_uint(v2) == kPartEmpty));
          if (!__builtin_amdgcn_ballot_w64(missing)) break;
          if (spin == (force != 0u ? force : (1u << 22))) {
            fail = kDevErrCombineWait;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          if (missing) fetch(off, wg, v, v2);
        }
        // add the batch in workgroup order (lane group 0 keeps the sums)
        const uint64_t have = __builtin_amdgcn_ballot_w64(off != kNoEntry);
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) {
          const float vk = __shfl(v, (int)(n + 16u * k), 64);
          const float v2k = kTwo ? __shfl(v2, (int)(n + 16u * k), 64) : 0.0f;
          if ((have >> (16u * k)) & 1u) {
            g += vk;
            if (kTwo) u += v2k;
          }
        }
        if (off != kNoEntry) {
          store_coherent(ws.part + off, __uint_as_float(kPartEmpty));
          if (kTwo) store_coherent(ws.part + off + 16u, __uint_as_float(kPartEmpty));
        }
      }
      if (grp == 0u && row < rows) store_sums(row, g, u);
      if (lane == 0u)
        (void)__hip_atomic_exchange(ws.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (lane == 0u) {
    lds_write_b32(sbase + L.cnt + 4u * slot, 0u);
    lds_write_b32(sbase + L.owner + 4u * slot, pr.lt + slots);
  }
}

// K-sliced launches, for matrices of few tiles and long rows (a down
// projection): the stages of every tile are cut into S slices as even as the
// stage count allows, and workgroup g = S tg + s works on slice s of the tiles
// tg, tg + Gs, tg + 2 Gs, ... (Gs = G / S).  A workgroup then holds the
// activation images of its slice only, so it builds a 1 / S share of them
// before its first stage.  The S slice sums of a tile meet in the workspace:
// the wave that completes a slice publishes its 16 sums in entry
// tile * S + s and counts them on the tile's counter, and the wave that
// completes the count adds the S entries in slice order and stores the rows
// (deterministic).  Launch constants: S, Gs, the slices' stage counts
// (ns_lo, and ns_lo + 1 for slices s < rem) and their division constants.
struct SliceArgs {
  uint32_t slices, m_slices, tgroups, m_tgroups;
  uint32_t ns_lo, rem, m_ns_lo, m_ns_hi;
};
struct SliceSched {
  uint32_t s, tg, r_lo, ns, npairs;
  uint32_t slices, tgroups;
  uint32_t pstride;  // partials per ring slot: the longest slice's stage count
  FastDiv by_ns, by_slots;
};
__device__ __forceinline__ SliceSched make_slice_sched(uint32_t ntiles, const SliceArgs& a,
                                                       const SchedArgs& sa) {
  SliceSched s;
  const uint32_t g = blockIdx.x;
  const uint32_t tg = quo(g, FastDiv{a.slices, a.m_slices});
  const uint32_t sl = g - tg * a.slices;
  const bool longer = sl < a.rem;
  const uint32_t ntl =
      tg < ntiles ? quo(ntiles - 1u - tg, FastDiv{a.tgroups, a.m_tgroups}) + 1u : 0u;
  s.s = sl;
  s.tg = tg;
  s.ns = a.ns_lo + (longer ? 1u : 0u);
  s.r_lo = sl * a.ns_lo + min(sl, a.rem);
  s.npairs = ntl * s.ns;
  s.slices = a.slices;
  s.tgroups = a.tgroups;
  s.pstride = a.ns_lo + (a.rem != 0u ? 1u : 0u);
  s.by_ns = FastDiv{s.ns, longer ? a.m_ns_hi : a.m_ns_lo};
  s.by_slots = FastDiv{sa.packed & 0xffu, sa.m_slots};
  return s;
}
// Pair k of a sliced workgroup: local tile lt = k / ns, stage r_lo + k % ns;
// [lo, hi) is the slice.
__device__ __forceinline__ Pair pair_at(const SliceSched& s, uint32_t k) {
  Pair p;
  const uint32_t lt = quo(k, s.by_ns);
  p.tile = s.tg + s.tgroups * lt;
  p.r = s.r_lo + (k - lt * s.ns);
  p.lt = lt;
  p.lo = s.r_lo;
  p.hi = s.r_lo + s.ns;
  return p;
}

// hand_off for a sliced launch (one matrix): the wave that completes the
// workgroup's slice of the tile adds its partials in stage order, frees the
// ring slot, publishes the 16 sums and counts them; the wave that completes
// the tile's count of S adds the S entries in slice order (lane group k
// reads slice k of each batch of four; the first batch is read before the
// count goes out, so the last slice waits about one memory round trip),
// stores the rows and returns the entries and the counter to their empty
// state.  The wait for an entry is bounded like hand_off's.  TWO (row pairs):
// every row has two sums, rowsum for y[2 row] and rowsum2 for y[2 row + 1];
// the LDS keeps 2 pstride partials per slot and an entry 32 floats (the
// second sums at +16).
template <bool TWO = false>
__device__ __forceinline__ void hand_off_slice(uint32_t sbase, const Layout& L,
                                               const SliceSched& sc, const Pair& pr, float rowsum,
                                               uint32_t lane, uint32_t rows, float* __restrict__ y,
                                               SplitWs ws, uint32_t& fail, float rowsum2 = 0.0f) {
  constexpr uint32_t kSums = TWO ? 2u : 1u;
  const uint32_t slots = sc.by_slots.d;
  const uint32_t slot = pr.lt - quo(pr.lt, sc.by_slots) * slots;
  wait_slot(sbase + L.owner + 4u * slot, pr.lt, fail);
  const uint32_t pbase = sbase + L.part + 64u * kSums * sc.pstride * slot + 4u * (lane & 15u);
  const uint32_t pbase2 = pbase + 64u * sc.pstride;  // TWO: the second sums
  if ((lane >> 4) == 0u) {
    lds_write_b32(pbase + 64u * (pr.r - pr.lo), __float_as_uint(rowsum));
    if constexpr (TWO) lds_write_b32(pbase2 + 64u * (pr.r - pr.lo), __float_as_uint(rowsum2));
  }
  uint32_t old = 0u;
  if (lane == 0u) old = lds_add_rtn(sbase + L.cnt + 4u * slot, 1u);
  const uint32_t done = __builtin_amdgcn_readlane(old, 0);
  if (done != sc.ns - 1u) return;
  float sum = 0.0f, sum2 = 0.0f;
  for (uint32_t k = 0; k < sc.ns; ++k) {
    sum += __uint_as_float(lds_read_b32(pbase + 64u * k));
    if constexpr (TWO) sum2 += __uint_as_float(lds_read_b32(pbase2 + 64u * k));
  }
  // the partials are in registers: the slot can take the workgroup's next tile
  if (lane == 0u) {
    lds_write_b32(sbase + L.cnt + 4u * slot, 0u);
    lds_write_b32(sbase + L.owner + 4u * slot, pr.lt + slots);
  }
  // (the lane's indices are taken afresh behind a compiler barrier, so that
  // none of this path's addresses stays live through the caller's loop)
  uint32_t ln = lane;
  asm volatile("" : "+v"(ln));
  const uint32_t grp = ln >> 4, n = ln & 15u;
  const uint32_t S = sc.slices;
  // slice k at ent + 16 kSums k (its second sums 16 floats on)
  float* const ent = ws.part + (size_t)pr.tile * S * 16u * kSums + n;
  if (grp == 0u) {
    store_coherent(ent + 16u * kSums * sc.s, sum);
    if constexpr (TWO) store_coherent(ent + 16u * kSums * sc.s + 16u, sum2);
  }
  auto fetch = [&](uint32_t k, float& v, float& v2) {
    if (k == sc.s) {
      v = sum;
      v2 = sum2;
    } else if (k < S) {
      v = load_coherent(ent + 16u * kSums * k);
      if constexpr (TWO) v2 = load_coherent(ent + 16u * kSums * k + 16u);
    }
  };
  float v = 0.0f, v2 = 0.0f;
  fetch(grp, v, v2);
  const uint32_t force = __builtin_amdgcn_readfirstlane(give_up_polls(ws.cnt));
  uint32_t before = 0u;
  if (lane == 0u)
    before = __hip_atomic_fetch_add(ws.cnt + pr.tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  before = __builtin_amdgcn_readlane(before, 0);
  if (before + 1u != S) return;
  float total = 0.0f, total2 = 0.0f;
  for (uint32_t base = 0; base < S; base += 4u) {
    const uint32_t k = base + grp;
    if (base != 0u) fetch(k, v, v2);
    for (uint32_t spin = 0;; ++spin) {
      const bool missing =
          k < S && k != sc.s &&
          (force != 0u || __float_as_uint(v) == kPartEmpty ||
           (TWO && __float_as_uint(v2) == kPartEmpty));
      if (!__builtin_amdgcn_ballot_w64(missing)) break;
      if (spin == (force != 0u ? force : (1u << 22))) {
        fail = kDevErrCombineWait;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if (missing) fetch(k, v, v2);
    }
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) {
      const float vj = __shfl(v, (int)(n + 16u * j), 64);
      if (base + j < S) total += vj;
      if constexpr (TWO) {
        const float wj = __shfl(v2, (int)(n + 16u * j), 64);
        if (base + j < S) total2 += wj;
      }
    }
    if (k < S) {
      store_coherent(ent + 16u * kSums * k, __uint_as_float(kPartEmpty));
      if constexpr (TWO) store_coherent(ent + 16u * kSums * k + 16u, __uint_as_float(kPartEmpty));
    }
  }
  const uint32_t row = pr.tile * 16u + n;
  if (grp == 0u && row < rows) {
    if constexpr (TWO) {
      y[2u * row] = total;
      y[2u * row + 1u] = total2;
    } else {
      y[row] = total;
    }
  }
  if (lane == 0u)
    (void)__hip_atomic_exchange(ws.cnt + pr.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The launch constants of a sliced launch of ntiles tiles of nstages stages
// in S slices over at most `cus` workgroups, or false when the shape does not
// fit: every slice at least one stage, the tiles' counters and S entries each
// inside the workspace (below the argmax area), the quotients exact.
struct SliceShape {
  uint32_t groups, tiles_per_group, ns_max;
  SliceArgs args;
};
inline bool slice_shape(uint32_t ntiles, uint32_t nstages, uint32_t S, uint32_t cus,
                        size_t ws_bytes, SliceShape* out, uint32_t entry_bytes = 64u) {
  if (S < 2u || S > 64u || nstages < S || ntiles == 0u || cus < S) return false;
  const uint32_t gs = min(ntiles, cus / S);
  if ((size_t)ntiles * 4u + 64u > kCounterBytes ||
      kCounterBytes + (size_t)ntiles * S * entry_bytes + 4096u > ws_bytes)
    return false;
  const uint32_t ns_lo = nstages / S, rem = nstages % S;
  out->groups = gs * S;
  out->tiles_per_group = (ntiles + gs - 1u) / gs;
  out->ns_max = ns_lo + (rem != 0u ? 1u : 0u);
  // pair quotients: k < tiles_per_group * ns_max, times ns
  if ((uint64_t)out->tiles_per_group * out->ns_max * out->ns_max >= (1ull << 32)) return false;
  out->args = SliceArgs{S, div_magic(S), gs, div_magic(gs), ns_lo, rem, div_magic(ns_lo),
                        div_magic(ns_lo + 1u)};
  return true;
}

inline int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

inline int cu_count() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    return n;
  }();
  return cus;
}

// Workgroups of a launch: one per CU, fewer when there are fewer pairs.
// Launch shape of a matrix-core matvec: workgroups, whether tiles are split
// (fewer rounds of pairs per wave than with whole tiles, in a launch of at
// least three rounds), and the most tiles one workgroup touches.
struct LaunchShape {
  uint32_t groups;
  bool split;
  uint32_t tiles_per_group;
};
// Pair and tile indices divided with FastDiv stay below ntiles * tparts and
// the ring's tile count below ntiles; the kernels need those times their
// divisor below 2^32.
inline bool quotients_fit(uint32_t ntiles, uint32_t tparts) {
  // ring slots are at most 8192 / 64 = 128
  return (uint64_t)ntiles * tparts * tparts < (1ull << 32) &&
         (uint64_t)ntiles * 128u < (1ull << 32);
}

inline LaunchShape launch_shape(uint32_t ntiles, uint32_t tparts, uint32_t waves,
                                size_t ws_bytes, uint32_t mats) {
  LaunchShape ls;
  const uint32_t cus = (uint32_t)cu_count();
  const uint32_t g0 = min(ntiles, cus);
  const uint64_t rounds0 = ((uint64_t)(ntiles + g0 - 1u) / g0 * tparts + waves - 1u) / waves;
  const uint32_t g1 = (uint32_t)min((uint64_t)cus, (uint64_t)ntiles * tparts);
  const uint32_t q = ntiles / g1;
  const uint64_t lpairs = (uint64_t)(ntiles - q * g1) * tparts;
  const uint64_t most = (uint64_t)q * tparts + (lpairs + g1 - 1u) / g1;
  const uint64_t rounds1 = (most + waves - 1u) / waves;
  // the cross-workgroup exchange costs about a round in a short launch, so
  // split only launches of three or more rounds
  ls.split = rounds1 < rounds0 && rounds0 >= 3u && split_ws_fits(ws_bytes, g1, ntiles, mats);
  ls.groups = ls.split ? g1 : g0;
  ls.tiles_per_group = ls.split ? q + (uint32_t)(((lpairs + g1 - 1u) / g1 + tparts - 1u) / tparts) + 1u
                                : (ntiles + g0 - 1u) / g0;
  return ls;
}

// hand_off for NTOK activation vectors at once, whole tiles only: partial r
// of the tile holds 16 rows x NTOK sums; the finishing wave stores
// y[tok * rows + row] for every token.  In two halves for kernels that write
// one vector's sums at a time: token_slot waits until the tile owns its ring
// slot and returns the LDS address of this lane's row in partial pr.r (vector
// t at + 64 t); token_slot_done counts the partial and, in the wave that
// completes the tile, adds the partials in order and stores the rows.
__device__ __forceinline__ uint32_t token_slot(uint32_t sbase, const Layout& L,
                                               const FastDiv& by_slots, const Pair& pr,
                                               uint32_t tparts, uint32_t ntok, uint32_t lane,
                                               uint32_t& fail) {
  const uint32_t slots = by_slots.d;
  const uint32_t slot = pr.lt - quo(pr.lt, by_slots) * slots;
  wait_slot(sbase + L.owner + 4u * slot, pr.lt, fail);
  return sbase + L.part + 64u * ntok * (slot * tparts + pr.r) + 4u * (lane & 15u);
}
template <int NTOK>
__device__ __forceinline__ void token_slot_done(uint32_t sbase, const Layout& L,
                                                const FastDiv& by_slots, const Pair& pr,
                                                uint32_t tparts, uint32_t lane, uint32_t rows,
                                                float* __restrict__ y) {
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t slots = by_slots.d;
  const uint32_t slot = pr.lt - quo(pr.lt, by_slots) * slots;
  uint32_t old = 0u;
  if (lane == 0u) old = lds_add_rtn(sbase + L.cnt + 4u * slot, 1u);
  const uint32_t done = __builtin_amdgcn_readlane(old, 0);
  if (done != tparts - 1u) return;
  // lane group g stores tokens g, g + 4, ...
  const uint32_t row = pr.tile * 16u + n;
  for (uint32_t t = grp; t < (uint32_t)NTOK; t += 4u) {
    float sum = 0.0f;
    for (uint32_t st = 0; st < tparts; ++st)
      sum += __uint_as_float(
          lds_read_b32(sbase + L.part + 64u * NTOK * (slot * tparts + st) + 64u * t + 4u * n));
    if (row < rows) y[(size_t)t * rows + row] = sum;
  }
  if (lane == 0u) {
    lds_write_b32(sbase + L.cnt + 4u * slot, 0u);
    lds_write_b32(sbase + L.owner + 4u * slot, pr.lt + slots);
  }
}
template <int NTOK>
__device__ __forceinline__ void hand_off_tokens(uint32_t sbase, const Layout& L,
                                                const FastDiv& by_slots, const Pair& pr,
                                                uint32_t tparts, const float (&rowsum)[NTOK],
                                                uint32_t lane, uint32_t rows,
                                                float* __restrict__ y, uint32_t& fail) {
  const uint32_t base = token_slot(sbase, L, by_slots, pr, tparts, NTOK, lane, fail);
  if ((lane >> 4) == 0u) {
#pragma unroll
    for (int t = 0; t < NTOK; ++t) lds_write_b32(base + 64u * t, __float_as_uint(rowsum[t]));
  }
  token_slot_done<NTOK>(sbase, L, by_slots, pr, tparts, lane, rows, y);
}

// hand_off_tokens for kernels that keep vector g's row sums in lane group g
// (lane 16 g + n holds vector g, row n): every lane writes its own sum; the
// finishing wave's lane group g stores vector g's rows (g < ntok).
__device__ __forceinline__ void hand_off_lane_tokens(uint32_t sbase, const Layout& L,
                                                     const FastDiv& by_slots, const Pair& pr,
                                                     uint32_t tparts, float rowsum, uint32_t lane,
                                                     uint32_t rows, uint32_t ntok,
                                                     float* __restrict__ y, uint32_t& fail) {
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t slots = by_slots.d;
  const uint32_t slot = pr.lt - quo(pr.lt, by_slots) * slots;
  wait_slot(sbase + L.owner + 4u * slot, pr.lt, fail);
  // the slot's partial r holds [vector][16 rows], 256 bytes
  lds_write_b32(sbase + L.part + 256u * (slot * tparts + pr.r) + 4u * lane,
                __float_as_uint(rowsum));
  uint32_t old = 0u;
  if (lane == 0u) old = lds_add_rtn(sbase + L.cnt + 4u * slot, 1u);
  const uint32_t done = __builtin_amdgcn_readlane(old, 0);
  if (done != tparts - 1u) return;
  const uint32_t row = pr.tile * 16u + n;
  float sum = 0.0f;
  for (uint32_t st = 0; st < tparts; ++st)
    sum += __uint_as_float(lds_read_b32(sbase + L.part + 256u * (slot * tparts + st) + 4u * lane));
  if (grp < ntok && row < rows) y[(size_t)grp * rows + row] = sum;
  if (lane == 0u) {
    lds_write_b32(sbase + L.cnt + 4u * slot, 0u);
    lds_write_b32(sbase + L.owner + 4u * slot, pr.lt + slots);
  }
}

// The schedule constants of a launch, or false when a multiply-high quotient
// of the schedule could be inexact (x * d >= 2^32 for some quotient taken) or
// the counts do not fit their fields.
inline bool make_sched_args(uint32_t ntiles, uint32_t tparts, uint32_t slots,
                            const LaunchShape& ls, SchedArgs* out) {
  const uint64_t G = ls.groups;
  if (G == 0u || G > 0xffffu || slots == 0u || slots > 0xffu) return false;
  if ((uint64_t)ntiles * G >= (1ull << 32)) return false;  // tile / G quotients
  if (ls.split) {
    const uint64_t lpairs = (uint64_t)(ntiles - ntiles / ls.groups * ls.groups) * tparts;
    if (lpairs * G * G >= (1ull << 32)) return false;  // range starts: (g + 1) L / G
  }
  out->packed = (uint32_t)(G << 16) | (ls.split ? 0x100u : 0u) | slots;
  out->m_groups = div_magic((uint32_t)G);
  out->m_parts = div_magic(tparts);
  out->m_slots = div_magic(slots);
  return true;
}

// Slots of the ring: enough for every wave to be a few tiles ahead, within
// 8 KB of partials.
inline uint32_t ring_slots(uint32_t waves, uint32_t depth, uint32_t tiles_per_wg,
                           uint32_t tparts) {
  uint32_t slots = min(tiles_per_wg, max(4u, (2u * waves * depth + tparts - 1u) / tparts + 2u));
  while (slots > 2u && slots * tparts * 64u > 8192u) --slots;
  return slots;
}

// kernels_q6k_mfma.hip: a group of Q6_K matrices (GroupArgs) in one launch.
bool launch_q6k_matvec_group(const GroupArgs& ga, uint32_t total_rows, uint32_t cols,
                             const float* x, float* y, const Workspace& ws, hipStream_t s,
                             hipError_t* err);

}  // namespace mfma
}  // namespace sihip
