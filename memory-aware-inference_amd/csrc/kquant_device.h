// Device-side GGUF K-quant decode primitives for gfx950.
//
// Block layouts (src/quant.rs:8-16, 18-174):
//   Q4_K 144 B: d f16 | dmin f16 | scales[12] | qs[128]
//   Q5_K 176 B: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
//   Q6_K 210 B: ql[128] | qh[64] | scales[16] (int8) | d f16
//
// Every block is handled as eight 32-weight "units".  Unit u of a Q4_K/Q5_K
// block is the 32 weights that share the (scale, min) pair u: group g = u/2,
// low nibbles of qs[32g..32g+32) for even u, high nibbles for odd u.  Unit u
// of a Q6_K block is half h = u/4, quartet q = u%4 (elements 128h+32q+i),
// whose 32 weights use int8 scales 8h+2q (i<16) and 8h+2q+1 (i>=16).
//
// The exact decoders reproduce quant.rs rounding step by step with
// __fmul_rn/__fsub_rn so the compiler cannot contract them into an FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sihip {

constexpr uint32_t kBlockElems = 256;
constexpr uint32_t kQ4Bytes = 144;
constexpr uint32_t kQ5Bytes = 176;
constexpr uint32_t kQ6Bytes = 210;
constexpr uint32_t kTypeQ4K = 12;
constexpr uint32_t kTypeQ5K = 13;
constexpr uint32_t kTypeQ6K = 14;

template <uint32_t T> struct BlockBytes;
template <> struct BlockBytes<kTypeQ4K> { static constexpr uint32_t value = kQ4Bytes; };
template <> struct BlockBytes<kTypeQ5K> { static constexpr uint32_t value = kQ5Bytes; };
template <> struct BlockBytes<kTypeQ6K> { static constexpr uint32_t value = kQ6Bytes; };

// quant.rs:187-207 restated with integer operations only, so NaN payloads,
// infinities and subnormal halves come out exactly as the CPU decoder gives.
__device__ __forceinline__ float half_bits_to_float_exact(uint32_t bits) {
  const uint32_t sign = (bits & 0x8000u) << 16;
  const uint32_t exponent = (bits >> 10) & 0x1fu;
  uint32_t fraction = bits & 0x3ffu;
  uint32_t value;
  if (exponent == 0x1fu) {
    value = sign | 0x7f800000u | (fraction << 13);
  } else if (exponent != 0) {
    value = sign | ((exponent + 112u) << 23) | (fraction << 13);
  } else if (fraction == 0) {
    value = sign;
  } else {
    // normalise: leading one of the 10-bit fraction moves to bit 10
    const uint32_t lead = 31u - __clz(fraction);  // 0..9
    const uint32_t shift = 10u - lead;
    fraction = (fraction << shift) & 0x3ffu;
    value = sign | ((uint32_t)(127 - 14 - (int)shift) << 23) | (fraction << 13);
  }
  return __uint_as_float(value);
}

// Hardware conversion; exact for every finite half and for infinities
// (quiets signalling NaNs, which the dot products do not care about).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  const unsigned short b = (unsigned short)(bits & 0xffffu);
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// quant.rs:176-185 on the 12 scale bytes held as three little-endian words.
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t* s, uint32_t& sc,
                                             uint32_t& mn) {
  if (j < 4) {
    sc = s[j] & 63u;
    mn = s[j + 4] & 63u;
  } else {
    sc = (s[j + 4] & 0x0fu) | ((s[j - 4] >> 6) << 4);
    mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// Exact per-weight value of a Q4_K/Q5_K weight (quant.rs:45-59, 99-122):
// d1 = d*sc, m1 = dmin*m, v = d1*q - m1, each rounded on its own.
__device__ __forceinline__ float k4_value_exact(float d1, float m1, uint32_t q) {
  return __fsub_rn(__fmul_rn(d1, (float)q), m1);
}

// Exact Q6_K value (quant.rs:164-169): (d*scale)*q.
__device__ __forceinline__ float k6_value_exact(float d, int scale, int q) {
  return __fmul_rn(__fmul_rn(d, (float)scale), (float)q);
}

// Decode one 32-weight unit of a block to exact f32 values (quant.rs order).
// `blk` points at the block's first byte (any alignment).
template <uint32_t T>
__device__ __forceinline__ void decode_unit_exact(const uint8_t* __restrict__ blk, uint32_t unit,
                                                  float out[32]) {
  if constexpr (T == kTypeQ4K || T == kTypeQ5K) {
    const float d = half_bits_to_float_exact(blk[0] | (blk[1] << 8));
    const float dmin = half_bits_to_float_exact(blk[2] | (blk[3] << 8));
    uint32_t sc, mn;
    scale_min_k4(unit, blk + 4, sc, mn);
    const float d1 = __fmul_rn(d, (float)sc);
    const float m1 = __fmul_rn(dmin, (float)mn);
    const uint32_t group = unit >> 1;
    const uint32_t shift = (unit & 1u) * 4u;
    const uint8_t* qs = blk + (T == kTypeQ4K ? 16 : 48) + 32 * group;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t q = (qs[i] >> shift) & 0x0fu;
      if constexpr (T == kTypeQ5K) {
        const uint32_t hbit = (blk[16 + i] >> unit) & 1u;  // mask 1<<2g or 2<<2g
        q += hbit << 4;
      }
      out[i] = k4_value_exact(d1, m1, q);
    }
  } else {
    const float d = half_bits_to_float_exact(blk[208] | (blk[209] << 8));
    const uint32_t half = unit >> 2;
    const uint32_t quartet = unit & 3u;
    const uint8_t* ql = blk + 64 * half + 32 * (quartet & 1u);
    const uint8_t* qh = blk + 128 + 32 * half;
    const int8_t* sc = (const int8_t*)(blk + 192 + 8 * half + 2 * quartet);
    const uint32_t nib_shift = (quartet >> 1) * 4u;
    const uint32_t h_shift = quartet * 2u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int q = (int)(((ql[i] >> nib_shift) & 0x0fu) | (((qh[i] >> h_shift) & 3u) << 4)) - 32;
      out[i] = k6_value_exact(d, sc[i >> 4], q);
    }
  }
}

}  // namespace sihip
