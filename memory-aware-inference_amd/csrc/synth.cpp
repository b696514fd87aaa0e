// Seeded synthetic K-quant blocks and activations (include/si_hip_synth.h).
// Host-only; no counterpart in the reference.
#include "si_hip_synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// word `index` of the stream `seed`
inline uint64_t stream_word(uint64_t seed, uint64_t index) {
  return splitmix64(splitmix64(seed ^ 0x5eed5eed5eed5eedull) + index * 0x9e3779b97f4a7c15ull);
}

// Inverse standard-normal CDF: Acklam's rational approximation followed by
// one Halley step on erfc, accurate to about 1e-15 on (0, 1).
double inverse_normal_cdf(double p) {
  static const double a[] = {-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
                             1.383577518672690e+02,  -3.066479806614716e+01, 2.506628277459239e+00};
  static const double b[] = {-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
                             6.680131188771972e+01,  -1.328068155288572e+01};
  static const double c[] = {-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
                             -2.549732539343734e+00, 4.374664141464968e+00,  2.938163982698783e+00};
  static const double d[] = {7.784695709041462e-03, 3.224671290700398e-01, 2.445134137142996e+00,
                             3.754408661907416e+00};
  const double lo = 0.02425, hi = 1 - lo;
  double x;
  if (p < lo) {
    double q = std::sqrt(-2 * std::log(p));
    x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
        ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1);
  } else if (p <= hi) {
    double q = p - 0.5, r = q * q;
    x = (((((a[0] * r + a[1]) * r + a[2]) * r + a[3]) * r + a[4]) * r + a[5]) * q /
        (((((b[0] * r + b[1]) * r + b[2]) * r + b[3]) * r + b[4]) * r + 1);
  } else {
    double q = std::sqrt(-2 * std::log(1 - p));
    x = -(((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
        ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1);
  }
  const double e = 0.5 * std::erfc(-x / std::sqrt(2.0)) - p;
  const double u = e * std::sqrt(2 * M_PI) * std::exp(x * x / 2);
  return x - u / (1 + x * u / 2);
}

const float *normal_table() {
  static float table[65536];
  static std::once_flag once;
  std::call_once(once, [] {
    for (int i = 0; i < 65536; ++i) table[i] = (float)inverse_normal_cdf((i + 0.5) / 65536.0);
  });
  return table;
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  const int e = (int)(ax >> 23) - 127;
  const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
  if (ax == 0) return (uint16_t)sign;
  if (e < -14) {
    // subnormal half: q = mant * 2^(e+1), rounded to nearest even
    const int s = -e - 1;
    if (s > 25) return (uint16_t)sign;
    uint32_t q = s >= 32 ? 0 : mant >> s;
    const uint32_t rem = mant & ((1u << s) - 1u);
    const uint32_t halfway = 1u << (s - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = mant >> 13;
  const uint32_t rem = mant & 0x1fffu;
  uint32_t he = (uint32_t)(e + 15);
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  if (q == 0x800u) {
    q = 0x400u;
    ++he;
  }
  if (he >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (he << 10) | (q & 0x3ffu));
}

uint16_t abs_normal_f16(uint64_t word, float sigma) {
  const float z = normal_table()[word & 0xffffu];
  return f32_to_f16(sigma * std::fabs(z));
}

void synth_block(uint32_t type, uint64_t seed, uint64_t block, uint8_t *out) {
  uint64_t words[32];
  for (int j = 0; j < 32; ++j) words[j] = stream_word(seed, block * 32 + (uint64_t)j);
  uint8_t raw[256];
  std::memcpy(raw, words, sizeof raw);  // little-endian byte stream of the words
  if (type == 14) {
    std::memcpy(out, raw, 210);
    for (int i = 0; i < 16; ++i) out[192 + i] = (uint8_t)(int8_t)((int)(raw[192 + i] & 63u) - 32);
    const uint16_t d = abs_normal_f16(words[30], 0.01f);
    out[208] = (uint8_t)(d & 0xff);
    out[209] = (uint8_t)(d >> 8);
  } else {
    const size_t bytes = type == 12 ? 144 : 176;
    std::memcpy(out, raw, bytes);
    const uint16_t d = abs_normal_f16(words[30], 0.02f);
    const uint16_t dmin = abs_normal_f16(words[31], 0.02f);
    out[0] = (uint8_t)(d & 0xff);
    out[1] = (uint8_t)(d >> 8);
    out[2] = (uint8_t)(dmin & 0xff);
    out[3] = (uint8_t)(dmin >> 8);
  }
}

size_t block_bytes(uint32_t type) {
  return type == 12 ? 144 : type == 13 ? 176 : type == 14 ? 210 : 0;
}

}  // namespace

extern "C" {

uint16_t si_hip_synth_f32_to_f16(float value) { return f32_to_f16(value); }

int si_hip_synth_blocks(uint32_t type, uint64_t seed, uint64_t first_block, size_t n_blocks,
                        uint8_t *out, size_t out_len, int threads) {
  const size_t bb = block_bytes(type);
  if (bb == 0) return -5;
  if (!out) return -1;
  if (n_blocks > SIZE_MAX / bb || out_len != n_blocks * bb) return -3;
  normal_table();
  const size_t hw = std::max(1u, std::thread::hardware_concurrency());
  size_t t = threads <= 1 ? 1 : std::min<size_t>((size_t)threads, hw);
  if (n_blocks < 4096) t = 1;
  auto work = [&](size_t b0, size_t b1) {
    for (size_t b = b0; b < b1; ++b) synth_block(type, seed, first_block + b, out + b * bb);
  };
  if (t == 1) {
    work(0, n_blocks);
    return 0;
  }
  std::vector<std::thread> pool;
  for (size_t i = 0; i < t; ++i) pool.emplace_back(work, n_blocks * i / t, n_blocks * (i + 1) / t);
  for (auto &th : pool) th.join();
  return 0;
}

int si_hip_synth_normal_f32(uint64_t seed, uint64_t first_index, size_t n, float scale, float *out) {
  if (!out) return -1;
  for (size_t i = 0; i < n; ++i) {
    const uint64_t k = first_index + i;
    const uint64_t pair = k >> 1;
    const uint64_t w1 = stream_word(seed ^ 0x6e6f726d616cull, 2 * pair);
    const uint64_t w2 = stream_word(seed ^ 0x6e6f726d616cull, 2 * pair + 1);
    const double u1 = ((double)(w1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);  // (0, 1]
    const double u2 = (double)(w2 >> 11) * (1.0 / 9007199254740992.0);          // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double z = (k & 1) ? r * std::sin(2.0 * M_PI * u2) : r * std::cos(2.0 * M_PI * u2);
    out[i] = scale * (float)z;
  }
  return 0;
}

int si_hip_synth_token_ids(uint64_t seed, size_t n, uint32_t vocab, uint32_t *out) {
  if (!out || vocab == 0) return -1;
  for (size_t i = 0; i < n; ++i)
    out[i] = (uint32_t)(((unsigned __int128)stream_word(seed ^ 0x746f6b656eull, i) * vocab) >> 64);
  return 0;
}

}  // extern "C"
