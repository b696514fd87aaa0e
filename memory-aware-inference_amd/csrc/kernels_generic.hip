// Generic K-quant kernels for gfx950: exact dequantisation (test support and
// the Q4_K embedding gather), the correctness-first row matvec used for
// shapes the tuned kernels do not cover, the batched verify fallback, the
// fused gate/up fallback, and the greedy-argmax reduction over logits.
//
// Reference kernels these stand in for: si_q{4,5,6}_k_matvec and
// si_q{4,5,6}_k_matmul_many (src/metal.rs:310-373, 770-836, 895-950,
// 1083-1262), si_q4_k_fused_gate_up (498-587), si_q4_k_embedding_row
// (589-625).  One wavefront (64 lanes) owns one output row; lane l decodes
// 32-weight units l, l+64, ... of that row exactly as quant.rs does and
// accumulates them into f32 with FMA; the wave reduces with cross-lane
// shuffles.
#include "kquant_device.h"
#include "si_hip_internal.h"

namespace sihip {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// One wavefront per row; `batch` candidate inputs (batch-major, K each).
template <uint32_t T, int MAXB>
__global__ __launch_bounds__(256) void matvec_generic_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ x, float* __restrict__ y,
    uint32_t rows, uint32_t cols, uint32_t batch) {
  constexpr uint32_t BB = BlockBytes<T>::value;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const uint32_t nb = cols / kBlockElems;
  const uint8_t* wrow = w + (size_t)row * nb * BB;
  float acc[MAXB];
#pragma unroll
  for (int b = 0; b < MAXB; ++b) acc[b] = 0.0f;
  for (uint32_t u = lane; u < nb * 8u; u += kWave) {
    float v[32];
    decode_unit_exact<T>(wrow + (size_t)(u >> 3) * BB, u & 7u, v);
    // element offset of this unit inside the row
    uint32_t col0;
    if constexpr (T == kTypeQ6K) {
      col0 = (u >> 3) * 256u + ((u & 7u) >> 2) * 128u + (u & 3u) * 32u;
    } else {
      col0 = (u >> 3) * 256u + (u & 7u) * 32u;
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      if (b < (int)batch) {
        const float4* xv = reinterpret_cast<const float4*>(x + (size_t)b * cols + col0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float4 xx = xv[i];
          acc[b] = fmaf(v[4 * i + 0], xx.x, acc[b]);
          acc[b] = fmaf(v[4 * i + 1], xx.y, acc[b]);
          acc[b] = fmaf(v[4 * i + 2], xx.z, acc[b]);
          acc[b] = fmaf(v[4 * i + 3], xx.w, acc[b]);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < MAXB; ++b) {
    if (b < (int)batch) {
      const float s = wave_sum(acc[b]);
      if (lane == 0) y[(size_t)b * rows + row] = s;
    }
  }
}

// One row of nb blocks by one workgroup: thread t decodes units t, t + 256,
// ... exactly as quant.rs does, the four waves' sums meet in LDS.
template <uint32_t T>
__global__ __launch_bounds__(256) void row_dot_kernel(const uint8_t* __restrict__ w,
                                                      const float* __restrict__ x,
                                                      float* __restrict__ y, uint32_t cols) {
  constexpr uint32_t BB = BlockBytes<T>::value;
  __shared__ float part[4];
  const uint32_t nb = cols / kBlockElems;
  float acc = 0.0f;
  for (uint32_t u = threadIdx.x; u < nb * 8u; u += 256u) {
    float v[32];
    decode_unit_exact<T>(w + (size_t)(u >> 3) * BB, u & 7u, v);
    uint32_t col0;
    if constexpr (T == kTypeQ6K) {
      col0 = (u >> 3) * 256u + ((u & 7u) >> 2) * 128u + (u & 3u) * 32u;
    } else {
      col0 = (u >> 3) * 256u + (u & 7u) * 32u;
    }
    const float4* xv = reinterpret_cast<const float4*>(x + col0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 xx = xv[i];
      acc = fmaf(v[4 * i + 0], xx.x, acc);
      acc = fmaf(v[4 * i + 1], xx.y, acc);
      acc = fmaf(v[4 * i + 2], xx.z, acc);
      acc = fmaf(v[4 * i + 3], xx.w, acc);
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0u) y[0] = (part[0] + part[1]) + (part[2] + part[3]);
}

// silu(g) * u with both projections Q4_K (si_q4_k_fused_gate_up, metal.rs:585).
__global__ __launch_bounds__(256) void fused_gate_up_generic_kernel(
    const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, const float* __restrict__ x,
    float* __restrict__ h, uint32_t rows, uint32_t cols) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const uint32_t nb = cols / kBlockElems;
  const size_t row_off = (size_t)row * nb * kQ4Bytes;
  float g = 0.0f, u = 0.0f;
  for (uint32_t unit = lane; unit < nb * 8u; unit += kWave) {
    float vg[32], vu[32];
    decode_unit_exact<kTypeQ4K>(gate + row_off + (size_t)(unit >> 3) * kQ4Bytes, unit & 7u, vg);
    decode_unit_exact<kTypeQ4K>(up + row_off + (size_t)(unit >> 3) * kQ4Bytes, unit & 7u, vu);
    const float4* xv = reinterpret_cast<const float4*>(x + (unit >> 3) * 256u + (unit & 7u) * 32u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 xx = xv[i];
      g = fmaf(vg[4 * i + 0], xx.x, g);
      g = fmaf(vg[4 * i + 1], xx.y, g);
      g = fmaf(vg[4 * i + 2], xx.z, g);
      g = fmaf(vg[4 * i + 3], xx.w, g);
      u = fmaf(vu[4 * i + 0], xx.x, u);
      u = fmaf(vu[4 * i + 1], xx.y, u);
      u = fmaf(vu[4 * i + 2], xx.z, u);
      u = fmaf(vu[4 * i + 3], xx.w, u);
    }
  }
  g = wave_sum(g);
  u = wave_sum(u);
  if (lane == 0) h[row] = silu_times(g, u);
}

// Exact dequantisation of whole blocks: one thread per 32-weight unit.
// `row_index` (optional) maps output row r to source row row_index[r]
// (the embedding gather); otherwise output row r is source row r.  An index
// of table_rows or more reads nothing: its output row is NaN and the kernel
// reports kDevErrTokenId through the workspace `ws` (when not null).
template <uint32_t T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      const uint32_t* __restrict__ row_index,
                                                      float* __restrict__ out, uint32_t out_rows,
                                                      uint32_t cols, uint32_t table_rows,
                                                      void* ws) {
  constexpr uint32_t BB = BlockBytes<T>::value;
  const uint32_t nb = cols / kBlockElems;
  const uint64_t units_total = (uint64_t)out_rows * nb * 8u;
  const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= units_total) return;
  const uint32_t r = (uint32_t)(id / ((uint64_t)nb * 8u));
  const uint32_t rem = (uint32_t)(id % ((uint64_t)nb * 8u));
  const uint32_t blk = rem >> 3;
  const uint32_t unit = rem & 7u;
  const uint64_t src_row = row_index ? row_index[r] : r;
  float v[32];
  if (src_row < table_rows) {
    decode_unit_exact<T>(w + (src_row * nb + blk) * BB, unit, v);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __builtin_nanf("");
    if (ws && blk == 0u && unit == 0u) report_device_error(ws, kDevErrTokenId);
  }
  uint32_t col0;
  if constexpr (T == kTypeQ6K) {
    col0 = blk * 256u + (unit >> 2) * 128u + (unit & 3u) * 32u;
  } else {
    col0 = blk * 256u + unit * 32u;
  }
  float4* o = reinterpret_cast<float4*>(out + (uint64_t)r * cols + col0);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

}  // namespace

hipError_t launch_matvec_generic(uint32_t type, const uint8_t* w, const float* x, float* y,
                                 uint32_t rows, uint32_t cols, uint32_t batch, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((rows + 3) / 4);
#define SIHIP_MV(T, B)                                                                      \
  hipLaunchKernelGGL((matvec_generic_kernel<T, B>), grid, block, 0, s, w, x, y, rows, cols, \
                     batch)
  const int bucket = batch <= 1 ? 1 : batch <= 4 ? 4 : batch <= 8 ? 8 : 16;
  switch (type) {
    case kTypeQ4K:
      if (bucket == 1) SIHIP_MV(kTypeQ4K, 1); else if (bucket == 4) SIHIP_MV(kTypeQ4K, 4);
      else if (bucket == 8) SIHIP_MV(kTypeQ4K, 8); else SIHIP_MV(kTypeQ4K, 16);
      break;
    case kTypeQ5K:
      if (bucket == 1) SIHIP_MV(kTypeQ5K, 1); else if (bucket == 4) SIHIP_MV(kTypeQ5K, 4);
      else if (bucket == 8) SIHIP_MV(kTypeQ5K, 8); else SIHIP_MV(kTypeQ5K, 16);
      break;
    case kTypeQ6K:
      if (bucket == 1) SIHIP_MV(kTypeQ6K, 1); else if (bucket == 4) SIHIP_MV(kTypeQ6K, 4);
      else if (bucket == 8) SIHIP_MV(kTypeQ6K, 8); else SIHIP_MV(kTypeQ6K, 16);
      break;
    default:
      return hipErrorInvalidValue;
  }
#undef SIHIP_MV
  return hipGetLastError();
}

hipError_t launch_row_dot(uint32_t type, const uint8_t* w, const float* x, float* y,
                          uint32_t cols, hipStream_t s) {
  switch (type) {
    case kTypeQ4K:
      hipLaunchKernelGGL(row_dot_kernel<kTypeQ4K>, dim3(1), dim3(256), 0, s, w, x, y, cols);
      break;
    case kTypeQ5K:
      hipLaunchKernelGGL(row_dot_kernel<kTypeQ5K>, dim3(1), dim3(256), 0, s, w, x, y, cols);
      break;
    case kTypeQ6K:
      hipLaunchKernelGGL(row_dot_kernel<kTypeQ6K>, dim3(1), dim3(256), 0, s, w, x, y, cols);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fused_gate_up_generic(const uint8_t* gate, const uint8_t* up, const float* x,
                                        float* h, uint32_t rows, uint32_t cols, hipStream_t s) {
  hipLaunchKernelGGL(fused_gate_up_generic_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, gate,
                     up, x, h, rows, cols);
  return hipGetLastError();
}

hipError_t launch_dequant(uint32_t type, const uint8_t* w, const uint32_t* row_index, float* out,
                          uint32_t out_rows, uint32_t cols, hipStream_t s, uint32_t table_rows,
                          void* ws) {
  const uint64_t units = (uint64_t)out_rows * (cols / kBlockElems) * 8u;
  const dim3 grid((uint32_t)((units + 255) / 256));
  switch (type) {
    case kTypeQ4K:
      hipLaunchKernelGGL(dequant_kernel<kTypeQ4K>, grid, dim3(256), 0, s, w, row_index, out,
                         out_rows, cols, table_rows, ws);
      break;
    case kTypeQ5K:
      hipLaunchKernelGGL(dequant_kernel<kTypeQ5K>, grid, dim3(256), 0, s, w, row_index, out,
                         out_rows, cols, table_rows, ws);
      break;
    case kTypeQ6K:
      hipLaunchKernelGGL(dequant_kernel<kTypeQ6K>, grid, dim3(256), 0, s, w, row_index, out,
                         out_rows, cols, table_rows, ws);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sihip
