// F32 matvec and RMSNorm kernels: the GGUF F32 tensors and the norms around
// the K-quant projections of a decoder block (si_f32_matvec, metal.rs:263-305;
// si_rms_norm / si_rms_norm_heads / si_rms_norm_gated, metal.rs:121-213).
//
// Both are HBM- or latency-bound: the F32 matvec streams 4 bytes per weight
// with one wave per row (16-byte loads, each lane a sequential partial, then a
// fixed-order wave reduction); an RMSNorm head is one workgroup (thread
// partials of x^2, a fixed-order reduction, 1 / sqrt(mean + eps) correctly
// rounded, then the scaled output).
#include "si_hip_internal.h"

namespace sihip {
namespace {

constexpr uint32_t kRowsPerGroup = 4;  // one wave per row

// Sum over the 64 lanes of a wave, in a fixed order, broadcast to all lanes:
// each 16-lane row by DPP shifts (lane 15 of the row ends with the row's
// sum), then the four rows' sums added in row order.
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));
  const float r0 = __shfl(v, 15, 64), r1 = __shfl(v, 31, 64);
  const float r2 = __shfl(v, 47, 64), r3 = __shfl(v, 63, 64);
  return (r0 + r1) + (r2 + r3);
}

// y[r] = sum_c w[r * cols + c] * x[c].  VEC: cols % 4 == 0 and w, x 16-byte
// aligned, so lane l reads float4s l, l + 64, ... of the row (two in flight).
template <bool VEC>
__global__ __launch_bounds__(256) void f32_matvec_kernel(const float* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, uint32_t rows,
                                                         uint32_t cols) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t row = blockIdx.x * kRowsPerGroup + wave;
  if (row >= rows) return;  // whole waves
  const float* const wr = w + (size_t)row * cols;
  float a0 = 0.0f, a1 = 0.0f;
  if (VEC) {
    const float4* const w4 = reinterpret_cast<const float4*>(wr);
    const float4* const x4 = reinterpret_cast<const float4*>(x);
    const uint32_t n4 = cols / 4u;
    uint32_t i = lane;
    for (; i + 64u < n4; i += 128u) {
      const float4 p = w4[i], q = x4[i], p2 = w4[i + 64u], q2 = x4[i + 64u];
      a0 = fmaf(p.x, q.x, a0);
      a0 = fmaf(p.y, q.y, a0);
      a0 = fmaf(p.z, q.z, a0);
      a0 = fmaf(p.w, q.w, a0);
      a1 = fmaf(p2.x, q2.x, a1);
      a1 = fmaf(p2.y, q2.y, a1);
      a1 = fmaf(p2.z, q2.z, a1);
      a1 = fmaf(p2.w, q2.w, a1);
    }
    if (i < n4) {
      const float4 p = w4[i], q = x4[i];
      a0 = fmaf(p.x, q.x, a0);
      a0 = fmaf(p.y, q.y, a0);
      a0 = fmaf(p.z, q.z, a0);
      a0 = fmaf(p.w, q.w, a0);
    }
  } else {
    for (uint32_t c = lane; c < cols; c += 64u) a0 = fmaf(wr[c], x[c], a0);
  }
  const float total = wave_sum(a0 + a1);
  if (lane == 0u) y[row] = total;
}

// Workgroup sum of per-thread partials, fixed order, in every thread.
__device__ __forceinline__ float group_sum(float v, float* red) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  v = wave_sum(v);
  if (lane == 0u) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// MODE 0: y = x * inv * w (si_rms_norm); 1: y = x * inv * (1 + w)
// (si_rms_norm_heads); 2: y = x * inv * w * silu(g) (si_rms_norm_gated).
// One workgroup of 256 threads per head of head_dim values.
template <int MODE>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ gate,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ y, uint32_t head_dim,
                                                       float eps) {
  __shared__ float red[4];
  const size_t base = (size_t)blockIdx.x * head_dim;
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < head_dim; i += 256u) {
    const float v = x[base + i];
    ss = __fadd_rn(ss, __fmul_rn(v, v));  // x^2 rounded, then added (qwen35.rs:36-40)
  }
  const float total = group_sum(ss, red);
  // (sum / n + eps).sqrt().recip(), each step correctly rounded
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)head_dim), eps)));
  for (uint32_t i = threadIdx.x; i < head_dim; i += 256u) {
    float o = __fmul_rn(x[base + i], inv);
    if (MODE == 0) o = __fmul_rn(o, w[i]);
    if (MODE == 1) o = __fmul_rn(o, __fadd_rn(1.0f, w[i]));
    if (MODE == 2) {
      const float g = gate[base + i];
      o = __fmul_rn(__fmul_rn(o, w[i]), __fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
    }
    y[base + i] = o;
  }
}

}  // namespace

hipError_t launch_f32_matvec(const float* w, const float* x, float* y, uint32_t rows,
                             uint32_t cols, hipStream_t s) {
  if (rows == 0 || cols == 0) return hipErrorInvalidValue;
  const dim3 grid((rows + kRowsPerGroup - 1u) / kRowsPerGroup), block(256);
  const bool vec = cols % 4u == 0u && (reinterpret_cast<uintptr_t>(w) & 15u) == 0u &&
                   (reinterpret_cast<uintptr_t>(x) & 15u) == 0u;
  if (vec)
    hipLaunchKernelGGL(f32_matvec_kernel<true>, grid, block, 0, s, w, x, y, rows, cols);
  else
    hipLaunchKernelGGL(f32_matvec_kernel<false>, grid, block, 0, s, w, x, y, rows, cols);
  return hipGetLastError();
}

hipError_t launch_rms_norm(uint32_t mode, const float* x, const float* gate, const float* w,
                           float* y, uint32_t heads, uint32_t head_dim, float eps, hipStream_t s) {
  if (heads == 0 || head_dim == 0 || mode > 2u) return hipErrorInvalidValue;
  const dim3 grid(heads), block(256);
  switch (mode) {
    case 0: hipLaunchKernelGGL(rms_norm_kernel<0>, grid, block, 0, s, x, gate, w, y, head_dim, eps); break;
    case 1: hipLaunchKernelGGL(rms_norm_kernel<1>, grid, block, 0, s, x, gate, w, y, head_dim, eps); break;
    default: hipLaunchKernelGGL(rms_norm_kernel<2>, grid, block, 0, s, x, gate, w, y, head_dim, eps); break;
  }
  return hipGetLastError();
}

}  // namespace sihip
