// Shared parts of the kernels that put several activation vectors in the
// rows of the matrix-core A operand (q4k_tokens_mfma, q6k_tokens_mfma): the
// group images of four vectors at a time, built in LDS from copies of x,
// and the reduce kernel that adds the K slices' partial sums of a sliced
// launch in slice order.
//
// Group images (4 KB per block and group of four vectors): group g's block
// b at img + 4096 (g nbl + b), unit pair p at + 1024 p, then 16 bytes per
// A-operand lane l = 16 k + 4 t + d of v_mfma_i32_16x16x32_i8: the 8 bytes
// of digit d of vector 4 g + t over elements 8 k .. 8 k + 7 of unit 2 p,
// then those of unit 2 p + 1.
#pragma once

#include "mfma_common.h"

namespace sihip {
namespace mfma {
namespace {

// An 8-byte MFMA operand from two words.
__device__ __forceinline__ int64_t as_i64(uint32_t lo, uint32_t hi) {
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// The image blocks a wave owns: group-blocks q = wave, wave + WAVES, ... of
// the ng x nbl of a launch (group q / nbl, local block q % nbl), walked
// without a division.
template <int WAVES, typename F>
__device__ __forceinline__ void for_group_blocks(uint32_t ng, uint32_t nbl, uint32_t wave, F f) {
  uint32_t g = 0u, i = wave;
  while (i >= nbl && g < ng) {
    i -= nbl;
    ++g;
  }
  for (; g < ng;) {
    f(g, i);
    i += WAVES;
    while (i >= nbl && g < ng) {
      i -= nbl;
      ++g;
    }
  }
}

// Copies of the vectors' blocks blk0 .. blk0 + nbl - 1: vector 4 g + t's
// block blk0 + i at img + 4096 (g nbl + i) + 1024 t; the slots of vectors past
// ntok are cleared.
template <int WAVES>
__device__ __forceinline__ void copy_x_group(uint8_t* smem, uint32_t img, const float* x,
                                             uint32_t nb, uint32_t blk0, uint32_t nbl,
                                             uint32_t ng, uint32_t ntok, uint32_t wave,
                                             uint32_t lane) {
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x), 0, (int)(ntok * nb * 1024u), kBufferWord3);
  for_group_blocks<WAVES>(ng, nbl, wave, [&](uint32_t g, uint32_t i) {
    const uint32_t dst = img + 4096u * (g * nbl + i);
#pragma unroll
    for (uint32_t t = 0; t < 4u; ++t) {
      const uint32_t v = 4u * g + t;
      if (v < ntok)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(smem + dst + 1024u * t), 16,
                                                  (v * nb + blk0 + i) * 1024u + 16u * lane, 0, 0,
                                                  0);
      else
        lds_write_b128((uint32_t)(uintptr_t)smem + dst + 1024u * t + 16u * lane,
                       u32x4{0u, 0u, 0u, 0u});
    }
  });
}

// Group images, exponents, side lists and unit sums of the copied blocks, in
// place: a wave converts exactly the group-blocks it copied; lane (t, c)
// takes elements 16 c .. 16 c + 15 of vector 4 g + t.  Blocks follow
// build_images' rules (side elements, exponent kBadBlock for blocks that
// must take the exact path).  LIST: up to kSideMax side elements of a block
// are listed (and zero in the image) for the kernel to add exactly; without
// it every block with side elements is a rounded block, which the kernel
// checks with the block's error sums instead (the two- and four-group Q4_K
// and Q5_K kernels: the listed elements' exact decode took registers enough
// to spill their main loops).
template <int WAVES, bool LIST = true>
__device__ __forceinline__ void build_group_images(uint32_t sbase, const Layout& L, uint32_t nbl,
                                                   uint32_t ng, uint32_t wave, uint32_t lane) {
  const uint32_t t = lane >> 4, c = lane & 15u;
  const uint32_t u = c >> 1;                                  // unit of the lane's chunk
  const uint32_t g0 = 2u * (c & 1u);                          // K slice of its first 8
  const uint32_t woff = 1024u * (u >> 1) + 16u * (16u * g0 + 4u * t) + 8u * (u & 1u);
  for_group_blocks<WAVES>(ng, nbl, wave, [&](uint32_t g, uint32_t b) {
    const uint32_t blk = sbase + L.img + 4096u * (g * nbl + b);
    const uint32_t v = 4u * g + t;  // the lane's vector
    u32x4 xq[4];
    lds_read4<16>(blk + 1024u * t + 64u * c, xq);
    float xv[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[4 * k + i] = __uint_as_float(xq[k][i]);
    const ChunkSplit cs = split_chunk(xv);
    const bool bad_blk = (__builtin_amdgcn_ballot_w64(cs.bad) >> (16u * t)) & 0xffffull;
    const uint32_t meta = sbase + L.expo + v * L.expo_stride;
    const uint32_t list = meta + L.side_off + kSideBytes * b;
    uint32_t nside = 0u;
    bool rounded;
    if constexpr (LIST) {
      nside = __builtin_amdgcn_ballot_w64(cs.smask != 0u)
                  ? side_list(xv, cs.smask, c, list, !bad_blk)
                  : 0u;
      rounded = !bad_blk && nside > kSideMax;
    } else {
      rounded = !bad_blk &&
                ((__builtin_amdgcn_ballot_w64(cs.smask != 0u) >> (16u * t)) & 0xffffull) != 0u;
    }
    uint32_t uq[16];
    biased_values(cs, !rounded, uq);
    uint32_t dg[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      transpose_digits(uq[4 * k], uq[4 * k + 1], uq[4 * k + 2], uq[4 * k + 3], dg[k]);
    // the wave has read the whole block (lds_read4 waits) before any write
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      lds_write_b64(blk + woff + 16u * d, u32x2{dg[0][d], dg[1][d]});
      lds_write_b64(blk + woff + 16u * d + 256u, u32x2{dg[2][d], dg[3][d]});
    }
    if (rounded)  // chunk c's error sum at position c (read whole by tok_side)
      lds_write_b32(list + 4u * c, __float_as_uint(cs.err_side));
    const float xsum = unit_fixed_sum(uq);  // odd lanes: unit c / 2 (listed elements as 0)
    if (c & 1u)
      lds_write_b32(sbase + L.xsum + v * L.xsum_stride + 32u * b + 4u * u, __float_as_uint(xsum));
    if (c == 0u) {
      lds_write_b32(meta + 4u * b, (uint32_t)(bad_blk ? kBadBlock : cs.e - kFixBits));
      lds_write_b8(meta + count_pos(L, b), bad_blk ? 0u : rounded ? kSideRounded : nside);
    }
  });
}


// Sum of all 16 chunk error sums of a rounded block's side area.
__device__ __forceinline__ float rounded_err_all(uint32_t list) {
  return (rounded_err(list, 0u) + rounded_err(list, 1u)) +
         (rounded_err(list, 2u) + rounded_err(list, 3u));
}

// y[t * rows + row] = sum over the stages s of part[(s * nv + t) * rows + row],
// in stage order (the sliced launch's second kernel; a "stage" here is the
// first kernel's unit of partial sums, bps blocks).  A partial that holds
// kPartRedo (its lane failed a check in the first kernel) is the stage's
// exact dot instead: quant.rs's per-weight values of blocks bps s ..
// bps s + bps - 1 of the row (decode_unit_exact) times vector t of the
// batch-major x, summed in f64 and rounded once.  The workgroup's 256
// threads take such stages together from a queue in LDS, eight at a time,
// 32 threads (half a wave) per stage and 32-weight units l, l + 32, ... per
// thread, their f64 sums added with shuffles; a stage past the queue's room
// is taken by its own thread.  A thread with such a stage sums its rows'
// partials again in stage order, the first eight stages kept in registers.
// R rows per thread: 1, or 4 with 16-byte loads and stores (launch_tok_reduce
// takes 4 when the rows, y and the grid allow it); each row's sum is the same.
constexpr uint32_t kRedoQueue = 64;
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <uint32_t T>
__device__ __noinline__ float stage_exact(const uint8_t* __restrict__ w, uint32_t row,
                                          uint32_t nb, uint32_t b0, uint32_t b1,
                                          const float* __restrict__ x) {
  constexpr uint32_t kBytes = BlockBytes<T>::value;
  const uint8_t* const r = w + (size_t)row * nb * kBytes;
  double acc = 0.0;
  for (uint32_t b = b0; b < b1; ++b) {
    for (uint32_t u = 0; u < 8u; ++u) {
      float wv[32];
      decode_unit_exact<T>(r + (size_t)b * kBytes, u, wv);
      const float* const xu = x + (size_t)b * kBlockElems + 32u * u;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc = fma((double)wv[i], (double)xu[i], acc);
    }
  }
  return (float)acc;
}

template <uint32_t T, int R>
__global__ __launch_bounds__(256) void tok_reduce(const float* __restrict__ part,
                                                  float* __restrict__ y, uint32_t rows,
                                                  uint32_t nstages, uint32_t nv,
                                                  const uint8_t* __restrict__ w,
                                                  const float* __restrict__ x, uint32_t nb,
                                                  uint32_t bps) {
  static_assert(R == 1 || R == 4, "one or four rows per thread");
  constexpr uint32_t kBytes = BlockBytes<T>::value;
  __shared__ uint32_t queue[kRedoQueue];  // (row in the workgroup) << 16 | stage
  __shared__ float value[kRedoQueue];
  __shared__ uint32_t queued;
  const uint32_t tid = threadIdx.x, t = blockIdx.y;
  const uint32_t rw = (uint32_t)R * tid;                    // the thread's first row in the workgroup
  const uint32_t row = blockIdx.x * (256u * R) + rw;        // its rows row .. row + R - 1
  const float* const p = part + (size_t)t * rows + row;
  const float* const xt = x + (size_t)t * nb * kBlockElems;
  const size_t step = (size_t)nv * rows;
  if (tid == 0u) queued = 0u;
  __syncthreads();
  // stages base .. base + 7 of the thread's rows, eight loads in flight
  auto load8 = [&](uint32_t base, float (&v)[8][R]) {
#pragma unroll
    for (uint32_t i = 0; i < 8u; ++i) {
      if (base + i < nstages) {
        if constexpr (R == 4) {
          const f32x4 q = *reinterpret_cast<const f32x4*>(p + (base + i) * step);
#pragma unroll
          for (int c = 0; c < R; ++c) v[i][c] = q[c];
        } else {
          v[i][0] = p[(base + i) * step];
        }
      } else {
#pragma unroll
        for (int c = 0; c < R; ++c) v[i][c] = 0.0f;
      }
    }
  };
  // the stages' sums in stage order; the stages the thread's rows leave to
  // the workgroup go to the queue
  float sum[R];
  float first[8][R];
#pragma unroll
  for (int c = 0; c < R; ++c) sum[c] = 0.0f;
  bool mine = false;
  if (row < rows) {  // (rows a multiple of R)
    for (uint32_t base = 0; base < nstages; base += 8u) {
      float v[8][R];
      load8(base, v);
#pragma unroll
      for (uint32_t i = 0; i < 8u; ++i) {
        if (base == 0u) {
#pragma unroll
          for (int c = 0; c < R; ++c) first[i][c] = v[i][c];
        }
        if (base + i >= nstages) continue;
#pragma unroll
        for (int c = 0; c < R; ++c) {
          if (__float_as_uint(v[i][c]) == kPartRedo) {
            const uint32_t k = atomicAdd(&queued, 1u);
            if (k < kRedoQueue) queue[k] = ((rw + (uint32_t)c) << 16) | (base + i);
            mine = true;
          }
          sum[c] += v[i][c];
        }
      }
    }
  }
  if (__syncthreads_or(mine)) {
    // queued stages eight at a time, one per 32 threads (half a wave), which
    // sum their units' f64 dots with shuffles inside the half wave
    const uint32_t nq = min(queued, kRedoQueue);
    const uint32_t e = tid >> 5, l = tid & 31u;  // stage e of a batch; its units l, l + 32, ...
    for (uint32_t k0 = 0; k0 < nq; k0 += 8u) {
      const uint32_t k = k0 + e;
      double acc = 0.0;
      if (k < nq) {
        const uint32_t r = blockIdx.x * (256u * R) + (queue[k] >> 16), st = queue[k] & 0xffffu;
        for (uint32_t uu = l; uu < 8u * bps; uu += 32u) {
          const uint32_t b = bps * st + (uu >> 3), u = uu & 7u;  // unit u of block b
          if (b < nb) {
            float wv[32];
            decode_unit_exact<T>(w + ((size_t)r * nb + b) * kBytes, u, wv);
            const float* const xu = xt + (size_t)b * kBlockElems + 32u * u;
#pragma unroll
            for (int i = 0; i < 32; ++i) acc = fma((double)wv[i], (double)xu[i], acc);
          }
        }
      }
#pragma unroll
      for (int h = 16; h > 0; h >>= 1) acc += __shfl_xor(acc, h, 32);
      if (l == 0u && k < nq) value[k] = (float)acc;
    }
    __syncthreads();
  }
  if (row >= rows) return;
  if (mine) {  // the sums again, with the recomputed stages (unchanged for rows without one)
    const uint32_t nq = min(queued, kRedoQueue);
#pragma unroll
    for (int c = 0; c < R; ++c) sum[c] = 0.0f;
    for (uint32_t base = 0; base < nstages; base += 8u) {
      float v[8][R];
      if (base == 0u) {
#pragma unroll
        for (uint32_t i = 0; i < 8u; ++i)
#pragma unroll
          for (int c = 0; c < R; ++c) v[i][c] = first[i][c];
      } else {
        load8(base, v);
      }
#pragma unroll
      for (uint32_t i = 0; i < 8u; ++i) {
        if (base + i >= nstages) continue;
        const uint32_t st = base + i;
#pragma unroll
        for (int c = 0; c < R; ++c) {
          float vc = v[i][c];
          if (__float_as_uint(vc) == kPartRedo) {
            const uint32_t key = ((rw + (uint32_t)c) << 16) | st;
            uint32_t k = 0;
            while (k < nq && queue[k] != key) ++k;
            vc = k < nq ? value[k]
                        : stage_exact<T>(w, row + (uint32_t)c, nb, bps * st,
                                         min(bps * st + bps, nb), xt);
          }
          sum[c] += vc;
        }
      }
    }
  }
  float* const yo = y + (size_t)t * rows + row;
  if constexpr (R == 4) {
    *reinterpret_cast<f32x4*>(yo) = f32x4{sum[0], sum[1], sum[2], sum[3]};
  } else {
    yo[0] = sum[0];
  }
}

// The reduce of a sliced launch of ntok vectors: four rows a thread when the
// row count is a multiple of 4, y is 16-byte aligned (the scratch always is)
// and the grid still gives every CU two workgroups, else one.  The Q6_K head
// (151,936 rows) at M = 4 / 8 / 16: 144.6 / 180.1 / 321.5 -> 143.6 / 176.8 /
// 317.4 us a call; Q4_K 17408 rows at M = 16 (one workgroup a CU) lost
// 0.4 us, so it keeps one row a thread.
template <uint32_t T>
void launch_tok_reduce(const float* part, float* y, uint32_t rows, uint32_t nstages, uint32_t nv,
                       uint32_t ntok, const uint8_t* w, const float* x, uint32_t nb, uint32_t bps,
                       hipStream_t s) {
  const uint32_t g4 = (rows + 1023u) / 1024u;
  if (rows % 4u == 0u && ((uintptr_t)y & 15u) == 0u &&
      (uint64_t)g4 * ntok >= 2u * (uint64_t)cu_count())
    hipLaunchKernelGGL((tok_reduce<T, 4>), dim3(g4, ntok), dim3(256), 0, s, part, y, rows, nstages,
                       nv, w, x, nb, bps);
  else
    hipLaunchKernelGGL((tok_reduce<T, 1>), dim3((rows + 255u) / 256u, ntok), dim3(256), 0, s, part,
                       y, rows, nstages, nv, w, x, nb, bps);
}

}  // namespace
}  // namespace mfma
}  // namespace sihip
