// Tuned gfx950 kernels (kernels_tuned.hip, kernels_q4k_mfma.hip, kernels_q6k_mfma.hip).  Each launcher returns false when
// the shape is outside what the tuned kernel handles; the caller then uses
// the generic kernels.  When it returns true, *err holds the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "si_hip_internal.h"

namespace sihip {

bool launch_matvec_tuned(uint32_t type, const uint8_t* w, const float* x, float* y, uint32_t rows,
                         uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                         hipError_t* err);
// Q4_K, one vector, on the matrix cores (rows of more than 128 blocks, and
// long rows over few tiles, in K slices; up to 2048 blocks of 256, where 64
// slices of at most 8 stages still fit the LDS).
bool launch_q4k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err);
// Q4_K, batch >= 2 vectors (batch-major x and y): two in one pass of the
// one-vector-per-MFMA kernel, three to sixteen in one pass of the
// vectors-in-rows kernel (the weights decoded once per pass).
bool launch_q4k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err);
// Q5_K, one vector / batch >= 2 vectors, on the matrix cores (the Q4_K kernels
// reading 176-byte blocks; batches as for Q4_K).
bool launch_q5k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err);
bool launch_q5k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err);
constexpr size_t kMaxGroupWeights = 8;  // = kMaxGroup of the kernels
// One vector, 2..8 matrices of one type (Q4_K, Q5_K or Q6_K) and one K (rows
// of each but the last a multiple of 16) in one launch: y holds their outputs
// one after the other.
bool launch_matvec_group(uint32_t type, const uint8_t* const* w, const uint32_t* rows,
                         uint32_t count, uint32_t cols, const float* x, float* y,
                         const Workspace& ws, hipStream_t s, hipError_t* err);
// Q6_K, one vector / batch >= 2 vectors (two in one pass of the per-vector
// loop, three to sixteen in one pass of the vectors-in-rows kernel), on the
// matrix cores.
bool launch_q6k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err);
// The Q6_K matvec with the greedy argmax of its output fused (rule: an
// ArgmaxRule): y gets the logits, *result the packed winning candidate
// (0 when no logit qualifies).
bool launch_q6k_matvec_argmax_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                                   uint32_t cols, uint32_t rule, uint64_t* result,
                                   const Workspace& ws, hipStream_t s, hipError_t* err);
bool launch_q6k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err);
// Fused SwiGLU gate/up (both Q4_K) on the matrix cores: h = silu(gate.x) * (up.x).
bool launch_q4k_gate_up_mfma(const uint8_t* gate, const uint8_t* up, const float* x, float* h,
                             uint32_t rows, uint32_t cols, const Workspace& ws, hipStream_t s,
                             hipError_t* err);
bool launch_fused_gate_up_tuned(const uint8_t* gate, const uint8_t* up, const float* x, float* h,
                                uint32_t rows, uint32_t cols, const Workspace& ws, hipStream_t s,
                                hipError_t* err);

}  // namespace sihip
