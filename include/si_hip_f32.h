/* F32 matvec and RMSNorm: the other ops of a decoder block around the K-quant
 * projections (the GGUF F32 tensors and the block's norms).
 *
 * Same conventions as si_hip.h: SI_HIP_OK or a negative SI_HIP_ERR_* code, the
 * reference's message in si_hip_last_error(), validation before the context
 * is touched.  Host-pointer calls are synchronous (copy in, run, copy out, one
 * wait); *_device calls are asynchronous on the context's stream (recorded
 * while a capture is open).  Results are not bit-identical to the reference's
 * Metal kernels (their reduction order is Apple's); they are within a few
 * units in the last place of the exact value (RMSNorm) and within
 * 2e-5 * sum|w*x| (matvec). */
#ifndef SI_HIP_F32_H
#define SI_HIP_F32_H

#include <stddef.h>
#include <stdint.h>

#include "si_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* MetalContext::f32_matvec (metal.rs:2983-3049): y[r] = sum_c w[r*cols+c] x[c]
 * for a row-major rows x cols matrix of `values` floats.  "F32 matvec
 * dimensions overflow", "F32 matvec dimensions or byte length are invalid". */
int si_hip_f32_matvec(si_hip_context *ctx, const float *w, size_t values, size_t rows, size_t cols,
                      const float *x, size_t x_len, float *y);
/* MetalContext::f32_matvec_bytes (metal.rs:3051-3072): the same over raw GGUF
 * bytes; "F32 matvec byte length overflows", "F32 matvec byte length is
 * invalid", "F32 matvec bytes are not 4-byte aligned". */
int si_hip_f32_matvec_bytes(si_hip_context *ctx, const uint8_t *bytes, size_t len, size_t rows,
                            size_t cols, const float *x, size_t x_len, float *y);
/* Several matrices with the same columns and one input, one submission
 * (the command buffer of f32_matvec_many_gguf_tensors, metal.rs:4780-4870);
 * matrix i has rows[i] rows, its result goes to ys[i]. */
int si_hip_f32_matvec_many(si_hip_context *ctx, const float *const *ws, const size_t *rows,
                           size_t count, size_t cols, const float *x, size_t x_len,
                           float *const *ys);
/* Device-resident form (no counterpart in the reference, which has no
 * device-pointer calls): d_y = W d_x, all pointers device memory. */
int si_hip_f32_matvec_device(si_hip_context *ctx, const float *d_w, size_t rows, size_t cols,
                             const float *d_x, float *d_y);

/* MetalContext::rms_norm (metal.rs:2641-2700): y = x * inv * w over one
 * vector, inv = 1 / sqrt(mean(x^2) + eps); "RMSNorm input and weight must have
 * equal non-zero length". */
int si_hip_rms_norm(si_hip_context *ctx, const float *x, size_t x_len, const float *w, size_t w_len,
                    float eps, float *y);
/* MetalContext::rms_norm_heads (metal.rs:2856-2926; CPU form qwen35.rs:53-87):
 * heads vectors of head_dim values, y = x * inv * (1 + w); "head RMSNorm
 * dimensions overflow", "head RMSNorm dimensions are invalid" (eps must be
 * finite and positive). */
int si_hip_rms_norm_heads(si_hip_context *ctx, const float *x, size_t x_len, const float *w,
                          size_t w_len, size_t heads, size_t head_dim, float eps, float *y);
/* MetalContext::rms_norm_gated (metal.rs:2773-2854; CPU form qwen35.rs:14-50):
 * y = x * inv * w * silu(gate), silu(g) = g / (1 + exp(-g)); "Gated RMSNorm
 * dimensions overflow", "Gated RMSNorm dimensions are invalid". */
int si_hip_rms_norm_gated(si_hip_context *ctx, const float *x, size_t x_len, const float *gate,
                          size_t gate_len, const float *w, size_t w_len, size_t heads,
                          size_t head_dim, float eps, float *y);
/* Device-resident form of the three (no counterpart in the reference): mode
 * 0 = rms_norm (heads must be 1), 1 = rms_norm_heads, 2 = rms_norm_gated
 * (d_gate used only there). */
int si_hip_rms_norm_device(si_hip_context *ctx, uint32_t mode, const float *d_x, const float *d_gate,
                           const float *d_w, size_t heads, size_t head_dim, float eps, float *d_y);

#ifdef __cplusplus
}
#endif
#endif /* SI_HIP_F32_H */
