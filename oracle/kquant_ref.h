/*
 * CPU oracle for the GGUF K-quant matvec path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of super-inference's CPU reference path:
 *   - src/quant.rs (block constants, f16_to_f32, get_scale_min, the three
 *     lossless dequantizers and their rejection rules),
 *   - the host dot used by the reference's GPU tests (src/metal.rs:7478-7484:
 *     a sequential f32 left fold over `decoded[row*cols+c] * input[c]`),
 *   - SiLU (src/runtime.rs:4296-4298) and the two greedy argmax rules
 *     (src/runtime.rs:4301-4309 and src/qwen35_runtime.rs:2237-2244).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or as the timed CPU baseline.
 * The HIP product never links or calls it.
 *
 * Compile with -O2 -ffp-contract=off and no fast-math: quant.rs performs
 * every f32 multiply and subtract with its own rounding, so a fused
 * multiply-add here would change result bits.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   kq_f16_to_f32        exhaustive 65,536 patterns vs numpy float16->float32
 *   kq_get_scale_min     round trip through an independent 6-bit packer
 *                        (random scale/min sets), hand-worked byte values
 *                        for j >= 4, exhaustive over the two bytes j < 4 reads
 *   kq_dequantize_q*_k   the four quant.rs known-answer tests (committed
 *                        fixtures) + an independent numpy restatement,
 *                        bit-for-bit on random blocks + committed random
 *                        block fixtures
 *   kq_dot_*             exact-arithmetic identities (integer-valued inputs)
 *                        and a Python fractions.Fraction reference
 *   kq_argmax_*          crafted ties / NaN / +-0 / +-inf vectors with the
 *                        answers Rust's max_by(total_cmp) and the strict '>'
 *                        loop give by their documented definitions
 */
#ifndef KQUANT_REF_H
#define KQUANT_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/quant.rs:8-16 */
#define KQ_BLOCK_ELEMENTS 256u
#define KQ_Q4_K_BLOCK_BYTES 144u
#define KQ_Q5_K_BLOCK_BYTES 176u
#define KQ_Q6_K_BLOCK_BYTES 210u
#define KQ_GGML_TYPE_Q4_K 12u
#define KQ_GGML_TYPE_Q5_K 13u
#define KQ_GGML_TYPE_Q6_K 14u

/* Status codes.  quant.rs returns Err(QuantError(String)); the oracle keeps
 * one code per rejection class (quant.rs:19-34, 68-83, 128-143). */
#define KQ_OK 0
#define KQ_ERR_ELEMENTS (-1)   /* element count 0 or not a multiple of 256 */
#define KQ_ERR_BYTES (-2)      /* byte length != blocks * block_bytes */
#define KQ_ERR_OVERFLOW (-3)   /* blocks * block_bytes overflows */
#define KQ_ERR_TYPE (-4)       /* ggml type is not 12/13/14 */
#define KQ_ERR_NO_FINITE (-5)  /* argmax over no finite value */

float kq_f16_to_f32(uint16_t bits);
/* Same conversion returning the raw bits (no float round trip through a caller
 * that might quiet a signalling NaN). */
uint32_t kq_f16_to_f32_bits(uint16_t bits);
void kq_get_scale_min(unsigned index, const uint8_t *scales, uint8_t *scale, uint8_t *minimum);

int kq_dequantize_q4_k(const uint8_t *bytes, size_t len, size_t elements, float *out);
int kq_dequantize_q5_k(const uint8_t *bytes, size_t len, size_t elements, float *out);
int kq_dequantize_q6_k(const uint8_t *bytes, size_t len, size_t elements, float *out);
int kq_dequantize(uint32_t ggml_type, const uint8_t *bytes, size_t len, size_t elements, float *out);
size_t kq_block_bytes(uint32_t ggml_type); /* 0 for an unsupported type */

/* Sequential f32 left fold, exactly `(0..n).map(|c| w[c]*x[c]).sum::<f32>()`. */
float kq_dot_f32_sequential(const float *w, const float *x, size_t n);
/* f64 dot of the exact f32 products, and sum |w*x| in f64 (tolerance scale). */
double kq_dot_f64(const float *w, const float *x, size_t n);
double kq_abs_dot_f64(const float *w, const float *x, size_t n);

/*
 * Reference matvec: dequantize each row (quant.rs) then dot it with x.
 * Any of y_f32 / y_f64 / abs_f64 may be NULL.  rows*cols/256 blocks are read
 * from `bytes` (len must match exactly).  `threads` > 1 splits rows over
 * pthreads (used for the all-core CPU baseline); results are identical.
 */
int kq_matvec_ref(uint32_t ggml_type, const uint8_t *bytes, size_t len, size_t rows,
                  size_t cols, const float *x, float *y_f32, double *y_f64, double *abs_f64,
                  int threads);

/* silu(v) = v / (1 + exp(-v)) in f32 (src/runtime.rs:4296-4298). */
float kq_silu(float v);

/* src/runtime.rs:4301-4309: finite values only, total order, last max wins. */
int kq_argmax_last_finite(const float *v, size_t n, uint32_t *index);
/* src/qwen35_runtime.rs:2237-2244: strict '>' from -inf, first max wins,
 * NaN never selected, all-NaN/-inf input gives 0. */
uint32_t kq_argmax_first_greater(const float *v, size_t n);

#ifdef __cplusplus
}
#endif
#endif
