/*
 * CPU oracle for the F32 matvec and RMSNorm ops around the K-quant path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ as the checker, never by the
 * HIP product.
 *
 *   kq_f32_matvec_ref  the expected values of the reference's F32 matvec test
 *                      (src/metal.rs:7347-7353): per row a sequential f32
 *                      left fold of w[r*cols+c] * x[c], each product and each
 *                      sum rounded.
 *   kq_rms_norm_ref    mode 0: the reference's RMSNorm test expectation
 *                      (src/metal.rs:7260-7266): mean of x*x (sequential f32),
 *                      inverse = (mean + eps).sqrt().recip(), y = x*inv*w;
 *                      mode 1: rms_norm_heads (src/qwen35.rs:53-87), y =
 *                      x*inv*(1 + w) per head; mode 2: gated_rms_norm
 *                      (src/qwen35.rs:14-50), y = x*inv*w*silu(g) with
 *                      silu(g) = g / (1 + exp(-g)) (src/qwen35.rs:8-10).
 *
 * Compiled with -ffp-contract=off: every product and sum rounds on its own,
 * as Rust's f32 arithmetic does.  Pinned in tests/test_f32_oracle.py by
 * closed-form cases (exact small-integer vectors, powers of two, eps at its
 * limits), head independence, the scale invariance of the norm and f64
 * recomputation.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

int kq_f32_matvec_ref(const float *w, const float *x, size_t rows, size_t cols, float *out) {
  if (!w || !x || !out || rows == 0 || cols == 0) return -1;
  for (size_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (size_t c = 0; c < cols; ++c) {
      const float p = w[r * cols + c] * x[c];
      sum = sum + p;
    }
    out[r] = sum;
  }
  return 0;
}

static float silu_ref(float v) { return v / (1.0f + expf(-v)); }

int kq_rms_norm_ref(uint32_t mode, const float *x, const float *gate, const float *w,
                    size_t heads, size_t head_dim, float eps, float *out) {
  if (!x || !w || !out || heads == 0 || head_dim == 0 || mode > 2 || (mode == 2 && !gate))
    return -1;
  for (size_t h = 0; h < heads; ++h) {
    const float *xh = x + h * head_dim;
    float sum = 0.0f;
    for (size_t i = 0; i < head_dim; ++i) {
      const float sq = xh[i] * xh[i];
      sum = sum + sq;
    }
    const float mean = sum / (float)head_dim;
    const float inverse = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < head_dim; ++i) {
      float o = xh[i] * inverse;
      if (mode == 0) o = o * w[i];
      if (mode == 1) o = o * (1.0f + w[i]);
      if (mode == 2) {
        o = o * w[i];
        o = o * silu_ref(gate[h * head_dim + i]);
      }
      out[h * head_dim + i] = o;
    }
  }
  return 0;
}
