/*
 * CPU oracle for the GGUF K-quant matvec path.  TEST INFRASTRUCTURE ONLY.
 * See kquant_ref.h for what each function restates and how it is pinned.
 * Build: oracle/Makefile (-O2 -ffp-contract=off, no fast-math).
 */
#include "kquant_ref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* src/quant.rs:187-207.  Exact IEEE binary16 -> binary32 by bit surgery. */
float kq_f16_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t fraction = bits & 0x03ffu;
    uint32_t value;
    if (exponent == 0 && fraction == 0) {
        value = sign;
    } else if (exponent == 0) {
        /* subnormal: shift the fraction up until the hidden bit appears */
        int32_t e = -14;
        while ((fraction & 0x0400u) == 0) {
            fraction <<= 1;
            e -= 1;
        }
        fraction &= 0x03ffu;
        value = sign | ((uint32_t)(e + 127) << 23) | (fraction << 13);
    } else if (exponent == 0x1f) {
        value = sign | 0x7f800000u | (fraction << 13);
    } else {
        value = sign | ((exponent + 112u) << 23) | (fraction << 13);
    }
    float out;
    memcpy(&out, &value, sizeof out);
    return out;
}

uint32_t kq_f16_to_f32_bits(uint16_t bits) {
    float f = kq_f16_to_f32(bits);
    uint32_t out;
    memcpy(&out, &f, sizeof out);
    return out;
}

/* src/quant.rs:176-185.  6-bit (scale, min) pair `index` of the 12 packed bytes. */
void kq_get_scale_min(unsigned index, const uint8_t *scales, uint8_t *scale, uint8_t *minimum) {
    if (index < 4) {
        *scale = scales[index] & 0x3f;
        *minimum = scales[index + 4] & 0x3f;
    } else {
        *scale = (uint8_t)((scales[index + 4] & 0x0f) | ((scales[index - 4] >> 6) << 4));
        *minimum = (uint8_t)((scales[index + 4] >> 4) | ((scales[index] >> 6) << 4));
    }
}

size_t kq_block_bytes(uint32_t ggml_type) {
    switch (ggml_type) {
    case KQ_GGML_TYPE_Q4_K: return KQ_Q4_K_BLOCK_BYTES;
    case KQ_GGML_TYPE_Q5_K: return KQ_Q5_K_BLOCK_BYTES;
    case KQ_GGML_TYPE_Q6_K: return KQ_Q6_K_BLOCK_BYTES;
    default: return 0;
    }
}

/* Rejection rules shared by the three decoders (quant.rs:19-34, 68-83, 128-143). */
static int check_shape(size_t len, size_t elements, size_t block_bytes) {
    if (elements == 0 || elements % KQ_BLOCK_ELEMENTS != 0) return KQ_ERR_ELEMENTS;
    size_t blocks = elements / KQ_BLOCK_ELEMENTS;
    if (blocks > SIZE_MAX / block_bytes) return KQ_ERR_OVERFLOW;
    if (len != blocks * block_bytes) return KQ_ERR_BYTES;
    return KQ_OK;
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* One Q4_K block (quant.rs:39-63).  Output order per 64-group: 32 low
 * nibbles with pair 2g, then 32 high nibbles with pair 2g+1. */
static void dequant_q4_k_block(const uint8_t *block, float *out) {
    const float d = kq_f16_to_f32(le16(block));
    const float dmin = kq_f16_to_f32(le16(block + 2));
    const uint8_t *scales = block + 4;
    const uint8_t *quants = block + 16;
    for (unsigned group = 0; group < 4; ++group) {
        uint8_t sc, mn;
        kq_get_scale_min(2 * group, scales, &sc, &mn);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)mn;
        kq_get_scale_min(2 * group + 1, scales, &sc, &mn);
        const float d2 = d * (float)sc;
        const float m2 = dmin * (float)mn;
        const uint8_t *q = quants + 32 * group;
        for (unsigned i = 0; i < 32; ++i) out[64 * group + i] = d1 * (float)(q[i] & 0x0f) - m1;
        for (unsigned i = 0; i < 32; ++i) out[64 * group + 32 + i] = d2 * (float)(q[i] >> 4) - m2;
    }
}

/* One Q5_K block (quant.rs:92-123).  qh bit 2g adds 16 to the low nibble of
 * byte i in group g, bit 2g+1 to the high nibble. */
static void dequant_q5_k_block(const uint8_t *block, float *out) {
    const float d = kq_f16_to_f32(le16(block));
    const float dmin = kq_f16_to_f32(le16(block + 2));
    const uint8_t *scales = block + 4;
    const uint8_t *high = block + 16;
    const uint8_t *quants = block + 48;
    for (unsigned group = 0; group < 4; ++group) {
        uint8_t sc1, mn1, sc2, mn2;
        kq_get_scale_min(2 * group, scales, &sc1, &mn1);
        kq_get_scale_min(2 * group + 1, scales, &sc2, &mn2);
        const float d1 = d * (float)sc1;
        const float m1 = dmin * (float)mn1;
        const float d2 = d * (float)sc2;
        const float m2 = dmin * (float)mn2;
        const uint8_t low_mask = (uint8_t)(1u << (2 * group));
        const uint8_t high_mask = (uint8_t)(2u << (2 * group));
        const uint8_t *q = quants + 32 * group;
        for (unsigned i = 0; i < 32; ++i) {
            unsigned v = (q[i] & 0x0fu) + ((high[i] & low_mask) ? 16u : 0u);
            out[64 * group + i] = d1 * (float)v - m1;
        }
        for (unsigned i = 0; i < 32; ++i) {
            unsigned v = (q[i] >> 4) + ((high[i] & high_mask) ? 16u : 0u);
            out[64 * group + 32 + i] = d2 * (float)v - m2;
        }
    }
}

/* One Q6_K block (quant.rs:145-172).  v = (d * scale) * q, q in -32..31. */
static void dequant_q6_k_block(const uint8_t *block, float *out) {
    const uint8_t *ql_all = block;
    const uint8_t *qh_all = block + 128;
    const uint8_t *sc_all = block + 192;
    const float d = kq_f16_to_f32(le16(block + 208));
    for (unsigned half = 0; half < 2; ++half) {
        const uint8_t *ql = ql_all + 64 * half;
        const uint8_t *qh = qh_all + 32 * half;
        const int8_t *sc = (const int8_t *)(sc_all + 8 * half);
        float *base = out + 128 * half;
        for (unsigned i = 0; i < 32; ++i) {
            const unsigned s = i / 16;
            const uint8_t h = qh[i];
            const int q1 = (int)((ql[i] & 0x0f) | ((h & 0x03) << 4)) - 32;
            const int q2 = (int)((ql[i + 32] & 0x0f) | (((h >> 2) & 0x03) << 4)) - 32;
            const int q3 = (int)((ql[i] >> 4) | (((h >> 4) & 0x03) << 4)) - 32;
            const int q4 = (int)((ql[i + 32] >> 4) | ((h >> 6) << 4)) - 32;
            base[i] = d * (float)sc[s] * (float)q1;
            base[i + 32] = d * (float)sc[s + 2] * (float)q2;
            base[i + 64] = d * (float)sc[s + 4] * (float)q3;
            base[i + 96] = d * (float)sc[s + 6] * (float)q4;
        }
    }
}

typedef void (*block_fn)(const uint8_t *, float *);

static int dequant_all(const uint8_t *bytes, size_t len, size_t elements, float *out,
                       size_t block_bytes, block_fn fn) {
    int rc = check_shape(len, elements, block_bytes);
    if (rc != KQ_OK) return rc;
    size_t blocks = elements / KQ_BLOCK_ELEMENTS;
    for (size_t b = 0; b < blocks; ++b) fn(bytes + b * block_bytes, out + b * KQ_BLOCK_ELEMENTS);
    return KQ_OK;
}

/* src/quant.rs:18-65 */
int kq_dequantize_q4_k(const uint8_t *bytes, size_t len, size_t elements, float *out) {
    return dequant_all(bytes, len, elements, out, KQ_Q4_K_BLOCK_BYTES, dequant_q4_k_block);
}
/* src/quant.rs:67-125 */
int kq_dequantize_q5_k(const uint8_t *bytes, size_t len, size_t elements, float *out) {
    return dequant_all(bytes, len, elements, out, KQ_Q5_K_BLOCK_BYTES, dequant_q5_k_block);
}
/* src/quant.rs:127-174 */
int kq_dequantize_q6_k(const uint8_t *bytes, size_t len, size_t elements, float *out) {
    return dequant_all(bytes, len, elements, out, KQ_Q6_K_BLOCK_BYTES, dequant_q6_k_block);
}

static block_fn block_decoder(uint32_t ggml_type) {
    switch (ggml_type) {
    case KQ_GGML_TYPE_Q4_K: return dequant_q4_k_block;
    case KQ_GGML_TYPE_Q5_K: return dequant_q5_k_block;
    case KQ_GGML_TYPE_Q6_K: return dequant_q6_k_block;
    default: return NULL;
    }
}

int kq_dequantize(uint32_t ggml_type, const uint8_t *bytes, size_t len, size_t elements, float *out) {
    block_fn fn = block_decoder(ggml_type);
    if (!fn) return KQ_ERR_TYPE;
    return dequant_all(bytes, len, elements, out, kq_block_bytes(ggml_type), fn);
}

/* src/metal.rs:7478-7484: `.map(|c| w[c] * x[c]).sum::<f32>()`.  Rust's f32
 * Sum folds from -0.0 (only visible when every product is -0.0). */
float kq_dot_f32_sequential(const float *w, const float *x, size_t n) {
    float acc = -0.0f;
    for (size_t i = 0; i < n; ++i) {
        float p = w[i] * x[i];
        acc = acc + p;
    }
    return acc;
}

double kq_dot_f64(const float *w, const float *x, size_t n) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += (double)w[i] * (double)x[i];
    return acc;
}

double kq_abs_dot_f64(const float *w, const float *x, size_t n) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += fabs((double)w[i] * (double)x[i]);
    return acc;
}

typedef struct {
    block_fn fn;
    size_t block_bytes;
    const uint8_t *bytes;
    size_t row_begin, row_end, cols;
    const float *x;
    float *y_f32;
    double *y_f64, *abs_f64;
    int rc;
} matvec_job;

static void *matvec_rows(void *arg) {
    matvec_job *job = (matvec_job *)arg;
    const size_t blocks_per_row = job->cols / KQ_BLOCK_ELEMENTS;
    const size_t row_bytes = blocks_per_row * job->block_bytes;
    float *row = (float *)malloc(job->cols * sizeof(float));
    if (!row) {
        job->rc = KQ_ERR_OVERFLOW;
        return NULL;
    }
    for (size_t r = job->row_begin; r < job->row_end; ++r) {
        const uint8_t *src = job->bytes + r * row_bytes;
        for (size_t b = 0; b < blocks_per_row; ++b)
            job->fn(src + b * job->block_bytes, row + b * KQ_BLOCK_ELEMENTS);
        if (job->y_f32) job->y_f32[r] = kq_dot_f32_sequential(row, job->x, job->cols);
        if (job->y_f64) job->y_f64[r] = kq_dot_f64(row, job->x, job->cols);
        if (job->abs_f64) job->abs_f64[r] = kq_abs_dot_f64(row, job->x, job->cols);
    }
    free(row);
    job->rc = KQ_OK;
    return NULL;
}

int kq_matvec_ref(uint32_t ggml_type, const uint8_t *bytes, size_t len, size_t rows, size_t cols,
                  const float *x, float *y_f32, double *y_f64, double *abs_f64, int threads) {
    block_fn fn = block_decoder(ggml_type);
    if (!fn) return KQ_ERR_TYPE;
    if (rows == 0 || cols == 0 || cols % KQ_BLOCK_ELEMENTS != 0) return KQ_ERR_ELEMENTS;
    if (rows > SIZE_MAX / cols) return KQ_ERR_OVERFLOW;
    int rc = check_shape(len, rows * cols, kq_block_bytes(ggml_type));
    if (rc != KQ_OK) return rc;
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)rows;
    matvec_job *jobs = (matvec_job *)calloc((size_t)threads, sizeof(matvec_job));
    pthread_t *tids = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        return KQ_ERR_OVERFLOW;
    }
    for (int t = 0; t < threads; ++t) {
        matvec_job *j = &jobs[t];
        j->fn = fn;
        j->block_bytes = kq_block_bytes(ggml_type);
        j->bytes = bytes;
        j->row_begin = rows * (size_t)t / (size_t)threads;
        j->row_end = rows * (size_t)(t + 1) / (size_t)threads;
        j->cols = cols;
        j->x = x;
        j->y_f32 = y_f32;
        j->y_f64 = y_f64;
        j->abs_f64 = abs_f64;
    }
    if (threads == 1) {
        matvec_rows(&jobs[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, matvec_rows, &jobs[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    rc = KQ_OK;
    for (int t = 0; t < threads; ++t)
        if (jobs[t].rc != KQ_OK) rc = jobs[t].rc;
    free(jobs);
    free(tids);
    return rc;
}

/* src/runtime.rs:4296-4298 */
float kq_silu(float v) { return v / (1.0f + expf(-v)); }

/* Key that orders f32 bit patterns like Rust's f32::total_cmp. */
static int32_t total_order_key(float v) {
    int32_t bits;
    memcpy(&bits, &v, sizeof bits);
    return bits ^ (int32_t)((uint32_t)(bits >> 31) >> 1);
}

/* src/runtime.rs:4301-4309: filter(is_finite).max_by(total_cmp); Iterator::max_by
 * returns the last of several equal maxima. */
int kq_argmax_last_finite(const float *v, size_t n, uint32_t *index) {
    int found = 0;
    int32_t best_key = 0;
    uint32_t best = 0;
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(v[i])) continue;
        int32_t key = total_order_key(v[i]);
        if (!found || key >= best_key) {
            best_key = key;
            best = (uint32_t)i;
            found = 1;
        }
    }
    if (!found) return KQ_ERR_NO_FINITE;
    *index = best;
    return KQ_OK;
}

/* src/qwen35_runtime.rs:2237-2244 */
uint32_t kq_argmax_first_greater(const float *v, size_t n) {
    uint32_t best = 0;
    float best_value = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        if (v[i] > best_value) {
            best_value = v[i];
            best = (uint32_t)i;
        }
    }
    return best;
}
