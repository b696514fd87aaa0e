/*
 * si_hip_synth.h: seeded synthetic GGUF K-quant data for benchmarks and tests.
 *
 * No counterpart in the reference (its probes read real GGUF files); these
 * host-only helpers generate the synthetic workloads of the benchmark
 * configurations without a model file.  Counter-based: block b of a stream
 * depends only on (seed, b), so any block of a multi-GB set can be
 * regenerated on its own to spot-check it.
 *
 *   Q4_K / Q5_K: every byte uniform, then d and dmin replaced by
 *                f16(|N(0, 0.02)|) (round to nearest even).
 *   Q6_K:        ql / qh uniform, 16 int8 scales uniform in [-32, 31],
 *                d = f16(|N(0, 0.01)|).
 * Normals for d/dmin come from a 65,536-entry inverse-CDF table
 * (Phi^-1((i + 0.5) / 65536)); activations use Box-Muller in f64 rounded
 * to f32.
 */
#ifndef SI_HIP_SYNTH_H
#define SI_HIP_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Writes n_blocks packed blocks (block_bytes * n_blocks bytes) starting at
 * block index first_block.  `threads` <= 1 runs on the calling thread. */
int si_hip_synth_blocks(uint32_t ggml_type, uint64_t seed, uint64_t first_block, size_t n_blocks,
                        uint8_t *out, size_t out_len, int threads);
/* out[i] = scale * N(0,1) sample i of the stream `seed`. */
int si_hip_synth_normal_f32(uint64_t seed, uint64_t first_index, size_t n, float scale, float *out);
/* Uniform token ids in [0, vocab). */
int si_hip_synth_token_ids(uint64_t seed, size_t n, uint32_t vocab, uint32_t *out);
/* IEEE binary32 -> binary16, round to nearest even (NaN stays NaN). */
uint16_t si_hip_synth_f32_to_f16(float value);

#ifdef __cplusplus
}
#endif
#endif /* SI_HIP_SYNTH_H */
