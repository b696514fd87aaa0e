/*
 * si_hip.h: C ABI of the MI355X (gfx950) GGUF K-quant matvec path.
 *
 * Drop-in boundary for super-inference's K-quant surface on `MetalContext`
 * (src/metal.rs).  A Rust `hip` backend module binds these symbols with an
 * `extern "C"` block and wraps them in a `HipContext` whose methods keep the
 * names and `Result<_, String>` behaviour of the Metal methods cited below.
 *
 * Conventions
 *   - Every entry point returns an int status: SI_HIP_OK (0) or a negative
 *     SI_HIP_ERR_* code.  On failure si_hip_last_error() returns a message
 *     for the calling thread (the reference's Err(String)).
 *   - Argument validation runs on the host, before any device work, in the
 *     same order as the reference; it needs no GPU, so every rejection can be
 *     exercised on a machine without one (pass ctx = NULL: shape errors are
 *     reported before the context is checked).
 *   - "rows"/"columns" follow the reference: a GGUF 2-D tensor has
 *     shape[0] = columns (contiguous) and shape[1] = rows (metal.rs:4356-4357);
 *     rows are packed 256-weight super-blocks, row-major.
 *   - Block bytes: Q4_K 144, Q5_K 176, Q6_K 210 per 256 weights
 *     (src/quant.rs:8-16); ggml type ids 12 / 13 / 14.
 *   - Host-pointer entry points are synchronous (the reference commits and
 *     waits, metal.rs:2320-2337): they copy inputs to HBM, run, copy results
 *     back, and return.  *_device entry points take device pointers and only
 *     enqueue on the context's compute stream (see si_hip_synchronize).
 *   - A context may be shared by several host threads; calls on one context
 *     are serialised internally.
 */
#ifndef SI_HIP_H
#define SI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SI_HIP_ABI_VERSION 1u

/* ---- status codes ------------------------------------------------------ */
#define SI_HIP_OK 0
#define SI_HIP_ERR_NULL (-1)              /* null context, handle or buffer */
#define SI_HIP_ERR_DIMENSIONS (-2)        /* rows/cols 0, cols % 256, input length */
#define SI_HIP_ERR_BYTE_LENGTH (-3)       /* byte length != rows*cols/256*block */
#define SI_HIP_ERR_OVERFLOW (-4)          /* checked_mul overflow / > u32 limits */
#define SI_HIP_ERR_UNSUPPORTED_TYPE (-5)  /* ggml type not 12/13/14 (or not Q4_K) */
#define SI_HIP_ERR_BATCH (-6)             /* batch outside 1..=SI_HIP_MAX_BATCH */
#define SI_HIP_ERR_RANGE (-7)             /* row range / token id / view range */
#define SI_HIP_ERR_NO_FINITE (-8)         /* argmax over logits with no finite value */
#define SI_HIP_ERR_DEVICE (-9)            /* HIP runtime or launch failure */
#define SI_HIP_ERR_OUT_OF_MEMORY (-10)
#define SI_HIP_ERR_EMPTY (-11)            /* empty weight upload */
#define SI_HIP_ERR_STATE (-12)            /* graph capture already open / not open */

#define SI_HIP_GGML_TYPE_Q4_K 12u
#define SI_HIP_GGML_TYPE_Q5_K 13u
#define SI_HIP_GGML_TYPE_Q6_K 14u

/* The reference caps candidate batches at 8 (metal.rs:4076, 1096); the HIP
 * path accepts up to 16 (the multi-token verify sweep goes to M = 16). */
#define SI_HIP_MAX_BATCH 16u

/* Greedy argmax tie rules. */
#define SI_HIP_ARGMAX_LAST_FINITE 0u   /* runtime.rs:4301-4309: finite only,
                                          total_cmp, last maximum wins */
#define SI_HIP_ARGMAX_FIRST_GREATER 1u /* qwen35_runtime.rs:2237-2244: strict
                                          '>' from -inf, first maximum wins */

typedef struct si_hip_context si_hip_context;
typedef struct si_hip_quant_weight si_hip_quant_weight;

/* CommandStatsSnapshot (metal.rs:1891-1946). */
typedef struct si_hip_command_stats {
  uint64_t submitted;
  uint64_t async_submitted;
  uint64_t waited;
  uint64_t wait_nanos;
} si_hip_command_stats;

/* ---- errors ------------------------------------------------------------ */
const char *si_hip_last_error(void);       /* thread-local; "" after success */
const char *si_hip_status_name(int status);
uint32_t si_hip_abi_version(void);

/* ---- context: MetalContext::new (metal.rs:2170-2310) ------------------- */
int si_hip_context_new(int device_ordinal, si_hip_context **out);
void si_hip_context_free(si_hip_context *ctx);

/* ---- quantized weights: QuantWeight (metal.rs:1840-1880) --------------- */
/* upload_quant_weight_private (metal.rs:2502-2542): packed blocks copied
 * as-is into a new HBM allocation on the upload stream. */
int si_hip_upload_quant_weight_private(si_hip_context *ctx, const uint8_t *weight_bytes,
                                       size_t weight_len, uint32_t ggml_type,
                                       si_hip_quant_weight **out);
/* bind_quant_weight_mapped (metal.rs:2549-2580).  MI355X cannot execute from
 * the host mapping, so the bytes are uploaded once; the handle is marked
 * mapped and counted as active (not persistent) weight memory. */
int si_hip_bind_quant_weight_mapped(si_hip_context *ctx, const uint8_t *weight_bytes,
                                    size_t weight_len, uint32_t ggml_type,
                                    si_hip_quant_weight **out);
/* Offset view of a parent's buffer, as PrivateStagedQwenLayer::quant_weight
 * (metal.rs:1858-1868) hands out views of one staged layer buffer.  The
 * view shares (and keeps alive) the parent's device memory. */
int si_hip_quant_weight_view(const si_hip_quant_weight *parent, uint64_t offset, uint64_t bytes,
                             uint32_t ggml_type, si_hip_quant_weight **out);
void si_hip_quant_weight_free(si_hip_quant_weight *weight);
uint64_t si_hip_quant_weight_byte_len(const si_hip_quant_weight *weight); /* metal.rs:1873 */
uint32_t si_hip_quant_weight_ggml_type(const si_hip_quant_weight *weight); /* metal.rs:1877 */
int si_hip_quant_weight_is_mapped(const si_hip_quant_weight *weight);
/* Device address of the first packed byte (for callers that build their own
 * launches or copies; valid while the handle or a view of it lives). */
const void *si_hip_quant_weight_device_ptr(const si_hip_quant_weight *weight);

/* ---- matvec: y[rows] = W[rows x columns] . input[columns] -------------- */
/* q4_k_matvec (metal.rs:3357-3397), q5_k_matvec (4307-4323),
 * q6_k_matvec (4325-4341): packed bytes from host memory, uploaded per call. */
int si_hip_q4_k_matvec(si_hip_context *ctx, const uint8_t *weight_bytes, size_t weight_len,
                       size_t rows, size_t columns, const float *input, size_t input_len,
                       float *output);
int si_hip_q5_k_matvec(si_hip_context *ctx, const uint8_t *weight_bytes, size_t weight_len,
                       size_t rows, size_t columns, const float *input, size_t input_len,
                       float *output);
int si_hip_q6_k_matvec(si_hip_context *ctx, const uint8_t *weight_bytes, size_t weight_len,
                       size_t rows, size_t columns, const float *input, size_t input_len,
                       float *output);
/* gguf_quant_matvec_bytes (metal.rs:4000-4061) */
int si_hip_gguf_quant_matvec_bytes(si_hip_context *ctx, uint32_t ggml_type,
                                   const uint8_t *weight_bytes, size_t weight_len, size_t rows,
                                   size_t columns, const float *input, size_t input_len,
                                   float *output);
/* gguf_quant_matvec_weight (metal.rs:3923-3995): HBM-resident weight. */
int si_hip_gguf_quant_matvec_weight(si_hip_context *ctx, const si_hip_quant_weight *weight,
                                    size_t rows, size_t columns, const float *input,
                                    size_t input_len, float *output);
/* quant_k_matvec_tensor_rows / q4_k_matvec_tensor_rows (metal.rs:4346-4467,
 * 4505-4527): rows [row_start, row_start+row_count) of a resident rank-2
 * tensor of shape [shape_columns, shape_rows]. */
int si_hip_gguf_quant_matvec_tensor_rows(si_hip_context *ctx, const si_hip_quant_weight *tensor,
                                         size_t shape_columns, size_t shape_rows,
                                         size_t row_start, size_t row_count, const float *input,
                                         size_t input_len, float *output);
/* gguf_quant_matvec_many_weights (metal.rs:4652-4775): several matvecs over
 * one shared input, one submission and one wait. */
int si_hip_gguf_quant_matvec_many_weights(si_hip_context *ctx,
                                          const si_hip_quant_weight *const *weights,
                                          const size_t *rows, size_t count, size_t columns,
                                          const float *input, size_t input_len,
                                          float *const *outputs);
/* gguf_quant_matvec_many_bytes (metal.rs:4878-5001): several matvecs over
 * host bytes (tensor i: types[i], bytes[i] of lens[i], rows[i] x columns[i]),
 * one input, one submission and one wait. */
int si_hip_gguf_quant_matvec_many_bytes(si_hip_context *ctx, const uint32_t *types,
                                        const uint8_t *const *bytes, const size_t *lens,
                                        const size_t *rows, const size_t *columns, size_t count,
                                        const float *input, size_t input_len,
                                        float *const *outputs);

/* ---- fused SwiGLU ------------------------------------------------------ */
/* q4_k_fused_gate_up (metal.rs:3402-3486): out = silu(gate.x) * (up.x). */
int si_hip_q4_k_fused_gate_up(si_hip_context *ctx, const uint8_t *gate_bytes, size_t gate_len,
                              const uint8_t *up_bytes, size_t up_len, size_t rows,
                              size_t columns, const float *input, size_t input_len,
                              float *output);
/* q4_k_fused_gate_up_weights (metal.rs:3489-3562) */
int si_hip_q4_k_fused_gate_up_weights(si_hip_context *ctx, const si_hip_quant_weight *gate,
                                      const si_hip_quant_weight *up, size_t rows, size_t columns,
                                      const float *input, size_t input_len, float *output);
/* gguf_quant_fused_mlp_weights (metal.rs:3569-3732): gate/up (Q4_K) then the
 * Q4_K/Q5_K/Q6_K down projection with the intermediate kept in HBM. */
int si_hip_gguf_quant_fused_mlp_weights(si_hip_context *ctx, const si_hip_quant_weight *gate,
                                        const si_hip_quant_weight *up,
                                        const si_hip_quant_weight *down, size_t gate_rows,
                                        size_t columns, size_t down_rows, const float *input,
                                        size_t input_len, float *output);

/* q4_k_matvec_tensor_rows / q5_k / q6_k and gguf_quant_matvec_tensor_rows
 * (metal.rs:4346-4527) on a GgufTensorView: its name, type, GGUF shape
 * [columns, rows] (n_dims entries) and borrowed payload bytes, with the
 * reference's checks and messages.  The whole payload is what stays resident
 * (see residency below), so calls on different row ranges share one copy. */
int si_hip_gguf_quant_matvec_view_rows(si_hip_context *ctx, const char *name, uint32_t ggml_type,
                                       const uint64_t *shape, uint32_t n_dims,
                                       const uint8_t *payload, size_t payload_len,
                                       size_t row_start, size_t row_count, const float *input,
                                       size_t input_len, float *output);

/* ---- embedding (bit-exact dequantisation of table rows) --------------- */
/* q4_k_embedding_tensor (metal.rs:3785-3810) on a GgufTensorView (type,
 * shape, borrowed payload): the reference's checks in order; the table stays
 * resident when it fits the residency budget, else the row alone is copied. */
int si_hip_q4_k_embedding_view(si_hip_context *ctx, uint32_t ggml_type, const uint64_t *shape,
                               uint32_t n_dims, const uint8_t *payload, size_t payload_len,
                               size_t token_id, float *output);
/* q4_k_embedding_row (metal.rs:3734-3783) */
int si_hip_q4_k_embedding_row(si_hip_context *ctx, const uint8_t *row_bytes, size_t row_len,
                              size_t columns, float *output);
/* q4_k_embedding_tensor (metal.rs:3785-3810), for a resident table. */
int si_hip_q4_k_embedding_tensor(si_hip_context *ctx, const si_hip_quant_weight *table,
                                 size_t shape_columns, size_t shape_rows, size_t token_id,
                                 float *output);
/* The same for n token ids in one launch: output is [n][shape_columns]. */
int si_hip_q4_k_embedding_tokens(si_hip_context *ctx, const si_hip_quant_weight *table,
                                 size_t shape_columns, size_t shape_rows,
                                 const uint32_t *token_ids, size_t n_tokens, float *output);

/* ---- multi-token verify: Y[b][rows] = W . X[b][columns], b < batch ----- */
/* gguf_quant_matmul_many_bytes (metal.rs:4067-4158) */
int si_hip_gguf_quant_matmul_many_bytes(si_hip_context *ctx, uint32_t ggml_type,
                                        const uint8_t *weight_bytes, size_t weight_len,
                                        size_t rows, size_t columns, size_t batch,
                                        const float *inputs, size_t inputs_len, float *outputs);
/* gguf_quant_matmul_many_weight (metal.rs:4161-4241) */
int si_hip_gguf_quant_matmul_many_weight(si_hip_context *ctx, const si_hip_quant_weight *weight,
                                         size_t rows, size_t columns, size_t batch,
                                         const float *inputs, size_t inputs_len,
                                         float *outputs);

/* ---- output head + greedy argmax -------------------------------------- */
/* Qwen35Runtime::logits' head matvec (qwen35_runtime.rs:2132-2192) followed
 * by argmax (runtime.rs:4301-4309, or the first-wins rule of
 * qwen35_runtime.rs:2237-2244), on the device; only the token id (and,
 * when logits is non-NULL, the logits) come back.  A Q6_K head runs as one
 * launch with the argmax fused into the matvec (which then stores no logits
 * when logits is NULL). */
int si_hip_gguf_quant_matvec_argmax_weight(si_hip_context *ctx, const si_hip_quant_weight *head,
                                           size_t rows, size_t columns, const float *input,
                                           size_t input_len, uint32_t rule, uint32_t *token,
                                           float *logits);

/* ---- dequantisation (quant.rs dequantize_q4_k/q5_k/q6_k on the GPU) ---- */
int si_hip_dequantize(si_hip_context *ctx, uint32_t ggml_type, const uint8_t *bytes, size_t len,
                      size_t elements, float *output);

/* ---- device-resident API (async on the compute stream) ----------------- */
int si_hip_device_alloc(si_hip_context *ctx, size_t bytes, void **device_ptr);
int si_hip_device_free(si_hip_context *ctx, void *device_ptr);
int si_hip_copy_to_device(si_hip_context *ctx, void *device_dst, const void *host_src,
                          size_t bytes);
int si_hip_copy_from_device(si_hip_context *ctx, void *host_dst, const void *device_src,
                            size_t bytes);
/* Device-to-device copy on the compute stream (asynchronous).  Plumbing with
 * no counterpart in metal.rs; the benchmark uses it as the plain-copy yardstick
 * for HBM traffic counters. */
int si_hip_copy_device(si_hip_context *ctx, void *device_dst, const void *device_src,
                       size_t bytes);
int si_hip_synchronize(si_hip_context *ctx);
int si_hip_quant_matvec_device(si_hip_context *ctx, const si_hip_quant_weight *weight,
                               size_t rows, size_t columns, const float *d_input,
                               float *d_output);
/* gguf_quant_matvec_many_weights (metal.rs:4652-4775) on device buffers:
 * weight i's rows land in d_output after those of weights 0..i-1.  Groups
 * of 2..8 weights of one type (Q4_K, Q5_K or Q6_K) whose row counts (all but
 * the last) are multiples of 16 run as one launch. */
int si_hip_quant_matvec_many_device(si_hip_context *ctx, const si_hip_quant_weight *const *weights,
                                    const size_t *rows, size_t count, size_t columns,
                                    const float *d_input, float *d_output);
int si_hip_q4_k_fused_gate_up_device(si_hip_context *ctx, const si_hip_quant_weight *gate,
                                     const si_hip_quant_weight *up, size_t rows, size_t columns,
                                     const float *d_input, float *d_output);
/* d_hidden: gate_rows floats of caller-owned device scratch. */
int si_hip_fused_mlp_device(si_hip_context *ctx, const si_hip_quant_weight *gate,
                            const si_hip_quant_weight *up, const si_hip_quant_weight *down,
                            size_t gate_rows, size_t columns, size_t down_rows,
                            const float *d_input, float *d_hidden, float *d_output);
int si_hip_matmul_many_device(si_hip_context *ctx, const si_hip_quant_weight *weight,
                              size_t rows, size_t columns, size_t batch, const float *d_inputs,
                              float *d_outputs);
/* d_logits: rows floats; d_result: one uint64 packed (key<<32 | index),
 * decoded by si_hip_argmax_result_index.  packed == 0 means no logit
 * qualified: under SI_HIP_ARGMAX_FIRST_GREATER (no logit beat -inf: all NaN
 * or -inf) the index is 0, the id the reference's scan keeps
 * (qwen35_runtime.rs:2237-2244); under SI_HIP_ARGMAX_LAST_FINITE (no finite
 * logit, runtime.rs:4301-4309 returns an error) it is SI_HIP_ARGMAX_NONE,
 * which no vocabulary row has. */
#define SI_HIP_ARGMAX_NONE 0xffffffffu
int si_hip_matvec_argmax_device(si_hip_context *ctx, const si_hip_quant_weight *head,
                                size_t rows, size_t columns, const float *d_input,
                                uint32_t rule, float *d_logits, uint64_t *d_result);
uint32_t si_hip_argmax_result_index(uint64_t packed, uint32_t rule);
/* q4_k_embedding_tensor (metal.rs:3785-3810) for n_tokens device-resident
 * ids.  The table checks run here; the ids are checked by the kernel: an id
 * beyond the rows the table holds yields a row of NaNs, and the next
 * synchronisation (si_hip_synchronize or any synchronous call) returns
 * SI_HIP_ERR_DEVICE. */
int si_hip_embedding_device(si_hip_context *ctx, const si_hip_quant_weight *table,
                            size_t shape_columns, size_t shape_rows, const uint32_t *d_ids,
                            size_t n_tokens, float *d_output);

/* Measurement probe, no counterpart in the reference (it is not part of the
 * path): `iters` back-to-back launches on the compute stream, launch i
 * reading weights[i % n] (Q4_K or Q5_K, rows x columns) with the weight
 * copies of the one-vector matrix-core kernel -- its grid, twelve waves per
 * CU, 16-row x 64-byte buffer->LDS copies, one stage in flight per wave --
 * and no arithmetic.  mode 0: the kernels' default cache policy; 1: the
 * nontemporal bit; 2: an empty kernel of the same launch shape; 3: the same
 * stages read as 4-row x 256-byte copies.  Modes 4 and 5 (Q4_K, the matrix
 * 128-byte aligned) deal the (tile, stage) pairs evenly to the workgroups,
 * as the kernel's split schedule does: 4 copies each stage as the whole
 * 128-byte lines of its rows (the one-vector kernel's copies; columns / 256
 * = 4 mod 8); 5 loads each lane's matrix-core operands straight into
 * registers (16-byte loads, eight waves per CU, two stages in flight per
 * wave); 6 the same with the nontemporal bit.  Timed with the event slots,
 * it bounds what the matvec can reach on its copy path. */
int si_hip_stream_probe(si_hip_context *ctx, const si_hip_quant_weight *const *weights, size_t n,
                        size_t rows, size_t columns, uint32_t mode, size_t iters);

/* Timing on the compute stream: 16 event slots. */
int si_hip_event_record(si_hip_context *ctx, uint32_t slot);
int si_hip_event_elapsed_ms(si_hip_context *ctx, uint32_t start_slot, uint32_t end_slot,
                            float *ms);
/* Enqueue `iterations` matvecs back to back, cycling through n_weights
 * resident copies (weights[i % n_weights]); used to time HBM streaming
 * without host launch gaps. */
int si_hip_quant_matvec_device_repeat(si_hip_context *ctx,
                                      const si_hip_quant_weight *const *weights,
                                      size_t n_weights, size_t rows, size_t columns,
                                      const float *d_input, float *d_output, size_t iterations);

/* ---- matvec that allocates nothing -------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  y = W x for one Q4_K / Q5_K / Q6_K matrix of `rows` x
 * `columns` whose packed GGUF bytes (`weight_bytes`, exactly rows * columns /
 * 256 blocks) are at device address `weights`; d_input / d_output are device
 * buffers of `columns` / `rows` floats; `stream` is a hipStream_t (NULL: the
 * null stream), and the call only enqueues on it.  No context is needed.
 * The kernels' cross-workgroup workspace is a file-scope device array of
 * SI_HIP_NOALLOC_WORKSPACE_BYTES per GPU (held until the process ends), set
 * up on the first call on each device and left in its rest state by every
 * call; calls that overlap on one GPU race on it.  rows above
 * SI_HIP_NOALLOC_MAX_ROWS (the tiles whose counters it holds) are rejected. */
#define SI_HIP_NOALLOC_WORKSPACE_BYTES (2u << 20)
#define SI_HIP_NOALLOC_MAX_ROWS 4194048u
int si_hip_quant_matvec_noalloc(uint32_t ggml_type, const void *weights, size_t weight_bytes,
                                size_t rows, size_t columns, const float *d_input,
                                float *d_output, void *stream);
/* No counterpart in the reference; for the callers of
 * si_hip_quant_matvec_noalloc.  A kernel that gives up one of its bounded
 * waits (the workgroups' exchange of split-tile sums, seconds of polling)
 * records it in a device word of the current GPU instead of failing the
 * call, and may leave the shared workspace out of its rest state.  This call
 * waits for `stream`, reads and clears that word, and when it was set puts
 * the workspace back into its rest state and returns SI_HIP_ERR_DEVICE
 * (results of no-alloc calls since the last check may then be wrong); else 0.
 * Not under graph capture.  Allocates nothing. */
int si_hip_noalloc_check(void *stream);
/* Test hook, no counterpart in the reference: the no-alloc workspace's
 * bounded waits give up after `polls` polls (0: their normal course); puts
 * the workspace into its rest state, waiting for `stream`.  Not under graph
 * capture. */
int si_hip_noalloc_debug_set_wait_give_up(uint32_t polls, void *stream);

/* ---- captured submission (HIP graphs) ------------------------------------
 * No counterpart in the reference: every Metal call there commits its command
 * buffer and waits (metal.rs:2320-2337).  For callers that repeat the same
 * device-resident work -- a decode step's projections, the 64-layer streaming
 * aggregate -- the *_device calls (and si_hip_copy_device) made between
 * si_hip_capture_begin and si_hip_capture_end are recorded instead of run, and
 * si_hip_graph_launch replays them on the compute stream with less launch
 * overhead per kernel.  The other calls keep running immediately while a
 * capture is open.  One capture per context at a time; record from one
 * thread.  A graph reads the weights and device buffers it was recorded with:
 * keep them alive while it may run. */
typedef struct si_hip_graph si_hip_graph;
int si_hip_capture_begin(si_hip_context *ctx);
int si_hip_capture_end(si_hip_context *ctx, si_hip_graph **out_graph);
int si_hip_graph_launch(si_hip_context *ctx, const si_hip_graph *graph);
uint64_t si_hip_graph_calls(const si_hip_graph *graph);  /* device calls recorded */
void si_hip_graph_free(si_hip_graph *graph);

/* ---- kernel selection (the reference picks variants via SI_QK_* env) --- */
#define SI_HIP_KERNEL_AUTO 0u     /* tuned gfx950 kernels where they apply */
#define SI_HIP_KERNEL_GENERIC 1u  /* one wavefront per row, exact per-weight decode */
/* Failure reporting.  Kernels that cannot finish their work correctly -- a
 * bounded cross-wave or cross-workgroup wait that gave up, a device-side
 * token id beyond the table -- still end normally, and report the failure
 * through a host-visible word of the context; the next synchronisation
 * returns SI_HIP_ERR_DEVICE (all device work since the previous one is then
 * invalid) and puts the context's workspace back into its rest state.
 *
 * Test hook, no counterpart in the reference: with polls > 0 the bounded
 * waits of the split-tile combine and of the argmax reduction take every
 * entry for missing and give up after `polls` polls, so that tests can drive
 * the reporting path while every kernel still ends; 0 restores normal
 * waits. */
int si_hip_debug_set_wait_give_up(si_hip_context *ctx, uint32_t polls);

int si_hip_set_kernel_policy(si_hip_context *ctx, uint32_t policy);

/* ---- telemetry (metal.rs:2312-2442) ------------------------------------ */
uint64_t si_hip_current_allocated_bytes(const si_hip_context *ctx);
uint64_t si_hip_peak_allocated_bytes(const si_hip_context *ctx);
uint64_t si_hip_peak_active_weight_bytes(const si_hip_context *ctx);
void si_hip_reset_peaks(si_hip_context *ctx);
/* sample_allocated (metal.rs:2374-2378): peak = max(peak, current). */
void si_hip_sample_allocated(si_hip_context *ctx);
int si_hip_get_command_stats(const si_hip_context *ctx, si_hip_command_stats *out);

/* ---- residency of borrowed weight bytes -----------------------------------
 * The reference's byte-slice entry points (q4_k_matvec / q5_k / q6_k,
 * gguf_quant_matvec_bytes, gguf_quant_matvec_many_bytes, q4_k_fused_gate_up,
 * gguf_quant_matmul_many_bytes, f32_matvec_bytes / f32_matvec_many; metal.rs
 * 3357-4100, 4652-4775) bind the caller's host bytes to the GPU without a
 * copy (unified memory, new_buffer_with_bytes_no_copy).  MI355X executes from
 * HBM, so a context keeps an HBM copy of each borrowed byte range, keyed by
 * (host address, length), and evicts the least recently used ranges beyond a
 * byte budget; the GGUF store's tensor calls borrow the mapped file this way.
 * A resident range is copied again when its fingerprint changes: the length
 * and 64 windows of 64 bytes spread evenly over the range.  Bytes changed in
 * place outside those windows go unseen: after changing borrowed bytes in
 * place, call si_hip_residency_evict.  Resident bytes count as allocated
 * device memory (si_hip_current_allocated_bytes).  No counterpart in the
 * reference. */
#define SI_HIP_DEFAULT_RESIDENCY_BUDGET (16ull << 30)
typedef struct si_hip_residency_stats {
  uint64_t hits;            /* ranges found resident and unchanged */
  uint64_t uploads;         /* ranges copied: first use, changed, or not kept */
  uint64_t uploaded_bytes;  /* bytes of those copies */
  uint64_t evictions;
  uint64_t resident_ranges;
  uint64_t resident_bytes;
  uint64_t budget_bytes;
} si_hip_residency_stats;
/* 0 turns residency off (every call copies its bytes); a smaller budget
 * evicts at once. */
int si_hip_set_residency_budget(si_hip_context *ctx, uint64_t bytes);
/* Drops every resident range that overlaps [host_bytes, host_bytes + len)
 * (len 0: every range). */
int si_hip_residency_evict(si_hip_context *ctx, const void *host_bytes, size_t len);
int si_hip_get_residency_stats(si_hip_context *ctx, si_hip_residency_stats *out);

#ifdef __cplusplus
}
#endif
#endif /* SI_HIP_H */
