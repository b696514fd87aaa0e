// C ABI of the gfx950 K-quant path (include/si_hip.h).
//
// Host side of the boundary: validation in the reference's order, HBM
// residency of packed weights, staging of host inputs/outputs, stream and
// event management, telemetry, and kernel selection.  Kernels live in the
// *.hip files; this file only launches them through si_hip_internal.h.
#include "si_hip.h"
#include "si_hip_f32.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "si_hip_internal.h"
#include "si_hip_shared.h"
#include "si_hip_tuned.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int ok() {
  g_last_error.clear();
  return SI_HIP_OK;
}

}  // namespace

namespace sihip {
int set_error(int status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}
int clear_error() { return ok(); }
}  // namespace sihip

namespace {

size_t block_bytes_of(uint32_t t) {
  switch (t) {
    case SI_HIP_GGML_TYPE_Q4_K: return 144;
    case SI_HIP_GGML_TYPE_Q5_K: return 176;
    case SI_HIP_GGML_TYPE_Q6_K: return 210;
    default: return 0;
  }
}

const char *type_label(uint32_t t) {
  switch (t) {
    case SI_HIP_GGML_TYPE_Q4_K: return "Q4_K";
    case SI_HIP_GGML_TYPE_Q5_K: return "Q5_K";
    case SI_HIP_GGML_TYPE_Q6_K: return "Q6_K";
    default: return "unsupported";
  }
}

bool checked_mul(size_t a, size_t b, size_t *out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

bool checked_add(size_t a, size_t b, size_t *out) {
  if (b > SIZE_MAX - a) return false;
  *out = a + b;
  return true;
}

// rows * (columns/256) * block_bytes with the reference's overflow checks.
int expected_weight_bytes(size_t rows, size_t columns, size_t block_bytes, const char *label,
                          size_t *out) {
  size_t blocks;
  if (!checked_mul(rows, columns / 256, &blocks))
    return fail(SI_HIP_ERR_OVERFLOW, "%s matvec block count overflows", label);
  if (!checked_mul(blocks, block_bytes, out))
    return fail(SI_HIP_ERR_OVERFLOW, "%s matvec byte length overflows", label);
  return SI_HIP_OK;
}

int check_u32(size_t rows, size_t columns, const char *label) {
  if (rows > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "%s rows exceed HIP limits", label);
  if (columns > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "%s columns exceed HIP limits", label);
  return SI_HIP_OK;
}

// Allocation counters shared by a context and every buffer/handle it made,
// so handles may outlive the context (metal.rs:2339-2442).
struct Telemetry {
  std::atomic<uint64_t> allocated{0};
  std::atomic<uint64_t> peak_allocated{0};
  std::atomic<uint64_t> active_weights{0};
  std::atomic<uint64_t> peak_active_weights{0};

  void note_alloc(uint64_t b) {
    const uint64_t now = allocated.fetch_add(b) + b;
    uint64_t prev = peak_allocated.load();
    while (now > prev && !peak_allocated.compare_exchange_weak(prev, now)) {
    }
  }
  void note_free(uint64_t b) { allocated.fetch_sub(b); }
  void note_active(int64_t delta) {
    const uint64_t now = active_weights.fetch_add((uint64_t)delta) + (uint64_t)delta;
    uint64_t prev = peak_active_weights.load();
    while (delta > 0 && now > prev && !peak_active_weights.compare_exchange_weak(prev, now)) {
    }
  }
};

struct DeviceBuffer {
  void *ptr = nullptr;
  size_t bytes = 0;
  std::shared_ptr<Telemetry> tel;
  ~DeviceBuffer() {
    if (ptr) {
      (void)hipFree(ptr);
      if (tel) tel->note_free(bytes);
    }
  }
};

// Pinned host memory that the synchronous host-pointer calls stage their
// inputs and outputs through (a bump region per call).
struct PinnedStage {
  uint8_t *ptr = nullptr;
  size_t cap = 0;
  size_t used = 0;
};
// An output copy waiting for its call's synchronisation: `bytes` from the
// pinned staging at `src` to the caller's `dst`.
struct PendingOut {
  void *dst;
  const void *src;
  size_t bytes;
};

// HBM copies of borrowed host byte ranges, keyed by (host address, length).
struct Resident {
  std::shared_ptr<DeviceBuffer> buf;
  uint64_t fingerprint = 0;
  uint64_t used = 0;  // the call that last used it
};
struct Residency {
  std::map<std::pair<uintptr_t, size_t>, Resident> ranges;
  uint64_t budget = SI_HIP_DEFAULT_RESIDENCY_BUDGET;
  uint64_t bytes = 0;
  uint64_t tick = 0;
  si_hip_residency_stats stats{};
};

}  // namespace

struct si_hip_context {
  int device = 0;
  hipStream_t stream = nullptr;         // compute queue (metal.rs `queue`)
  hipStream_t upload_stream = nullptr;  // metal.rs `upload_queue`
  std::mutex mu;
  uint32_t policy = SI_HIP_KERNEL_AUTO;
  // grow-only staging for the synchronous host-pointer API
  void *stage_in = nullptr;
  size_t stage_in_bytes = 0;
  void *stage_out = nullptr;
  size_t stage_out_bytes = 0;
  void *stage_weights = nullptr;
  size_t stage_weights_bytes = 0;
  void *stage_aux = nullptr;
  size_t stage_aux_bytes = 0;
  // cross-workgroup combine area of the matrix-core kernels (kept zeroed)
  sihip::Workspace ws;
  // the host-visible word kernels report failures in (sihip::DeviceError),
  // its device address (in the workspace's report slot) and the test hook's
  // poll count (0 outside tests)
  volatile uint32_t *dev_error = nullptr;
  uint64_t dev_error_addr = 0;
  uint32_t give_up_polls = 0;
  // pinned staging of the synchronous calls' inputs and outputs; buffers
  // outgrown during a call are freed after its synchronisation
  PinnedStage pin_in, pin_out;
  std::vector<PendingOut> pending;
  std::vector<void *> pin_retired;
  // borrowed weight bytes kept resident in HBM
  Residency res;
  hipEvent_t events[16] = {};
  // graph capture: while `capturing`, the *_device calls go to capture_stream,
  // where HIP records them instead of running them
  hipStream_t capture_stream = nullptr;
  bool capturing = false;
  uint64_t captured_calls = 0;
  // telemetry
  std::shared_ptr<Telemetry> tel = std::make_shared<Telemetry>();
  std::atomic<uint64_t> submitted{0}, async_submitted{0}, waited{0}, wait_nanos{0};
};

struct si_hip_quant_weight {
  std::shared_ptr<Telemetry> tel;
  std::shared_ptr<DeviceBuffer> buffer;
  uint64_t offset = 0;
  uint64_t bytes = 0;
  uint32_t ggml_type = 0;
  bool mapped = false;
  bool owner = false;  // counts toward active weight bytes
  const uint8_t *data() const { return static_cast<const uint8_t *>(buffer->ptr) + offset; }
};

struct si_hip_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int device = 0;
  uint64_t calls = 0;  // device calls recorded
};

namespace {

int hip_fail(hipError_t e, const char *what) {
  return fail(SI_HIP_ERR_DEVICE, "HIP %s failed: %s", what, hipGetErrorString(e));
}

#define SIHIP_CHECK(expr, what)            \
  do {                                     \
    hipError_t _e = (expr);                \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

int grow(si_hip_context *ctx, void **buf, size_t *cap, size_t need) {
  if (need <= *cap) return SI_HIP_OK;
  size_t want = std::max(need, *cap * 2);
  if (*buf) {
    (void)hipFree(*buf);
    ctx->tel->note_free(*cap);
    *buf = nullptr;
    *cap = 0;
  }
  if (hipMalloc(buf, want) != hipSuccess) {
    *buf = nullptr;
    return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate %zu staging bytes", want);
  }
  *cap = want;
  ctx->tel->note_alloc(want);
  return SI_HIP_OK;
}

// ---- pinned staging of host inputs and outputs ---------------------------------
// Pageable host memory is copied through the runtime's own bounce buffers,
// several times slower than DMA from pinned memory: the synchronous calls
// copy their inputs into the context's pinned staging and read their outputs
// from it after the wait.  Large transfers go direct.
constexpr size_t kPinnedMaxCopy = size_t(16) << 20;

uint8_t *pin_take(si_hip_context *ctx, PinnedStage &st, size_t bytes) {
  const size_t chunk = (bytes + 255) & ~size_t(255);
  if (st.used + chunk > st.cap) {
    const size_t cap = std::max({st.used + chunk, 2 * st.cap, size_t(1) << 20});
    void *p = nullptr;
    if (hipHostMalloc(&p, cap, hipHostMallocDefault) != hipSuccess) return nullptr;
    // chunks already handed out in this call stay valid until its wait
    if (st.ptr) ctx->pin_retired.push_back(st.ptr);
    st.ptr = static_cast<uint8_t *>(p);
    st.cap = cap;
    st.used = 0;
  }
  uint8_t *r = st.ptr + st.used;
  st.used += chunk;
  return r;
}

hipError_t copy_in(si_hip_context *ctx, void *dev, const void *host, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  if (bytes <= kPinnedMaxCopy) {
    uint8_t *p = pin_take(ctx, ctx->pin_in, bytes);
    if (!p) return hipErrorOutOfMemory;
    std::memcpy(p, host, bytes);
    return hipMemcpyAsync(dev, p, bytes, hipMemcpyHostToDevice, ctx->stream);
  }
  return hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream);
}

hipError_t copy_out(si_hip_context *ctx, void *host, const void *dev, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  if (bytes <= kPinnedMaxCopy) {
    uint8_t *p = pin_take(ctx, ctx->pin_out, bytes);
    if (!p) return hipErrorOutOfMemory;
    ctx->pending.push_back({host, p, bytes});
    return hipMemcpyAsync(p, dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
  }
  return hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
}

// Where a synchronous call's kernel stores an output: a pinned region when
// the bytes fit there (the kernel's stores cross PCIe; the bytes reach the
// caller's buffer after the stream wait, with no copy back), else the
// device staging buffer, which `deliver` copies out.
struct OutStage {
  float *ptr;
  bool pinned;
};

OutStage out_stage(si_hip_context *ctx, size_t bytes) {
  if (bytes > 0 && bytes <= kPinnedMaxCopy)
    if (uint8_t *p = pin_take(ctx, ctx->pin_out, bytes)) return {reinterpret_cast<float *>(p), true};
  return {static_cast<float *>(ctx->stage_out), false};
}

// The `floats` values at o.ptr + off to the caller's buffer `host`.
hipError_t deliver(si_hip_context *ctx, void *host, const OutStage &o, size_t off, size_t floats) {
  if (!o.pinned) return copy_out(ctx, host, o.ptr + off, floats * sizeof(float));
  if (floats) ctx->pending.push_back({host, o.ptr + off, floats * sizeof(float)});
  return hipSuccess;
}

// After the stream has drained: outputs to the caller, staging reset.
void finish_staging(si_hip_context *ctx, bool deliver) {
  if (deliver)
    for (const PendingOut &o : ctx->pending) std::memcpy(o.dst, o.src, o.bytes);
  ctx->pending.clear();
  ctx->pin_in.used = ctx->pin_out.used = 0;
  for (void *p : ctx->pin_retired) (void)hipHostFree(p);
  ctx->pin_retired.clear();
}

// The context's lock for one call.  A synchronous call that returns before
// its wait (an error after some copies were enqueued) leaves staging in use:
// the scope then drains the stream and drops the undelivered outputs.
class CallScope {
 public:
  explicit CallScope(si_hip_context *ctx) : ctx_(ctx), lock_(ctx->mu) {}
  ~CallScope() {
    if (!ctx_->pending.empty() || ctx_->pin_in.used || ctx_->pin_out.used ||
        !ctx_->pin_retired.empty()) {
      (void)hipStreamSynchronize(ctx_->stream);
      finish_staging(ctx_, false);
    }
  }
  CallScope(const CallScope &) = delete;
  CallScope &operator=(const CallScope &) = delete;

 private:
  si_hip_context *ctx_;
  std::lock_guard<std::mutex> lock_;
};

// The workspace's rest state on the context's stream, waited for: counters
// zero, entries empty, then the reserved words (the error word's address and
// the test hook's poll count).
int reset_workspace(si_hip_context *ctx) {
  uint8_t *p = static_cast<uint8_t *>(ctx->ws.ptr);
  static_assert(sihip::kWorkspaceReportSlot + 8 == sihip::kWorkspaceGiveUpWord &&
                    sihip::kWorkspaceGiveUpWord + 4 == sihip::kWorkspaceArgmaxCounter,
                "reserved words in one 16-byte run");
  const uint32_t reserved[4] = {(uint32_t)ctx->dev_error_addr, (uint32_t)(ctx->dev_error_addr >> 32),
                                ctx->give_up_polls, 0u};
  SIHIP_CHECK(hipMemsetAsync(p, 0, sihip::kWorkspaceCounterBytes, ctx->stream), "workspace clear");
  SIHIP_CHECK(hipMemsetD32Async(p + sihip::kWorkspaceCounterBytes, (int)sihip::kWorkspaceEmpty,
                                (sihip::kWorkspaceBytes - sihip::kWorkspaceCounterBytes) / 4,
                                ctx->stream),
              "workspace clear");
  SIHIP_CHECK(hipMemcpyAsync(p + sihip::kWorkspaceReportSlot, reserved, sizeof reserved,
                             hipMemcpyHostToDevice, ctx->stream),
              "workspace clear");
  SIHIP_CHECK(hipStreamSynchronize(ctx->stream), "workspace clear");
  return SI_HIP_OK;
}

const char *device_error_text(uint32_t code) {
  switch (code) {
    case sihip::kDevErrSlotWait: return "a kernel gave up waiting for a tile's LDS slot";
    case sihip::kDevErrCombineWait: return "a kernel gave up waiting for a split tile's partial sums";
    case sihip::kDevErrArgmaxWait: return "a kernel gave up waiting for a workgroup's argmax candidate";
    case sihip::kDevErrTokenId: return "an embedding token id lies beyond the table";
    default: return "a kernel reported an unknown failure";
  }
}

// After the stream has drained: a failure a kernel reported since the last
// check fails the call (the work since then is not valid) and puts the
// workspace back into its rest state for the next commands.
int check_device_error(si_hip_context *ctx) {
  const uint32_t code = ctx->dev_error ? *ctx->dev_error : 0u;
  if (code == 0u) return SI_HIP_OK;
  *ctx->dev_error = 0u;
  int rc = reset_workspace(ctx);
  if (rc) return rc;
  return fail(SI_HIP_ERR_DEVICE, "%s (code %u); the device work since the last synchronisation "
              "is not valid", device_error_text(code), code);
}

int wait_stream(si_hip_context *ctx, const char *what) {
  ctx->submitted.fetch_add(1);
  const auto t0 = std::chrono::steady_clock::now();
  hipError_t e = hipStreamSynchronize(ctx->stream);
  const auto t1 = std::chrono::steady_clock::now();
  ctx->waited.fetch_add(1);
  ctx->wait_nanos.fetch_add(
      (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count());
  if (e != hipSuccess) {
    finish_staging(ctx, false);
    return fail(SI_HIP_ERR_DEVICE, "HIP %s failed: %s", what, hipGetErrorString(e));
  }
  finish_staging(ctx, true);
  return check_device_error(ctx);
}

// ---------------------------------------------------------------------------
// Kernel dispatch.
int dispatch_matvec(si_hip_context *ctx, uint32_t type, const uint8_t *w, const float *x,
                    float *y, uint32_t rows, uint32_t cols, uint32_t batch,
                    hipStream_t stream) {
  hipError_t e = hipErrorInvalidValue;
  bool done = false;
  if (ctx->policy == SI_HIP_KERNEL_AUTO) {
    done = sihip::launch_matvec_tuned(type, w, x, y, rows, cols, batch, ctx->ws, stream, &e);
  }
  if (!done) e = sihip::launch_matvec_generic(type, w, x, y, rows, cols, batch, stream);
  if (e != hipSuccess) return hip_fail(e, "matvec launch");
  return SI_HIP_OK;
}

// Several matvecs over one x into consecutive outputs (y of weight i at the
// sum of the earlier rows): one launch when a matrix-core kernel takes the
// group (2..8 matrices of one of Q4_K, Q5_K, Q6_K, rows of all but the last a
// multiple of 16), else one launch per matrix.
int dispatch_matvec_group(si_hip_context *ctx, const uint32_t *types, const uint8_t *const *w,
                          const size_t *rows, size_t count, const float *x, float *y,
                          uint32_t cols, hipStream_t stream) {
  if (ctx->policy == SI_HIP_KERNEL_AUTO && count >= 2 && count <= sihip::kMaxGroupWeights) {
    bool same = true;
    uint32_t r[sihip::kMaxGroupWeights];
    for (size_t i = 0; i < count; ++i) {
      same = same && types[i] == types[0];
      r[i] = (uint32_t)rows[i];
    }
    hipError_t e = hipErrorInvalidValue;
    if (same && sihip::launch_matvec_group(types[0], w, r, (uint32_t)count, cols, x, y, ctx->ws,
                                           stream, &e)) {
      if (e != hipSuccess) return hip_fail(e, "grouped matvec launch");
      return SI_HIP_OK;
    }
  }
  size_t off = 0;
  for (size_t i = 0; i < count; ++i) {
    int rc = dispatch_matvec(ctx, types[i], w[i], x, y + off, (uint32_t)rows[i], cols, 1, stream);
    if (rc) return rc;
    off += rows[i];
  }
  return SI_HIP_OK;
}

int dispatch_weight_group(si_hip_context *ctx, const si_hip_quant_weight *const *ws,
                          const size_t *rows, size_t count, const float *x, float *y,
                          uint32_t cols, hipStream_t stream) {
  std::vector<uint32_t> types(count);
  std::vector<const uint8_t *> w(count);
  for (size_t i = 0; i < count; ++i) {
    types[i] = ws[i]->ggml_type;
    w[i] = ws[i]->data();
  }
  return dispatch_matvec_group(ctx, types.data(), w.data(), rows, count, x, y, cols, stream);
}

int dispatch_gate_up(si_hip_context *ctx, const uint8_t *g, const uint8_t *u, const float *x,
                     float *h, uint32_t rows, uint32_t cols, hipStream_t stream) {
  hipError_t e = hipErrorInvalidValue;
  bool done = false;
  if (ctx->policy == SI_HIP_KERNEL_AUTO) {
    done = sihip::launch_fused_gate_up_tuned(g, u, x, h, rows, cols, ctx->ws, stream, &e);
  }
  if (!done) e = sihip::launch_fused_gate_up_generic(g, u, x, h, rows, cols, stream);
  if (e != hipSuccess) return hip_fail(e, "fused gate/up launch");
  return SI_HIP_OK;
}

// Stream of the device-resident calls: the capture stream while a graph is
// being recorded, else the compute stream.
hipStream_t device_stream(const si_hip_context *ctx) {
  return ctx->capturing ? ctx->capture_stream : ctx->stream;
}

// Validation shared by the byte-slice matvec entry points
// (quant_k_matvec_dispatch, metal.rs:3847-3858 and 3884-3887).
int validate_matvec(uint32_t type, size_t weight_len, size_t rows, size_t columns,
                    size_t input_len, const char *label) {
  if (rows == 0 || columns == 0 || columns % 256 != 0 || input_len != columns)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s matvec dimensions are invalid", label);
  size_t expected;
  int rc = expected_weight_bytes(rows, columns, block_bytes_of(type), label, &expected);
  if (rc) return rc;
  if (weight_len != expected) return fail(SI_HIP_ERR_BYTE_LENGTH, "%s matvec byte length is invalid", label);
  return check_u32(rows, columns, label);
}

int run_matvec_host(si_hip_context *ctx, uint32_t type, const uint8_t *dev_w, size_t rows,
                    size_t columns, size_t batch, const float *input, float *output,
                    const char *what) {
  const size_t in_bytes = batch * columns * sizeof(float);
  const size_t out_bytes = batch * rows * sizeof(float);
  int rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, in_bytes);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, out_bytes);
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, input, in_bytes),
              "input copy");
  const OutStage o = out_stage(ctx, out_bytes);
  rc = dispatch_matvec(ctx, type, dev_w, static_cast<const float *>(ctx->stage_in), o.ptr,
                       (uint32_t)rows, (uint32_t)columns, (uint32_t)batch, ctx->stream);
  if (rc) return rc;
  SIHIP_CHECK(deliver(ctx, output, o, 0, batch * rows), "output copy");
  rc = wait_stream(ctx, what);
  if (rc) return rc;
  return ok();
}

// ---- borrowed weight bytes ----------------------------------------------------
// Length and 64 evenly spread 64-byte windows, mixed (a change detector for
// resident ranges, not a content hash).
uint64_t fingerprint(const uint8_t *p, size_t len) {
  auto mix = [](uint64_t h) {
    h ^= h >> 33;
    h *= 0xff51afd7ed558ccdull;
    h ^= h >> 33;
    h *= 0xc4ceb9fe1a85ec53ull;
    return h ^ (h >> 33);
  };
  uint64_t h = mix(0x9e3779b97f4a7c15ull ^ len);
  constexpr size_t kWin = 64, kWindows = 64;
  if (len <= kWin * kWindows) {
    for (size_t i = 0; i < len; i += 8) {
      uint64_t v = 0;
      std::memcpy(&v, p + i, std::min<size_t>(8, len - i));
      h = mix(h ^ v);
    }
    return h;
  }
  for (size_t w = 0; w < kWindows; ++w) {
    const size_t off = (len - kWin) / (kWindows - 1) * w;
    for (size_t i = 0; i < kWin; i += 8) {
      uint64_t v;
      std::memcpy(&v, p + off + i, 8);
      h = mix(h ^ v);
    }
  }
  return h;
}

void evict_range(si_hip_context *ctx, std::map<std::pair<uintptr_t, size_t>, Resident>::iterator it) {
  ctx->res.bytes -= it->first.second;
  ctx->res.stats.evictions += 1;
  ctx->res.ranges.erase(it);  // the last reference frees the HBM copy
}

// HBM addresses of n borrowed host byte ranges for one call, enqueued on the
// context's stream: resident copies (copied again when changed), new ones
// under the budget, or -- residency off or the call's ranges over the budget
// -- one staging copy per call.
int borrow_weights(si_hip_context *ctx, size_t n, const uint8_t *const *ptrs, const size_t *lens,
                   const uint8_t **devs, bool keep = true) {
  Residency &R = ctx->res;
  uint64_t total = 0;
  for (size_t i = 0; i < n; ++i) total += lens[i];
  if (!keep || R.budget == 0 || total > R.budget) {
    size_t staged = 0;
    for (size_t i = 0; i < n; ++i) staged += (lens[i] + 255) & ~size_t(255);
    int rc = grow(ctx, &ctx->stage_weights, &ctx->stage_weights_bytes, staged);
    if (rc) return rc;
    size_t off = 0;
    for (size_t i = 0; i < n; ++i) {
      uint8_t *d = static_cast<uint8_t *>(ctx->stage_weights) + off;
      SIHIP_CHECK(hipMemcpyAsync(d, ptrs[i], lens[i], hipMemcpyHostToDevice, ctx->stream),
                  "weight copy");
      devs[i] = d;
      off += (lens[i] + 255) & ~size_t(255);
      R.stats.uploads += 1;
      R.stats.uploaded_bytes += lens[i];
    }
    return SI_HIP_OK;
  }
  const uint64_t now = ++R.tick;
  for (size_t i = 0; i < n; ++i) {
    const auto key = std::make_pair((uintptr_t)ptrs[i], lens[i]);
    const uint64_t fp = fingerprint(ptrs[i], lens[i]);
    auto it = R.ranges.find(key);
    if (it != R.ranges.end()) {
      Resident &r = it->second;
      r.used = now;
      if (r.fingerprint == fp) {
        R.stats.hits += 1;
      } else {
        SIHIP_CHECK(hipMemcpyAsync(r.buf->ptr, ptrs[i], lens[i], hipMemcpyHostToDevice, ctx->stream),
                    "weight copy");
        r.fingerprint = fp;
        R.stats.uploads += 1;
        R.stats.uploaded_bytes += lens[i];
      }
      devs[i] = static_cast<const uint8_t *>(r.buf->ptr);
      continue;
    }
    // room under the budget: the least recently used ranges this call does
    // not use (the call's own ranges fit: total <= budget)
    while (R.bytes + lens[i] > R.budget) {
      auto victim = R.ranges.end();
      for (auto j = R.ranges.begin(); j != R.ranges.end(); ++j)
        if (j->second.used != now && (victim == R.ranges.end() || j->second.used < victim->second.used))
          victim = j;
      if (victim == R.ranges.end()) break;
      evict_range(ctx, victim);
    }
    auto buf = std::make_shared<DeviceBuffer>();
    if (hipMalloc(&buf->ptr, lens[i]) != hipSuccess) {
      buf->ptr = nullptr;
      return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate %zu bytes for borrowed weights",
                  lens[i]);
    }
    buf->bytes = lens[i];
    buf->tel = ctx->tel;
    ctx->tel->note_alloc(lens[i]);
    SIHIP_CHECK(hipMemcpyAsync(buf->ptr, ptrs[i], lens[i], hipMemcpyHostToDevice, ctx->stream),
                "weight copy");
    devs[i] = static_cast<const uint8_t *>(buf->ptr);
    R.ranges.emplace(key, Resident{std::move(buf), fp, now});
    R.bytes += lens[i];
    R.stats.uploads += 1;
    R.stats.uploaded_bytes += lens[i];
  }
  return SI_HIP_OK;
}

// One borrowed range (keep = false: a per-call staging copy).
int stage_weights(si_hip_context *ctx, const uint8_t *bytes, size_t len, const uint8_t **dev,
                  bool keep = true) {
  return borrow_weights(ctx, 1, &bytes, &len, dev, keep);
}

int typed_matvec(si_hip_context *ctx, uint32_t type, const uint8_t *weight_bytes,
                 size_t weight_len, size_t rows, size_t columns, const float *input,
                 size_t input_len, float *output) {
  const char *label = type_label(type);
  int rc = validate_matvec(type, weight_len, rows, columns, input_len, label);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!weight_bytes || !input || !output) return fail(SI_HIP_ERR_NULL, "%s matvec buffer is null", label);
  CallScope scope(ctx);
  const uint8_t *dev_w = nullptr;
  rc = stage_weights(ctx, weight_bytes, weight_len, &dev_w);
  if (rc) return rc;
  char what[64];
  snprintf(what, sizeof what, "%s matvec command", label);
  return run_matvec_host(ctx, type, dev_w, rows, columns, 1, input, output, what);
}

int make_weight(si_hip_context *ctx, const uint8_t *bytes, size_t len, uint32_t type, bool mapped,
                si_hip_quant_weight **out) {
  if (!out) return fail(SI_HIP_ERR_NULL, "output handle pointer is null");
  *out = nullptr;
  if (len == 0 || block_bytes_of(type) == 0)
    return fail(len == 0 ? SI_HIP_ERR_EMPTY : SI_HIP_ERR_UNSUPPORTED_TYPE,
                mapped ? "unsupported or empty mapped quantized weight"
                       : "unsupported or empty quantized weight");
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!bytes) return fail(SI_HIP_ERR_NULL, "quantized weight bytes are null");
  auto buf = std::make_shared<DeviceBuffer>();
  if (hipMalloc(&buf->ptr, len) != hipSuccess) {
    buf->ptr = nullptr;
    return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate %zu weight bytes", len);
  }
  buf->bytes = len;
  buf->tel = ctx->tel;
  ctx->tel->note_alloc(len);
  hipError_t e = hipMemcpyAsync(buf->ptr, bytes, len, hipMemcpyHostToDevice, ctx->upload_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->upload_stream);
  ctx->submitted.fetch_add(1);
  ctx->waited.fetch_add(1);
  if (e != hipSuccess) return hip_fail(e, "quantized weight upload");
  auto *w = new si_hip_quant_weight;
  w->tel = ctx->tel;
  w->buffer = std::move(buf);
  w->bytes = len;
  w->ggml_type = type;
  w->mapped = mapped;
  w->owner = true;
  ctx->tel->note_active((int64_t)len);
  *out = w;
  return ok();
}

int check_weight(const si_hip_quant_weight *w, const char *what) {
  if (!w) return fail(SI_HIP_ERR_NULL, "%s weight handle is null", what);
  return SI_HIP_OK;
}

}  // namespace

// ===========================================================================
extern "C" {

const char *si_hip_last_error(void) { return g_last_error.c_str(); }

const char *si_hip_status_name(int s) {
  switch (s) {
    case SI_HIP_OK: return "SI_HIP_OK";
    case SI_HIP_ERR_NULL: return "SI_HIP_ERR_NULL";
    case SI_HIP_ERR_DIMENSIONS: return "SI_HIP_ERR_DIMENSIONS";
    case SI_HIP_ERR_BYTE_LENGTH: return "SI_HIP_ERR_BYTE_LENGTH";
    case SI_HIP_ERR_OVERFLOW: return "SI_HIP_ERR_OVERFLOW";
    case SI_HIP_ERR_UNSUPPORTED_TYPE: return "SI_HIP_ERR_UNSUPPORTED_TYPE";
    case SI_HIP_ERR_BATCH: return "SI_HIP_ERR_BATCH";
    case SI_HIP_ERR_RANGE: return "SI_HIP_ERR_RANGE";
    case SI_HIP_ERR_NO_FINITE: return "SI_HIP_ERR_NO_FINITE";
    case SI_HIP_ERR_DEVICE: return "SI_HIP_ERR_DEVICE";
    case SI_HIP_ERR_OUT_OF_MEMORY: return "SI_HIP_ERR_OUT_OF_MEMORY";
    case SI_HIP_ERR_EMPTY: return "SI_HIP_ERR_EMPTY";
    case SI_HIP_ERR_STATE: return "SI_HIP_ERR_STATE";
    default: return "SI_HIP_ERR_UNKNOWN";
  }
}

uint32_t si_hip_abi_version(void) { return SI_HIP_ABI_VERSION; }

int si_hip_context_new(int device_ordinal, si_hip_context **out) {
  if (!out) return fail(SI_HIP_ERR_NULL, "output context pointer is null");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) return fail(SI_HIP_ERR_DEVICE, "no HIP device is available");
  if (device_ordinal < 0 || device_ordinal >= count)
    return fail(SI_HIP_ERR_RANGE, "HIP device %d does not exist (%d visible)", device_ordinal, count);
  SIHIP_CHECK(hipSetDevice(device_ordinal), "set device");
  auto ctx = std::make_unique<si_hip_context>();
  ctx->device = device_ordinal;
  SIHIP_CHECK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "stream create");
  SIHIP_CHECK(hipStreamCreateWithFlags(&ctx->upload_stream, hipStreamNonBlocking), "stream create");
  for (auto &ev : ctx->events) SIHIP_CHECK(hipEventCreate(&ev), "event create");
  {
    void *p = nullptr;
    constexpr size_t total = sihip::kWorkspaceBytes + sihip::kWorkspaceScratchBytes;
    if (hipMalloc(&p, total) != hipSuccess)
      return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate the %zu-byte workspace",
                  total);
    ctx->ws.ptr = p;
    ctx->ws.bytes = sihip::kWorkspaceBytes;
    ctx->ws.scratch = reinterpret_cast<float *>(static_cast<uint8_t *>(p) + sihip::kWorkspaceBytes);
    ctx->ws.scratch_bytes = sihip::kWorkspaceScratchBytes;
    ctx->tel->note_alloc(total);
    void *word = nullptr, *word_dev = nullptr;
    if (hipHostMalloc(&word, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
      return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate the device error word");
    ctx->dev_error = static_cast<volatile uint32_t *>(word);
    *ctx->dev_error = 0u;
    SIHIP_CHECK(hipHostGetDevicePointer(&word_dev, word, 0), "error word mapping");
    ctx->dev_error_addr = (uint64_t)(uintptr_t)word_dev;
    // rest state, set on the context's own (non-blocking) stream before any
    // kernel
    int rc = reset_workspace(ctx.get());
    if (rc) return rc;
  }
  // the device's workspace of si_hip_quant_matvec_noalloc (no allocation;
  // done here so that callers of that entry point under graph capture find
  // it ready)
  int rc = sihip::noalloc_setup(ctx->stream);
  if (rc) return rc;
  *out = ctx.release();
  return ok();
}

void si_hip_context_free(si_hip_context *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (void *p : {ctx->stage_in, ctx->stage_out, ctx->stage_weights, ctx->stage_aux, ctx->ws.ptr})
    if (p) (void)hipFree(p);
  ctx->tel->note_free(ctx->stage_in_bytes + ctx->stage_out_bytes + ctx->stage_weights_bytes +
                      ctx->stage_aux_bytes + ctx->ws.bytes + ctx->ws.scratch_bytes);
  if (ctx->dev_error) (void)hipHostFree(const_cast<uint32_t *>(ctx->dev_error));
  finish_staging(ctx, false);
  for (PinnedStage *st : {&ctx->pin_in, &ctx->pin_out})
    if (st->ptr) (void)hipHostFree(st->ptr);
  ctx->res.ranges.clear();
  for (auto &ev : ctx->events)
    if (ev) (void)hipEventDestroy(ev);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  if (ctx->upload_stream) (void)hipStreamDestroy(ctx->upload_stream);
  if (ctx->capture_stream) {
    if (ctx->capturing) {
      hipGraph_t g = nullptr;
      if (hipStreamEndCapture(ctx->capture_stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    }
    (void)hipStreamDestroy(ctx->capture_stream);
  }
  delete ctx;
}

int si_hip_upload_quant_weight_private(si_hip_context *ctx, const uint8_t *weight_bytes,
                                       size_t weight_len, uint32_t ggml_type,
                                       si_hip_quant_weight **out) {
  return make_weight(ctx, weight_bytes, weight_len, ggml_type, false, out);
}

int si_hip_bind_quant_weight_mapped(si_hip_context *ctx, const uint8_t *weight_bytes,
                                    size_t weight_len, uint32_t ggml_type,
                                    si_hip_quant_weight **out) {
  return make_weight(ctx, weight_bytes, weight_len, ggml_type, true, out);
}

int si_hip_quant_weight_view(const si_hip_quant_weight *parent, uint64_t offset, uint64_t bytes,
                             uint32_t ggml_type, si_hip_quant_weight **out) {
  if (!out) return fail(SI_HIP_ERR_NULL, "output handle pointer is null");
  *out = nullptr;
  if (!parent) return fail(SI_HIP_ERR_NULL, "parent weight handle is null");
  if (block_bytes_of(ggml_type) == 0) return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported quantized view type");
  if (bytes == 0 || offset > parent->bytes || bytes > parent->bytes - offset)
    return fail(SI_HIP_ERR_RANGE, "quantized weight view [%llu, +%llu) is outside its parent",
                (unsigned long long)offset, (unsigned long long)bytes);
  auto *w = new si_hip_quant_weight;
  w->tel = parent->tel;
  w->buffer = parent->buffer;
  w->offset = parent->offset + offset;
  w->bytes = bytes;
  w->ggml_type = ggml_type;
  w->mapped = parent->mapped;
  w->owner = false;
  *out = w;
  return ok();
}

void si_hip_quant_weight_free(si_hip_quant_weight *w) {
  if (!w) return;
  if (w->owner && w->tel) w->tel->note_active(-(int64_t)w->bytes);
  delete w;
}

uint64_t si_hip_quant_weight_byte_len(const si_hip_quant_weight *w) { return w ? w->bytes : 0; }
uint32_t si_hip_quant_weight_ggml_type(const si_hip_quant_weight *w) { return w ? w->ggml_type : 0; }
int si_hip_quant_weight_is_mapped(const si_hip_quant_weight *w) { return w && w->mapped ? 1 : 0; }
const void *si_hip_quant_weight_device_ptr(const si_hip_quant_weight *w) { return w ? w->data() : nullptr; }

// ---- matvec ---------------------------------------------------------------
int si_hip_q4_k_matvec(si_hip_context *ctx, const uint8_t *wb, size_t wl, size_t rows, size_t cols,
                       const float *in, size_t in_len, float *out) {
  return typed_matvec(ctx, SI_HIP_GGML_TYPE_Q4_K, wb, wl, rows, cols, in, in_len, out);
}
int si_hip_q5_k_matvec(si_hip_context *ctx, const uint8_t *wb, size_t wl, size_t rows, size_t cols,
                       const float *in, size_t in_len, float *out) {
  return typed_matvec(ctx, SI_HIP_GGML_TYPE_Q5_K, wb, wl, rows, cols, in, in_len, out);
}
int si_hip_q6_k_matvec(si_hip_context *ctx, const uint8_t *wb, size_t wl, size_t rows, size_t cols,
                       const float *in, size_t in_len, float *out) {
  return typed_matvec(ctx, SI_HIP_GGML_TYPE_Q6_K, wb, wl, rows, cols, in, in_len, out);
}

int si_hip_gguf_quant_matvec_bytes(si_hip_context *ctx, uint32_t type, const uint8_t *wb, size_t wl,
                                   size_t rows, size_t cols, const float *in, size_t in_len,
                                   float *out) {
  if (block_bytes_of(type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported staged quantized weight type");
  return typed_matvec(ctx, type, wb, wl, rows, cols, in, in_len, out);
}

}  // extern "C"

int sihip::quant_matvec_tensor_range(si_hip_context *ctx, uint32_t type, const uint8_t *tensor,
                                     size_t tensor_len, size_t offset, size_t len, size_t rows,
                                     size_t cols, const float *in, size_t in_len, float *out) {
  if (block_bytes_of(type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported staged quantized weight type");
  const char *label = type_label(type);
  int rc = validate_matvec(type, len, rows, cols, in_len, label);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!tensor || !in || !out) return fail(SI_HIP_ERR_NULL, "%s matvec buffer is null", label);
  if (offset > tensor_len || len > tensor_len - offset)
    return fail(SI_HIP_ERR_RANGE, "%s row range is invalid", label);
  CallScope scope(ctx);
  const uint8_t *dev = nullptr;
  if (tensor_len <= ctx->res.budget) {
    rc = stage_weights(ctx, tensor, tensor_len, &dev);
    dev += offset;
  } else {
    rc = stage_weights(ctx, tensor + offset, len, &dev);
  }
  if (rc) return rc;
  char what[64];
  snprintf(what, sizeof what, "%s matvec command", label);
  return run_matvec_host(ctx, type, dev, rows, cols, 1, in, out, what);
}

extern "C" {

int si_hip_gguf_quant_matvec_view_rows(si_hip_context *ctx, const char *name, uint32_t type,
                                       const uint64_t *shape, uint32_t n_dims,
                                       const uint8_t *payload, size_t payload_len,
                                       size_t row_start, size_t row_count, const float *in,
                                       size_t in_len, float *out) {
  // gguf_quant_matvec_tensor_rows (metal.rs:4505-4527), then the checks of
  // q4_k_matvec_tensor_rows / quant_k_matvec_tensor_rows (4346-4467) in order
  if (block_bytes_of(type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "GGUF tensor %s has unsupported quantized type %u",
                name ? name : "", type);
  const char *label = type_label(type);
  if (n_dims != 2 || !shape)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "%s matvec requires a rank-2 %s tensor", label, label);
  const uint64_t cols = shape[0], rows = shape[1];
  if (row_count == 0 || row_start >= rows || row_count > rows - row_start)
    return fail(SI_HIP_ERR_RANGE, "%s row range is invalid", label);
  if (cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s tensor columns or input length is invalid", label);
  const size_t row_bytes = (size_t)cols / 256 * block_bytes_of(type);
  size_t start = 0, len = 0, end = 0;
  if (!checked_mul(row_start, row_bytes, &start))
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte range overflows", label);
  if (!checked_mul(row_count, row_bytes, &len))
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte length overflows", label);
  if (!checked_add(start, len, &end))
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte range overflows", label);
  if (end > payload_len)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "%s tensor payload is shorter than its shape", label);
  return sihip::quant_matvec_tensor_range(ctx, type, payload, payload_len, start, len, row_count,
                                          (size_t)cols, in, in_len, out);
}

int si_hip_gguf_quant_matvec_many_bytes(si_hip_context *ctx, const uint32_t *types,
                                        const uint8_t *const *bytes, const size_t *lens,
                                        const size_t *rows, const size_t *columns, size_t count,
                                        const float *in, size_t in_len, float *const *outputs) {
  // gguf_quant_matvec_many_bytes (metal.rs:4878-5001): the checks in its order
  if (count == 0)
    return fail(SI_HIP_ERR_EMPTY, "staged quantized matvec group requires at least one tensor");
  if (!types || !bytes || !lens || !rows || !columns || !outputs)
    return fail(SI_HIP_ERR_NULL, "staged grouped matvec arrays are null");
  const size_t cols = columns[0];
  if (cols == 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "staged quantized matvec group input length is invalid");
  for (size_t i = 0; i < count; ++i) {
    if (rows[i] == 0 || columns[i] != cols || cols % 256 != 0)
      return fail(SI_HIP_ERR_DIMENSIONS, "staged quantized matvec group shapes differ");
    const size_t bb = block_bytes_of(types[i]);
    if (bb == 0) return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported staged quantized tensor type");
    size_t expected;
    if (!checked_mul(rows[i], cols / 256, &expected) || !checked_mul(expected, bb, &expected))
      return fail(SI_HIP_ERR_OVERFLOW, "staged quantized matvec group byte length overflows");
    if (expected != lens[i])
      return fail(SI_HIP_ERR_BYTE_LENGTH, "staged quantized matvec tensor byte length is invalid");
  }
  if (cols > UINT32_MAX)
    return fail(SI_HIP_ERR_OVERFLOW, "staged grouped quantized columns exceed HIP limits");
  uint64_t total_rows = 0;
  for (size_t i = 0; i < count; ++i) {
    if (rows[i] > UINT32_MAX)
      return fail(SI_HIP_ERR_OVERFLOW, "staged grouped quantized rows exceed HIP limits");
    total_rows += rows[i];
  }
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in) return fail(SI_HIP_ERR_NULL, "staged grouped matvec input is null");
  for (size_t i = 0; i < count; ++i)
    if (!bytes[i] || !outputs[i])
      return fail(SI_HIP_ERR_NULL, "staged grouped matvec buffer %zu is null", i);
  CallScope scope(ctx);
  std::vector<const uint8_t *> dev(count);
  int rc = borrow_weights(ctx, count, bytes, lens, dev.data());
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, total_rows * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  const OutStage o = out_stage(ctx, total_rows * sizeof(float));
  rc = dispatch_matvec_group(ctx, types, dev.data(), rows, count,
                             static_cast<const float *>(ctx->stage_in), o.ptr, (uint32_t)cols,
                             ctx->stream);
  if (rc) return rc;
  size_t off = 0;
  for (size_t i = 0; i < count; ++i) {
    SIHIP_CHECK(deliver(ctx, outputs[i], o, off, rows[i]), "output copy");
    off += rows[i];
  }
  rc = wait_stream(ctx, "staged grouped quantized matvec command");
  if (rc) return rc;
  return ok();
}

int si_hip_gguf_quant_matvec_weight(si_hip_context *ctx, const si_hip_quant_weight *w, size_t rows,
                                    size_t cols, const float *in, size_t in_len, float *out) {
  int rc = check_weight(w, "retained matvec");
  if (rc) return rc;
  if (block_bytes_of(w->ggml_type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported retained quantized weight type");
  const char *label = type_label(w->ggml_type);
  if (rows == 0 || cols == 0 || cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s retained matvec dimensions are invalid", label);
  size_t expected;
  rc = expected_weight_bytes(rows, cols, block_bytes_of(w->ggml_type), label, &expected);
  if (rc) return rc;
  if ((uint64_t)expected != w->bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "%s retained matvec byte length is invalid", label);
  rc = check_u32(rows, cols, label);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in || !out) return fail(SI_HIP_ERR_NULL, "%s matvec buffer is null", label);
  CallScope scope(ctx);
  char what[64];
  snprintf(what, sizeof what, "%s retained matvec command", label);
  return run_matvec_host(ctx, w->ggml_type, w->data(), rows, cols, 1, in, out, what);
}

int si_hip_gguf_quant_matvec_tensor_rows(si_hip_context *ctx, const si_hip_quant_weight *t,
                                         size_t shape_cols, size_t shape_rows, size_t row_start,
                                         size_t row_count, const float *in, size_t in_len,
                                         float *out) {
  int rc = check_weight(t, "tensor");
  if (rc) return rc;
  if (block_bytes_of(t->ggml_type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "GGUF tensor has unsupported quantized type %u", t->ggml_type);
  const char *label = type_label(t->ggml_type);
  if (row_count == 0 || row_start >= shape_rows || row_count > shape_rows - row_start)
    return fail(SI_HIP_ERR_RANGE, "%s row range is invalid", label);
  if (shape_cols % 256 != 0 || in_len != shape_cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s tensor columns or input length is invalid", label);
  const size_t row_bytes = shape_cols / 256 * block_bytes_of(t->ggml_type);
  size_t byte_start, byte_len;
  if (!checked_mul(row_start, row_bytes, &byte_start))
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte range overflows", label);
  if (!checked_mul(row_count, row_bytes, &byte_len))
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte length overflows", label);
  if (byte_start > SIZE_MAX - byte_len)
    return fail(SI_HIP_ERR_OVERFLOW, "%s row byte range overflows", label);
  if (byte_start + byte_len > t->bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "%s tensor payload is shorter than its shape", label);
  rc = check_u32(row_count, shape_cols, label);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in || !out) return fail(SI_HIP_ERR_NULL, "%s matvec buffer is null", label);
  CallScope scope(ctx);
  char what[64];
  snprintf(what, sizeof what, "%s matvec command", label);
  return run_matvec_host(ctx, t->ggml_type, t->data() + byte_start, row_count, shape_cols, 1, in,
                         out, what);
}

int si_hip_gguf_quant_matvec_many_weights(si_hip_context *ctx,
                                          const si_hip_quant_weight *const *weights,
                                          const size_t *rows, size_t count, size_t cols,
                                          const float *in, size_t in_len, float *const *outputs) {
  if (!weights || !rows || !outputs) return fail(SI_HIP_ERR_NULL, "grouped matvec arrays are null");
  if (count == 0) return fail(SI_HIP_ERR_DIMENSIONS, "grouped quantized matvec needs at least one weight");
  if (cols == 0 || cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "grouped quantized matvec dimensions are invalid");
  size_t total_rows = 0;
  for (size_t i = 0; i < count; ++i) {
    int rc = check_weight(weights[i], "grouped matvec");
    if (rc) return rc;
    const uint32_t t = weights[i]->ggml_type;
    if (block_bytes_of(t) == 0)
      return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported grouped quantized weight type");
    if (rows[i] == 0) return fail(SI_HIP_ERR_DIMENSIONS, "grouped quantized matvec rows are invalid");
    size_t expected;
    rc = expected_weight_bytes(rows[i], cols, block_bytes_of(t), type_label(t), &expected);
    if (rc) return rc;
    if ((uint64_t)expected != weights[i]->bytes)
      return fail(SI_HIP_ERR_BYTE_LENGTH, "grouped %s matvec byte length is invalid", type_label(t));
    rc = check_u32(rows[i], cols, type_label(t));
    if (rc) return rc;
    if (!outputs[i]) return fail(SI_HIP_ERR_NULL, "grouped matvec output %zu is null", i);
    total_rows += rows[i];
  }
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in) return fail(SI_HIP_ERR_NULL, "grouped matvec input is null");
  CallScope scope(ctx);
  int rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, total_rows * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  const OutStage o = out_stage(ctx, total_rows * sizeof(float));
  rc = dispatch_weight_group(ctx, weights, rows, count, static_cast<const float *>(ctx->stage_in),
                             o.ptr, (uint32_t)cols, ctx->stream);
  if (rc) return rc;
  size_t off = 0;
  for (size_t i = 0; i < count; ++i) {
    SIHIP_CHECK(deliver(ctx, outputs[i], o, off, rows[i]), "output copy");
    off += rows[i];
  }
  rc = wait_stream(ctx, "grouped quantized matvec command");
  if (rc) return rc;
  return ok();
}

// ---- fused gate/up ----------------------------------------------------------
int si_hip_q4_k_fused_gate_up(si_hip_context *ctx, const uint8_t *gate, size_t gate_len,
                              const uint8_t *up, size_t up_len, size_t rows, size_t cols,
                              const float *in, size_t in_len, float *out) {
  if (rows == 0 || cols == 0 || cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "Q4_K fused gate/up dimensions are invalid");
  size_t blocks, expected;
  if (!checked_mul(rows, cols / 256, &blocks))
    return fail(SI_HIP_ERR_OVERFLOW, "Q4_K fused gate/up block count overflows");
  if (!checked_mul(blocks, 144, &expected))
    return fail(SI_HIP_ERR_OVERFLOW, "Q4_K fused gate/up byte length overflows");
  if (gate_len != expected || up_len != expected)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "Q4_K fused gate/up byte length is invalid");
  int rc = check_u32(rows, cols, "Q4_K fused gate/up");
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!gate || !up || !in || !out) return fail(SI_HIP_ERR_NULL, "Q4_K fused gate/up buffer is null");
  CallScope scope(ctx);
  const uint8_t *const borrowed[2] = {gate, up};
  const size_t blens[2] = {expected, expected};
  const uint8_t *dgu[2] = {nullptr, nullptr};
  rc = borrow_weights(ctx, 2, borrowed, blens, dgu);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, rows * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  const OutStage o = out_stage(ctx, rows * sizeof(float));
  rc = dispatch_gate_up(ctx, dgu[0], dgu[1], static_cast<const float *>(ctx->stage_in), o.ptr,
                        (uint32_t)rows, (uint32_t)cols, ctx->stream);
  if (rc) return rc;
  SIHIP_CHECK(deliver(ctx, out, o, 0, rows), "output copy");
  rc = wait_stream(ctx, "Q4_K fused gate/up command");
  if (rc) return rc;
  return ok();
}

namespace {
int validate_gate_up_weights(const si_hip_quant_weight *g, const si_hip_quant_weight *u, size_t rows,
                             size_t cols, size_t in_len, const char *invalid, const char *overflow,
                             const char *bad_len) {
  if (!g || !u) return fail(SI_HIP_ERR_NULL, "gate/up weight handle is null");
  if (g->ggml_type != SI_HIP_GGML_TYPE_Q4_K || u->ggml_type != SI_HIP_GGML_TYPE_Q4_K ||
      g->bytes != u->bytes || rows == 0 || cols == 0 || cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s", invalid);
  size_t blocks, expected;
  if (!checked_mul(rows, cols / 256, &blocks) || !checked_mul(blocks, 144, &expected))
    return fail(SI_HIP_ERR_OVERFLOW, "%s", overflow);
  if (g->bytes != (uint64_t)expected) return fail(SI_HIP_ERR_BYTE_LENGTH, "%s", bad_len);
  return check_u32(rows, cols, "Q4_K fused gate/up");
}
}  // namespace

int si_hip_q4_k_fused_gate_up_weights(si_hip_context *ctx, const si_hip_quant_weight *g,
                                      const si_hip_quant_weight *u, size_t rows, size_t cols,
                                      const float *in, size_t in_len, float *out) {
  int rc = validate_gate_up_weights(g, u, rows, cols, in_len,
                                    "retained Q4_K fused gate/up dimensions are invalid",
                                    "retained Q4_K fused gate/up byte length overflows",
                                    "retained Q4_K fused gate/up byte length is invalid");
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in || !out) return fail(SI_HIP_ERR_NULL, "Q4_K fused gate/up buffer is null");
  CallScope scope(ctx);
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, rows * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  const OutStage o = out_stage(ctx, rows * sizeof(float));
  rc = dispatch_gate_up(ctx, g->data(), u->data(), static_cast<const float *>(ctx->stage_in), o.ptr,
                        (uint32_t)rows, (uint32_t)cols, ctx->stream);
  if (rc) return rc;
  SIHIP_CHECK(deliver(ctx, out, o, 0, rows), "output copy");
  rc = wait_stream(ctx, "retained Q4_K fused gate/up command");
  if (rc) return rc;
  return ok();
}

namespace {
int validate_mlp(const si_hip_quant_weight *g, const si_hip_quant_weight *u,
                 const si_hip_quant_weight *d, size_t gate_rows, size_t cols, size_t down_rows,
                 size_t in_len) {
  if (!g || !u || !d) return fail(SI_HIP_ERR_NULL, "fused MLP weight handle is null");
  if (g->ggml_type != SI_HIP_GGML_TYPE_Q4_K || u->ggml_type != SI_HIP_GGML_TYPE_Q4_K ||
      g->bytes != u->bytes || gate_rows == 0 || cols == 0 || down_rows == 0 || cols % 256 != 0 ||
      in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "fused quantized MLP dimensions are invalid");
  size_t blocks, gate_bytes;
  if (!checked_mul(gate_rows, cols / 256, &blocks) || !checked_mul(blocks, 144, &gate_bytes))
    return fail(SI_HIP_ERR_OVERFLOW, "fused quantized MLP gate byte length overflows");
  if (g->bytes != (uint64_t)gate_bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "fused quantized MLP gate byte length is invalid");
  const size_t down_block = block_bytes_of(d->ggml_type);
  if (down_block == 0) return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported fused quantized MLP down type");
  if (gate_rows % 256 != 0)
    return fail(SI_HIP_ERR_DIMENSIONS, "fused quantized MLP down columns are invalid");
  size_t down_bytes;
  if (!checked_mul(down_rows, gate_rows / 256, &blocks) || !checked_mul(blocks, down_block, &down_bytes))
    return fail(SI_HIP_ERR_OVERFLOW, "fused quantized MLP down byte length overflows");
  if (d->bytes != (uint64_t)down_bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "fused quantized MLP down byte length is invalid");
  int rc = check_u32(gate_rows, cols, "fused quantized MLP");
  if (rc) return rc;
  return check_u32(down_rows, gate_rows, "fused quantized MLP");
}
}  // namespace

int si_hip_gguf_quant_fused_mlp_weights(si_hip_context *ctx, const si_hip_quant_weight *g,
                                        const si_hip_quant_weight *u, const si_hip_quant_weight *d,
                                        size_t gate_rows, size_t cols, size_t down_rows,
                                        const float *in, size_t in_len, float *out) {
  int rc = validate_mlp(g, u, d, gate_rows, cols, down_rows, in_len);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in || !out) return fail(SI_HIP_ERR_NULL, "fused MLP buffer is null");
  CallScope scope(ctx);
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_aux, &ctx->stage_aux_bytes, gate_rows * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, down_rows * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  float *hidden = static_cast<float *>(ctx->stage_aux);
  rc = dispatch_gate_up(ctx, g->data(), u->data(), static_cast<const float *>(ctx->stage_in), hidden,
                        (uint32_t)gate_rows, (uint32_t)cols, ctx->stream);
  if (rc) return rc;
  const OutStage o = out_stage(ctx, down_rows * sizeof(float));
  rc = dispatch_matvec(ctx, d->ggml_type, d->data(), hidden, o.ptr, (uint32_t)down_rows,
                       (uint32_t)gate_rows, 1, ctx->stream);
  if (rc) return rc;
  SIHIP_CHECK(deliver(ctx, out, o, 0, down_rows), "output copy");
  char what[64];
  snprintf(what, sizeof what, "fused MLP %s command", type_label(d->ggml_type));
  rc = wait_stream(ctx, what);
  if (rc) return rc;
  return ok();
}

// ---- embedding --------------------------------------------------------------
int si_hip_q4_k_embedding_row(si_hip_context *ctx, const uint8_t *row, size_t row_len, size_t cols,
                              float *out) {
  if (cols == 0 || cols % 256 != 0) return fail(SI_HIP_ERR_DIMENSIONS, "Q4_K embedding dimension is invalid");
  if (row_len != cols / 256 * 144) return fail(SI_HIP_ERR_BYTE_LENGTH, "Q4_K embedding row byte length is invalid");
  if (cols > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "embedding dimension exceeds HIP limits");
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!row || !out) return fail(SI_HIP_ERR_NULL, "Q4_K embedding buffer is null");
  CallScope scope(ctx);
  const uint8_t *dev = nullptr;
  int rc = stage_weights(ctx, row, row_len, &dev, false);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, cols * sizeof(float));
  if (rc) return rc;
  const OutStage o = out_stage(ctx, cols * sizeof(float));
  hipError_t e = sihip::launch_dequant(SI_HIP_GGML_TYPE_Q4_K, dev, nullptr, o.ptr, 1, (uint32_t)cols,
                                       ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "embedding launch");
  SIHIP_CHECK(deliver(ctx, out, o, 0, cols), "output copy");
  rc = wait_stream(ctx, "Q4_K embedding command");
  if (rc) return rc;
  return ok();
}

namespace {
// q4_k_embedding_tensor's checks (src/metal.rs:3785-3810) in its order: the
// tensor type, the token id and the dimension, the row's start and end
// offsets, then that row alone against the payload (a table shorter than its
// shape still serves the rows it holds); q4_k_embedding_row's dimension check
// (metal.rs:3735-3737) and the u32 launch limit follow.
int validate_embedding_row(const si_hip_quant_weight *t, size_t cols, size_t rows, size_t id) {
  if (!t) return fail(SI_HIP_ERR_NULL, "embedding table handle is null");
  if (t->ggml_type != SI_HIP_GGML_TYPE_Q4_K)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "Q4_K embedding requires a rank-2 Q4_K tensor");
  if (id >= rows || cols % 256 != 0)
    return fail(SI_HIP_ERR_RANGE, "Q4_K embedding token id or dimension is invalid");
  const size_t row_bytes = cols / 256 * 144;
  size_t start = 0, end = 0;
  if (!checked_mul(id, row_bytes, &start)) return fail(SI_HIP_ERR_OVERFLOW, "Q4_K embedding row offset overflows");
  if (!checked_add(start, row_bytes, &end)) return fail(SI_HIP_ERR_OVERFLOW, "Q4_K embedding row end overflows");
  if (end > t->bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "Q4_K embedding tensor payload is shorter than its shape");
  if (cols == 0) return fail(SI_HIP_ERR_DIMENSIONS, "Q4_K embedding dimension is invalid");
  if (cols > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "embedding dimension exceeds HIP limits");
  return SI_HIP_OK;
}

// The rows of the table a kernel may read: those of its shape that its
// payload holds whole.
uint32_t embedding_table_rows(const si_hip_quant_weight *t, size_t cols, size_t rows) {
  const size_t held = t->bytes / (cols / 256 * 144);
  return (uint32_t)std::min<size_t>({rows, held, (size_t)UINT32_MAX});
}
}  // namespace

int si_hip_q4_k_embedding_tokens(si_hip_context *ctx, const si_hip_quant_weight *t, size_t cols,
                                 size_t rows, const uint32_t *ids, size_t n, float *out) {
  if (n == 0) return fail(SI_HIP_ERR_DIMENSIONS, "Q4_K embedding needs at least one token id");
  if (!ids) return fail(SI_HIP_ERR_NULL, "token id buffer is null");
  for (size_t i = 0; i < n; ++i) {
    int rc = validate_embedding_row(t, cols, rows, ids[i]);
    if (rc) return rc;
  }
  if (n > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "too many token ids");
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!out) return fail(SI_HIP_ERR_NULL, "Q4_K embedding output is null");
  CallScope scope(ctx);
  int rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, n * sizeof(uint32_t));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, n * cols * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, ids, n * sizeof(uint32_t)),
              "token id copy");
  const OutStage o = out_stage(ctx, n * cols * sizeof(float));
  hipError_t e = sihip::launch_dequant(SI_HIP_GGML_TYPE_Q4_K, t->data(),
                                       static_cast<const uint32_t *>(ctx->stage_in), o.ptr,
                                       (uint32_t)n, (uint32_t)cols, ctx->stream,
                                       embedding_table_rows(t, cols, rows), ctx->ws.ptr);
  if (e != hipSuccess) return hip_fail(e, "embedding launch");
  SIHIP_CHECK(deliver(ctx, out, o, 0, n * cols), "output copy");
  rc = wait_stream(ctx, "Q4_K embedding command");
  if (rc) return rc;
  return ok();
}

int si_hip_q4_k_embedding_view(si_hip_context *ctx, uint32_t type, const uint64_t *shape,
                               uint32_t n_dims, const uint8_t *payload, size_t payload_len,
                               size_t token_id, float *out) {
  // q4_k_embedding_tensor (metal.rs:3785-3810) in its order, then
  // q4_k_embedding_row's checks (3734-3741)
  if (type != SI_HIP_GGML_TYPE_Q4_K || n_dims != 2 || !shape)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "Q4_K embedding requires a rank-2 Q4_K tensor");
  const uint64_t cols = shape[0], rows = shape[1];
  if (token_id >= rows || cols % 256 != 0)
    return fail(SI_HIP_ERR_RANGE, "Q4_K embedding token id or dimension is invalid");
  const size_t row_bytes = (size_t)cols / 256 * 144;
  size_t start = 0, end = 0;
  if (!checked_mul(token_id, row_bytes, &start))
    return fail(SI_HIP_ERR_OVERFLOW, "Q4_K embedding row offset overflows");
  if (!checked_add(start, row_bytes, &end)) return fail(SI_HIP_ERR_OVERFLOW, "Q4_K embedding row end overflows");
  if (end > payload_len)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "Q4_K embedding tensor payload is shorter than its shape");
  if (cols == 0) return fail(SI_HIP_ERR_DIMENSIONS, "Q4_K embedding dimension is invalid");
  if (cols > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "embedding dimension exceeds HIP limits");
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!payload || !out) return fail(SI_HIP_ERR_NULL, "Q4_K embedding buffer is null");
  CallScope scope(ctx);
  // the whole table stays resident when it fits the budget (later lookups
  // copy nothing); otherwise the row alone is copied
  const bool whole = payload_len <= ctx->res.budget;
  const uint8_t *dev = nullptr;
  int rc = whole ? stage_weights(ctx, payload, payload_len, &dev)
                 : stage_weights(ctx, payload + start, row_bytes, &dev, false);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, (size_t)cols * sizeof(float));
  if (rc) return rc;
  const OutStage o = out_stage(ctx, (size_t)cols * sizeof(float));
  hipError_t e = sihip::launch_dequant(SI_HIP_GGML_TYPE_Q4_K, whole ? dev + start : dev, nullptr,
                                       o.ptr, 1, (uint32_t)cols, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "embedding launch");
  SIHIP_CHECK(deliver(ctx, out, o, 0, cols), "output copy");
  rc = wait_stream(ctx, "Q4_K embedding command");
  if (rc) return rc;
  return ok();
}

int si_hip_q4_k_embedding_tensor(si_hip_context *ctx, const si_hip_quant_weight *t, size_t cols,
                                 size_t rows, size_t token_id, float *out) {
  int rc = validate_embedding_row(t, cols, rows, token_id);
  if (rc) return rc;
  const uint32_t id = (uint32_t)token_id;
  return si_hip_q4_k_embedding_tokens(ctx, t, cols, rows, &id, 1, out);
}

// ---- matmul many ----------------------------------------------------------
namespace {
int validate_many(uint32_t type, size_t weight_len, size_t rows, size_t cols, size_t batch,
                  size_t inputs_len, bool retained) {
  if (batch == 0 || batch > SI_HIP_MAX_BATCH || rows == 0 || cols == 0 || cols % 256 != 0)
    return fail(batch == 0 || batch > SI_HIP_MAX_BATCH ? SI_HIP_ERR_BATCH : SI_HIP_ERR_DIMENSIONS,
                retained ? "batched retained quantized dimensions are invalid"
                         : "batched quantized matvec dimensions are invalid");
  size_t want;
  if (!checked_mul(batch, cols, &want) || inputs_len != want)
    return fail(SI_HIP_ERR_DIMENSIONS, retained ? "batched retained quantized input length is invalid"
                                                : "batched quantized input length is invalid");
  const size_t bb = block_bytes_of(type);
  if (bb == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, retained ? "unsupported retained batched quantized type"
                                                      : "unsupported batched quantized weight type");
  size_t blocks, expected;
  if (!checked_mul(rows, cols / 256, &blocks) || !checked_mul(blocks, bb, &expected))
    return fail(SI_HIP_ERR_OVERFLOW, retained ? "retained batched weight byte length overflows"
                                              : "batched quantized weight byte length overflows");
  if (weight_len != expected)
    return fail(SI_HIP_ERR_BYTE_LENGTH, retained ? "retained batched weight byte length is invalid"
                                                 : "batched quantized weight byte length is invalid");
  size_t out_elems;
  if (!checked_mul(batch, rows, &out_elems))
    return fail(SI_HIP_ERR_OVERFLOW, "batched quantized output dimensions overflow");
  return check_u32(rows, cols, "batched");
}
}  // namespace

int si_hip_gguf_quant_matmul_many_bytes(si_hip_context *ctx, uint32_t type, const uint8_t *wb,
                                        size_t wl, size_t rows, size_t cols, size_t batch,
                                        const float *inputs, size_t inputs_len, float *outputs) {
  int rc = validate_many(type, wl, rows, cols, batch, inputs_len, false);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!wb || !inputs || !outputs) return fail(SI_HIP_ERR_NULL, "batched matvec buffer is null");
  CallScope scope(ctx);
  const uint8_t *dev_w = nullptr;
  rc = stage_weights(ctx, wb, wl, &dev_w);
  if (rc) return rc;
  return run_matvec_host(ctx, type, dev_w, rows, cols, batch, inputs, outputs,
                         "batched quantized matvec command");
}

int si_hip_gguf_quant_matmul_many_weight(si_hip_context *ctx, const si_hip_quant_weight *w,
                                         size_t rows, size_t cols, size_t batch,
                                         const float *inputs, size_t inputs_len, float *outputs) {
  int rc = check_weight(w, "batched");
  if (rc) return rc;
  rc = validate_many(w->ggml_type, (size_t)w->bytes, rows, cols, batch, inputs_len, true);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!inputs || !outputs) return fail(SI_HIP_ERR_NULL, "batched matvec buffer is null");
  CallScope scope(ctx);
  return run_matvec_host(ctx, w->ggml_type, w->data(), rows, cols, batch, inputs, outputs,
                         "retained batched quantized matvec command");
}

// ---- head + argmax ------------------------------------------------------------
namespace {
int validate_head(const si_hip_quant_weight *w, size_t rows, size_t cols, size_t in_len, uint32_t rule) {
  int rc = check_weight(w, "output head");
  if (rc) return rc;
  if (block_bytes_of(w->ggml_type) == 0)
    return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported output head quantized type");
  const char *label = type_label(w->ggml_type);
  if (rows == 0 || cols == 0 || cols % 256 != 0 || in_len != cols)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s output head dimensions are invalid", label);
  size_t expected;
  rc = expected_weight_bytes(rows, cols, block_bytes_of(w->ggml_type), label, &expected);
  if (rc) return rc;
  if ((uint64_t)expected != w->bytes)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "%s output head byte length is invalid", label);
  if (rule != SI_HIP_ARGMAX_LAST_FINITE && rule != SI_HIP_ARGMAX_FIRST_GREATER)
    return fail(SI_HIP_ERR_RANGE, "unknown argmax tie rule %u", rule);
  if (rows >= sihip::kArgmaxMaxRows)
    return fail(SI_HIP_ERR_OVERFLOW, "%s output head rows exceed the argmax's %u", label,
                (unsigned)sihip::kArgmaxMaxRows);
  return check_u32(rows, cols, label);
}
// The head's logits and greedy argmax on `stream`: the Q6_K matrix-core
// kernel with the argmax fused into it (storing the logits only when
// `logits_wanted`), else the matvec into d_logits, then the argmax kernel.
// The fused launch stores the logits (when wanted) at fused_logits, which
// may be pinned host staging (that kernel never reads them back), and sets
// *fused; the matvec + argmax_kernel pair stores them at d_logits (device
// memory, which argmax_kernel reads).
int dispatch_head(si_hip_context *ctx, const si_hip_quant_weight *w, const float *d_in,
                  float *d_logits, float *fused_logits, bool logits_wanted, uint32_t rows,
                  uint32_t cols, uint32_t rule, uint64_t *d_result, hipStream_t stream,
                  bool *fused) {
  hipError_t e = hipErrorInvalidValue;
  *fused = false;
  if (ctx->policy == SI_HIP_KERNEL_AUTO && w->ggml_type == SI_HIP_GGML_TYPE_Q6_K &&
      sihip::launch_q6k_matvec_argmax_mfma(w->data(), d_in, logits_wanted ? fused_logits : nullptr,
                                           rows, cols, rule, d_result, ctx->ws, stream, &e)) {
    if (e != hipSuccess) return hip_fail(e, "output head launch");
    *fused = true;
    return SI_HIP_OK;
  }
  int rc = dispatch_matvec(ctx, w->ggml_type, w->data(), d_in, d_logits, rows, cols, 1, stream);
  if (rc) return rc;
  e = sihip::launch_argmax(d_logits, rows, rule, ctx->ws, d_result, stream);
  if (e != hipSuccess) return hip_fail(e, "argmax launch");
  return SI_HIP_OK;
}
}  // namespace

int si_hip_gguf_quant_matvec_argmax_weight(si_hip_context *ctx, const si_hip_quant_weight *w,
                                           size_t rows, size_t cols, const float *in, size_t in_len,
                                           uint32_t rule, uint32_t *token, float *logits) {
  int rc = validate_head(w, rows, cols, in_len, rule);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!in || !token) return fail(SI_HIP_ERR_NULL, "output head buffer is null");
  CallScope scope(ctx);
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, rows * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_aux, &ctx->stage_aux_bytes, sizeof(uint64_t));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, in, cols * sizeof(float)),
              "input copy");
  float *d_logits = static_cast<float *>(ctx->stage_out);
  // the packed token (a plain store of the reducing wave) and a fused
  // launch's logits go straight into pinned staging when they fit there
  const OutStage lo = logits ? out_stage(ctx, rows * sizeof(float)) : OutStage{d_logits, false};
  uint8_t *pinned_token = pin_take(ctx, ctx->pin_out, sizeof(uint64_t));
  uint64_t *aux = pinned_token ? reinterpret_cast<uint64_t *>(pinned_token)
                               : static_cast<uint64_t *>(ctx->stage_aux);
  bool fused = false;
  rc = dispatch_head(ctx, w, static_cast<const float *>(ctx->stage_in), d_logits, lo.ptr,
                     logits != nullptr, (uint32_t)rows, (uint32_t)cols, rule, aux, ctx->stream,
                     &fused);
  if (rc) return rc;
  uint64_t packed = 0;
  if (pinned_token)
    ctx->pending.push_back({&packed, pinned_token, sizeof packed});
  else
    SIHIP_CHECK(copy_out(ctx, &packed, aux, sizeof packed), "argmax copy");
  if (logits) {
    if (fused)
      SIHIP_CHECK(deliver(ctx, logits, lo, 0, rows), "logits copy");
    else
      SIHIP_CHECK(copy_out(ctx, logits, d_logits, rows * sizeof(float)), "logits copy");
  }
  rc = wait_stream(ctx, "output head argmax command");
  if (rc) return rc;
  if (packed == 0) {
    if (rule == SI_HIP_ARGMAX_LAST_FINITE) return fail(SI_HIP_ERR_NO_FINITE, "logits contain no finite values");
    *token = 0;
  } else {
    *token = sihip::argmax_candidate_index(packed, rule);
  }
  return ok();
}

// ---- F32 matvec and RMSNorm (metal.rs:2641-3110) ---------------------------------
namespace {
// f32_matvec's checks (metal.rs:2983-2998), then the launch limits.
int validate_f32_matvec(size_t values, size_t rows, size_t cols, size_t input_len) {
  size_t expected;
  if (!checked_mul(rows, cols, &expected)) return fail(SI_HIP_ERR_OVERFLOW, "F32 matvec dimensions overflow");
  if (rows == 0 || cols == 0 || input_len != cols || values != expected)
    return fail(SI_HIP_ERR_DIMENSIONS, "F32 matvec dimensions or byte length are invalid");
  if (cols > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "F32 matvec columns exceed HIP limits");
  if (rows > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "F32 matvec rows exceed HIP limits");
  return SI_HIP_OK;
}

// Copies of the weights and x in, y out, one wait (the reference's command
// buffer with commit_and_wait).
int run_f32_matvec_host(si_hip_context *ctx, const float *w, size_t rows, size_t cols,
                        const float *x, float *y) {
  const size_t wb = rows * cols * sizeof(float);
  const size_t xb = cols * sizeof(float), yb = rows * sizeof(float);
  const uint8_t *dw = nullptr;
  int rc = stage_weights(ctx, reinterpret_cast<const uint8_t *>(w), wb, &dw);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, xb);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, yb);
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, x, xb), "input copy");
  const OutStage o = out_stage(ctx, yb);
  hipError_t e = sihip::launch_f32_matvec(reinterpret_cast<const float *>(dw),
                                          static_cast<const float *>(ctx->stage_in), o.ptr,
                                          (uint32_t)rows, (uint32_t)cols, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "F32 matvec launch");
  SIHIP_CHECK(deliver(ctx, y, o, 0, rows), "output copy");
  rc = wait_stream(ctx, "F32 matvec command");
  if (rc) return rc;
  return ok();
}

// rms_norm / rms_norm_heads / rms_norm_gated's checks (metal.rs:2648-2650,
// 2864-2875, 2782-2794).
int validate_rms(uint32_t mode, size_t x_len, size_t gate_len, size_t w_len, size_t heads,
                 size_t head_dim, float eps) {
  if (mode == 0) {
    if (x_len == 0 || x_len != w_len)
      return fail(SI_HIP_ERR_DIMENSIONS, "RMSNorm input and weight must have equal non-zero length");
  } else {
    const char *label = mode == 1 ? "head RMSNorm" : "Gated RMSNorm";
    size_t n;
    if (!checked_mul(heads, head_dim, &n)) return fail(SI_HIP_ERR_OVERFLOW, "%s dimensions overflow", label);
    if (heads == 0 || head_dim == 0 || !std::isfinite(eps) || eps <= 0.0f || x_len != n ||
        (mode == 2 && gate_len != n) || w_len != head_dim)
      return fail(SI_HIP_ERR_DIMENSIONS, "%s dimensions are invalid", label);
  }
  if (heads > UINT32_MAX || head_dim > UINT32_MAX)
    return fail(SI_HIP_ERR_OVERFLOW, "RMSNorm dimensions exceed HIP limits");
  return SI_HIP_OK;
}

int run_rms_host(si_hip_context *ctx, uint32_t mode, const float *x, const float *gate,
                 const float *w, size_t heads, size_t head_dim, float eps, float *y) {
  const size_t n = heads * head_dim, xb = n * sizeof(float), wb = head_dim * sizeof(float);
  // staging: x (and the gate after it) in, the weight in aux, y out
  int rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, mode == 2 ? 2 * xb : xb);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_aux, &ctx->stage_aux_bytes, wb);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, xb);
  if (rc) return rc;
  float *dx = static_cast<float *>(ctx->stage_in);
  float *dg = mode == 2 ? dx + n : nullptr;
  SIHIP_CHECK(copy_in(ctx, dx, x, xb), "input copy");
  if (dg) SIHIP_CHECK(copy_in(ctx, dg, gate, xb), "gate copy");
  SIHIP_CHECK(hipMemcpyAsync(ctx->stage_aux, w, wb, hipMemcpyHostToDevice, ctx->stream), "weight copy");
  const OutStage o = out_stage(ctx, xb);
  hipError_t e = sihip::launch_rms_norm(mode, dx, dg, static_cast<const float *>(ctx->stage_aux),
                                        o.ptr, (uint32_t)heads, (uint32_t)head_dim, eps, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "RMSNorm launch");
  SIHIP_CHECK(deliver(ctx, y, o, 0, n), "output copy");
  rc = wait_stream(ctx, "RMSNorm command");
  if (rc) return rc;
  return ok();
}
}  // namespace

int si_hip_f32_matvec(si_hip_context *ctx, const float *w, size_t values, size_t rows, size_t cols,
                      const float *x, size_t x_len, float *y) {
  int rc = validate_f32_matvec(values, rows, cols, x_len);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!w || !x || !y) return fail(SI_HIP_ERR_NULL, "F32 matvec buffer is null");
  CallScope scope(ctx);
  return run_f32_matvec_host(ctx, w, rows, cols, x, y);
}

int si_hip_f32_matvec_bytes(si_hip_context *ctx, const uint8_t *bytes, size_t len, size_t rows,
                            size_t cols, const float *x, size_t x_len, float *y) {
  // f32_matvec_bytes (metal.rs:3051-3072)
  size_t expected;
  if (!checked_mul(rows, cols, &expected) || !checked_mul(expected, sizeof(float), &expected))
    return fail(SI_HIP_ERR_OVERFLOW, "F32 matvec byte length overflows");
  if (len != expected) return fail(SI_HIP_ERR_BYTE_LENGTH, "F32 matvec byte length is invalid");
  if (reinterpret_cast<uintptr_t>(bytes) % alignof(float) != 0)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "F32 matvec bytes are not 4-byte aligned");
  return si_hip_f32_matvec(ctx, reinterpret_cast<const float *>(bytes), len / sizeof(float), rows,
                           cols, x, x_len, y);
}

int si_hip_f32_matvec_device(si_hip_context *ctx, const float *d_w, size_t rows, size_t cols,
                             const float *d_x, float *d_y) {
  int rc = validate_f32_matvec(rows * cols, rows, cols, cols);
  if (rc) return rc;
  if (!ctx || !d_w || !d_x || !d_y) return fail(SI_HIP_ERR_NULL, "device F32 matvec argument is null");
  CallScope scope(ctx);
  hipError_t e = sihip::launch_f32_matvec(d_w, d_x, d_y, (uint32_t)rows, (uint32_t)cols,
                                          device_stream(ctx));
  if (e != hipSuccess) return hip_fail(e, "F32 matvec launch");
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_f32_matvec_many(si_hip_context *ctx, const float *const *ws, const size_t *rows,
                           size_t count, size_t cols, const float *x, size_t x_len,
                           float *const *ys) {
  // one submission for a group of F32 matvecs sharing x (the command buffer of
  // f32_matvec_many_gguf_tensors, metal.rs:4780-4870)
  if (count == 0) return fail(SI_HIP_ERR_EMPTY, "F32 matvec group requires at least one matrix");
  if (!ws || !rows || !ys) return fail(SI_HIP_ERR_NULL, "F32 matvec group argument is null");
  size_t ytotal = 0;
  for (size_t i = 0; i < count; ++i) {
    int rc = validate_f32_matvec(rows[i] * cols, rows[i], cols, x_len);
    if (rc) return rc;
    if (!ws[i] || !ys[i]) return fail(SI_HIP_ERR_NULL, "F32 matvec buffer is null");
    ytotal += rows[i];
  }
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!x) return fail(SI_HIP_ERR_NULL, "F32 matvec buffer is null");
  CallScope scope(ctx);
  std::vector<const uint8_t *> wptr(count), dws(count);
  std::vector<size_t> wlen(count);
  for (size_t i = 0; i < count; ++i) {
    wptr[i] = reinterpret_cast<const uint8_t *>(ws[i]);
    wlen[i] = rows[i] * cols * sizeof(float);
  }
  int rc = borrow_weights(ctx, count, wptr.data(), wlen.data(), dws.data());
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_in, &ctx->stage_in_bytes, cols * sizeof(float));
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, ytotal * sizeof(float));
  if (rc) return rc;
  SIHIP_CHECK(copy_in(ctx, ctx->stage_in, x, cols * sizeof(float)),
              "input copy");
  const OutStage o = out_stage(ctx, ytotal * sizeof(float));
  size_t off = 0;
  for (size_t i = 0; i < count; ++i) {
    hipError_t e = sihip::launch_f32_matvec(reinterpret_cast<const float *>(dws[i]),
                                            static_cast<const float *>(ctx->stage_in), o.ptr + off,
                                            (uint32_t)rows[i], (uint32_t)cols, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "F32 matvec launch");
    SIHIP_CHECK(deliver(ctx, ys[i], o, off, rows[i]), "output copy");
    off += rows[i];
  }
  rc = wait_stream(ctx, "F32 matvec group command");
  if (rc) return rc;
  return ok();
}

int si_hip_rms_norm(si_hip_context *ctx, const float *x, size_t x_len, const float *w, size_t w_len,
                    float eps, float *y) {
  int rc = validate_rms(0, x_len, 0, w_len, 1, x_len, eps);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!x || !w || !y) return fail(SI_HIP_ERR_NULL, "RMSNorm buffer is null");
  CallScope scope(ctx);
  return run_rms_host(ctx, 0, x, nullptr, w, 1, x_len, eps, y);
}

int si_hip_rms_norm_heads(si_hip_context *ctx, const float *x, size_t x_len, const float *w,
                          size_t w_len, size_t heads, size_t head_dim, float eps, float *y) {
  int rc = validate_rms(1, x_len, 0, w_len, heads, head_dim, eps);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!x || !w || !y) return fail(SI_HIP_ERR_NULL, "head RMSNorm buffer is null");
  CallScope scope(ctx);
  return run_rms_host(ctx, 1, x, nullptr, w, heads, head_dim, eps, y);
}

int si_hip_rms_norm_gated(si_hip_context *ctx, const float *x, size_t x_len, const float *gate,
                          size_t gate_len, const float *w, size_t w_len, size_t heads,
                          size_t head_dim, float eps, float *y) {
  int rc = validate_rms(2, x_len, gate_len, w_len, heads, head_dim, eps);
  if (rc) return rc;
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!x || !gate || !w || !y) return fail(SI_HIP_ERR_NULL, "Gated RMSNorm buffer is null");
  CallScope scope(ctx);
  return run_rms_host(ctx, 2, x, gate, w, heads, head_dim, eps, y);
}

int si_hip_rms_norm_device(si_hip_context *ctx, uint32_t mode, const float *d_x, const float *d_gate,
                           const float *d_w, size_t heads, size_t head_dim, float eps, float *d_y) {
  if (mode > 2u) return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported RMSNorm mode %u", mode);
  const size_t n = heads * head_dim;
  int rc = validate_rms(mode, mode == 0 ? head_dim : n, n, head_dim, mode == 0 ? 1 : heads,
                        head_dim, eps);
  if (rc) return rc;
  if (mode == 0 && heads != 1) return fail(SI_HIP_ERR_DIMENSIONS, "RMSNorm input and weight must have equal non-zero length");
  if (!ctx || !d_x || !d_w || !d_y || (mode == 2 && !d_gate))
    return fail(SI_HIP_ERR_NULL, "device RMSNorm argument is null");
  CallScope scope(ctx);
  hipError_t e = sihip::launch_rms_norm(mode, d_x, d_gate, d_w, d_y, (uint32_t)heads,
                                        (uint32_t)head_dim, eps, device_stream(ctx));
  if (e != hipSuccess) return hip_fail(e, "RMSNorm launch");
  ctx->async_submitted.fetch_add(1);
  return ok();
}

// ---- dequantisation -----------------------------------------------------------
int si_hip_dequantize(si_hip_context *ctx, uint32_t type, const uint8_t *bytes, size_t len,
                      size_t elements, float *out) {
  const size_t bb = block_bytes_of(type);
  if (bb == 0) return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported quantized type %u", type);
  const char *label = type_label(type);
  if (elements == 0 || elements % 256 != 0)
    return fail(SI_HIP_ERR_DIMENSIONS, "%s element count must be a non-zero multiple of 256", label);
  size_t expected;
  if (!checked_mul(elements / 256, bb, &expected)) return fail(SI_HIP_ERR_OVERFLOW, "%s byte count overflows", label);
  if (len != expected)
    return fail(SI_HIP_ERR_BYTE_LENGTH, "%s data has %zu bytes; expected %zu", label, len, expected);
  if (elements / 256 > UINT32_MAX) return fail(SI_HIP_ERR_OVERFLOW, "%s block count exceeds HIP limits", label);
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!bytes || !out) return fail(SI_HIP_ERR_NULL, "dequantize buffer is null");
  CallScope scope(ctx);
  const uint8_t *dev = nullptr;
  int rc = stage_weights(ctx, bytes, len, &dev, false);
  if (rc) return rc;
  rc = grow(ctx, &ctx->stage_out, &ctx->stage_out_bytes, elements * sizeof(float));
  if (rc) return rc;
  // treat the blocks as one row-major [blocks x 256] matrix
  const OutStage o = out_stage(ctx, elements * sizeof(float));
  hipError_t e = sihip::launch_dequant(type, dev, nullptr, o.ptr, (uint32_t)(elements / 256), 256,
                                       ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  SIHIP_CHECK(deliver(ctx, out, o, 0, elements), "output copy");
  rc = wait_stream(ctx, "dequantize command");
  if (rc) return rc;
  return ok();
}

// ---- device-resident API --------------------------------------------------------
int si_hip_device_alloc(si_hip_context *ctx, size_t bytes, void **p) {
  if (!ctx || !p) return fail(SI_HIP_ERR_NULL, "device_alloc argument is null");
  *p = nullptr;
  if (bytes == 0) return fail(SI_HIP_ERR_DIMENSIONS, "device_alloc of zero bytes");
  if (hipMalloc(p, bytes) != hipSuccess) {
    *p = nullptr;
    return fail(SI_HIP_ERR_OUT_OF_MEMORY, "HIP could not allocate %zu bytes", bytes);
  }
  ctx->tel->note_alloc(bytes);
  return ok();
}

int si_hip_device_free(si_hip_context *ctx, void *p) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (!p) return ok();
  size_t bytes = 0;
  void *base = nullptr;
  if (hipMemGetAddressRange((hipDeviceptr_t *)&base, &bytes, (hipDeviceptr_t)p) == hipSuccess)
    ctx->tel->note_free(bytes);
  SIHIP_CHECK(hipFree(p), "free");
  return ok();
}

int si_hip_copy_to_device(si_hip_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || !dst || !src) return fail(SI_HIP_ERR_NULL, "copy argument is null");
  CallScope scope(ctx);
  SIHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "copy to device");
  SIHIP_CHECK(hipStreamSynchronize(ctx->stream), "copy to device");
  return ok();
}

int si_hip_copy_from_device(si_hip_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || !dst || !src) return fail(SI_HIP_ERR_NULL, "copy argument is null");
  CallScope scope(ctx);
  SIHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "copy from device");
  SIHIP_CHECK(hipStreamSynchronize(ctx->stream), "copy from device");
  int rc = check_device_error(ctx);
  if (rc) return rc;
  return ok();
}

int si_hip_copy_device(si_hip_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || !dst || !src) return fail(SI_HIP_ERR_NULL, "copy argument is null");
  SIHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, device_stream(ctx)),
              "device copy");
  return ok();
}

int si_hip_synchronize(si_hip_context *ctx) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  CallScope scope(ctx);
  int rc = wait_stream(ctx, "synchronize");
  if (rc) return rc;
  return ok();
}

namespace {
int validate_device_matvec(const si_hip_quant_weight *w, size_t rows, size_t cols, size_t batch) {
  int rc = check_weight(w, "device matvec");
  if (rc) return rc;
  rc = validate_many(w->ggml_type, (size_t)w->bytes, rows, cols, batch, batch * cols, true);
  return rc;
}
}  // namespace

int si_hip_quant_matvec_device(si_hip_context *ctx, const si_hip_quant_weight *w, size_t rows,
                               size_t cols, const float *d_in, float *d_out) {
  int rc = validate_device_matvec(w, rows, cols, 1);
  if (rc) return rc;
  if (!ctx || !d_in || !d_out) return fail(SI_HIP_ERR_NULL, "device matvec argument is null");
  CallScope scope(ctx);
  rc = dispatch_matvec(ctx, w->ggml_type, w->data(), d_in, d_out, (uint32_t)rows, (uint32_t)cols, 1, device_stream(ctx));
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_quant_matvec_many_device(si_hip_context *ctx, const si_hip_quant_weight *const *ws,
                                    const size_t *rows, size_t count, size_t cols,
                                    const float *d_in, float *d_out) {
  if (!ws || !rows) return fail(SI_HIP_ERR_NULL, "grouped matvec arrays are null");
  if (count == 0) return fail(SI_HIP_ERR_DIMENSIONS, "grouped quantized matvec needs at least one weight");
  uint64_t total = 0;
  for (size_t i = 0; i < count; ++i) {
    int rc = validate_device_matvec(ws[i], rows[i], cols, 1);
    if (rc) return rc;
    total += rows[i];
  }
  if (total > 0xffffffffu) return fail(SI_HIP_ERR_DIMENSIONS, "grouped quantized matvec rows overflow");
  if (!ctx || !d_in || !d_out) return fail(SI_HIP_ERR_NULL, "device matvec argument is null");
  CallScope scope(ctx);
  int rc = dispatch_weight_group(ctx, ws, rows, count, d_in, d_out, (uint32_t)cols,
                                 device_stream(ctx));
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_quant_matvec_device_repeat(si_hip_context *ctx, const si_hip_quant_weight *const *ws,
                                      size_t n, size_t rows, size_t cols, const float *d_in,
                                      float *d_out, size_t iters) {
  if (!ws || n == 0) return fail(SI_HIP_ERR_NULL, "repeat needs at least one weight");
  for (size_t i = 0; i < n; ++i) {
    int rc = validate_device_matvec(ws[i], rows, cols, 1);
    if (rc) return rc;
    if (ws[i]->ggml_type != ws[0]->ggml_type)
      return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "repeat weights must share one type");
  }
  if (!ctx || !d_in || !d_out) return fail(SI_HIP_ERR_NULL, "device matvec argument is null");
  CallScope scope(ctx);
  for (size_t i = 0; i < iters; ++i) {
    const si_hip_quant_weight *w = ws[i % n];
    int rc = dispatch_matvec(ctx, w->ggml_type, w->data(), d_in, d_out, (uint32_t)rows, (uint32_t)cols, 1, device_stream(ctx));
    if (rc) return rc;
  }
  ctx->async_submitted.fetch_add(iters);
  return ok();
}

int si_hip_stream_probe(si_hip_context *ctx, const si_hip_quant_weight *const *ws, size_t n,
                        size_t rows, size_t cols, uint32_t mode, size_t iters) {
  if (!ws || n == 0) return fail(SI_HIP_ERR_NULL, "stream probe needs at least one weight");
  if (mode > sihip::kProbeRegistersNontemporal)
    return fail(SI_HIP_ERR_RANGE, "unknown stream probe mode %u", mode);
  for (size_t i = 0; i < n; ++i) {
    int rc = validate_device_matvec(ws[i], rows, cols, 1);
    if (rc) return rc;
    if (ws[i]->ggml_type != SI_HIP_GGML_TYPE_Q4_K && ws[i]->ggml_type != SI_HIP_GGML_TYPE_Q5_K)
      return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "the stream probe reads Q4_K or Q5_K weights");
  }
  if (mode >= sihip::kProbeLines) {
    for (size_t i = 0; i < n; ++i) {
      if (ws[i]->ggml_type != SI_HIP_GGML_TYPE_Q4_K)
        return fail(SI_HIP_ERR_UNSUPPORTED_TYPE, "stream probe mode %u reads Q4_K weights", mode);
      if ((reinterpret_cast<uintptr_t>(ws[i]->data()) & 127u) != 0u)
        return fail(SI_HIP_ERR_RANGE, "stream probe mode %u needs 128-byte aligned weights", mode);
    }
    if (mode == sihip::kProbeLines && (cols / 256u) % 8u != 4u)
      return fail(SI_HIP_ERR_DIMENSIONS, "stream probe mode 4 needs rows of 4 mod 8 blocks");
  }
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  int cus = 0;
  SIHIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device),
              "device query");
  CallScope scope(ctx);
  for (size_t i = 0; i < iters; ++i) {
    const si_hip_quant_weight *w = ws[i % n];
    hipError_t e = sihip::launch_stream_probe(mode, w->data(), (uint32_t)rows, (uint32_t)cols,
                                              (uint32_t)block_bytes_of(w->ggml_type),
                                              (uint32_t)cus, device_stream(ctx));
    if (e != hipSuccess) return hip_fail(e, "stream probe launch");
  }
  ctx->async_submitted.fetch_add(iters);
  return ok();
}

int si_hip_q4_k_fused_gate_up_device(si_hip_context *ctx, const si_hip_quant_weight *g,
                                     const si_hip_quant_weight *u, size_t rows, size_t cols,
                                     const float *d_in, float *d_out) {
  int rc = validate_gate_up_weights(g, u, rows, cols, cols,
                                    "retained Q4_K fused gate/up dimensions are invalid",
                                    "retained Q4_K fused gate/up byte length overflows",
                                    "retained Q4_K fused gate/up byte length is invalid");
  if (rc) return rc;
  if (!ctx || !d_in || !d_out) return fail(SI_HIP_ERR_NULL, "device gate/up argument is null");
  CallScope scope(ctx);
  rc = dispatch_gate_up(ctx, g->data(), u->data(), d_in, d_out, (uint32_t)rows, (uint32_t)cols, device_stream(ctx));
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_fused_mlp_device(si_hip_context *ctx, const si_hip_quant_weight *g,
                            const si_hip_quant_weight *u, const si_hip_quant_weight *d,
                            size_t gate_rows, size_t cols, size_t down_rows, const float *d_in,
                            float *d_hidden, float *d_out) {
  int rc = validate_mlp(g, u, d, gate_rows, cols, down_rows, cols);
  if (rc) return rc;
  if (!ctx || !d_in || !d_hidden || !d_out) return fail(SI_HIP_ERR_NULL, "device MLP argument is null");
  CallScope scope(ctx);
  rc = dispatch_gate_up(ctx, g->data(), u->data(), d_in, d_hidden, (uint32_t)gate_rows, (uint32_t)cols, device_stream(ctx));
  if (rc) return rc;
  rc = dispatch_matvec(ctx, d->ggml_type, d->data(), d_hidden, d_out, (uint32_t)down_rows,
                       (uint32_t)gate_rows, 1, device_stream(ctx));
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_matmul_many_device(si_hip_context *ctx, const si_hip_quant_weight *w, size_t rows,
                              size_t cols, size_t batch, const float *d_in, float *d_out) {
  int rc = validate_device_matvec(w, rows, cols, batch);
  if (rc) return rc;
  if (!ctx || !d_in || !d_out) return fail(SI_HIP_ERR_NULL, "device matmul argument is null");
  CallScope scope(ctx);
  rc = dispatch_matvec(ctx, w->ggml_type, w->data(), d_in, d_out, (uint32_t)rows, (uint32_t)cols,
                       (uint32_t)batch, device_stream(ctx));
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_matvec_argmax_device(si_hip_context *ctx, const si_hip_quant_weight *w, size_t rows,
                                size_t cols, const float *d_in, uint32_t rule, float *d_logits,
                                uint64_t *d_result) {
  int rc = validate_head(w, rows, cols, cols, rule);
  if (rc) return rc;
  if (!ctx || !d_in || !d_logits || !d_result) return fail(SI_HIP_ERR_NULL, "device head argument is null");
  CallScope scope(ctx);
  bool fused = false;
  rc = dispatch_head(ctx, w, d_in, d_logits, d_logits, true, (uint32_t)rows, (uint32_t)cols, rule,
                     d_result, device_stream(ctx), &fused);
  if (rc) return rc;
  ctx->async_submitted.fetch_add(1);
  return ok();
}

uint32_t si_hip_argmax_result_index(uint64_t packed, uint32_t rule) {
  return sihip::argmax_candidate_index(packed, rule);
}

int si_hip_embedding_device(si_hip_context *ctx, const si_hip_quant_weight *t, size_t cols,
                            size_t rows, const uint32_t *d_ids, size_t n, float *d_out) {
  // the ids live on the device: the table checks here (those of row 0, which
  // every non-empty table passes), the ids' in the kernel, which gives an id
  // beyond the rows the table holds a NaN row and reports it at the next
  // synchronisation
  if (rows == 0) return fail(SI_HIP_ERR_RANGE, "Q4_K embedding token id or dimension is invalid");
  int rc = validate_embedding_row(t, cols, rows, 0);
  if (rc) return rc;
  if (n == 0 || n > UINT32_MAX) return fail(SI_HIP_ERR_DIMENSIONS, "embedding token count is invalid");
  if (!ctx || !d_ids || !d_out) return fail(SI_HIP_ERR_NULL, "device embedding argument is null");
  CallScope scope(ctx);
  hipError_t e = sihip::launch_dequant(SI_HIP_GGML_TYPE_Q4_K, t->data(), d_ids, d_out, (uint32_t)n,
                                       (uint32_t)cols, device_stream(ctx),
                                       embedding_table_rows(t, cols, rows), ctx->ws.ptr);
  if (e != hipSuccess) return hip_fail(e, "embedding launch");
  ctx->async_submitted.fetch_add(1);
  return ok();
}

int si_hip_event_record(si_hip_context *ctx, uint32_t slot) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (slot >= 16) return fail(SI_HIP_ERR_RANGE, "event slot %u out of range", slot);
  SIHIP_CHECK(hipEventRecord(ctx->events[slot], ctx->stream), "event record");
  return ok();
}

int si_hip_event_elapsed_ms(si_hip_context *ctx, uint32_t a, uint32_t b, float *ms) {
  if (!ctx || !ms) return fail(SI_HIP_ERR_NULL, "event argument is null");
  if (a >= 16 || b >= 16) return fail(SI_HIP_ERR_RANGE, "event slot out of range");
  SIHIP_CHECK(hipEventSynchronize(ctx->events[b]), "event synchronize");
  SIHIP_CHECK(hipEventElapsedTime(ms, ctx->events[a], ctx->events[b]), "event elapsed");
  return ok();
}

// ---- captured submission -------------------------------------------------------
int si_hip_capture_begin(si_hip_context *ctx) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  CallScope scope(ctx);
  if (ctx->capturing) return fail(SI_HIP_ERR_STATE, "a graph capture is already open");
  if (!ctx->capture_stream)
    SIHIP_CHECK(hipStreamCreateWithFlags(&ctx->capture_stream, hipStreamNonBlocking),
                "capture stream create");
  SIHIP_CHECK(hipStreamBeginCapture(ctx->capture_stream, hipStreamCaptureModeRelaxed),
              "begin capture");
  ctx->capturing = true;
  ctx->captured_calls = ctx->async_submitted.load();
  return ok();
}

int si_hip_capture_end(si_hip_context *ctx, si_hip_graph **out) {
  if (!ctx || !out) return fail(SI_HIP_ERR_NULL, "capture_end argument is null");
  *out = nullptr;
  CallScope scope(ctx);
  if (!ctx->capturing) return fail(SI_HIP_ERR_STATE, "no graph capture is open");
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  SIHIP_CHECK(hipStreamEndCapture(ctx->capture_stream, &g), "end capture");
  if (!g) return fail(SI_HIP_ERR_DEVICE, "HIP returned no captured graph");
  auto graph = std::make_unique<si_hip_graph>();
  graph->graph = g;
  graph->device = ctx->device;
  graph->calls = ctx->async_submitted.load() - ctx->captured_calls;
  // the recorded calls did not run
  ctx->async_submitted.fetch_sub(graph->calls);
  hipError_t e = hipGraphInstantiate(&graph->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "graph instantiate");
  }
  *out = graph.release();
  return ok();
}

int si_hip_graph_launch(si_hip_context *ctx, const si_hip_graph *graph) {
  if (!ctx || !graph) return fail(SI_HIP_ERR_NULL, "graph launch argument is null");
  if (graph->device != ctx->device)
    return fail(SI_HIP_ERR_RANGE, "graph was captured on device %d, context is on %d",
                graph->device, ctx->device);
  CallScope scope(ctx);
  SIHIP_CHECK(hipGraphLaunch(graph->exec, ctx->stream), "graph launch");
  ctx->async_submitted.fetch_add(graph->calls);
  return ok();
}

uint64_t si_hip_graph_calls(const si_hip_graph *graph) { return graph ? graph->calls : 0; }

void si_hip_graph_free(si_hip_graph *graph) {
  if (!graph) return;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
}

int si_hip_debug_set_wait_give_up(si_hip_context *ctx, uint32_t polls) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  CallScope scope(ctx);
  if (ctx->capturing) return fail(SI_HIP_ERR_STATE, "the wait hook cannot change during a graph capture");
  SIHIP_CHECK(hipStreamSynchronize(ctx->stream), "wait hook");
  ctx->give_up_polls = polls;
  int rc = reset_workspace(ctx);
  if (rc) return rc;
  return ok();
}

int si_hip_set_kernel_policy(si_hip_context *ctx, uint32_t policy) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  if (policy != SI_HIP_KERNEL_AUTO && policy != SI_HIP_KERNEL_GENERIC)
    return fail(SI_HIP_ERR_RANGE, "unknown kernel policy %u", policy);
  CallScope scope(ctx);
  ctx->policy = policy;
  return ok();
}

uint64_t si_hip_current_allocated_bytes(const si_hip_context *ctx) {
  return ctx ? ctx->tel->allocated.load() : 0;
}
uint64_t si_hip_peak_allocated_bytes(const si_hip_context *ctx) {
  return ctx ? ctx->tel->peak_allocated.load() : 0;
}
uint64_t si_hip_peak_active_weight_bytes(const si_hip_context *ctx) {
  return ctx ? ctx->tel->peak_active_weights.load() : 0;
}
void si_hip_reset_peaks(si_hip_context *ctx) {
  if (!ctx) return;
  ctx->tel->peak_allocated.store(ctx->tel->allocated.load());
  ctx->tel->peak_active_weights.store(ctx->tel->active_weights.load());
}
void si_hip_sample_allocated(si_hip_context *ctx) {
  // sample_allocated (metal.rs:2374-2378): the peak takes the current device
  // allocation.  Allocations here already raise the peak as they happen, so a
  // sample only matters after reset_peaks.
  if (!ctx) return;
  const uint64_t now = ctx->tel->allocated.load();
  uint64_t prev = ctx->tel->peak_allocated.load();
  while (now > prev && !ctx->tel->peak_allocated.compare_exchange_weak(prev, now)) {
  }
}
int si_hip_set_residency_budget(si_hip_context *ctx, uint64_t bytes) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  CallScope scope(ctx);
  ctx->res.budget = bytes;
  while (ctx->res.bytes > bytes) {
    auto victim = ctx->res.ranges.begin();
    for (auto j = ctx->res.ranges.begin(); j != ctx->res.ranges.end(); ++j)
      if (j->second.used < victim->second.used) victim = j;
    evict_range(ctx, victim);
  }
  return ok();
}

int si_hip_residency_evict(si_hip_context *ctx, const void *host_bytes, size_t len) {
  if (!ctx) return fail(SI_HIP_ERR_NULL, "HIP context is null");
  CallScope scope(ctx);
  const uintptr_t lo = (uintptr_t)host_bytes;
  const uintptr_t hi = len == 0 ? UINTPTR_MAX : (len > UINTPTR_MAX - lo ? UINTPTR_MAX : lo + len);
  for (auto it = ctx->res.ranges.begin(); it != ctx->res.ranges.end();) {
    const uintptr_t a = it->first.first, b = a + it->first.second;
    auto next = std::next(it);
    if (len == 0 || (a < hi && lo < b)) evict_range(ctx, it);
    it = next;
  }
  return ok();
}

int si_hip_get_residency_stats(si_hip_context *ctx, si_hip_residency_stats *out) {
  if (!ctx || !out) return fail(SI_HIP_ERR_NULL, "residency stats argument is null");
  CallScope scope(ctx);
  *out = ctx->res.stats;
  out->resident_ranges = ctx->res.ranges.size();
  out->resident_bytes = ctx->res.bytes;
  out->budget_bytes = ctx->res.budget;
  return ok();
}

int si_hip_get_command_stats(const si_hip_context *ctx, si_hip_command_stats *out) {
  if (!ctx || !out) return fail(SI_HIP_ERR_NULL, "command stats argument is null");
  out->submitted = ctx->submitted.load();
  out->async_submitted = ctx->async_submitted.load();
  out->waited = ctx->waited.load();
  out->wait_nanos = ctx->wait_nanos.load();
  return ok();
}

}  // extern "C"
