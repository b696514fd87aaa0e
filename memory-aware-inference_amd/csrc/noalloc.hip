// si_hip_quant_matvec_noalloc: the device-resident matvec without a context
// and without any device allocation, for callers that cannot allocate (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  No counterpart in the reference.
//
// The matrix-core kernels combine the partial sums of tiles split across
// workgroups through a workspace (per-tile counters that start at zero, then
// entries that read kWorkspaceEmpty when they hold no sum; si_hip_internal.h).
// A context allocates one; here it is the file-scope device array `scratch`,
// one copy per GPU for the life of the process.  Its device address is taken
// once per device with hipGetSymbolAddress (the array's name in host code is
// only a stand-in) and filled into its rest state by a small kernel on the
// first call's stream.  Every kernel leaves the workspace in that state, so
// later calls find it ready.  Calls that overlap on one GPU would race on it.
//
// A kernel that gives up one of its bounded waits (report_device_error)
// stores its code into the file-scope device word `failure`, whose address the
// workspace's report slot holds; the workspace may then be out of its rest
// state.  si_hip_noalloc_check reads the word, and when it is set clears it,
// puts the workspace back into its rest state and returns SI_HIP_ERR_DEVICE.
#include <mutex>

#include "kquant_device.h"
#include "si_hip.h"
#include "si_hip_internal.h"
#include "si_hip_status.h"
#include "si_hip_tuned.h"

static __device__ __align__(256) uint8_t scratch[sihip::kWorkspaceBytes];
static __device__ __align__(16) uint32_t failure;

namespace {

static_assert(SI_HIP_NOALLOC_WORKSPACE_BYTES == sihip::kWorkspaceBytes, "the header's figure");
// the kernels split tiles only while every tile has a counter below the
// argmax's reserved words (the last 64 bytes of the counter region)
static_assert((SI_HIP_NOALLOC_MAX_ROWS / 16u) * 4u + 64u <= sihip::kWorkspaceCounterBytes,
              "counters for every tile");

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, once set up
uint32_t* g_failure[kMaxDevices];  // device address of `failure` per device
uint32_t g_give_up[kMaxDevices];   // the test hook's poll count per device

// Rest state of the workspace: counters 0, entries empty, the reserved words
// (the report slot: the address of `failure`; the test hook's poll count;
// the argmax counter 0), and the failure word 0.
constexpr uint32_t kReservedWord = (uint32_t)(sihip::kWorkspaceReportSlot / 4);
__global__ __launch_bounds__(256) void workspace_rest(uint32_t* w, uint32_t counter_words,
                                                       uint32_t words, uint32_t* fail,
                                                       uint32_t give_up) {
  static_assert(sihip::kWorkspaceReportSlot + 8 == sihip::kWorkspaceGiveUpWord &&
                    sihip::kWorkspaceGiveUpWord + 4 == sihip::kWorkspaceArgmaxCounter,
                "reserved words in one 16-byte run");
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < words; i += gridDim.x * 256u) {
    uint32_t v = i < counter_words ? 0u : sihip::kWorkspaceEmpty;
    if (i == kReservedWord) v = (uint32_t)(uintptr_t)fail;
    if (i == kReservedWord + 1u) v = (uint32_t)((uint64_t)(uintptr_t)fail >> 32);
    if (i == kReservedWord + 2u) v = give_up;
    w[i] = v;
  }
  if (blockIdx.x == 0u && threadIdx.x == 0u) *fail = 0u;
}

// The rest state on `stream`, waited for.
hipError_t put_to_rest(void* p, uint32_t* fail, uint32_t give_up, hipStream_t stream) {
  constexpr uint32_t words = (uint32_t)(sihip::kWorkspaceBytes / 4);
  constexpr uint32_t counter_words = (uint32_t)(sihip::kWorkspaceCounterBytes / 4);
  hipLaunchKernelGGL(workspace_rest, dim3(512), dim3(256), 0, stream, static_cast<uint32_t*>(p),
                     counter_words, words, fail, give_up);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return e;
}

// The current device's workspace: on its first use, its address and its
// rest state (a fill kernel on `stream`, waited for, so that calls on any
// stream find it ready).  A first use under graph capture is refused: the
// fill would only run when the graph does.
int device_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP device query failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "device %d beyond the no-alloc workspace table", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess)
      return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP capture query failed: %s", hipGetErrorString(e));
    if (cap != hipStreamCaptureStatusNone)
      return sihip::set_error(SI_HIP_ERR_STATE,
                              "the no-alloc workspace of device %d is set up by a call outside "
                              "graph capture (or by creating a context on the device)", dev);
    void* p = nullptr;
    void* f = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipGetSymbolAddress(&f, HIP_SYMBOL(failure));
    if (e != hipSuccess || !p || !f)
      return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP symbol address of the workspace failed: %s",
                              hipGetErrorString(e));
    e = put_to_rest(p, static_cast<uint32_t*>(f), 0u, stream);
    if (e != hipSuccess)
      return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP no-alloc workspace set-up failed: %s",
                              hipGetErrorString(e));
    g_failure[dev] = static_cast<uint32_t*>(f);
    g_give_up[dev] = 0u;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return SI_HIP_OK;
}

// The current device's index (set up: device_scratch has run on it).
int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP device query failed: %s", hipGetErrorString(e));
  return SI_HIP_OK;
}

// The workspace of the current device back in its rest state (with the test
// hook's poll count `give_up`), outside graph capture.
int rest_outside_capture(hipStream_t stream, uint32_t give_up, const char* what) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP capture query failed: %s", hipGetErrorString(e));
  if (cap != hipStreamCaptureStatusNone)
    return sihip::set_error(SI_HIP_ERR_STATE, "%s cannot run under graph capture", what);
  void* p = nullptr;
  int rc = device_scratch(stream, &p);
  if (rc) return rc;
  int dev = 0;
  rc = current_device(&dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  e = put_to_rest(p, g_failure[dev], give_up, stream);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP no-alloc workspace reset failed: %s",
                            hipGetErrorString(e));
  g_give_up[dev] = give_up;
  return SI_HIP_OK;
}

size_t block_bytes_of(uint32_t type) {
  return type == sihip::kTypeQ4K ? sihip::kQ4Bytes
         : type == sihip::kTypeQ5K ? sihip::kQ5Bytes
         : type == sihip::kTypeQ6K ? sihip::kQ6Bytes
                                   : 0u;
}

}  // namespace

int sihip::noalloc_setup(hipStream_t stream) {
  void* p = nullptr;
  return device_scratch(stream, &p);
}

extern "C" int si_hip_quant_matvec_noalloc(uint32_t ggml_type, const void* weights,
                                           size_t weight_bytes, size_t rows, size_t columns,
                                           const float* d_input, float* d_output, void* stream) {
  const size_t bb = block_bytes_of(ggml_type);
  if (bb == 0) return sihip::set_error(SI_HIP_ERR_UNSUPPORTED_TYPE, "unsupported no-alloc quantized weight type");
  if (rows == 0 || columns == 0 || columns % 256 != 0)
    return sihip::set_error(SI_HIP_ERR_DIMENSIONS, "no-alloc quantized matvec dimensions are invalid");
  if (rows > SI_HIP_NOALLOC_MAX_ROWS)
    return sihip::set_error(SI_HIP_ERR_DIMENSIONS,
                            "no-alloc quantized matvec rows %zu exceed the workspace's %u", rows,
                            (unsigned)SI_HIP_NOALLOC_MAX_ROWS);
  if (columns > 0xffffffffu)
    return sihip::set_error(SI_HIP_ERR_OVERFLOW, "no-alloc quantized matvec columns exceed u32");
  const unsigned __int128 want = (unsigned __int128)rows * (columns / 256) * bb;
  if (want != weight_bytes)
    return sihip::set_error(SI_HIP_ERR_BYTE_LENGTH, "no-alloc quantized weight byte length is invalid");
  if (!weights || !d_input || !d_output)
    return sihip::set_error(SI_HIP_ERR_NULL, "no-alloc matvec argument is null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws_ptr = nullptr;
  int rc = device_scratch(s, &ws_ptr);
  if (rc) return rc;
  sihip::Workspace ws;
  ws.ptr = ws_ptr;
  ws.bytes = sihip::kWorkspaceBytes;  // no scratch region: one vector needs none
  const uint8_t* w = static_cast<const uint8_t*>(weights);
  hipError_t e = hipErrorInvalidValue;
  if (!sihip::launch_matvec_tuned(ggml_type, w, d_input, d_output, (uint32_t)rows,
                                  (uint32_t)columns, 1u, ws, s, &e))
    e = sihip::launch_matvec_generic(ggml_type, w, d_input, d_output, (uint32_t)rows,
                                     (uint32_t)columns, 1u, s);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP no-alloc matvec launch failed: %s", hipGetErrorString(e));
  return sihip::clear_error();
}

extern "C" int si_hip_noalloc_check(void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP capture query failed: %s", hipGetErrorString(e));
  if (cap != hipStreamCaptureStatusNone)
    return sihip::set_error(SI_HIP_ERR_STATE, "the no-alloc check cannot run under graph capture");
  void* p = nullptr;
  int rc = device_scratch(s, &p);
  if (rc) return rc;
  int dev = 0;
  rc = current_device(&dev);
  if (rc) return rc;
  uint32_t code = 0;
  e = hipMemcpyAsync(&code, g_failure[dev], sizeof code, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess)
    return sihip::set_error(SI_HIP_ERR_DEVICE, "HIP no-alloc failure word read failed: %s",
                            hipGetErrorString(e));
  if (code == 0u) return sihip::clear_error();
  rc = rest_outside_capture(s, g_give_up[dev], "the no-alloc check");
  if (rc) return rc;
  return sihip::set_error(SI_HIP_ERR_DEVICE,
                          "a no-alloc matvec kernel gave up a bounded wait (code %u): results "
                          "since the last check may be wrong; the workspace is back in its rest "
                          "state",
                          code);
}

extern "C" int si_hip_noalloc_debug_set_wait_give_up(uint32_t polls, void* stream) {
  int rc = rest_outside_capture(static_cast<hipStream_t>(stream), polls, "the no-alloc wait hook");
  if (rc) return rc;
  return sihip::clear_error();
}
