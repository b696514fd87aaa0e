// Functions the C-ABI translation units (api.cpp, gguf.cpp) share beyond the
// public headers.  Plain C++: no HIP types.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "si_hip.h"

namespace sihip {

// gguf_quant_matvec_bytes over bytes [offset, offset + len) of the borrowed
// range [tensor, tensor + tensor_len) (a GGUF tensor's payload in the mapped
// file): the whole tensor is what stays resident in HBM when it fits the
// context's residency budget, so that calls on different row ranges of one
// tensor share one copy.  offset + len <= tensor_len.
int quant_matvec_tensor_range(si_hip_context *ctx, uint32_t type, const uint8_t *tensor,
                              size_t tensor_len, size_t offset, size_t len, size_t rows,
                              size_t cols, const float *in, size_t in_len, float *out);

}  // namespace sihip
