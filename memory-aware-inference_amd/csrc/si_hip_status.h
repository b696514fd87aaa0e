// Status reporting shared by the C-ABI translation units: the thread-local
// message behind si_hip_last_error().
#pragma once

namespace sihip {
// Sets the calling thread's message (printf format) and returns `status`.
int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns SI_HIP_OK.
int clear_error();
}  // namespace sihip
