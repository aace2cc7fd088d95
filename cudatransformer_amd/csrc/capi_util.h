// Shared helpers of the C-ABI entry points: the per-thread error message and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {
namespace capi {

extern thread_local char g_err[512];

// Sets the calling thread's message and returns `code`.
int fail(hipError_t code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns 0.
int ok();
// Turns a launch status into the entry point's return value; with CTATTN_SYNC_CHECK=1 also
// synchronises the stream and reports asynchronous kernel errors.
int finish(const char *fn, hipError_t e, hipStream_t stream);

constexpr int64_t kAlign = 256;  // workspace sub-buffer alignment (bytes)
int64_t align_up(int64_t x);

}  // namespace capi
}  // namespace ctattn
