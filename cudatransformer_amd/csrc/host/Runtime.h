// Host runtime glue: one process-wide HIP stream and error translation.
//
// Replaces the reference's implicit legacy-default-stream model (headers.cu:195-215 syncs the
// whole device after every allocation).  Here every allocation, copy and kernel of the host
// layer is enqueued on one stream; the host waits only where data crosses to the CPU.
#pragma once

#include <hip/hip_runtime_api.h>

#include <mutex>
#include <stdexcept>
#include <string>

#include "ctattn.h"

namespace ct {

inline void hipCheck(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// ctattn_* return 0 or a hipError_t value; argument errors become std::invalid_argument
// (Python ValueError), everything else std::runtime_error (Python RuntimeError).
inline void ctattnCheck(int rc, const char *what) {
    if (rc == 0) return;
    std::string msg = std::string(what) + ": " + ctattn_last_error();
    if (rc == hipErrorInvalidValue || rc == hipErrorNotSupported) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

class Runtime {
public:
    // The stream every host-side operation is ordered on (created on first use, on the
    // device current at that time; default priority).
    static hipStream_t stream() {
        static Runtime rt;
        return rt.stream_;
    }

    static void synchronize() { hipCheck(hipStreamSynchronize(stream()), "hipStreamSynchronize"); }

private:
    Runtime() { hipCheck(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate"); }
    ~Runtime() = default;  // the stream lives until process exit
    hipStream_t stream_ = nullptr;
};

}  // namespace ct
