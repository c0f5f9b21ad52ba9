// HIP error checks that turn runtime failures into qne::Error(QNE_EDEVICE).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "error.hpp"

namespace qne {

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(QNE_EDEVICE, std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

#define QNE_HIP(expr) ::qne::hip_check((expr), #expr)

// Waits for the stream like the reference's device poll (kernels/src/lib.rs:399-405): an error
// after 30 s instead of blocking forever.
void wait_stream(hipStream_t st, double timeout_s = 30.0);

}  // namespace qne
