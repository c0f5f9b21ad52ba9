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
// after timeout_s instead of blocking forever.
void wait_stream(hipStream_t st, double timeout_s = 30.0);

// Host deadline for work of `units` dependent device steps (decode-program phases, prefill
// passes, batched steps): 30 s plus 2 ms per step, about 250 times what a decode-program phase
// of the 2B model takes (8 us), so a long prompt or window never times out while the device is
// still making progress, and a genuinely stuck stream still ends in an error.
inline double work_deadline_s(double units) { return 30.0 + 2e-3 * (units > 0 ? units : 0.0); }

}  // namespace qne
