// Host-side helpers shared by the library's translation units: error reporting for the C-ABI and the
// optional per-kernel HIP-event timing (implemented once, in slotscan.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slothost {

// Store `msg` as this thread's last error and return `code`.
int fail(int code, const char* msg);
// Store "<where>: <HIP error string>" and return SLOTSCAN_ERR_HIP.
int hip_fail(hipError_t e, const char* where);

// While timing is enabled (slotscan_profile(1)), records one hipEvent on `st` at construction and one at
// destruction, filed under kernel id `kid`; a no-op otherwise.
struct Scope {
    int kid;
    hipStream_t st;
    hipEvent_t a = nullptr;
    Scope(int k, hipStream_t s);
    ~Scope();
};

inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The library's second stream on the current device (non-blocking, default priority) and a pool of
// timing-free events, for fork/join pipelines inside one entry point.  Created on first use per device and
// kept until the process ends.  Returns 0, or SLOTSCAN_ERR_HIP with the message set.
int side_stream(hipStream_t* side, hipEvent_t** ev, int nev);

}  // namespace slothost
