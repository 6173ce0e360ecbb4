// Host-side helpers shared by the library's translation units: error reporting for the C-ABI and the
// optional per-kernel HIP-event timing (implemented once, in slotscan.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

namespace slothost {

// Store `msg` as this thread's last error and return `code`.
int fail(int code, const char* msg);
// Store "<where>: <HIP error string>" and return SLOTSCAN_ERR_HIP.
int hip_fail(hipError_t e, const char* where);

// While timing is enabled (slotscan_profile(1)), a Scope takes two events and becomes the calling thread's
// current scope.  The next slothost::launch on the scope's stream hands them to hipExtLaunchKernel, which
// stamps them with that kernel's own start and end, so timing adds no packets between launches.  The pair
// is filed under kernel id `kid` when the scope ends.  A no-op while timing is disabled.
struct Scope {
    int kid;
    hipStream_t st;
    hipEvent_t a = nullptr, b = nullptr;
    bool used = false;
    Scope* prev = nullptr;
    Scope(int k, hipStream_t s);
    ~Scope();
};
Scope*& current_scope();                                // per calling thread

// Every kernel launch of the library goes through here.
template <typename F, typename... Args>
inline void launch(F kernel, const dim3& grid, const dim3& block, uint32_t shm, hipStream_t st, Args... args) {
    Scope* sc = current_scope();
    hipEvent_t a = nullptr, b = nullptr;
    if (sc && sc->a && !sc->used && sc->st == st) { a = sc->a; b = sc->b; sc->used = true; }
    hipExtLaunchKernelGGL(kernel, grid, block, shm, st, a, b, 0u, args...);
}

inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The library's second stream on the current device (non-blocking, default priority) and a pool of
// timing-free events, for fork/join pipelines inside one entry point.  Created on first use per device and
// kept until the process ends.  Returns 0, or SLOTSCAN_ERR_HIP with the message set.
int side_stream(hipStream_t* side, hipEvent_t** ev, int nev);

}  // namespace slothost
