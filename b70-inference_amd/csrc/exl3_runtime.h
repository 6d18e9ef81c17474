// Host-side runtime shared by the EXL3 C-ABI entry points: status codes, the thread-local error message, and the
// per-device workspace (split-K partials, arrival counters, routing tables, intermediate activations).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/exl3mi.h"

namespace exl3 {

// Records a message for exl3_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define EXL3_CHECK_ARG(cond, ...) \
    do { if (!(cond)) return ::exl3::fail(EXL3_ERR_INVALID, __VA_ARGS__); } while (0)
#define EXL3_CHECK_HIP(expr)                                                                          \
    do {                                                                                              \
        hipError_t e_ = (expr);                                                                       \
        if (e_ != hipSuccess) return ::exl3::fail(EXL3_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// Device workspace of the current device. `bytes` of plain scratch (256-byte aligned) and `ncounters` int32 arrival
// counters that are zero between calls (kernels that use a counter reset it before they exit), plus `status`, the
// device address of a host-mapped word that a kernel sets (system-scope store) when one of its bounded waits gives
// up. Calls that share a device must be ordered on one stream (as the reference's library-owned scratch,
// glm/xpu/csrc/exl3_ops.sycl:202-207).
// Growing allocates new buffers and keeps the old ones alive (kernels already queued and captured graphs still point
// at them) until exl3_release_workspace; it never synchronises, the new counters are zeroed by a fill kernel on
// `stream`, and it is refused while `stream` is being captured (exl3_reserve_workspace beforehand).
// Before anything else it checks the status word (a host read, no synchronisation): when a wait has timed out it
// zeroes every counters buffer of the device (current and outgrown) on `stream`, clears the word and fails with
// EXL3_ERR_HIP; under stream capture it fails without the reset and leaves the word set.
struct Workspace {
    char* scratch = nullptr;
    size_t scratch_bytes = 0;
    int* counters = nullptr;
    size_t ncounters = 0;
    int* status = nullptr;
};
int workspace(size_t bytes, size_t ncounters, hipStream_t stream, Workspace* out);

// Wait bound of the kernels' cross-workgroup waits (polls): EXL3MI_SPIN_LIMIT, default 2^20. A small value makes a
// wait give up early (failure-path tests); every kernel still exits.
int spin_limit();

// A second per-device buffer for data a call builds before it runs on the workspace (e.g. expert tables); same
// growth rules as the workspace (retired, never freed under queued work; refused under capture).
int aux_buffer(size_t bytes, hipStream_t stream, void** out);
int device_status(int* out);
int release_workspace();

// Marks the status word (device code; `status` from Workspace).
__device__ __forceinline__ void report_timeout(int* status) {
    __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Two library-owned side streams (default priority) and three events of the current device, created on first use:
// a launch sequence forks onto them with events and joins back, which also works under stream capture.
struct AuxStreams {
    hipStream_t s[2];
    hipEvent_t ev[3];
};
int aux_streams(AuxStreams* out);

// Workgroups of `threads` threads of kernel `fn` that the current device holds at once (occupancy x CUs), cached
// per device and kernel.
int resident_blocks(const void* fn, int threads, int* out);

// Integer tuning knob from the environment (read at every call), `dflt` when unset or not a positive number.
int env_int(const char* name, int dflt);

// Bump allocator over one workspace request.
struct Carve {
    char* p;
    size_t left;
    template <typename T>
    T* take(size_t n) {
        size_t b = (n * sizeof(T) + 255) & ~(size_t)255;
        if (b > left) return nullptr;
        T* r = reinterpret_cast<T*>(p);
        p += b;
        left -= b;
        return r;
    }
};
inline size_t carve_size(size_t n, size_t elem) { return (n * elem + 255) & ~(size_t)255; }

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Opt-in kernel timing (exl3_profile_enable): every library launch gets a HIP event pair that the runtime records
// with the dispatch itself (hipExtLaunchKernel start/stop events: the kernel's own begin and end, no queue gaps),
// aggregated per kernel name by exl3_profile_read. Off by default; never used under graph capture.
// With repeat R > 1 every profiled launch runs R times back to back, the first carrying the start event and the
// last the stop event (all library kernels are idempotent: they rewrite their outputs and leave their arrival
// counters at zero); exl3_profile_read reports the per-launch average.
struct ProfEvents {
    hipEvent_t a, b;                    // both null when profiling is off
};
ProfEvents prof_begin(const char* name);
int prof_repeat();

#define EXL3_LAUNCH(name, kernel, grid, block, lds, stream, ...)                                          \
    do {                                                                                                \
        const ::exl3::ProfEvents pe_ = ::exl3::prof_begin(name);                                        \
        if (pe_.a) {                                                                                    \
            const int reps_ = ::exl3::prof_repeat();                                                    \
            for (int rep_ = 0; rep_ < reps_; ++rep_)                                                    \
                hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, rep_ == 0 ? pe_.a : nullptr,    \
                                      rep_ == reps_ - 1 ? pe_.b : nullptr, 0u, __VA_ARGS__);            \
        } else {                                                                                        \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                          \
        }                                                                                               \
        EXL3_CHECK_HIP(hipGetLastError());                                                              \
    } while (0)

}  // namespace exl3
