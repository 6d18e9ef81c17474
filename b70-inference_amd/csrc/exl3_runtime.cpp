// Status/error reporting and the per-device workspace behind the C-ABI.
#include "exl3_runtime.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

namespace exl3 {

static thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_ws_mu;
Workspace g_ws[kMaxDevices];
}  // namespace

int workspace(size_t bytes, size_t ncounters, Workspace* out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[dev];
    if (bytes > w.scratch_bytes) {
        size_t nb = bytes + bytes / 4;
        nb = (nb + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        char* p = nullptr;
        EXL3_CHECK_HIP(hipDeviceSynchronize());
        if (w.scratch) EXL3_CHECK_HIP(hipFree(w.scratch));
        w.scratch = nullptr;
        w.scratch_bytes = 0;
        EXL3_CHECK_HIP(hipMalloc(&p, nb));
        w.scratch = p;
        w.scratch_bytes = nb;
    }
    if (ncounters > w.ncounters) {
        size_t nc = ncounters < 65536 ? 65536 : ncounters * 2;
        int* c = nullptr;
        EXL3_CHECK_HIP(hipDeviceSynchronize());
        if (w.counters) EXL3_CHECK_HIP(hipFree(w.counters));
        w.counters = nullptr;
        w.ncounters = 0;
        EXL3_CHECK_HIP(hipMalloc(&c, nc * sizeof(int)));
        EXL3_CHECK_HIP(hipMemset(c, 0, nc * sizeof(int)));
        EXL3_CHECK_HIP(hipDeviceSynchronize());
        w.counters = c;
        w.ncounters = nc;
    }
    *out = w;
    return EXL3_OK;
}

}  // namespace exl3

extern "C" {

const char* exl3_last_error(void) { return exl3::g_err; }

int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

int exl3_reserve_workspace(int64_t bytes, int64_t ncounters) {
    if (bytes < 0 || ncounters < 0) return exl3::fail(EXL3_ERR_INVALID, "negative workspace size");
    exl3::Workspace w;
    return exl3::workspace((size_t)bytes, (size_t)ncounters, &w);
}

}  // extern "C"
