// Status/error reporting and the per-device workspace behind the C-ABI.
#include "exl3_runtime.h"

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>

#include <mutex>
#include <string>
#include <string.h>
#include <utility>
#include <vector>

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
int* g_status_host[kMaxDevices];   // host view of each device's status word (Workspace::status is its device address)
}  // namespace

namespace {
AuxStreams g_aux[kMaxDevices];
bool g_aux_ok[kMaxDevices];
}  // namespace

int aux_streams(AuxStreams* out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (!g_aux_ok[dev]) {
        AuxStreams a{};
        for (int i = 0; i < 2; ++i) EXL3_CHECK_HIP(hipStreamCreateWithFlags(&a.s[i], hipStreamNonBlocking));
        for (int i = 0; i < 3; ++i) EXL3_CHECK_HIP(hipEventCreateWithFlags(&a.ev[i], hipEventDisableTiming));
        g_aux[dev] = a;
        g_aux_ok[dev] = true;
    }
    *out = g_aux[dev];
    return EXL3_OK;
}

namespace {
struct ResidentRec {
    int dev;
    const void* fn;
    int threads, blocks;
};
std::vector<ResidentRec> g_resident;
}  // namespace

int resident_blocks(const void* fn, int threads, int* out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ws_mu);
    for (const ResidentRec& r : g_resident)
        if (r.dev == dev && r.fn == fn && r.threads == threads) {
            *out = r.blocks;
            return EXL3_OK;
        }
    int per_cu = 0, cus = 0;
    EXL3_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0));
    EXL3_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int blocks = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    g_resident.push_back({dev, fn, threads, blocks});
    *out = blocks;
    return EXL3_OK;
}

namespace {
std::vector<void*> g_retired[kMaxDevices];   // outgrown workspace buffers, freed by exl3_release_workspace
// Outgrown counter buffers (a subset of g_retired) with their sizes: graphs captured while one of them was current
// still use it, so a timeout reset zeroes them too.
std::vector<std::pair<int*, size_t>> g_retired_counters[kMaxDevices];

__global__ void zero_ints_kernel(int* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

int zero_ints(int* p, size_t n, hipStream_t st) {
    if (!p || !n) return EXL3_OK;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, st, p, n);
    EXL3_CHECK_HIP(hipGetLastError());
    return EXL3_OK;
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
}  // namespace

int workspace(size_t bytes, size_t ncounters, hipStream_t st, Workspace* out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[dev];
    if (!w.status) {
        if (capturing(st))
            return fail(EXL3_ERR_INVALID, "workspace: first use of device %d under stream capture; call "
                                          "exl3_reserve_workspace before capturing", dev);
        int* h = nullptr;
        EXL3_CHECK_HIP(hipHostMalloc(reinterpret_cast<void**>(&h), 64, hipHostMallocMapped | hipHostMallocCoherent));
        *h = 0;
        int* d = nullptr;
        EXL3_CHECK_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&d), h, 0));
        g_status_host[dev] = h;
        w.status = d;
    }
    if (*reinterpret_cast<volatile int*>(g_status_host[dev]) != 0) {
        // A reset recorded into a graph would not run now: under capture the word stays set and the next call
        // outside capture resets.
        if (capturing(st))
            return fail(EXL3_ERR_HIP, "a launch on device %d gave up waiting for its inputs (fused MoE layer: gate|up "
                                      "partials; split-K GEMV: other splits' partials); the counter buffers are reset "
                                      "by the next library call outside stream capture", dev);
        int rc = zero_ints(w.counters, w.ncounters, st);
        for (const auto& c : g_retired_counters[dev])
            if (!rc) rc = zero_ints(c.first, c.second, st);
        if (rc) return rc;
        *reinterpret_cast<volatile int*>(g_status_host[dev]) = 0;
        return fail(EXL3_ERR_HIP, "a launch on device %d gave up waiting for its inputs (fused MoE layer: gate|up "
                                  "partials; split-K GEMV: other splits' partials; its outputs are incomplete, and so "
                                  "may be those of calls queued behind it); every counter buffer has been reset, later "
                                  "calls and graph replays run normally", dev);
    }
    if (bytes > w.scratch_bytes) {
        if (capturing(st))
            return fail(EXL3_ERR_INVALID, "workspace: %zu bytes of scratch needed under stream capture, %zu reserved; "
                                          "call exl3_reserve_workspace before capturing", bytes, w.scratch_bytes);
        size_t nb = bytes + bytes / 4;
        nb = (nb + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        char* p = nullptr;
        EXL3_CHECK_HIP(hipMalloc(&p, nb));
        if (w.scratch) g_retired[dev].push_back(w.scratch);
        w.scratch = p;
        w.scratch_bytes = nb;
    }
    if (ncounters > w.ncounters) {
        if (capturing(st))
            return fail(EXL3_ERR_INVALID, "workspace: %zu counters needed under stream capture, %zu reserved; call "
                                          "exl3_reserve_workspace before capturing", ncounters, w.ncounters);
        size_t nc = ncounters < 65536 ? 65536 : ncounters * 2;
        int* c = nullptr;
        EXL3_CHECK_HIP(hipMalloc(&c, nc * sizeof(int)));
        const int rc = zero_ints(c, nc, st);
        if (rc) {
            (void)hipFree(c);
            return rc;
        }
        if (w.counters) {
            g_retired[dev].push_back(w.counters);
            g_retired_counters[dev].push_back({w.counters, w.ncounters});
        }
        w.counters = c;
        w.ncounters = nc;
    }
    *out = w;
    return EXL3_OK;
}

int spin_limit() { return env_int("EXL3MI_SPIN_LIMIT", 1 << 20); }

namespace {
char* g_auxbuf[kMaxDevices];
size_t g_auxbuf_bytes[kMaxDevices];
}  // namespace

int aux_buffer(size_t bytes, hipStream_t st, void** out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (bytes > g_auxbuf_bytes[dev]) {
        if (capturing(st))
            return fail(EXL3_ERR_INVALID, "aux buffer: %zu bytes needed under stream capture, %zu held; run the call "
                                          "once before capturing", bytes, g_auxbuf_bytes[dev]);
        const size_t nb = ((bytes + bytes / 4) + 4095) & ~(size_t)4095;
        char* p = nullptr;
        EXL3_CHECK_HIP(hipMalloc(&p, nb));
        if (g_auxbuf[dev]) g_retired[dev].push_back(g_auxbuf[dev]);
        g_auxbuf[dev] = p;
        g_auxbuf_bytes[dev] = nb;
    }
    *out = g_auxbuf[dev];
    return EXL3_OK;
}

int device_status(int* out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    *out = g_status_host[dev] ? *reinterpret_cast<volatile int*>(g_status_host[dev]) : 0;
    return EXL3_OK;
}

int release_workspace() {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    EXL3_CHECK_HIP(hipDeviceSynchronize());
    std::lock_guard<std::mutex> lk(g_ws_mu);
    for (void* p : g_retired[dev]) EXL3_CHECK_HIP(hipFree(p));
    g_retired[dev].clear();
    g_retired_counters[dev].clear();
    return EXL3_OK;
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    long x = strtol(v, nullptr, 10);
    return x > 0 && x < (1L << 30) ? (int)x : dflt;
}

namespace {
struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};
bool g_prof_on = false;
int g_prof_rep = 1;
std::vector<hipEvent_t> g_pool;
size_t g_pool_used = 0;
std::vector<ProfRec> g_recs;
bool g_prof_overflow = false;

hipEvent_t take_event() {
    if (g_pool_used == g_pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        g_pool.push_back(e);
    }
    return g_pool[g_pool_used++];
}
}  // namespace

ProfEvents prof_begin(const char* name) {
    if (!g_prof_on) return {nullptr, nullptr};
    if (g_recs.size() >= 100000) {
        g_prof_overflow = true;
        return {nullptr, nullptr};
    }
    ProfRec r{name, take_event(), take_event()};
    if (!r.a || !r.b) return {nullptr, nullptr};
    g_recs.push_back(r);
    return {r.a, r.b};
}

int prof_repeat() { return g_prof_on ? g_prof_rep : 1; }

}  // namespace exl3

extern "C" {

int exl3_profile_enable(int on) {
    exl3::g_prof_on = on != 0;
    exl3::g_prof_rep = on > 1 ? on : 1;
    exl3::g_recs.clear();
    exl3::g_pool_used = 0;
    exl3::g_prof_overflow = false;
    return EXL3_OK;
}

int exl3_profile_read(char* out, int64_t cap) {
    using namespace exl3;
    std::vector<std::pair<std::string, std::pair<double, long>>> agg;
    for (const ProfRec& r : g_recs) {
        EXL3_CHECK_HIP(hipEventSynchronize(r.b));
        float ms = 0.f;
        EXL3_CHECK_HIP(hipEventElapsedTime(&ms, r.a, r.b));
        size_t i = 0;
        while (i < agg.size() && agg[i].first != r.name) ++i;
        if (i == agg.size()) agg.push_back({r.name, {0.0, 0}});
        agg[i].second.first += ms * 1000.0 / g_prof_rep;
        agg[i].second.second += 1;
    }
    std::string txt;
    char line[256];
    for (auto& a : agg) {
        snprintf(line, sizeof(line), "%s %ld %.4f\n", a.first.c_str(), a.second.second,
                 a.second.first / (double)a.second.second);
        txt += line;
    }
    if (cap > 0 && out) {
        size_t n = txt.size() < (size_t)cap - 1 ? txt.size() : (size_t)cap - 1;
        memcpy(out, txt.data(), n);
        out[n] = 0;
    }
    return (int64_t)txt.size() < cap ? EXL3_OK : fail(EXL3_ERR_INVALID, "exl3_profile_read: buffer too small");
}


const char* exl3_last_error(void) { return exl3::g_err; }

int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

int exl3_reserve_workspace(int64_t bytes, int64_t ncounters) {
    if (bytes < 0 || ncounters < 0) return exl3::fail(EXL3_ERR_INVALID, "negative workspace size");
    exl3::Workspace w;
    const int rc = exl3::workspace((size_t)bytes, (size_t)ncounters, nullptr, &w);
    if (rc) return rc;
    EXL3_CHECK_HIP(hipDeviceSynchronize());   // counters zeroed for every stream
    return EXL3_OK;
}

int exl3_device_status(int* status) {
    if (!status) return exl3::fail(EXL3_ERR_INVALID, "exl3_device_status: null output");
    return exl3::device_status(status);
}

int exl3_release_workspace(void) { return exl3::release_workspace(); }

}  // extern "C"
