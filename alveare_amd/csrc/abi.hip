// Error reporting and per-stream workspace of libalveare_q4.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>
#include <vector>
#include <algorithm>

#include "q4_host.h"

namespace alv {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return ALV_OK;
    return fail(ALV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {
// Split-K arrival counters: one block per device holding
// kWsStreams sets, handed out to streams on first use. The blocks are
// allocated (the words zeroed) at the first call on the device; a stream's
// later first use takes a set without allocating, so it may happen during
// graph capture.
constexpr int kWsStreams = 64;
std::mutex g_ws_mu;
struct DeviceWs {
    uint32_t* block = nullptr;
    size_t words = 0;  // per set
    std::map<hipStream_t, int> slot;
};
std::map<int, DeviceWs> g_ws;
}  // namespace

int get_workspace(hipStream_t s, size_t counters, Workspace* out) {
    int dev = 0;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    DeviceWs& w = g_ws[dev];
    if (!w.block) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (int rc = hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing")) return rc;
        if (cs != hipStreamCaptureStatusNone)
            return fail(ALV_ERR_ARG,
                        "the split-K counters of this device are allocated on its first call, which cannot "
                        "happen during graph capture: run one call on this device before capturing");
        const size_t all = (size_t)kSplitCounters;
        const size_t words = counters > all ? counters : all;
        if (hipMalloc(&w.block, words * kWsStreams * sizeof(uint32_t)) != hipSuccess) {
            w.block = nullptr;
            return fail(ALV_ERR_HIP, "hipMalloc of the split-K counters failed");
        }
        if (int rc = hip_check(hipMemset(w.block, 0, words * kWsStreams * sizeof(uint32_t)), "hipMemset")) return rc;
        w.words = words;
    }
    if (counters > w.words) return fail(ALV_ERR_ARG, "%zu counters requested, %zu available", counters, w.words);
    auto it = w.slot.find(s);
    int idx;
    if (it != w.slot.end()) {
        idx = it->second;
    } else {
        if ((int)w.slot.size() >= kWsStreams)
            return fail(ALV_ERR_ARG, "more than %d streams use split-K launches on device %d", kWsStreams, dev);
        idx = (int)w.slot.size();
        w.slot[s] = idx;
    }
    out->counters = w.block + (size_t)idx * w.words;
    out->counter_count = w.words;
    return ALV_OK;
}

namespace {
// A slot's current block and the blocks it outgrew. An outgrown block is never
// freed: a HIP graph captured while it was current keeps its address in the
// captured kernel arguments and may be replayed at any later time. Capacity at
// least doubles on each growth, so the retired blocks of a slot total less than
// its current one.
struct Scratch {
    void* p = nullptr;
    size_t cap = 0;
    std::vector<void*> retired;
};
std::map<std::tuple<int, hipStream_t, int>, Scratch> g_scratch;
}  // namespace

int get_scratch(hipStream_t s, int slot, size_t bytes, void** out) {
    int dev = 0;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Scratch& sc = g_scratch[{dev, s, slot}];
    if (bytes > sc.cap) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (int rc = hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing")) return rc;
        if (cs != hipStreamCaptureStatusNone)
            return fail(ALV_ERR_ARG, "scratch of %zu bytes must grow, which cannot happen during graph capture: "
                        "run one call of this shape on this stream before capturing", bytes);
        size_t cap = std::max(bytes, 2 * sc.cap);
        cap = (cap + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        void* p = nullptr;
        if (int rc = hip_check(hipMalloc(&p, cap), "hipMalloc(scratch)")) return rc;
        if (int rc = hip_check(hipMemsetAsync(p, 0, cap, s), "hipMemsetAsync(scratch)")) {
            (void)hipFree(p);
            return rc;
        }
        if (sc.p) sc.retired.push_back(sc.p);
        sc.p = p;
        sc.cap = cap;
    }
    *out = sc.p;
    return ALV_OK;
}

int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

int small_wg_per_cu() {
    const char* e = getenv("ALV_GEMM_SMALL_WG_PER_CU");
    if (!e || !*e) return 1;
    const long v = strtol(e, nullptr, 10);
    return v >= 1 && v <= 16 ? (int)v : 1;
}

int small_tile_max_m() {
    const char* e = getenv("ALV_GEMM_SMALL_TILE_MAX_M");
    if (!e || !*e) return kSmallTileMaxM;
    const long v = strtol(e, nullptr, 10);
    return v >= 0 && v <= (1 << 30) ? (int)v : kSmallTileMaxM;
}

int tiled_min_m(bool fp32_x) {
    const int dflt = fp32_x ? kTiledMinMF32 : kTiledMinMBf16;
    const char* e = getenv("ALV_TILED_MIN_M");
    if (!e || !*e) return dflt;
    const long v = strtol(e, nullptr, 10);
    return v >= 1 && v <= (1 << 30) ? (int)v : dflt;
}

}  // namespace alv

extern "C" const char* alv_last_error(void) { return alv::g_err; }

extern "C" const char* alv_version(void) { return "alveare_q4 1.0 gfx950"; }
