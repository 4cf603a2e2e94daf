// Error reporting and per-stream workspace of libalveare_q4.
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>
#include <utility>

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
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
}  // namespace

int get_workspace(hipStream_t s, size_t counters, Workspace* out) {
    int dev = 0;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[{dev, s}];
    if (w.counter_count < counters) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (int rc = hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing")) return rc;
        if (cs != hipStreamCaptureStatusNone)
            return fail(ALV_ERR_ARG,
                        "the synchronisation words of this stream are allocated on its first call, which "
                        "cannot happen during graph capture: run one call on this stream before capturing");
        // The old words may still be used by queued kernels.
        if (int rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
        if (w.counters) (void)hipFree(w.counters);
        w = Workspace{};
        if (hipMalloc(&w.counters, counters * sizeof(uint32_t)) != hipSuccess)
            return fail(ALV_ERR_HIP, "hipMalloc of %zu counters failed", counters);
        if (int rc = hip_check(hipMemset(w.counters, 0, counters * sizeof(uint32_t)), "hipMemset")) return rc;
        w.counter_count = counters;
    }
    *out = w;
    return ALV_OK;
}

}  // namespace alv

extern "C" const char* alv_last_error(void) { return alv::g_err; }

extern "C" const char* alv_version(void) { return "alveare_q4 1.0 gfx950"; }
