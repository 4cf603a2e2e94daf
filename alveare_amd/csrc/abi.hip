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

int get_workspace(hipStream_t s, size_t partial_floats, size_t counters, Workspace* out) {
    int dev = 0;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[{dev, s}];
    if (w.partial_floats < partial_floats || w.counter_count < counters) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (int rc = hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing")) return rc;
        if (cs != hipStreamCaptureStatusNone)
            return fail(ALV_ERR_ARG,
                        "split-K workspace of this stream must grow, which cannot happen during graph "
                        "capture: run the same call once on this stream before capturing");
        // The old buffers may still be read by queued kernels.
        if (int rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
        size_t pf = w.partial_floats > partial_floats ? w.partial_floats : partial_floats;
        size_t cc = w.counter_count > counters ? w.counter_count : counters;
        if (w.partial) (void)hipFree(w.partial);
        if (w.counters) (void)hipFree(w.counters);
        w = Workspace{};
        if (pf && hipMalloc(&w.partial, pf * sizeof(float)) != hipSuccess)
            return fail(ALV_ERR_HIP, "hipMalloc of %zu partial floats failed", pf);
        if (cc) {
            if (hipMalloc(&w.counters, cc * sizeof(uint32_t)) != hipSuccess)
                return fail(ALV_ERR_HIP, "hipMalloc of %zu counters failed", cc);
            if (int rc = hip_check(hipMemset(w.counters, 0, cc * sizeof(uint32_t)), "hipMemset"))
                return rc;
        }
        w.partial_floats = pf;
        w.counter_count = cc;
    }
    *out = w;
    return ALV_OK;
}

}  // namespace alv

extern "C" const char* alv_last_error(void) { return alv::g_err; }

extern "C" const char* alv_version(void) { return "alveare_q4 1.0 gfx950"; }
