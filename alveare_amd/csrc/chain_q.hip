// alv_chain_run: a sequence of registered projections and FFN layers enqueued
// in one call -- the device-resident form of the reference's per-layer
// dispatch, where the host calls run_gemv / run_ffn_fused one after another
// and waits on each (runtime/cpp/src/model.cpp:265-420,
// runtime/py/model.py:632-818). The ops run as ordinary launches in stream
// order, which satisfies every dependency; the host never waits between them.
#include "q4_device.h"
#include "q4_host.h"

using namespace alv;

namespace {

int check_op(const alv_chain_op& c, int i, int dev) {
    const bool is_w = c.weight != nullptr, is_f = c.ffn != nullptr;
    if (is_w == is_f) return fail(ALV_ERR_ARG, "chain op %d needs exactly one of weight and ffn", i);
    if (is_w && c.weight->magic != kWeightMagic) return fail(ALV_ERR_HANDLE, "chain op %d: invalid weight handle", i);
    if (is_f && c.ffn->magic != kFfnMagic) return fail(ALV_ERR_HANDLE, "chain op %d: invalid FFN handle", i);
    const int hdev = is_w ? c.weight->device : c.ffn->device;
    if (hdev != dev) return fail(ALV_ERR_HANDLE, "chain op %d: handle belongs to device %d, current device is %d", i, hdev, dev);
    if (!c.x || !c.y) return fail(ALV_ERR_ARG, "chain op %d: null activation pointer", i);
    if (reinterpret_cast<uintptr_t>(c.x) % 4 || reinterpret_cast<uintptr_t>(c.y) % 4)
        return fail(ALV_ERR_ALIGN, "chain op %d: x and y need 4-byte alignment", i);
    if (c.dep >= i) return fail(ALV_ERR_ARG, "chain op %d depends on op %d, not an earlier one", i, c.dep);
    return ALV_OK;
}

}  // namespace

extern "C" int alv_chain_run(const alv_chain_op* ops, int n, int M, void* stream) {
    if (!ops || n < 1) return fail(ALV_ERR_ARG, "empty chain");
    if (M < 1 || M > kGemvMaxM) return fail(ALV_ERR_ARG, "chains take 1 <= M <= %d tokens (got %d)", kGemvMaxM, M);
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    for (int i = 0; i < n; ++i)
        if (int rc = check_op(ops[i], i, dev)) return rc;
    hipStream_t s = (hipStream_t)stream;
    for (int i = 0; i < n; ++i) {
        const alv_chain_op& c = ops[i];
        if (c.weight) {
            GemvLaunch L;
            weight_launch(c.weight, L);
            L.X = c.x;
            L.ldx = c.weight->K;
            L.Y = c.y;
            L.ldy = c.weight->N;
            L.M = M;
            L.parts = 3;
            if (int rc = launch_gemv(L, s)) return rc;
        } else {
            GemvLaunch two[2];
            ffn_ops(c.ffn, c.ffn->a, c.x, c.ffn->H, c.y, c.ffn->H, M, two);
            if (int rc = launch_gemv(two[0], s)) return rc;
            if (int rc = launch_gemv(two[1], s)) return rc;
            c.ffn->last_a = c.ffn->a;
            c.ffn->a_rows = M;
        }
    }
    return ALV_OK;
}
