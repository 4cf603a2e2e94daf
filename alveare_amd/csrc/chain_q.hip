// alv_chain_run / alv_check_async: a sequence of registered projections and
// FFN layers enqueued in one call -- the device-resident form of the
// reference's per-layer dispatch, where the host calls run_gemv /
// run_ffn_fused one after another and waits on each
// (runtime/cpp/src/model.cpp:265-420, runtime/py/model.py:632-818). By default
// the ops run as separate one-shot launches in stream order; with
// ALV_CHAIN_FUSED=1 they run as few launches of the op-chain executor
// (stream_q.hip), each op waiting on the device for the op whose output it
// reads.
#include <stdlib.h>

#include <algorithm>
#include <vector>

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

namespace {

// The ops one after another on the stream (stream order satisfies every dep).
int run_ops(const alv_chain_op* ops, int n, int M, hipStream_t s) {
    for (int i = 0; i < n; ++i) {
        const alv_chain_op& c = ops[i];
        if (c.weight) {
            GemvLaunch L;
            L.W0 = c.weight->w;
            L.X = c.x;
            L.ldx = c.weight->K;
            L.Y = c.y;
            L.ldy = c.weight->N;
            L.M = M;
            L.N = c.weight->N;
            L.K = c.weight->K;
            L.parts = 3;
            L.tiled = true;
            if (int rc = launch_gemv(L, s)) return rc;
        } else {
            if ((size_t)M * c.ffn->I > c.ffn->a_cap) return fail(ALV_ERR_ARG, "chain op %d: FFN scratch holds %zu activations", i, c.ffn->a_cap);
            ExecOp two[2];
            ffn_ops(c.ffn, c.x, c.ffn->H, c.y, c.ffn->H, M, two);
            if (int rc = launch_gemv(two[0], s)) return rc;
            if (int rc = launch_gemv(two[1], s)) return rc;
            c.ffn->a_rows = M;
        }
    }
    return ALV_OK;
}

// Expand into executor ops and cut into launches of at most kMaxOps. An op
// whose producer ran in an earlier launch needs no wait (stream order); an FFN
// handle appears at most once per launch (it owns its scratch).
int run_fused(const alv_chain_op* ops, int n, int M, hipStream_t s) {
    std::vector<ExecOp> cur;
    std::vector<int> last_exec(n, -1);  // executor index of chain op i's output in the current launch
    std::vector<alv_ffn_t> ffns;
    int base = 0;  // first chain op of the current launch
    auto flush = [&](int upto) -> int {
        if (cur.empty()) return ALV_OK;
        if (int rc = exec_chain(cur.data(), (int)cur.size(), true, s)) return rc;
        for (alv_ffn_t f : ffns) f->a_rows = M;
        cur.clear();
        ffns.clear();
        base = upto;
        return ALV_OK;
    };
    for (int i = 0; i < n; ++i) {
        const alv_chain_op& c = ops[i];
        const int need = c.ffn ? 2 : 1;
        const bool repeat = c.ffn && std::find(ffns.begin(), ffns.end(), c.ffn) != ffns.end();
        if ((int)cur.size() + need > kMaxOps || repeat)
            if (int rc = flush(i)) return rc;
        const int dep = c.dep >= base ? last_exec[c.dep] : -1;
        if (c.weight) {
            ExecOp op{};
            op.W0 = c.weight->w;
            op.X = c.x;
            op.ldx = c.weight->K;
            op.Y = c.y;
            op.ldy = c.weight->N;
            op.M = M;
            op.N = c.weight->N;
            op.K = c.weight->K;
            op.parts = 3;
            op.tiled = true;
            op.dep = dep;
            cur.push_back(op);
        } else {
            if ((size_t)M * c.ffn->I > c.ffn->a_cap) return fail(ALV_ERR_ARG, "chain op %d: FFN scratch holds %zu activations", i, c.ffn->a_cap);
            ExecOp two[2];
            ffn_ops(c.ffn, c.x, c.ffn->H, c.y, c.ffn->H, M, two);
            two[0].dep = dep;
            two[1].dep = (int)cur.size();
            cur.push_back(two[0]);
            cur.push_back(two[1]);
            ffns.push_back(c.ffn);
        }
        last_exec[i] = (int)cur.size() - 1;
    }
    return flush(n);
}

}  // namespace

extern "C" int alv_chain_run(const alv_chain_op* ops, int n, int M, void* stream) {
    if (!ops || n < 1) return fail(ALV_ERR_ARG, "empty chain");
    if (M < 1 || M > kGemvMaxM) return fail(ALV_ERR_ARG, "chains take 1 <= M <= %d tokens (got %d)", kGemvMaxM, M);
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    for (int i = 0; i < n; ++i)
        if (int rc = check_op(ops[i], i, dev)) return rc;
    // Separate one-shot launches measure faster than the fused executor on
    // the decode shapes; ALV_CHAIN_FUSED=1 selects the fused executor.
    const char* e = getenv("ALV_CHAIN_FUSED");
    if (e && e[0] == '1') return run_fused(ops, n, M, (hipStream_t)stream);
    return run_ops(ops, n, M, (hipStream_t)stream);
}

extern "C" int alv_check_async(void* stream) { return check_async((hipStream_t)stream); }
