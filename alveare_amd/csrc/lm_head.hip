// alv_lm_head: the LM head of a decode step on a registered projection --
// logits = softcap(bf16(W x)) over the first `vocab` rows and the greedy
// token, the index of the largest logit.
//
// The reference runs the head as one Q4 GEMV (in 16384-row chunks on the
// NPU, runtime/cpp/src/generator.cpp:28-52; whole in Python,
// runtime/py/model.py:904-916), rounds the logits to bf16 (the GEMV's output
// type), slices them to the vocabulary, applies 30 tanh(x / 30) in float32
// (model.py:915) and picks np.argmax (runtime/py/sampler.py:9: the first
// index of the maximum; NaN counts as the maximum). The C++ generator skips
// the softcap because it is monotonic (generator.cpp:15-26, :48): softcap 0
// here gives those raw bf16 logits.
//
// Three launches: the streaming GEMV (gemv1_q.hip) into `logits` (fp32);
// head_kernel, which rewrites each logit in place and folds each workgroup's
// slice to one (value, index) pair in the stream's scratch; head_fold_kernel,
// one workgroup folding the pairs into the token. The order is total, so the
// token does not depend on the fold's shape. alv_lm_head_bf16 takes the
// activation as bf16 (one MFMA term; the fp32 entry splits its activation
// into three, and a bf16-valued fp32 activation gives the same bits) and can
// advance a device-resident decode position in its last launch.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

constexpr int kHeadThreads = 1024;
constexpr int kHeadGroups = 256;

// (value, index) ordering of np.argmax: NaN above everything (the first NaN
// wins), then larger values, then the smaller index.
__device__ __forceinline__ bool head_better(float v, int i, float bv, int bi) {
    const bool n = v != v, bn = bv != bv;
    if (n != bn) return n;
    if (n) return i < bi;
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void head_fold(float& v, int& i, float ov, int oi) {
    if (head_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// The reference's logit: bf16 of the GEMV's fp32 value, then (cap > 0)
// cap * tanh(l / cap) in float32 -- a correctly rounded divide, tanh of the
// float32 quotient rounded from float64, a float32 product.
__device__ __forceinline__ float head_logit(float y, float cap) {
    const float l = bf16_round(y);
    if (!(cap > 0.0f)) return l;
    const float q = __fdiv_rn(l, cap);
    const float t = (float)tanh((double)q);
    return cap * t;
}

// Fold (v, i) across the workgroup in a fixed tree: shuffles within each
// wave, then wave 0's lane 0 over the waves in order. Returns in thread 0.
__device__ __forceinline__ void head_fold_block(float& v, int& i) {
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(i, o);
        head_fold(v, i, ov, oi);
    }
    __shared__ float sv[kHeadThreads / 64];
    __shared__ int si[kHeadThreads / 64];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = v;
        si[w] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k) head_fold(v, i, sv[k], si[k]);
}

// Each logit rewritten in place; workgroup b's best (value, index) to pair b.
__global__ void __launch_bounds__(kHeadThreads) head_kernel(float* logits, int vocab, float cap, float* pv, int* pi) {
    float bv = -__builtin_inff();
    int bi = 0x7FFFFFFF;  // an empty lane loses to every logit (its index is the largest)
    const int per = (vocab + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * per, hi = min(vocab, lo + per);
    for (int i = lo + threadIdx.x; i < hi; i += kHeadThreads) {
        const float v = head_logit(logits[i], cap);
        logits[i] = v;
        head_fold(bv, bi, v, i);
    }
    head_fold_block(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

// The pairs of head_kernel's `groups` workgroups folded into the token. With
// a position (pos non-null) the token is -1 when *pos >= max_pos, and *pos
// then advances by one.
__global__ void __launch_bounds__(kHeadThreads) head_fold_kernel(const float* pv, const int* pi, int groups,
                                                                int32_t* argmax, int32_t* pos, int max_pos) {
    float v = -__builtin_inff();
    int i = 0x7FFFFFFF;
    for (int b = threadIdx.x; b < groups; b += kHeadThreads) head_fold(v, i, pv[b], pi[b]);
    head_fold_block(v, i);
    if (threadIdx.x == 0) {
        if (pos) {
            const int p = *pos;
            if (p >= max_pos) i = -1;
            *pos = p + 1;
        }
        *argmax = i;
    }
}

}  // namespace

}  // namespace alv

using namespace alv;

namespace {

int lm_head(alv_weight_t w, const float* x, const uint16_t* xb, float* logits, int vocab, float softcap,
            int32_t* argmax, int32_t* pos, int max_pos, void* stream, const ResidStep* step = nullptr) {
    if (!w || w->magic != kWeightMagic) return fail(ALV_ERR_HANDLE, "invalid weight handle");
    if ((!x && !xb) || !logits || !argmax) return fail(ALV_ERR_ARG, "null pointer");
    if (vocab < 1 || vocab > w->N) return fail(ALV_ERR_ARG, "vocab=%d outside the head's %d rows", vocab, w->N);
    if (!(softcap >= 0.0f) || softcap == __builtin_inff())
        return fail(ALV_ERR_ARG, "softcap must be 0 (none) or a positive finite cap");
    if (reinterpret_cast<uintptr_t>(logits) % 4 || reinterpret_cast<uintptr_t>(argmax) % 4 ||
        reinterpret_cast<uintptr_t>(pos) % 4)
        return fail(ALV_ERR_ALIGN, "logits, argmax and pos need 4-byte alignment");
    if (x ? reinterpret_cast<uintptr_t>(x) % 4 : reinterpret_cast<uintptr_t>(xb) % 16)
        return fail(ALV_ERR_ALIGN, "x needs 4-byte (fp32) or 16-byte (bf16) alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "weight handle belongs to device %d, current device is %d", w->device, dev);
    hipStream_t s = (hipStream_t)stream;
    void* part = nullptr;
    if (int rc = get_scratch(s, kScratchHead, 2 * kHeadGroups * sizeof(float), &part)) return rc;
    float* pv = static_cast<float*>(part);
    int* pi = reinterpret_cast<int*>(pv + kHeadGroups);
    // The GEMV over the first `vocab` rows (rows are independent).
    GemvLaunch L;
    weight_launch(w, L);
    L.X = x;
    L.Xb = xb;
    L.ldx = w->K;
    L.Y = logits;
    L.ldy = vocab;
    L.M = 1;
    L.N = std::min(vocab, w->Ne);  // rows past the registered extent are zero logits
    L.Nz = vocab;
    L.parts = xb ? 1 : 3;
    L.step = step;
    if (int rc = launch_gemv(L, s)) return rc;
    const int groups = std::min(kHeadGroups, (vocab + 63) / 64);
    hipLaunchKernelGGL(head_kernel, dim3(groups), dim3(kHeadThreads), 0, s, logits, vocab, softcap, pv, pi);
    if (int rc = hip_check(hipGetLastError(), "head_kernel launch")) return rc;
    hipLaunchKernelGGL(head_fold_kernel, dim3(1), dim3(kHeadThreads), 0, s, pv, pi, groups, argmax, pos, max_pos);
    return hip_check(hipGetLastError(), "head_fold_kernel launch");
}

}  // namespace

extern "C" int alv_lm_head(alv_weight_t w, const float* x, float* logits, int vocab, float softcap,
                           int32_t* argmax, void* stream) {
    if (!x) return fail(ALV_ERR_ARG, "null pointer");
    return lm_head(w, x, nullptr, logits, vocab, softcap, argmax, nullptr, 0, stream);
}

extern "C" int alv_lm_head_bf16(alv_weight_t w, const uint16_t* x, float* logits, int vocab, float softcap,
                                int32_t* argmax, int32_t* pos_dev, int max_pos, void* stream) {
    if (!x) return fail(ALV_ERR_ARG, "null pointer");
    return lm_head(w, nullptr, x, logits, vocab, softcap, argmax, pos_dev, max_pos, stream);
}

extern "C" int alv_lm_head_bf16_addnorm(alv_weight_t w, const uint16_t* resid, const uint16_t* y, const float* w_y,
                                        int norm_y, float scale, int scale_mode, uint16_t* sum_out, const float* w_x,
                                        float eps, int hidden, float* logits, int vocab, float softcap,
                                        int32_t* argmax, int32_t* pos_dev, int max_pos, void* stream) {
    if (!resid) return fail(ALV_ERR_ARG, "null pointer");
    if (!w || w->magic != kWeightMagic) return fail(ALV_ERR_HANDLE, "invalid weight handle");
    if (hidden < 8 || hidden > w->K)
        return fail(ALV_ERR_ARG, "hidden=%d outside [8, the head's K=%d]", hidden, w->K);
    ResidStep st;
    st.resid = resid;
    st.y = y;
    st.w_y = w_y;
    st.norm_y = norm_y;
    st.scale = scale;
    st.scale_mode = scale_mode;
    st.sum_out = sum_out;
    st.w_x = w_x;
    st.eps = eps;
    st.k = hidden;
    return lm_head(w, nullptr, y ? y : resid, logits, vocab, softcap, argmax, pos_dev, max_pos, stream, &st);
}
