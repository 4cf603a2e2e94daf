// Registration-time repack of Q4 weights into the kernels' tiled layout
// (q4_device.h::TileGeom) and the registered-weight entry points
// alv_q4_tiled_bytes / alv_q4_tile / alv_weight_register / alv_weight_shape /
// alv_gemv / alv_weight_release.
//
// The repack is a pure byte permutation of the combined layout plus zero
// padding of the last 128-column run and the last row tile (the reference does
// the same kind of registration-time permutation for its FFN weights,
// runtime/cpp/src/weights.cpp:94-190).
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

// One thread per output dword. A dword of the tiled layout is 4 consecutive
// bytes of one row's 80-byte run, so it is one aligned dword of the source row
// (or zero past the row / matrix end).
__global__ void __launch_bounds__(256) tile_kernel(const uint8_t* W, uint32_t* out, int N, int K) {
    const TileGeom tg = tile_geom(K);
    const uint32_t rs = (uint32_t)tg.nb * kBlockBytes;
    const int RT = (N + 15) / 16;
    const uint64_t total = (uint64_t)RT * tg.rtb / 4;
    for (uint64_t d = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; d < total;
         d += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t byte = d * 4;
        const int rt = (int)(byte / tg.rtb);
        const uint32_t off = (uint32_t)(byte - (uint64_t)rt * tg.rtb);
        const int ss = min((int)(off / 5120u), tg.nss - 1);
        const uint32_t toff = off - (uint32_t)ss * 5120u;
        const int ng = ss == tg.nss - 1 ? tg.ng_last : 4;
        const uint32_t pstride = 256u * (uint32_t)ng;
        const uint32_t i = toff / pstride;
        const uint32_t within = toff - i * pstride;
        const uint32_t lane = within / 16;
        const int g = (int)(lane / 16), j = (int)(lane % 16);
        const int row = rt * 16 + j;
        const uint32_t src = (uint32_t)(ss * 16 + g * 4) * kBlockBytes + i * 16 + (within % 16);
        uint32_t v = 0;
        if (row < N && src < rs) v = *reinterpret_cast<const uint32_t*>(W + (size_t)row * rs + src);
        out[d] = v;
    }
}

}  // namespace

uint64_t tile_bytes(int N, int K) { return (uint64_t)((N + 15) / 16) * tile_geom(K).rtb; }

int launch_tile(const uint8_t* W, uint8_t* out, int N, int K, hipStream_t s) {
    const uint64_t dwords = tile_bytes(N, K) / 4;
    const int grid = (int)std::min<uint64_t>((dwords + 255) / 256, 16384);
    hipLaunchKernelGGL(tile_kernel, dim3(grid), dim3(256), 0, s, W, reinterpret_cast<uint32_t*>(out), N, K);
    return hip_check(hipGetLastError(), "tile_kernel launch");
}

}  // namespace alv

using namespace alv;


namespace {


int check_weight(alv_weight_t w) {
    if (!w || w->magic != kWeightMagic) return fail(ALV_ERR_HANDLE, "invalid weight handle");
    return ALV_OK;
}

int check_shape(int N, int K) {
    if (N < 1 || K < 32 || K % 32) return fail(ALV_ERR_ARG, "bad shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
    if (tile_bytes(N, K) >= 0xFFFFE000ull) return fail(ALV_ERR_RANGE, "weight matrix exceeds the 4 GiB buffer range");
    return ALV_OK;
}

}  // namespace

extern "C" uint64_t alv_q4_tiled_bytes(int N, int K) {
    if (N < 1 || K < 32 || K % 32) return 0;
    return tile_bytes(N, K);
}

extern "C" int alv_q4_tile(const uint8_t* W, uint8_t* out, int N, int K, void* stream) {
    if (!W || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (int rc = check_shape(N, K)) return rc;
    if (reinterpret_cast<uintptr_t>(W) % 4 || reinterpret_cast<uintptr_t>(out) % 4)
        return fail(ALV_ERR_ALIGN, "W and out need 4-byte alignment");
    return launch_tile(W, out, N, K, (hipStream_t)stream);
}

extern "C" int alv_weight_register(const uint8_t* W, int N, int K, alv_weight_t* out, void* stream) {
    if (!out) return fail(ALV_ERR_ARG, "null output handle pointer");
    *out = nullptr;
    if (!W) return fail(ALV_ERR_ARG, "null weight pointer");
    if (int rc = check_shape(N, K)) return rc;
    if (reinterpret_cast<uintptr_t>(W) % 4) return fail(ALV_ERR_ALIGN, "W needs 4-byte alignment");
    hipStream_t s = (hipStream_t)stream;
    alv_weight* h = new alv_weight{};
    h->magic = kWeightMagic;
    h->N = N;
    h->K = K;
    int rc = hip_check(hipGetDevice(&h->device), "hipGetDevice");
    if (!rc) rc = hip_check(hipMalloc(&h->w, tile_bytes(N, K)), "hipMalloc(weights)");
    if (!rc) rc = launch_tile(W, h->w, N, K, s);
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (rc) {
        if (h->w) (void)hipFree(h->w);
        h->magic = 0;
        delete h;
        return rc;
    }
    *out = h;
    return ALV_OK;
}

extern "C" int alv_weight_shape(alv_weight_t w, int* N, int* K) {
    if (int rc = check_weight(w)) return rc;
    if (N) *N = w->N;
    if (K) *K = w->K;
    return ALV_OK;
}

extern "C" int alv_gemv(alv_weight_t w, const float* X, float* Y, int M, int ldx, int ldy, void* stream) {
    if (int rc = check_weight(w)) return rc;
    if (!X || !Y) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || ldx < w->K || ldy < w->N)
        return fail(ALV_ERR_ARG, "bad M=%d ldx=%d ldy=%d for N=%d K=%d", M, ldx, ldy, w->N, w->K);
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(Y) % 4)
        return fail(ALV_ERR_ALIGN, "X and Y need 4-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "weight handle belongs to device %d, current device is %d", w->device, dev);
    GemvLaunch L;
    L.W0 = w->w;
    L.ldx = ldx;
    L.ldy = ldy;
    L.N = w->N;
    L.K = w->K;
    L.parts = 3;
    L.tiled = true;
    hipStream_t s = (hipStream_t)stream;
    if (M >= tiled_min_m(true)) {
        L.X = X;
        L.Y = Y;
        L.M = M;
        return launch_gemm_tiled(L, s);
    }
    for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
        L.X = X + (size_t)m0 * ldx;
        L.Y = Y + (size_t)m0 * ldy;
        L.M = std::min(kGemvMaxM, M - m0);
        if (int rc = launch_gemv(L, s)) return rc;
    }
    return ALV_OK;
}

extern "C" int alv_gemv_bf16(alv_weight_t w, const uint16_t* X, uint16_t* Y, int M, int ldx, int ldy, void* stream) {
    if (int rc = check_weight(w)) return rc;
    if (!X || !Y) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || ldx < w->K || ldy < w->N)
        return fail(ALV_ERR_ARG, "bad M=%d ldx=%d ldy=%d for N=%d K=%d", M, ldx, ldy, w->N, w->K);
    if (reinterpret_cast<uintptr_t>(X) % 16 || ldx % 8 || reinterpret_cast<uintptr_t>(Y) % 2)
        return fail(ALV_ERR_ALIGN, "X needs 16-byte aligned rows (ldx a multiple of 8), Y 2-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "weight handle belongs to device %d, current device is %d", w->device, dev);
    GemvLaunch L;
    L.W0 = w->w;
    L.ldx = ldx;
    L.ldy = ldy;
    L.N = w->N;
    L.K = w->K;
    L.parts = 1;
    L.tiled = true;
    hipStream_t s = (hipStream_t)stream;
    if (M >= tiled_min_m(false)) {
        L.Xb = X;
        L.Yb = Y;
        L.M = M;
        return launch_gemm_tiled(L, s);
    }
    for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
        L.Xb = X + (size_t)m0 * ldx;
        L.Yb = Y + (size_t)m0 * ldy;
        L.M = std::min(kGemvMaxM, M - m0);
        if (int rc = launch_gemv(L, s)) return rc;
    }
    return ALV_OK;
}

extern "C" int alv_gemv_bf16_addnorm(alv_weight_t w, const uint16_t* resid, const uint16_t* y, const float* w_y,
                                     int norm_y, float scale, int scale_mode, uint16_t* sum_out, const float* w_x,
                                     float eps, uint16_t* Y, void* stream) {
    if (int rc = check_weight(w)) return rc;
    if (!Y) return fail(ALV_ERR_ARG, "null output pointer");
    if (reinterpret_cast<uintptr_t>(Y) % 2) return fail(ALV_ERR_ALIGN, "Y needs 2-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "weight handle belongs to device %d, current device is %d", w->device, dev);
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
    GemvLaunch L;
    L.W0 = w->w;
    L.Xb = y;
    L.ldx = w->K;
    L.Yb = Y;
    L.ldy = w->N;
    L.M = 1;
    L.N = w->N;
    L.K = w->K;
    L.parts = 1;
    L.tiled = true;
    L.step = &st;
    return launch_gemv(L, (hipStream_t)stream);
}

extern "C" void alv_weight_release(alv_weight_t w) {
    if (!w || w->magic != kWeightMagic) return;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (cur != w->device) (void)hipSetDevice(w->device);
    (void)hipDeviceSynchronize();
    if (w->w) (void)hipFree(w->w);
    if (cur >= 0 && cur != w->device) (void)hipSetDevice(cur);
    w->magic = 0;
    delete w;
}
