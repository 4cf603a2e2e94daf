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
__global__ void __launch_bounds__(256) tile_kernel(const uint8_t* W, uint32_t* out, int N, int K, uint32_t W_rs) {
    const TileGeom tg = tile_geom(K);
    const uint32_t rs = (uint32_t)tg.nb * kBlockBytes;  // bytes of a row's K columns
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
        if (row < N && src < rs) v = *reinterpret_cast<const uint32_t*>(W + (size_t)row * W_rs + src);
        out[d] = v;
    }
}

// Nonzero extent of a combined-layout matrix (weight_extent): each thread
// folds the blocks it visits into (last row, last block) with a nonzero
// weight, the workgroup reduces, and one atomic max per workgroup and value
// publishes it (ext must be zero before the launch).
__global__ void __launch_bounds__(256) extent_kernel(const uint8_t* W, int N, int nb, uint32_t rs, int* ext) {
    int lr = 0, lb = 0;  // 1 + last row / block seen holding a nonzero weight
    const int64_t total = (int64_t)N * nb;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int row = (int)(i / nb);
        const int b = (int)(i - (int64_t)row * nb);
        const uint32_t* d = reinterpret_cast<const uint32_t*>(W + (size_t)row * rs + (size_t)b * kBlockBytes);
        const uint32_t codes = d[0] | d[1] | d[2] | d[3];
        const uint32_t sc = d[4] & 0xFFFFu;  // the bf16 scale, bytes 16-17
        const bool zero = (sc & 0x7FFFu) == 0u || (codes == 0u && (sc & 0x7F80u) != 0x7F80u);
        if (!zero) {
            lr = max(lr, row + 1);
            lb = max(lb, b + 1);
        }
    }
    __shared__ int red[2][4];
    for (int o = 32; o > 0; o >>= 1) {
        lr = max(lr, __shfl_xor(lr, o));
        lb = max(lb, __shfl_xor(lb, o));
    }
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = lr;
        red[1][threadIdx.x >> 6] = lb;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        lr = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
        lb = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
        if (lr) atomicMax(ext, lr);
        if (lb) atomicMax(ext + 1, lb);
    }
}

}  // namespace

uint64_t tile_bytes(int N, int K) { return (uint64_t)((N + 15) / 16) * tile_geom(K).rtb; }

int launch_tile(const uint8_t* W, uint8_t* out, int N, int K, hipStream_t s, uint32_t rs) {
    const uint64_t dwords = tile_bytes(N, K) / 4;
    const int grid = (int)std::min<uint64_t>((dwords + 255) / 256, 16384);
    if (!rs) rs = (uint32_t)(K / kBlockK) * kBlockBytes;
    hipLaunchKernelGGL(tile_kernel, dim3(grid), dim3(256), 0, s, W, reinterpret_cast<uint32_t*>(out), N, K, rs);
    return hip_check(hipGetLastError(), "tile_kernel launch");
}

int weight_extent(const uint8_t* W, int N, int K, uint32_t rs, hipStream_t s, int ext[2]) {
    ext[0] = ext[1] = 0;
    int* d = nullptr;
    int rc = hip_check(hipMalloc(&d, 2 * sizeof(int)), "hipMalloc(extent)");
    if (!rc) rc = hip_check(hipMemsetAsync(d, 0, 2 * sizeof(int), s), "hipMemsetAsync(extent)");
    if (!rc) {
        const int nb = K / kBlockK;
        const int64_t total = (int64_t)N * nb;
        const int grid = (int)std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, 2048));
        hipLaunchKernelGGL(extent_kernel, dim3(grid), dim3(256), 0, s, W, N, nb, rs, d);
        rc = hip_check(hipGetLastError(), "extent_kernel launch");
    }
    if (!rc) rc = hip_check(hipMemcpyAsync(ext, d, 2 * sizeof(int), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(extent)");
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (d) (void)hipFree(d);
    return rc;
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
    const uint32_t rs = (uint32_t)(K / kBlockK) * kBlockBytes;
    int ext[2] = {0, 0};
    int rc = hip_check(hipGetDevice(&h->device), "hipGetDevice");
    if (!rc) rc = weight_extent(W, N, K, rs, s, ext);
    // At least one row and one block stay, so an all-zero matrix still runs.
    h->Ne = std::max(1, ext[0]);
    h->Ke = kBlockK * std::max(1, ext[1]);
    if (!rc) rc = hip_check(hipMalloc(&h->w, tile_bytes(h->Ne, h->Ke)), "hipMalloc(weights)");
    if (!rc) rc = launch_tile(W, h->w, h->Ne, h->Ke, s, rs);
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

extern "C" int alv_weight_exec_shape(alv_weight_t w, int* N, int* K) {
    if (int rc = check_weight(w)) return rc;
    if (N) *N = w->Ne;
    if (K) *K = w->Ke;
    return ALV_OK;
}

namespace alv {

// The launch of a registered matrix: the executed (trimmed) shape, with the
// trimmed rows written as zeros up to the logical N.
void weight_launch(const alv_weight* w, GemvLaunch& L) {
    L.W0 = w->w;
    L.N = w->Ne;
    L.K = w->Ke;
    L.Nz = w->N;
    L.tiled = true;
}

}  // namespace alv

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
    weight_launch(w, L);
    L.ldx = ldx;
    L.ldy = ldy;
    L.parts = 3;
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
    weight_launch(w, L);
    L.ldx = ldx;
    L.ldy = ldy;
    L.parts = 1;
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
    if (w->Ke != w->K)
        return fail(ALV_ERR_ARG, "a fused residual step needs the whole row: this matrix registered with its "
                    "trailing all-zero columns trimmed (K=%d executed as %d)", w->K, w->Ke);
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
    weight_launch(w, L);
    L.Xb = y ? y : resid;
    L.ldx = w->K;
    L.Yb = Y;
    L.ldy = w->N;
    L.M = 1;
    L.parts = 1;
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
