// Fused FFN (gate/up projection, GLU activation, down projection) on gfx950:
// alv_ffn_register / alv_ffn_fused / alv_ffn_shape / alv_ffn_release.
//
// Decode (M <= 16): two launches of the streaming kernel (gemv_q.hip).
//   1. gate and up rows of one 16-row I-tile are streamed together by the same
//      waves against the same activation operands; the epilogue rounds both to
//      bf16, applies the GLU and rounds the activation to bf16 -- the
//      reference CPU path's three rounding points (runtime/py/model.py:798-803).
//      The activation (M x I bf16) stays in the handle's scratch, which is
//      L2/MALL-resident at these sizes.
//   2. down = Wd * a, with a single bf16 term per activation value (it is
//      bf16 by construction), summed entirely on the device -- the reference
//      sums per-core partials on the host (runtime/cpp/src/npu.cpp:360-377).
// Prefill (M >= 32): the same two steps with the MFMA tiled kernel (gemm_q.hip).
#include <string.h>

#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

struct alv_ffn {
    uint32_t magic;
    int device;
    int H, I, act;
    uint8_t* w;  // one allocation: gate | up | down, tiled layout (q4_device.h)
    size_t gate_bytes, down_bytes;
    uint16_t* a;  // activation scratch (bf16 bit patterns), a_cap elements
    size_t a_cap;
    int a_rows;  // tokens held in `a` after the last call
};

namespace {

constexpr uint32_t kFfnMagic = 0xA1FEED42u;

int check_handle(alv_ffn_t w) {
    if (!w || w->magic != kFfnMagic) return alv::fail(ALV_ERR_HANDLE, "invalid FFN handle");
    return ALV_OK;
}

}  // namespace

using namespace alv;

extern "C" int alv_ffn_register(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, int H, int I,
                                int act, alv_ffn_t* out, void* stream) {
    if (!out) return fail(ALV_ERR_ARG, "null output handle pointer");
    *out = nullptr;
    if (!Wg || !Wu || !Wd) return fail(ALV_ERR_ARG, "null weight pointer");
    if ((reinterpret_cast<uintptr_t>(Wg) | reinterpret_cast<uintptr_t>(Wu) | reinterpret_cast<uintptr_t>(Wd)) % 4)
        return fail(ALV_ERR_ALIGN, "FFN weights need 4-byte alignment");
    if (H < 32 || I < 32 || H % 32 || I % 32)
        return fail(ALV_ERR_ARG, "bad FFN shape H=%d I=%d (both must be positive multiples of 32)", H, I);
    if (act != ALV_ACT_GELU_TANH && act != ALV_ACT_SILU) return fail(ALV_ERR_ARG, "bad activation id %d", act);
    const size_t gate_bytes = tile_bytes(I, H);
    const size_t down_bytes = tile_bytes(H, I);
    if (gate_bytes >= 0xFFFFE000ull || down_bytes >= 0xFFFFE000ull)
        return fail(ALV_ERR_RANGE, "FFN matrices exceed the 4 GiB buffer range");
    hipStream_t s = (hipStream_t)stream;
    alv_ffn* h = new alv_ffn{};
    h->magic = kFfnMagic;
    h->H = H;
    h->I = I;
    h->act = act;
    h->gate_bytes = gate_bytes;
    h->down_bytes = down_bytes;
    int rc = hip_check(hipGetDevice(&h->device), "hipGetDevice");
    if (!rc) rc = hip_check(hipMalloc(&h->w, 2 * gate_bytes + down_bytes), "hipMalloc(FFN weights)");
    if (!rc) rc = launch_tile(Wg, h->w, I, H, s);
    if (!rc) rc = launch_tile(Wu, h->w + gate_bytes, I, H, s);
    if (!rc) rc = launch_tile(Wd, h->w + 2 * gate_bytes, H, I, s);
    h->a_cap = (size_t)I * kGemvMaxM;
    if (!rc) rc = hip_check(hipMalloc(&h->a, h->a_cap * sizeof(uint16_t)), "hipMalloc(FFN activation)");
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (rc) {
        if (h->w) (void)hipFree(h->w);
        if (h->a) (void)hipFree(h->a);
        h->magic = 0;
        delete h;
        return rc;
    }
    *out = h;
    return ALV_OK;
}

extern "C" int alv_ffn_shape(alv_ffn_t w, int* H, int* I, int* act) {
    if (int rc = check_handle(w)) return rc;
    if (H) *H = w->H;
    if (I) *I = w->I;
    if (act) *act = w->act;
    return ALV_OK;
}

extern "C" int alv_ffn_fused(alv_ffn_t w, const float* X, float* Y, int M, int ldx, int ldy, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!X || !Y) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || ldx < w->H || ldy < w->H) return fail(ALV_ERR_ARG, "bad M=%d ldx=%d ldy=%d for H=%d", M, ldx, ldy, w->H);
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(Y) % 4)
        return fail(ALV_ERR_ALIGN, "X and Y need 4-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    hipStream_t s = (hipStream_t)stream;
    const int chunk = M >= kTiledMinM ? M : std::min(M, kGemvMaxM);
    const size_t need = (size_t)chunk * w->I;
    if (need > w->a_cap) {
        if (int rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
        (void)hipFree(w->a);
        w->a = nullptr;
        w->a_cap = 0;
        if (int rc = hip_check(hipMalloc(&w->a, need * sizeof(uint16_t)), "hipMalloc(FFN activation)")) return rc;
        w->a_cap = need;
    }
    const uint8_t* wg = w->w;
    const uint8_t* wu = w->w + w->gate_bytes;
    const uint8_t* wd = w->w + 2 * w->gate_bytes;
    for (int m0 = 0; m0 < M; m0 += chunk) {
        const int mc = std::min(chunk, M - m0);
        GemvLaunch up;
        up.W0 = wg;
        up.W1 = wu;
        up.X = X + (size_t)m0 * ldx;
        up.ldx = ldx;
        up.Yb = w->a;
        up.ldy = w->I;
        up.M = mc;
        up.N = w->I;
        up.K = w->H;
        up.parts = 3;
        up.glu = true;
        up.tiled = true;
        up.act = w->act;
        GemvLaunch down;
        down.W0 = wd;
        down.Xb = w->a;
        down.ldx = w->I;
        down.Y = Y + (size_t)m0 * ldy;
        down.ldy = ldy;
        down.M = mc;
        down.N = w->H;
        down.K = w->I;
        down.parts = 1;
        down.tiled = true;
        const bool tiled = mc >= kTiledMinM;
        if (int rc = tiled ? launch_gemm_tiled(up, s) : launch_gemv(up, s)) return rc;
        if (int rc = tiled ? launch_gemm_tiled(down, s) : launch_gemv(down, s)) return rc;
        w->a_rows = mc;
    }
    return ALV_OK;
}

namespace {

__global__ void __launch_bounds__(256) bf16_to_f32_kernel(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = bf16_bits_to_f32(in[i]);
}

}  // namespace

extern "C" int alv_ffn_activation(alv_ffn_t w, float* out, int M, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!out) return fail(ALV_ERR_ARG, "null output pointer");
    if (M < 1 || M > w->a_rows) return fail(ALV_ERR_ARG, "M=%d outside the %d tokens of the last call", M, w->a_rows);
    const int64_t n = (int64_t)M * w->I;
    const int grid = (int)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, w->a, out, n);
    return hip_check(hipGetLastError(), "bf16_to_f32_kernel launch");
}

extern "C" void alv_ffn_release(alv_ffn_t w) {
    if (!w || w->magic != kFfnMagic) return;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (cur != w->device) (void)hipSetDevice(w->device);
    (void)hipDeviceSynchronize();
    if (w->w) (void)hipFree(w->w);
    if (w->a) (void)hipFree(w->a);
    if (cur >= 0 && cur != w->device) (void)hipSetDevice(cur);
    w->magic = 0;
    delete w;
}
