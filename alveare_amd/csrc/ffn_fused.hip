// Fused FFN (gate/up projection, GLU activation, down projection) on gfx950:
// alv_ffn_register / alv_ffn_fused / alv_ffn_shape / alv_ffn_release.
//
// One token (when the registration has the slice-ordered down matrix): one
// streaming launch plus a summing launch (gemv1_q.hip, q4_ffn1_kernel): each
// workgroup computes gate, up and the activation of 64 intermediate rows and
// multiplies their 64 down columns into a partial output, as the reference's
// NPU cores do with their slices (kernels/ffn_fused/ffn_fused.py:28-328); the
// partials are summed in a fixed order on the device.
// Decode (M <= 16) otherwise: two launches of the streaming kernel (gemv1_q.hip).
//   1. gate and up tiles of the same rows are streamed by the same workgroup
//      against the same activation operands; the epilogue rounds both to
//      bf16, applies the GLU and rounds the activation to bf16 -- the
//      reference CPU path's three rounding points (runtime/py/model.py:798-803).
//      The activation (M x I bf16) stays in the handle's buffer (16 x I,
//      allocated at registration and never moved), which is L2/MALL-resident
//      at these sizes.
//   2. down = Wd * a, with a single bf16 term per activation value (it is
//      bf16 by construction), summed entirely on the device -- the reference
//      sums per-core partials on the host (runtime/cpp/src/npu.cpp:360-377).
// Prefill (from 17 bf16 / 33 fp32 tokens): the same two steps with the MFMA
// tiled kernel (gemm_q.hip);
// the M x I activation lives in the stream's prefill scratch (q4_host.h).
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "q4_device.h"
#include "q4_host.h"


namespace {

int check_handle(alv_ffn_t w) {
    if (!w || w->magic != alv::kFfnMagic) return alv::fail(ALV_ERR_HANDLE, "invalid FFN handle");
    return ALV_OK;
}

// Down slices of the one-token FFN launch (gemv1_q.hip, q4_ffn1_kernel): a
// combined-layout matrix of G U 16 rows x 16 blocks whose row (u G + b) 16 + j
// holds, as block vb, the block (row 128 u + 16 (vb >> 1) + j, column block
// b + G (vb & 1)) of Wd (rows rs bytes apart). A byte permutation, like the
// reference's own FFN repack (runtime/cpp/src/weights.cpp:94-190).
__global__ void __launch_bounds__(256) ffn1_vdown_kernel(const uint8_t* Wd, uint32_t rs, int G, int U, uint32_t* out) {
    const int64_t total = (int64_t)G * U * 16 * 16 * 5;  // dwords: 16 blocks of 5 per virtual row
    for (int64_t d = (int64_t)blockIdx.x * 256 + threadIdx.x; d < total; d += (int64_t)gridDim.x * 256) {
        const int64_t blk = d / 5;
        const int e = (int)(d - blk * 5);
        const int vb = (int)(blk & 15);
        const int64_t vr = blk >> 4;
        const int j = (int)(vr & 15);
        const int64_t ub = vr >> 4;  // unit-major: tile u G + b
        const int b = (int)(ub % G), u = (int)(ub / G);
        const int row = 128 * u + 16 * (vb >> 1) + j;
        const int cb = b + G * (vb & 1);
        out[d] = *reinterpret_cast<const uint32_t*>(Wd + (size_t)row * rs + (size_t)cb * alv::kBlockBytes + 4 * e);
    }
}

// Whether one-token calls take the one-launch FFN (when the handle has it):
// the environment variable ALV_FFN_ONE (0 / 1), read at each call, overrides
// the default (on).
bool ffn1_on() {
    const char* e = getenv("ALV_FFN_ONE");
    if (e && *e) return atoi(e) != 0;
    return true;
}

}  // namespace

using namespace alv;

namespace alv {

// The two launches of one FFN call: gate/up with the GLU epilogue into the
// bf16 activation `act`, then down from it.
void ffn_ops(alv_ffn_t w, uint16_t* act, const float* X, int ldx, float* Y, int ldy, int M, GemvLaunch (&op)[2]) {
    GemvLaunch& up = op[0];
    up = GemvLaunch{};
    up.W0 = w->w;
    up.W1 = w->w + w->gate_bytes;
    up.X = X;
    up.ldx = ldx;
    up.Yb = act;
    up.ldy = w->I;
    up.M = M;
    up.N = w->Ie;
    up.K = w->He;
    up.Nz = w->I;  // the activation of trimmed (all-zero) rows is zero
    up.parts = 3;
    up.glu = true;
    up.tiled = true;
    up.act = w->act;
    GemvLaunch& down = op[1];
    down = GemvLaunch{};
    down.W0 = w->w + 2 * w->gate_bytes;
    down.Xb = act;
    down.ldx = w->I;
    down.Y = Y;
    down.ldy = ldy;
    down.M = M;
    down.N = w->He;
    down.K = w->Ie;
    down.Nz = w->H;
    down.parts = 1;
    down.tiled = true;
}

}  // namespace alv

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
    int rc = hip_check(hipGetDevice(&h->device), "hipGetDevice");
    // Trailing all-zero rows and columns (the reference's padded FFN, 15360 x
    // 3840 stored as 16384 x 4096) are trimmed: gate/up rows past Ie and
    // columns past He, down rows past He and columns past Ie hold only zero
    // weights, so the activation there is GLU(0, 0) = 0 and the output 0.
    int eg[2] = {0, 0}, eu[2] = {0, 0}, ed[2] = {0, 0};
    const uint32_t rs_h = (uint32_t)(H / kBlockK) * kBlockBytes, rs_i = (uint32_t)(I / kBlockK) * kBlockBytes;
    if (!rc) rc = weight_extent(Wg, I, H, rs_h, s, eg);
    if (!rc) rc = weight_extent(Wu, I, H, rs_h, s, eu);
    if (!rc) rc = weight_extent(Wd, H, I, rs_i, s, ed);
    auto up32 = [](int v) { return std::max(kBlockK, (v + kBlockK - 1) / kBlockK * kBlockK); };
    h->He = std::min(H, up32(std::max({kBlockK * eg[1], kBlockK * eu[1], ed[0]})));
    h->Ie = std::min(I, up32(std::max({eg[0], eu[0], kBlockK * ed[1]})));
    h->gate_bytes = tile_bytes(h->Ie, h->He);
    h->down_bytes = tile_bytes(h->He, h->Ie);
    if (!rc) rc = hip_check(hipMalloc(&h->w, 2 * h->gate_bytes + h->down_bytes), "hipMalloc(FFN weights)");
    if (!rc) rc = launch_tile(Wg, h->w, h->Ie, h->He, s, rs_h);
    if (!rc) rc = launch_tile(Wu, h->w + h->gate_bytes, h->Ie, h->He, s, rs_h);
    if (!rc) rc = launch_tile(Wd, h->w + 2 * h->gate_bytes, h->He, h->Ie, s, rs_i);
    h->a_cap = (size_t)I * kGemvMaxM;
    if (!rc) rc = hip_check(hipMalloc(&h->a, h->a_cap * sizeof(uint16_t)), "hipMalloc(FFN activation)");
    if (!rc) rc = hip_check(hipMemsetAsync(h->a, 0, h->a_cap * sizeof(uint16_t), s), "hipMemsetAsync(FFN activation)");
    h->last_a = h->a;
    // The one-token launch takes 64 intermediate rows per workgroup and down
    // units of 128 rows: Ie a multiple of 64, He of 128.
    uint8_t* vtmp = nullptr;
    if (!rc && h->Ie % 64 == 0 && h->He % 128 == 0 && h->He > 512 && h->Ie / 64 <= 256) {
        h->G1 = h->Ie / 64;
        h->U1 = h->He / 128;
        const int nv = h->G1 * h->U1 * 16;
        h->vdown_bytes = tile_bytes(nv, 512);
        rc = hip_check(hipMalloc(&vtmp, (size_t)nv * 16 * kBlockBytes), "hipMalloc(FFN down slices, staging)");
        if (!rc) rc = hip_check(hipMalloc(&h->vdown, h->vdown_bytes), "hipMalloc(FFN down slices)");
        if (!rc) rc = hip_check(hipMalloc(&h->part1, (size_t)h->G1 * h->He * sizeof(float)), "hipMalloc(FFN partials)");
        if (!rc) {
            hipLaunchKernelGGL(ffn1_vdown_kernel, dim3(4096), dim3(256), 0, s, Wd, rs_i, h->G1, h->U1,
                               reinterpret_cast<uint32_t*>(vtmp));
            rc = hip_check(hipGetLastError(), "ffn1_vdown_kernel launch");
        }
        if (!rc) rc = launch_tile(vtmp, h->vdown, nv, 512, s, 16 * kBlockBytes);
    }
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (vtmp) (void)hipFree(vtmp);
    if (rc) {
        if (h->w) (void)hipFree(h->w);
        if (h->a) (void)hipFree(h->a);
        if (h->vdown) (void)hipFree(h->vdown);
        if (h->part1) (void)hipFree(h->part1);
        h->magic = 0;
        delete h;
        return rc;
    }
    *out = h;
    return ALV_OK;
}

extern "C" int alv_ffn_exec_shape(alv_ffn_t w, int* H, int* I) {
    if (int rc = check_handle(w)) return rc;
    if (H) *H = w->He;
    if (I) *I = w->Ie;
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
    if (M >= tiled_min_m(true)) {
        // Prefill: the activation goes to the stream's scratch; the handle's
        // decode buffer keeps its size and address (graphs may hold it).
        void* act = nullptr;
        if (int rc = get_scratch(s, kScratchAct, (size_t)M * w->I * sizeof(uint16_t), &act)) return rc;
        GemvLaunch op[2];
        ffn_ops(w, static_cast<uint16_t*>(act), X, ldx, Y, ldy, M, op);
        if (int rc = launch_gemm_tiled(op[0], s)) return rc;
        if (int rc = launch_gemm_tiled(op[1], s)) return rc;
        w->last_a = static_cast<uint16_t*>(act);
        w->a_rows = M;
        return ALV_OK;
    }
    if (M == 1 && w->vdown && ffn1_on()) {
        GemvLaunch op[2];
        ffn_ops(w, w->a, X, ldx, Y, ldy, 1, op);
        if (int rc = launch_ffn1(op[0], w->vdown, w->vdown_bytes, w->part1, w->a, w->G1, w->U1, w->H, Y, nullptr, s))
            return rc;
        w->last_a = w->a;
        w->a_rows = 1;
        return ALV_OK;
    }
    for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
        const int mc = std::min(kGemvMaxM, M - m0);
        GemvLaunch op[2];
        ffn_ops(w, w->a, X + (size_t)m0 * ldx, ldx, Y + (size_t)m0 * ldy, ldy, mc, op);
        if (int rc = launch_gemv(op[0], s)) return rc;
        if (int rc = launch_gemv(op[1], s)) return rc;
        w->last_a = w->a;
        w->a_rows = mc;
    }
    return ALV_OK;
}

extern "C" int alv_ffn_fused_bf16(alv_ffn_t w, const uint16_t* X, uint16_t* Y, int M, int ldx, int ldy, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!X || !Y) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || ldx < w->H || ldy < w->H) return fail(ALV_ERR_ARG, "bad M=%d ldx=%d ldy=%d for H=%d", M, ldx, ldy, w->H);
    if (reinterpret_cast<uintptr_t>(X) % 16 || ldx % 8 || reinterpret_cast<uintptr_t>(Y) % 2)
        return fail(ALV_ERR_ALIGN, "X needs 16-byte aligned rows (ldx a multiple of 8), Y 2-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    hipStream_t s = (hipStream_t)stream;
    // The fp32 plan with bf16 ends: gate/up reads X as one bf16 term, down
    // writes bf16 (the reference's y_bf16, runtime/cpp/src/npu.cpp:340-378).
    auto bf16_ends = [&](GemvLaunch (&op)[2], const uint16_t* x, uint16_t* y) {
        op[0].X = nullptr;
        op[0].Xb = x;
        op[0].parts = 1;
        op[1].Y = nullptr;
        op[1].Yb = y;
    };
    if (M >= tiled_min_m(false)) {
        void* act = nullptr;
        if (int rc = get_scratch(s, kScratchAct, (size_t)M * w->I * sizeof(uint16_t), &act)) return rc;
        GemvLaunch op[2];
        ffn_ops(w, static_cast<uint16_t*>(act), nullptr, ldx, nullptr, ldy, M, op);
        bf16_ends(op, X, Y);
        if (int rc = launch_gemm_tiled(op[0], s)) return rc;
        if (int rc = launch_gemm_tiled(op[1], s)) return rc;
        w->last_a = static_cast<uint16_t*>(act);
        w->a_rows = M;
        return ALV_OK;
    }
    if (M == 1 && w->vdown && ffn1_on()) {
        GemvLaunch op[2];
        ffn_ops(w, w->a, nullptr, ldx, nullptr, ldy, 1, op);
        bf16_ends(op, X, Y);
        if (int rc = launch_ffn1(op[0], w->vdown, w->vdown_bytes, w->part1, w->a, w->G1, w->U1, w->H, nullptr, Y, s))
            return rc;
        w->last_a = w->a;
        w->a_rows = 1;
        return ALV_OK;
    }
    for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
        const int mc = std::min(kGemvMaxM, M - m0);
        GemvLaunch op[2];
        ffn_ops(w, w->a, nullptr, ldx, nullptr, ldy, mc, op);
        bf16_ends(op, X + (size_t)m0 * ldx, Y + (size_t)m0 * ldy);
        if (int rc = launch_gemv(op[0], s)) return rc;
        if (int rc = launch_gemv(op[1], s)) return rc;
        w->last_a = w->a;
        w->a_rows = mc;
    }
    return ALV_OK;
}

// ---- alv_ffn_fused_noalloc ------------------------------------------------------
// The decode FFN with its split-K temporaries (arrival counters, partial sums)
// in `scratch`, a fixed array in device memory that every GPU the library runs
// on holds until the process ends, instead of buffers allocated per stream:
// no call allocates. `scratch` names a host-side stand-in in host code; the
// device address comes from hipGetSymbolAddress, once per device.
namespace {

constexpr size_t kStaticCounterBytes = (size_t)kSplitCounters * sizeof(uint32_t);
constexpr size_t kStaticPartBytes = (size_t)16 << 20;  // split-K partial sums
static __device__ __align__(256) unsigned char scratch[kStaticCounterBytes + kStaticPartBytes];

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

std::mutex g_static_mu;
unsigned char* g_static_ptr[64];

// This device's copy of `scratch`. Its first use on a device also clears the
// counters, with a kernel on `s` (stream-ordered before the caller's launches).
int static_split(int dev, hipStream_t s, SplitBuf* out) {
    if (dev < 0 || dev >= 64) return fail(ALV_ERR_ARG, "device %d outside the 64 the library tracks", dev);
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static_ptr[dev]) {
        void* p = nullptr;
        if (int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
        if (!p) return fail(ALV_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
        hipLaunchKernelGGL(zero_words_kernel, dim3(4), dim3(256), 0, s, static_cast<uint32_t*>(p), (int)kSplitCounters);
        if (int rc = hip_check(hipGetLastError(), "zero_words_kernel launch")) return rc;
        g_static_ptr[dev] = static_cast<unsigned char*>(p);
    }
    out->counters = reinterpret_cast<uint32_t*>(g_static_ptr[dev]);
    out->part = reinterpret_cast<float*>(g_static_ptr[dev] + kStaticCounterBytes);
    out->part_bytes = kStaticPartBytes;
    return ALV_OK;
}

}  // namespace

extern "C" int alv_ffn_fused_bf16_addnorm(alv_ffn_t w, const uint16_t* resid, const uint16_t* y, const float* w_y,
                                          int norm_y, float scale, int scale_mode, uint16_t* sum_out,
                                          const float* w_x, float eps, uint16_t* Y, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!Y) return fail(ALV_ERR_ARG, "null output pointer");
    if (reinterpret_cast<uintptr_t>(Y) % 2) return fail(ALV_ERR_ALIGN, "Y needs 2-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    if (w->He != w->H)
        return fail(ALV_ERR_ARG, "a fused residual step needs the whole row: this FFN registered with its trailing "
                    "all-zero hidden columns trimmed (H=%d executed as %d)", w->H, w->He);
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
    hipStream_t s = (hipStream_t)stream;
    GemvLaunch op[2];
    ffn_ops(w, w->a, nullptr, w->H, nullptr, w->H, 1, op);
    op[0].X = nullptr;
    op[0].Xb = y ? y : resid;
    op[0].parts = 1;
    op[0].step = &st;
    op[1].Y = nullptr;
    op[1].Yb = Y;
    if (w->vdown && ffn1_on()) {
        if (int rc = launch_ffn1(op[0], w->vdown, w->vdown_bytes, w->part1, w->a, w->G1, w->U1, w->H, nullptr, Y, s))
            return rc;
        w->last_a = w->a;
        w->a_rows = 1;
        return ALV_OK;
    }
    if (int rc = launch_gemv(op[0], s)) return rc;
    if (int rc = launch_gemv(op[1], s)) return rc;
    w->last_a = w->a;
    w->a_rows = 1;
    return ALV_OK;
}

extern "C" int alv_ffn_fused_noalloc(alv_ffn_t w, const float* X, float* Y, int M, int ldx, int ldy,
                                     void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!X || !Y) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || M > kGemvMaxM || ldx < w->H || ldy < w->H)
        return fail(ALV_ERR_ARG, "bad M=%d ldx=%d ldy=%d for H=%d (1 <= M <= %d)", M, ldx, ldy, w->H, kGemvMaxM);
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(Y) % 4)
        return fail(ALV_ERR_ALIGN, "X and Y need 4-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    GemvLaunch op[2];
    ffn_ops(w, w->a, X, ldx, Y, ldy, M, op);
    if (M == 1 && w->vdown && ffn1_on()) {
        // The one-launch form, as alv_ffn_fused takes it: its partials live in
        // the handle (allocated at registration), so the call allocates nothing.
        if (int rc = launch_ffn1(op[0], w->vdown, w->vdown_bytes, w->part1, w->a, w->G1, w->U1, w->H, Y, nullptr,
                                 (hipStream_t)stream))
            return rc;
        w->last_a = w->a;
        w->a_rows = 1;
        return ALV_OK;
    }
    for (const GemvLaunch& L : op) {
        const int64_t need = gemv_split_bytes(L);
        if (need < 0) return fail(ALV_ERR_RANGE, "no launch plan for M=%d H=%d I=%d", M, w->H, w->I);
        if ((size_t)need > kStaticPartBytes)
            return fail(ALV_ERR_RANGE, "M=%d H=%d I=%d needs %lld bytes of split-K partial sums; the fixed scratch holds %zu",
                        M, w->H, w->I, (long long)need, kStaticPartBytes);
    }
    hipStream_t s = (hipStream_t)stream;
    SplitBuf sb;
    if (int rc = static_split(dev, s, &sb)) return rc;
    for (GemvLaunch& L : op) {
        L.split = &sb;
        if (int rc = launch_gemv(L, s)) return rc;
    }
    w->last_a = w->a;
    w->a_rows = M;
    return ALV_OK;
}

extern "C" int alv_ffn_gate_up(alv_ffn_t w, const float* X, int M, int ldx, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!X) return fail(ALV_ERR_ARG, "null activation pointer");
    if (M < 1 || M > kGemvMaxM || ldx < w->H) return fail(ALV_ERR_ARG, "bad M=%d ldx=%d for H=%d (1 <= M <= %d)", M, ldx, w->H, kGemvMaxM);
    if (reinterpret_cast<uintptr_t>(X) % 4) return fail(ALV_ERR_ALIGN, "X needs 4-byte alignment");
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    GemvLaunch op[2];
    ffn_ops(w, w->a, X, ldx, nullptr, w->H, M, op);
    if (int rc = launch_gemv(op[0], (hipStream_t)stream)) return rc;
    w->last_a = w->a;
    w->a_rows = M;
    return ALV_OK;
}

extern "C" int alv_ffn_partials(alv_ffn_t w, const float* X, float* P, int* slices, void* stream) {
    if (int rc = check_handle(w)) return rc;
    if (!X) return fail(ALV_ERR_ARG, "null activation pointer");
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(P) % 4)
        return fail(ALV_ERR_ALIGN, "X and P need 4-byte alignment");
    if (!w->vdown)
        return fail(ALV_ERR_ARG, "this FFN (H=%d I=%d executed as %d x %d) has no one-launch form: it needs the "
                    "executed I a multiple of 64 up to 16384 and H a multiple of 128 above 512", w->H, w->I, w->He, w->Ie);
    int dev = -1;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != w->device) return fail(ALV_ERR_HANDLE, "FFN handle belongs to device %d, current device is %d", w->device, dev);
    if (slices) *slices = w->G1;
    GemvLaunch op[2];
    ffn_ops(w, w->a, X, w->H, nullptr, w->H, 1, op);
    if (int rc = launch_ffn1(op[0], w->vdown, w->vdown_bytes, P ? P : w->part1, w->a, w->G1, w->U1, w->H, nullptr,
                             nullptr, (hipStream_t)stream, false))
        return rc;
    w->last_a = w->a;
    w->a_rows = 1;
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
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, w->last_a, out, n);
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
    if (w->vdown) (void)hipFree(w->vdown);
    if (w->part1) (void)hipFree(w->part1);
    if (cur >= 0 && cur != w->device) (void)hipSetDevice(cur);
    w->magic = 0;
    delete w;
}
