// Entry points on the combined layout: alv_gemv_q, alv_gemm_q (M < 32 via the
// streaming kernel of gemv1_q.hip, larger M via the MFMA tiled kernel of
// gemm_q.hip), the dequant and GLU parity kernels behind alv_dequant_q4 and
// alv_glu.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

// out[N, K] bf16 bits of dequant(W); one thread per block.
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* W, uint16_t* out, int N, int K) {
    const int nb = K >> 5;
    const int64_t total = (int64_t)N * nb;
    const uint32_t rs = (uint32_t)nb * kBlockBytes;
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
         b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = b / nb, kb = b - r * nb;
        const uint32_t* blk = reinterpret_cast<const uint32_t*>(W + r * rs + kb * kBlockBytes);
        uint32_t d[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) d[i] = blk[i];
        const uint32_t sbits = d[4] & 0xFFFFu;
        const Scale sc = make_scale(bf16_bits_to_f32(sbits));
        bf16x8* o = reinterpret_cast<bf16x8*>(out + r * K + kb * 32);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            // An exactly zero product keeps the IEEE sign of q * s (the fma in
            // dequant8 returns +0); only the sign of a zero total of a dot
            // product could see it, so the streaming kernels skip this.
            u32x4 bits = __builtin_bit_cast(u32x4, dequant8(d[t], sc));
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t w = bits[p];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int e = 2 * p + h;  // column 8t + e, nibble e of d[t]
                    if (((w >> (16 * h)) & 0x7FFFu) == 0) {
                        const uint32_t neg = ((d[t] >> (4 * e + 3)) & 1u) ^ (sbits >> 15);
                        w = (w & ~(0xFFFFu << (16 * h))) | ((neg << 15) << (16 * h));
                    }
                }
                bits[p] = w;
            }
            o[t] = __builtin_bit_cast(bf16x8, bits);
        }
    }
}

}  // namespace alv

using namespace alv;

static int check_common(const void* W, const void* x, const void* y, int N, int K) {
    if (!W || !x || !y) return fail(ALV_ERR_ARG, "null pointer");
    if (N < 1 || K < 32 || K % 32) return fail(ALV_ERR_ARG, "bad shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
    if (reinterpret_cast<uintptr_t>(W) % 4 || reinterpret_cast<uintptr_t>(x) % 4 || reinterpret_cast<uintptr_t>(y) % 4)
        return fail(ALV_ERR_ALIGN, "W, x and y need 4-byte alignment");
    return ALV_OK;
}

extern "C" int alv_gemv_q(const uint8_t* W, const float* x, float* y, int N, int K, void* stream) {
    if (int rc = check_common(W, x, y, N, K)) return rc;
    GemvLaunch L;
    L.W0 = W;
    L.X = x;
    L.ldx = K;
    L.Y = y;
    L.ldy = N;
    L.M = 1;
    L.N = N;
    L.K = K;
    L.parts = 3;
    return launch_gemv(L, (hipStream_t)stream);
}

extern "C" int alv_gemm_q(const uint8_t* W, const float* X, float* Y, int M, int N, int K, int ldx,
                          int ldy, void* stream) {
    if (int rc = check_common(W, X, Y, N, K)) return rc;
    if (M < 1) return fail(ALV_ERR_ARG, "bad M=%d", M);
    if (ldx < K || ldy < N) return fail(ALV_ERR_ARG, "leading dimensions ldx=%d ldy=%d below K=%d N=%d", ldx, ldy, K, N);
    GemvLaunch L;
    L.W0 = W;
    L.ldx = ldx;
    L.ldy = ldy;
    L.N = N;
    L.K = K;
    L.parts = 3;
    if (M >= tiled_min_m(true)) {
        L.X = X;
        L.Y = Y;
        L.M = M;
        return launch_gemm_tiled(L, (hipStream_t)stream);
    }
    for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
        L.X = X + (size_t)m0 * ldx;
        L.Y = Y + (size_t)m0 * ldy;
        L.M = std::min(kGemvMaxM, M - m0);
        if (int rc = launch_gemv(L, (hipStream_t)stream)) return rc;
    }
    return ALV_OK;
}

namespace {

__global__ void __launch_bounds__(256) glu_kernel(const float* g, const float* u, float* out, int64_t n, int act) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = alv::bf16_round(alv::glu_act(g[i], u[i], act));
}

}  // namespace

extern "C" int alv_glu(const float* g, const float* u, float* out, int64_t n, int act, void* stream) {
    if (!g || !u || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (n < 0) return fail(ALV_ERR_ARG, "negative length");
    if (act != ALV_ACT_GELU_TANH && act != ALV_ACT_SILU) return fail(ALV_ERR_ARG, "bad activation id %d", act);
    if (n == 0) return ALV_OK;
    const int grid = (int)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(glu_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, g, u, out, n, act);
    return hip_check(hipGetLastError(), "glu_kernel launch");
}

extern "C" int alv_dequant_q4(const uint8_t* W, uint16_t* out, int N, int K, void* stream) {
    if (int rc = check_common(W, out, out, N, K)) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 16) return fail(ALV_ERR_ALIGN, "out needs 16-byte alignment");
    const int64_t blocks = (int64_t)N * (K / 32);
    const int grid = (int)std::min<int64_t>((blocks + 255) / 256, 65535);
    hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, W, out, N, K);
    return hip_check(hipGetLastError(), "dequant_kernel launch");
}
