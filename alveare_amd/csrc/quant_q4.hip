// GPU quantizer: float32 weights -> Q4 combined layout (alv_quantize_q4), or
// straight into a registered weight (alv_weight_quantize).
//
// The reference quantizes on the host in numpy (tools/convert/gemv_q_convert.py:
// quantize_to_q4_0 :5-51, pack_to_combined :53-85), after zero-padding the
// matrix to the kernel shape (tools/quantize_gemma4.py:26-41). Per 32-weight
// block of a row:
//   scale = max|w| / 7 in float32 (a NaN anywhere in the block makes it NaN,
//           as np.max does); a zero scale becomes 1.0;
//   q     = clip(round_half_even(w / scale), -8, 7), where a NaN quotient (a
//           NaN block, or inf / inf) becomes -8 -- numpy's astype(int32) gives
//           INT32_MIN for NaN on x86-64, which the clip takes to -8;
//   bytes = 16 nibble pairs (even column low), the bf16 scale (round to
//           nearest even, NaN -> 0x7FC0) little-endian, two zero bytes.
// The quotient is a correctly rounded float32 division (__fdiv_rn) and the
// rounding is v_rndne_f32, so the codes match numpy's bit for bit.
//
// Eight lanes share a block: lane p holds columns 4p..4p+3, the group finds
// the block maximum with three xor shuffles, and each lane writes its two code
// bytes; lane 0 also writes the scale and the padding. Reads and writes of a
// wave are contiguous (8 blocks of one row).
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

__device__ __forceinline__ uint32_t bf16_bits_rne(float v) {
    if (v != v) return 0x7FC0u;
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__global__ void __launch_bounds__(256) quant_kernel(const float* W, int n_src, int k_src, int ldw, uint8_t* out,
                                                    int N, int K) {
    const int nb = K / 32;
    const uint64_t total = (uint64_t)N * nb;
    const int part = threadIdx.x & 7;
    const uint64_t step = ((uint64_t)gridDim.x * blockDim.x) >> 3;
    // Every lane of an 8-lane group has the same block, so a group is either
    // wholly inside the loop or wholly out of it (the shuffles stay in-group).
    for (uint64_t blk = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3; blk < total; blk += step) {
        const int r = (int)(blk / (uint64_t)nb);
        const int b = (int)(blk - (uint64_t)r * nb);
        const int c0 = b * 32 + part * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + e;
            v[e] = r < n_src && c < k_src ? W[(size_t)r * ldw + c] : 0.0f;
        }
        float m = 0.0f;
        int nan = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a = fabsf(v[e]);
            nan |= a != a;
            m = fmaxf(m, a);  // a NaN is tracked in `nan`, not in m
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            m = fmaxf(m, __shfl_xor(m, o));
            nan |= __shfl_xor(nan, o);
        }
        float s = nan ? __builtin_nanf("") : __fdiv_rn(m, 7.0f);
        if (s == 0.0f) s = 1.0f;
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float qf = rintf(__fdiv_rn(v[e], s));
            int q = qf != qf ? -8 : (int)qf;
            q = q < -8 ? -8 : (q > 7 ? 7 : q);
            packed |= (uint32_t)(q & 0xF) << (4 * e);
        }
        uint8_t* o = out + (size_t)r * nb * kBlockBytes + (size_t)b * kBlockBytes;
        *reinterpret_cast<uint16_t*>(o + 2 * part) = (uint16_t)packed;
        if (part == 0) *reinterpret_cast<uint32_t*>(o + 16) = bf16_bits_rne(s);
    }
}

int check_quant(const float* W, int n_src, int k_src, int ldw, const void* out, int N, int K) {
    if (!W || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (N < 1 || K < 32 || K % 32) return fail(ALV_ERR_ARG, "bad shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
    if (n_src < 0 || k_src < 0 || n_src > N || k_src > K || ldw < k_src)
        return fail(ALV_ERR_ARG, "source %d x %d (row stride %d) does not fit the %d x %d output", n_src, k_src, ldw, N, K);
    if (reinterpret_cast<uintptr_t>(W) % 4) return fail(ALV_ERR_ALIGN, "W needs 4-byte alignment");
    if ((uint64_t)N * (uint64_t)(K / 32) * kBlockBytes >= (1ull << 40))
        return fail(ALV_ERR_RANGE, "output of %d x %d exceeds 1 TiB", N, K);
    return ALV_OK;
}

int launch_quant(const float* W, int n_src, int k_src, int ldw, uint8_t* out, int N, int K, hipStream_t s) {
    const uint64_t threads = (uint64_t)N * (uint64_t)(K / 32) * 8;
    const int grid = (int)std::min<uint64_t>((threads + 255) / 256, 65536);
    hipLaunchKernelGGL(quant_kernel, dim3(grid), dim3(256), 0, s, W, n_src, k_src, ldw, out, N, K);
    return hip_check(hipGetLastError(), "quant_kernel launch");
}

}  // namespace

}  // namespace alv

using namespace alv;

extern "C" int alv_quantize_q4(const float* W, int n_src, int k_src, int ldw, uint8_t* out, int N, int K,
                               void* stream) {
    if (int rc = check_quant(W, n_src, k_src, ldw, out, N, K)) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 4) return fail(ALV_ERR_ALIGN, "out needs 4-byte alignment");
    return launch_quant(W, n_src, k_src, ldw, out, N, K, (hipStream_t)stream);
}

extern "C" int alv_weight_quantize(const float* W, int n_src, int k_src, int ldw, int N, int K, alv_weight_t* out,
                                   void* stream) {
    if (!out) return fail(ALV_ERR_ARG, "null output handle pointer");
    *out = nullptr;
    if (int rc = check_quant(W, n_src, k_src, ldw, W, N, K)) return rc;
    hipStream_t s = (hipStream_t)stream;
    uint8_t* tmp = nullptr;
    int rc = hip_check(hipMalloc(&tmp, (size_t)N * (K / 32) * kBlockBytes), "hipMalloc(quantized weights)");
    if (!rc) rc = launch_quant(W, n_src, k_src, ldw, tmp, N, K, s);
    // Registration tiles the combined bytes and waits for the stream, after
    // which the temporary can go.
    if (!rc) rc = alv_weight_register(tmp, N, K, out, stream);
    if (tmp) {
        const int rs = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        (void)hipFree(tmp);
        if (!rc) rc = rs;
    }
    if (rc && *out) {
        alv_weight_release(*out);
        *out = nullptr;
    }
    return rc;
}
