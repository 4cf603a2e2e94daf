// MFMA Q4 GEMM for prefill-sized batches (gfx950): the M >= 32 path of
// alv_gemm_q, alv_gemv and alv_ffn_fused (gate/up with the GLU epilogue, then
// down).
//
// C[M, N] = X[M, K] * dequant(W)[N, K]^T. A workgroup of 8 waves owns a
// 256-token x 128-weight-row tile and walks K 64 at a time (two Q4 blocks per
// row):
//   * the 128 x 64 weight tile is dequantized once into LDS as bf16
//     (q4_device.h::dequant8, exact), shared by 256 tokens;
//   * the 256 x 64 activation tile goes into LDS as bf16. fp32 activations
//     are split exactly into up to three bf16 terms (x = t0 + t1 + t2,
//     q4_device.h::split3), one pass over K per term: the first pass stages
//     t0 and notes whether any activation of the token tile has bits below
//     bf16 precision; only then do passes for t1 and t2 follow. Activations
//     that are already bf16-valued -- the reference's callers pass bf16
//     (runtime/py/model.py:399-485) -- cost one pass;
//   * each wave computes a 64 x 64 sub-tile with v_mfma_f32_16x16x32_bf16
//     (fp32 accumulation);
//   * the global loads of step k + 1 are issued before the MFMAs of step k and
//     land in the other half of a double-buffered LDS, so one barrier per step
//     separates them.
// Workgroups are numbered token-tile fastest: with the round-robin placement
// of workgroups on the 8 XCDs, the workgroups of one XCD share token tiles, so
// their activation reads hit that XCD's L2.
// LDS rows are padded to 72 bf16 (144 bytes) so the 16-byte operand reads of
// 16 lanes spread over the banks.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

constexpr int TM = 256;  // tokens per tile
constexpr int TN = 128;  // weight rows per tile
constexpr int TK = 64;   // k per step (two Q4 blocks)
constexpr int LDR = TK + 8;  // padded LDS row length in bf16
constexpr int kGemmThreads = 512;

struct GemmArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const void* X;           // fp32 activations (XF32) or bf16 bit patterns
    float* Y;                // fp32 output, or
    uint16_t* Yb;            // bf16 output (bit patterns)
    uint32_t wbytes;
    uint32_t xbytes;         // bytes of X (buffer range)
    int ldx, ldy, M, N, K, parts, act;
    TileGeom tg;
};

template <int NT, bool TILED, bool XF32>
__global__ void __launch_bounds__(kGemmThreads) gemm_q4_kernel(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    // [buffer][matrix][row][LDR] weights, then [buffer][token][LDR] activations.
    __bf16* wsm = reinterpret_cast<__bf16*>(smem);
    __bf16* xsm = wsm + 2 * NT * TN * LDR;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves of 64 x 64
    const int m0 = blockIdx.x * TM;
    const int n0 = blockIdx.y * TN;
    const int nsteps = (a.K + TK - 1) / TK;
    const int j = lane & 15, g = lane >> 4;
    const uint32_t rs = (uint32_t)(a.K >> 5) * kBlockBytes;

    // Staging roles. Weights: thread -> (matrix, row, block) of the
    // NT x 128 x 2 blocks of a step (threads past them stay idle).
    // Activations: thread -> 8 consecutive k of one token, 4 such pieces.
    const int wmat = tid >> 8;
    const int wr = (tid >> 1) & (TN - 1), wb = tid & 1;
    const bool wstage = wmat < NT;
    const int wrow = n0 + wr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wmat ? a.W1 : a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);

    f32x4 acc[NT][4][4];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc[n][i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int XV = XF32 ? 2 : 1;  // 16-byte loads per 8 activations
    uint32_t wreg[5];
    u32x4 xreg[4][XV];
    uint32_t lowbits = 0;  // OR of all fp32 activation bits seen by the first pass

    // Global loads of step s into registers.
    auto load = [&](int s) {
        const int kb = s * 2 + wb;
        const bool ok = wstage && wrow < a.N && kb < (a.K >> 5);
#pragma unroll
        for (int x = 0; x < 5; ++x) {
            uint32_t off = a.wbytes;
            if (ok) off = TILED ? tiled_offset(a.tg, wrow, kb, 4 * x) : (uint32_t)wrow * rs + (uint32_t)kb * kBlockBytes + 4 * x;
            wreg[x] = buf_load4(rw, off);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int piece = tid + i * kGemmThreads;  // 256 tokens x 8 pieces
            const int r = piece >> 3, c = (piece & 7) * 8;
            const int m = m0 + r, k = s * TK + c;
            const bool in = m < a.M && k < a.K;
            const uint32_t off = in ? (uint32_t)(((size_t)m * a.ldx + k) * (XF32 ? 4 : 2)) : a.xbytes;
#pragma unroll
            for (int v = 0; v < XV; ++v) xreg[i][v] = buf_load16(rx, off + 16 * v);
        }
    };
    // Registers of the last load into LDS buffer b, activations as term p.
    auto store = [&](int b, int p) {
        if (wstage) {
            const Scale sc = make_scale(bf16_bits_to_f32(wreg[4] & 0xFFFFu));
            __bf16* dst = wsm + ((size_t)(b * NT + wmat) * TN + wr) * LDR + 32 * wb;
#pragma unroll
            for (int t = 0; t < 4; ++t) *reinterpret_cast<bf16x8*>(dst + 8 * t) = dequant8(wreg[t], sc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int piece = tid + i * kGemmThreads;
            const int r = piece >> 3, c = (piece & 7) * 8;
            u32x4* dst = reinterpret_cast<u32x4*>(xsm + ((size_t)b * TM + r) * LDR + c);
            if constexpr (XF32) {
                bf16x8 t;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t bits = xreg[i][e >> 2][e & 3];
                    const float x = __builtin_bit_cast(float, bits);
                    if (p == 0) {
                        lowbits |= bits;
                        t[e] = (__bf16)x;
                    } else {
                        const Split3 sp = split3(x);
                        t[e] = p == 1 ? sp.p1 : sp.p2;
                    }
                }
                *dst = __builtin_bit_cast(u32x4, t);
            } else {
                *dst = xreg[i][0];
            }
        }
    };

    int nterms = 1;
    for (int p = 0; p < nterms; ++p) {
        load(0);
        store(0, p);
        __syncthreads();
        for (int s = 0; s < nsteps; ++s) {
            const int b = s & 1;
            if (s + 1 < nsteps) load(s + 1);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                bf16x8 bv[NT][4];
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
                        bv[n][jj] = *reinterpret_cast<const bf16x8*>(
                            wsm + ((size_t)(b * NT + n) * TN + wn * 64 + jj * 16 + j) * LDR + kk * 32 + 8 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bf16x8 av = *reinterpret_cast<const bf16x8*>(
                        xsm + ((size_t)b * TM + wm * 64 + i * 16 + j) * LDR + kk * 32 + 8 * g);
#pragma unroll
                    for (int n = 0; n < NT; ++n)
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) acc[n][i][jj] = mfma16x16x32(av, bv[n][jj], acc[n][i][jj]);
                }
            }
            if (s + 1 < nsteps) store(b ^ 1, p);
            __syncthreads();
        }
        // After the first pass: residual terms only for a token tile with
        // activations that are not bf16-valued.
        if (XF32 && p == 0 && a.parts == 3) nterms = __syncthreads_or((lowbits & 0xFFFFu) != 0) ? 3 : 1;
    }

    // ---- epilogue: D[4g + r][j] of each 16 x 16 sub-tile ----------------------------
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + 4 * g + r;
                const int n = n0 + wn * 64 + jj * 16 + j;
                if (m >= a.M || n >= a.N) continue;
                float out = acc[0][i][jj][r];
                if constexpr (NT == 2)
                    out = bf16_round(glu_act(bf16_round(acc[0][i][jj][r]), bf16_round(acc[1][i][jj][r]), a.act));
                if (a.Yb)
                    a.Yb[(size_t)m * a.ldy + n] = __builtin_bit_cast(uint16_t, (__bf16)out);
                else
                    a.Y[(size_t)m * a.ldy + n] = out;
            }
}

template <int NT, bool TILED, bool XF32>
hipError_t launch_gemm(const GemmArgs& a, dim3 grid, hipStream_t s) {
    const size_t lds = (size_t)2 * (NT * TN + TM) * LDR * sizeof(uint16_t);
    static bool attr[64] = {};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    if (dev >= 64 || !attr[dev]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_q4_kernel<NT, TILED, XF32>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        if (dev < 64) attr[dev] = true;
    }
    hipLaunchKernelGGL((gemm_q4_kernel<NT, TILED, XF32>), grid, dim3(kGemmThreads), lds, s, a);
    return hipGetLastError();
}

template <int NT, bool TILED>
hipError_t launch_gemm_x(const GemmArgs& a, bool xf32, dim3 grid, hipStream_t s) {
    return xf32 ? launch_gemm<NT, TILED, true>(a, grid, s) : launch_gemm<NT, TILED, false>(a, grid, s);
}

}  // namespace

int launch_gemm_tiled(const GemvLaunch& L, hipStream_t s) {
    const uint64_t wbytes = L.tiled ? tile_bytes(L.N, L.K) : (uint64_t)L.N * (uint64_t)(L.K / 32) * kBlockBytes;
    if (wbytes >= 0xFFFFFF00ull) return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    const bool xf32 = L.Xb == nullptr;
    const void* x = xf32 ? static_cast<const void*>(L.X) : static_cast<const void*>(L.Xb);
    // 16-byte activation loads: 4-byte aligned rows for fp32; for bf16 (the FFN's
    // own activation buffer) 16-byte aligned rows.
    if (xf32 ? reinterpret_cast<uintptr_t>(x) % 4 != 0 : reinterpret_cast<uintptr_t>(x) % 16 != 0 || L.ldx % 8 != 0)
        return fail(ALV_ERR_ALIGN, "prefill activations are not aligned for 16-byte loads");
    const uint64_t xbytes = ((uint64_t)(L.M - 1) * L.ldx + L.K) * (xf32 ? 4 : 2);
    if (xbytes >= 0xFFFFFF00ull) return fail(ALV_ERR_RANGE, "activations of %llu bytes exceed the 4 GiB buffer range", (unsigned long long)xbytes);
    GemmArgs a{};
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = x;
    a.Y = L.Y;
    a.Yb = L.Yb;
    a.wbytes = (uint32_t)wbytes;
    a.xbytes = (uint32_t)xbytes;
    a.ldx = L.ldx;
    a.ldy = L.ldy;
    a.M = L.M;
    a.N = L.N;
    a.K = L.K;
    a.parts = L.parts;
    a.act = L.act;
    a.tg = tile_geom(L.K);
    const dim3 grid((L.M + TM - 1) / TM, (L.N + TN - 1) / TN);
    hipError_t e;
    if (L.glu)
        e = L.tiled ? launch_gemm_x<2, true>(a, xf32, grid, s) : launch_gemm_x<2, false>(a, xf32, grid, s);
    else
        e = L.tiled ? launch_gemm_x<1, true>(a, xf32, grid, s) : launch_gemm_x<1, false>(a, xf32, grid, s);
    return hip_check(e, "gemm_q4_kernel launch");
}

}  // namespace alv
