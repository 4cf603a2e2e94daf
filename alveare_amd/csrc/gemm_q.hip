// MFMA tiled Q4 GEMM for prefill-sized batches (gfx950): the M >= 32 path of
// alv_gemm_q and of alv_ffn_fused (gate/up with the GLU epilogue, then down).
//
// C[M, N] = X[M, K] * dequant(W)[N, K]^T. A workgroup of 4 waves owns a
// 128-token x 128-weight-row tile and walks K one Q4 block (32 k) at a time:
//   * the 128 x 32 weight tile is dequantized once into LDS as bf16
//     (q4_device.h::dequant8, exact), so the dequant cost is shared by 128
//     tokens;
//   * the 128 x 32 activation tile is split exactly into three bf16 terms;
//     a term whose tile is all zero (every term past the first when the
//     activations are bf16-valued, as the reference's callers pass them) is
//     skipped with a workgroup-uniform branch;
//   * each wave computes a 64 x 64 sub-tile with 4 x 4
//     v_mfma_f32_16x16x32_bf16, fp32 accumulation.
// LDS rows are padded to 40 bf16 (80 bytes) so the 16-byte operand reads of
// 16 lanes land in distinct banks.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

constexpr int TM = 128;  // tokens per tile
constexpr int TN = 128;  // weight rows per tile
constexpr int LDR = 40;  // padded LDS row length in bf16

struct TiledArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const float* X;       // fp32 activations, or
    const uint16_t* Xb;   // bf16 activations (bit patterns)
    float* Y;             // fp32 output, or
    uint16_t* Yb;         // bf16 output (bit patterns)
    uint32_t wbytes;
    int ldx, ldy, M, N, K, parts, act;
    bool tiled;   // weights in the tiled layout (q4_device.h) instead of the combined one
    TileGeom tg;
};

template <bool GLU>
__global__ void __launch_bounds__(256) gemm_tiled_kernel(TiledArgs a) {
    constexpr int NT = GLU ? 2 : 1;
    __shared__ __align__(16) __bf16 ws[NT][TN * LDR];
    __shared__ __align__(16) __bf16 xs[3][TM * LDR];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * TN;
    const int m0 = blockIdx.y * TM;
    const int nb = a.K >> 5;
    const uint32_t rs = (uint32_t)nb * kBlockBytes;
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);

    // Staging roles: thread -> (tile row, 16-column half).
    const int srow = tid >> 1, half = tid & 1;
    const int wrow = n0 + srow;
    const bool wrow_ok = wrow < a.N;
    const int xrow = m0 + srow;
    const bool xrow_ok = xrow < a.M;

    f32x4 acc[NT][4][4];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc[n][i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int j = lane & 15, g = lane >> 4;
    for (int kb = 0; kb < nb; ++kb) {
        // ---- stage the weight tile (dequantized) --------------------------
        {
            uint32_t o0, o1, os;  // nibble dwords 2*half, 2*half+1 and the scale dword
            if (!wrow_ok) {
                o0 = o1 = os = a.wbytes;
            } else if (a.tiled) {
                o0 = tiled_offset(a.tg, wrow, kb, 8 * half);
                o1 = tiled_offset(a.tg, wrow, kb, 8 * half + 4);
                os = tiled_offset(a.tg, wrow, kb, 16);
            } else {
                const uint32_t off = (uint32_t)wrow * rs + (uint32_t)kb * kBlockBytes;
                o0 = off + 8 * half;
                o1 = off + 8 * half + 4;
                os = off + 16;
            }
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const __amdgpu_buffer_rsrc_t r = n ? r1 : r0;
                const uint32_t d0 = buf_load4(r, o0);
                const uint32_t d1 = buf_load4(r, o1);
                const uint32_t ds = buf_load4(r, os);
                const Scale sc = make_scale(bf16_bits_to_f32(ds & 0xFFFFu));
                __bf16* dst = &ws[n][srow * LDR + 16 * half];
                *reinterpret_cast<bf16x8*>(dst) = dequant8(d0, sc);
                *reinterpret_cast<bf16x8*>(dst + 8) = dequant8(d1, sc);
            }
        }
        // ---- stage the activation tile as exact bf16 terms ----------------
        int nz = 0;
        {
            bf16x8 p[3][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const size_t xi = (size_t)xrow * a.ldx + kb * 32 + 16 * half + 8 * h + e;
                    const float v = !xrow_ok ? 0.0f : a.Xb ? bf16_bits_to_f32(a.Xb[xi]) : a.X[xi];
                    if (a.parts == 3) {
                        const Split3 s = split3(v);
                        p[0][h][e] = s.p0;
                        p[1][h][e] = s.p1;
                        p[2][h][e] = s.p2;
                        nz |= ((float)s.p1 != 0.0f) | (((float)s.p2 != 0.0f) << 1);
                    } else {
                        p[0][h][e] = (__bf16)v;
                    }
                }
            }
#pragma unroll
            for (int pp = 0; pp < 3; ++pp) {
                if (pp >= a.parts) break;
                __bf16* dst = &xs[pp][srow * LDR + 16 * half];
                *reinterpret_cast<bf16x8*>(dst) = p[pp][0];
                *reinterpret_cast<bf16x8*>(dst + 8) = p[pp][1];
            }
        }
        const int any1 = __syncthreads_or(nz & 1);
        const int any2 = __syncthreads_or(nz & 2);

        // ---- MFMA ------------------------------------------------------------
        bf16x8 bv[NT][4];
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                bv[n][jj] = *reinterpret_cast<const bf16x8*>(&ws[n][(wn * 64 + jj * 16 + j) * LDR + 8 * g]);
#pragma unroll
        for (int pp = 0; pp < 3; ++pp) {
            if (pp == 1 && !any1) continue;
            if (pp == 2 && !any2) continue;
            if (pp >= a.parts) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(&xs[pp][(wm * 64 + i * 16 + j) * LDR + 8 * g]);
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) acc[n][i][jj] = mfma16x16x32(av, bv[n][jj], acc[n][i][jj]);
            }
        }
        __syncthreads();
    }

    // ---- epilogue: D[4g + r][j] of each 16 x 16 sub-tile --------------------
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
                if constexpr (GLU)
                    out = bf16_round(glu_act(bf16_round(acc[0][i][jj][r]), bf16_round(acc[NT - 1][i][jj][r]), a.act));
                if (a.Yb)
                    a.Yb[(size_t)m * a.ldy + n] = __builtin_bit_cast(uint16_t, (__bf16)out);
                else
                    a.Y[(size_t)m * a.ldy + n] = out;
            }
}

}  // namespace

int launch_gemm_tiled(const GemvLaunch& L, hipStream_t s) {
    const uint64_t wbytes = L.tiled ? tile_bytes(L.N, L.K) : (uint64_t)L.N * (uint64_t)(L.K / 32) * kBlockBytes;
    if (wbytes >= 0xFFFFFF00ull) return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    TiledArgs a{};
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = L.X;
    a.Xb = L.Xb;
    a.Y = L.Y;
    a.Yb = L.Yb;
    a.wbytes = (uint32_t)wbytes;
    a.ldx = L.ldx;
    a.ldy = L.ldy;
    a.M = L.M;
    a.N = L.N;
    a.K = L.K;
    a.parts = L.parts;
    a.act = L.act;
    a.tiled = L.tiled;
    a.tg = tile_geom(L.K);
    const dim3 grid((L.N + TN - 1) / TN, (L.M + TM - 1) / TM);
    if (L.glu)
        hipLaunchKernelGGL(gemm_tiled_kernel<true>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(gemm_tiled_kernel<false>, grid, dim3(256), 0, s, a);
    return hip_check(hipGetLastError(), "gemm_tiled_kernel launch");
}

}  // namespace alv
