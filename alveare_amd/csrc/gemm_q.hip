// MFMA Q4 GEMM for prefill-sized batches (gfx950): the path of alv_gemm_q,
// alv_gemv, alv_gemv_bf16, alv_ffn_fused and alv_ffn_fused_bf16 from 17 (bf16
// activations) or 33 (fp32) tokens (gate/up with the GLU epilogue, then down).
//
// C[M, N] = X[M, K] * dequant(W)[N, K]^T. A workgroup of 8 waves owns a
// TM-token x 128-weight-row tile -- TM = 256, or 64 up to 128 tokens (a
// quarter of the MFMA and LDS work per weight tile; measured 1.6-1.8x faster
// at M <= 128) -- and walks K 64 at a time (two Q4 blocks per row):
//   * the 128 x 64 weight tile is dequantized once into LDS as bf16
//     (q4_device.h::dequant8_mix, exact), shared by the TM tokens; with
//     64-token tiles this dequantization is most of the VALU work (SQ
//     counters: about 128 VALU instructions per wave and step against 16
//     MFMAs), so the streaming kernel stays faster below 32 tokens;
//   * the TM x 64 activation tile goes into LDS as bf16. fp32 activations
//     are split exactly into up to three bf16 terms (x = t0 + t1 + t2,
//     q4_device.h::split3), one pass over K per term: the first pass stages
//     t0 and notes whether any activation of the token tile has bits below
//     bf16 precision; only then do passes for t1 and t2 follow. Activations
//     that are already bf16-valued -- the reference's callers pass bf16
//     (runtime/py/model.py:399-485) -- cost one pass;
//   * each wave computes a 64-token x (64, or 16 for TM = 64) row sub-tile
//     with v_mfma_f32_16x16x32_bf16 (fp32 accumulation);
//   * the global loads of step k + S are issued before the MFMAs of step k
//     (S = 2 register stages for 256-token tiles, 4 for 64-token ones; one
//     stage for fp32 activations split in the kernel) and land in the other
//     half of a double-buffered LDS, so one barrier per step separates them;
//     the dequantization of step k + 1 sits between the two k-halves of step
//     k's MFMAs;
//   * fp32 activations are first split into three bf16 term arrays by
//     split_x_kernel (half the bytes per re-read, the token tile fits the
//     L2), with a per-token flag for the second and third terms;
//   * a grid that leaves half the CUs idle (the FFN's down projection: 30
//     weight tiles x 2 token tiles) splits K; the last workgroup of each tile
//     adds the partial tiles in split order (deterministic).
// Workgroups are numbered token-tile fastest: with the round-robin placement
// of workgroups on the 8 XCDs, the workgroups of one XCD share token tiles, so
// their activation reads hit that XCD's L2.
// LDS layout (conflict-free 16-byte operand reads, measured): each tile is
// split into 8 planes, one per 8-column octet of the step's 64 k, and a plane
// holds 16 bytes per row. A wave's operand read (16 consecutive rows x 4
// octets) then touches 16 consecutive 16-byte slots in each of 4 planes, and
// the weight stores (row per lane) are contiguous. Activation rows sit at
// slot token ^ (2 * plane) inside their aligned group of 16, so the
// 8 lanes that store one token's 8 octets (row-major global loads) hit 8
// different banks, and so do the stores of the next token.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

constexpr int TN = 128;  // weight rows per tile
constexpr int TK = 64;   // k per step (two Q4 blocks)
constexpr int KP = TK / 8;    // octet planes per step
constexpr int kGemmThreads = 512;

// Token tile TM (256, or 64 for small batches): the 8 waves form a
// (TM / 64) x (8 / (TM / 64)) grid over (tokens, weight rows); each wave
// computes 64 tokens x (TN / waves across rows) rows per matrix.
template <int TM>
struct GemmTile {
    static constexpr int WAVES_M = TM / 64;
    static constexpr int WAVES_N = 8 / WAVES_M;
    static constexpr int WN = TN / WAVES_N;   // weight rows per wave
    static constexpr int JJ = WN / 16;        // 16-row blocks per wave
    static constexpr int XI = TM / 64;        // activation loads per thread (64 tokens per pass)
};

// bf16 offset of 16-byte slot `row` of plane p in a tile of `rows` rows.
__device__ __forceinline__ size_t wslot(int p, int row) { return ((size_t)p * TN + row) * 8; }
template <int TM>
__device__ __forceinline__ size_t xslot(int p, int token) { return ((size_t)p * TM + (token ^ (2 * p))) * 8; }

struct GemmArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const void* X;           // fp32 activations (XF32) or bf16 bit patterns
    float* Y;                // fp32 output, or
    uint16_t* Yb;            // bf16 output (bit patterns)
    uint32_t wbytes;
    uint32_t xbytes;         // bytes of X (buffer range, all terms)
    int ldx, ldy, M, N, K, parts, act;
    TileGeom tg;
    // bf16 activations given as three term arrays tstride elements apart
    // (split_x_kernel): tflags[m] != 0 when token m has a nonzero second or
    // third term. Null: one term.
    const uint32_t* tflags;
    uint32_t tstride;
    // Split K (grid.z = ks): partial tiles and per-tile arrival counters.
    int ks;
    float* part;
    uint32_t* cnt;
};

template <int NT, bool TILED, bool XF32, int TM>
__global__ void __launch_bounds__(kGemmThreads) gemm_q4_kernel(GemmArgs a) {
    using G = GemmTile<TM>;
    constexpr int JJ = G::JJ, XI = G::XI;
    extern __shared__ __align__(16) unsigned char smem[];
    // [buffer][matrix][plane][row] weights, then [buffer][plane][token] activations.
    __bf16* wsm = reinterpret_cast<__bf16*>(smem);
    __bf16* xsm = wsm + (size_t)2 * NT * KP * TN * 8;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
    const int m0 = blockIdx.x * TM;
    const int n0 = blockIdx.y * TN;
    const int nsteps_all = (a.K + TK - 1) / TK;
    // Split K: this workgroup's steps [st0, st0 + nsteps).
    const int kq = blockIdx.z;
    const int st0 = kq * nsteps_all / a.ks;
    const int nsteps = (kq + 1) * nsteps_all / a.ks - st0;
    const int j = lane & 15, g = lane >> 4;
    const uint32_t rs = (uint32_t)(a.K >> 5) * kBlockBytes;

    // Staging roles. Weights: wave -> (block wb of the step's two, matrix
    // wmat, half of the 128 rows), lane -> row, so a thread's row is fixed and
    // the part of each load address that moves with the step is wave-uniform
    // (an SGPR soffset; no per-step address arithmetic per lane). Waves past
    // the NT x 2 x 2 roles stay idle. Activations: thread -> 8 consecutive k
    // of one token, 4 tokens 64 apart.
    const int wb = wave & 1;
    const int wmat = NT == 2 ? (wave >> 1) & 1 : 0;
    const int rh = NT == 2 ? wave >> 2 : wave >> 1;
    const bool wstage = rh < 2;
    const int wr = rh * 64 + lane;
    const int wrow = n0 + wr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wmat ? a.W1 : a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);
    // Lane parts of the addresses (past the range: the loads return zeros).
    const uint32_t wv = wstage && wrow < a.N ? (TILED ? (uint32_t)(wrow >> 4) * a.tg.rtb + (uint32_t)(wrow & 15) * 16u
                                                      : (uint32_t)wrow * rs)
                                             : a.wbytes;
    uint32_t xv[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int m = m0 + (tid >> 3) + 64 * i;
        xv[i] = m < a.M ? (uint32_t)(((size_t)m * a.ldx + (tid & 7) * 8) * (XF32 ? 4 : 2)) : a.xbytes;
    }

    f32x4 acc[NT][4][JJ];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < JJ; ++jj) acc[n][i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int XV = XF32 ? 2 : 1;  // 16-byte loads per 8 activations
    // One register stage for fp32 activations (twice the registers per
    // stage); bf16 activations keep S stages (below).
    uint32_t wreg0[5];
    u32x4 xreg0[XI][XV];
    uint32_t lowbits = 0;  // OR of all fp32 activation bits seen by the first pass

    // Global loads of step s (absolute) of activation term p into registers.
    // Activations past K (a last step half past it) read the next token's
    // values or zeros: finite, and their weights are zero. Issued on every
    // path -- past the last step (in = false) the loads read past the buffers
    // and return zeros -- so the compiler's wait counts stay exact and a wait
    // for one register stage never drains the other.
    auto load = [&](int s, bool in, int p, uint32_t (&wreg)[5], u32x4 (&xreg)[XI][XV]) __attribute__((always_inline)) {
        const int kb = s * 2 + wb;
        const bool ok = in && kb < (a.K >> 5);
#pragma unroll
        for (int x = 0; x < 5; ++x) {
            uint32_t so = a.wbytes;
            if (ok) {
                if constexpr (TILED) {
                    // Byte 4x of block kb within the row's run: super-step kb / 16,
                    // plane (20 bl + 4x) / 16, lane group g (q4_device.h tiled layout).
                    const int ss = kb >> 4, gq = (kb >> 2) & 3, rb = 20 * (kb & 3) + 4 * x;
                    const uint32_t ng = ss == a.tg.nss - 1 ? (uint32_t)a.tg.ng_last : 4u;
                    so = (uint32_t)ss * 5120u + (uint32_t)(rb >> 4) * 256u * ng + (uint32_t)gq * 256u + (uint32_t)(rb & 15);
                } else {
                    so = (uint32_t)kb * kBlockBytes + 4u * x;
                }
            }
            wreg[x] = __builtin_amdgcn_raw_buffer_load_b32(rw, wv, __builtin_amdgcn_readfirstlane(so), 0);
        }
        const uint32_t xo = __builtin_amdgcn_readfirstlane(
            in ? (uint32_t)(((size_t)s * TK + (XF32 ? 0 : (size_t)p * a.tstride)) * (XF32 ? 4 : 2)) : a.xbytes);
#pragma unroll
        for (int i = 0; i < XI; ++i)
#pragma unroll
            for (int v = 0; v < XV; ++v)
                xreg[i][v] = __builtin_amdgcn_raw_buffer_load_b128(rx, xv[i] + 16 * v, xo, 0);
    };
    // Registers of a load into LDS buffer b, activations as term p.
    auto store_w = [&](int b, const uint32_t (&wreg)[5]) __attribute__((always_inline)) {
        if (wstage) {
            const Scale2 sc = make_scale2(bf16_bits_to_f32(wreg[4] & 0xFFFFu));
            __bf16* tile = wsm + (size_t)(b * NT + wmat) * KP * TN * 8;
#pragma unroll
            for (int t = 0; t < 4; ++t) *reinterpret_cast<bf16x8*>(tile + wslot(4 * wb + t, wr)) = dequant8_mix(wreg[t], sc);
        }
    };
    auto store_x = [&](int b, int p, const u32x4 (&xreg)[XI][XV]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int r = (tid >> 3) + 64 * i, o = tid & 7;
            u32x4* dst = reinterpret_cast<u32x4*>(xsm + (size_t)b * KP * TM * 8 + xslot<TM>(o, r));
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
    auto store = [&](int b, int p, const uint32_t (&wreg)[5], const u32x4 (&xreg)[XI][XV]) __attribute__((always_inline)) {
        store_w(b, wreg);
        store_x(b, p, xreg);
    };

    int nterms = 1;
    if (!XF32 && a.tflags) {
        // Terms 1 and 2 only for a token tile with a token that has them.
        const int m = m0 + (tid & (TM - 1));
        nterms = __syncthreads_or(tid < TM && m < a.M && a.tflags[m] != 0) ? 3 : 1;
    }
    auto compute_kk = [&](int b, int kk) __attribute__((always_inline)) {
        {
            bf16x8 bv[NT][JJ];
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj)
                    bv[n][jj] = *reinterpret_cast<const bf16x8*>(
                        wsm + (size_t)(b * NT + n) * KP * TN * 8 + wslot(kk * 4 + g, wn * G::WN + jj * 16 + j));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(
                    xsm + (size_t)b * KP * TM * 8 + xslot<TM>(kk * 4 + g, wm * 64 + i * 16 + j));
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int jj = 0; jj < JJ; ++jj) acc[n][i][jj] = mfma16x16x32(av, bv[n][jj], acc[n][i][jj]);
            }
        }
    };
    auto compute = [&](int b) __attribute__((always_inline)) {
        compute_kk(b, 0);
        compute_kk(b, 1);
    };
    for (int p = 0; p < nterms; ++p) {
        if constexpr (XF32) {
            // fp32 activations take twice the registers per stage: one stage,
            // loads one step ahead.
            load(st0, true, p, wreg0, xreg0);
            store(0, p, wreg0, xreg0);
            __syncthreads();
            for (int s = 0; s < nsteps; ++s) {
                const int b = s & 1;
                load(st0 + s + 1, s + 1 < nsteps, p, wreg0, xreg0);
                compute(b);
                if (s + 1 < nsteps) store(b ^ 1, p, wreg0, xreg0);
                __syncthreads();
            }
        } else {
            // S register stages: stage t % S holds step t from its load (issued
            // S steps ahead) until its store into LDS buffer t & 1 during step
            // t - 1; then it is reloaded with step t + S. Step t computes
            // buffer t & 1 while the dequantization and activation stores of
            // step t + 1 sit between its two k halves, so VALU and matrix work
            // of one wave overlap. 64-token tiles take short steps and need
            // the deeper prefetch to cover the loads' latency.
            constexpr int S = TM == 64 ? 4 : 2;
            uint32_t wst[S][5];
            u32x4 xst[S][XI][XV];
#pragma unroll
            for (int q = 0; q < S; ++q) load(st0 + q, q < nsteps, p, wst[q], xst[q]);
            store(0, p, wst[0], xst[0]);
            __syncthreads();
            for (int s = 0; s < nsteps; s += S) {
#pragma unroll
                for (int q = 0; q < S; ++q) {
                    const int t = s + q;
                    if (t >= nsteps) break;
                    const int b = q & 1;
                    load(st0 + t + S, t + S < nsteps, p, wst[q], xst[q]);
                    compute_kk(b, 0);
                    if (t + 1 < nsteps) store_w(b ^ 1, wst[(q + 1) % S]);
                    compute_kk(b, 1);
                    if (t + 1 < nsteps) store_x(b ^ 1, p, xst[(q + 1) % S]);
                    __syncthreads();
                }
            }
        }
        // After the first pass: residual terms only for a token tile with
        // activations that are not bf16-valued.
        if (XF32 && p == 0 && a.parts == 3) nterms = __syncthreads_or((lowbits & 0xFFFFu) != 0) ? 3 : 1;
    }

    // ---- split K: the last workgroup of the tile adds the partial tiles -------------
    // Each workgroup writes its partial tile through (agent-scope stores) and
    // counts itself in once they have landed; the one that completes the count
    // reads all of them (sc1) and sums them in split order, so the result does
    // not depend on which came last, then resets the count.
    if (a.ks > 1) {
        // Each thread's accumulators go out as whole 16-byte pieces, thread
        // tid's f32x4 (n, i, jj) at ((n * 16 + 4 i + jj) * 512 + tid) * 16 bytes
        // of the split's partial tile, so a wave writes 1 KiB contiguous with
        // write-through (sc1) stores -- single-float write-through stores cost
        // a partial-line write each -- and the last workgroup's thread tid
        // reads back exactly the pieces it adds to its own accumulators.
        const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
        const size_t tsz = (size_t)NT * TM * TN;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.part + tile * a.ks * tsz, (uint32_t)(a.ks * tsz * sizeof(float)));
        auto piece = [&](int q, int n, int i, int jj) -> uint32_t {
            return (uint32_t)(((((size_t)q * NT + n) * 4 * JJ + JJ * i + jj) * kGemmThreads + tid) * 16);
        };
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[n][i][jj]), rp,
                                                           piece(kq, n, i, jj), 0, 16);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __shared__ int last;
        __syncthreads();
        if (tid == 0)
            last = __hip_atomic_fetch_add(&a.cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(a.ks - 1);
        __syncthreads();
        if (!last) return;
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj) acc[n][i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int q = 0; q < a.ks; ++q)
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int jj = 0; jj < JJ; ++jj)
                        acc[n][i][jj] += __builtin_bit_cast(f32x4, buf_load16_sc1(rp, piece(q, n, i, jj)));
        if (tid == 0) __hip_atomic_store(&a.cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- epilogue: D[4g + r][j] of each 16 x 16 sub-tile ----------------------------
    auto put = [&](int m, int n, float out) __attribute__((always_inline)) {
        if (a.Yb)
            a.Yb[(size_t)m * a.ldy + n] = __builtin_bit_cast(uint16_t, (__bf16)out);
        else
            a.Y[(size_t)m * a.ldy + n] = out;
    };
    if constexpr (NT == 2) {
        // GLU: the float32 path inside the unrolled loop; the few values it
        // cannot settle keep their (g, u) in LDS (free after the main loop)
        // and are finished one at a time on the float64 path, so the unrolled
        // code stays small and the accumulators stay in registers.
        __syncthreads();
        uint32_t* stash = reinterpret_cast<uint32_t*>(smem) + (size_t)tid * (16 * JJ);
        uint64_t miss = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + wm * 64 + i * 16 + 4 * g + r;
                    const int n = n0 + wn * G::WN + jj * 16 + j;
                    if (m >= a.M || n >= a.N) continue;
                    const float gb = bf16_round(acc[0][i][jj][r]), ub = bf16_round(acc[1][i][jj][r]);
                    float v;
                    if (glu_fast(gb, ub, a.act, &v)) {
                        put(m, n, bf16_round(v));
                    } else {
                        const int e = (i * JJ + jj) * 4 + r;
                        miss |= 1ull << e;
                        stash[e] = (__builtin_bit_cast(uint32_t, gb) >> 16) | (__builtin_bit_cast(uint32_t, ub) & 0xFFFF0000u);
                    }
                }
        while (miss) {
            const int e = __builtin_ctzll(miss);
            miss &= miss - 1;
            const uint32_t pk = stash[e];
            const float gb = __builtin_bit_cast(float, pk << 16), ub = __builtin_bit_cast(float, pk & 0xFFFF0000u);
            const int i = (e >> 2) / JJ, jj = (e >> 2) % JJ, r = e & 3;
            put(m0 + wm * 64 + i * 16 + 4 * g + r, n0 + wn * G::WN + jj * 16 + j, bf16_round(glu_exact(gb, ub, a.act)));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + 4 * g + r;
                const int n = n0 + wn * G::WN + jj * 16 + j;
                if (m >= a.M || n >= a.N) continue;
                put(m, n, acc[0][i][jj][r]);
            }
}

// Output rows [N, Nz) of every token as zeros (the all-zero trailing rows a
// registration trimmed off).
__global__ void __launch_bounds__(256) zero_rows_kernel(float* Y, uint16_t* Yb, int ldy, int M, int N, int Nz) {
    const int nz = Nz - N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)nz * M; i += (int64_t)gridDim.x * 256) {
        const int m = (int)(i / nz), r = N + (int)(i % nz);
        if (Yb)
            Yb[(size_t)m * ldy + r] = 0;
        else
            Y[(size_t)m * ldy + r] = 0.0f;
    }
}

// fp32 activations -> three bf16 term arrays (exact split, q4_device.h::split3)
// once per call, so the GEMM reads half the bytes per activation and its
// token tiles hold them in L2; flags[m] != 0 when token m has a nonzero second
// or third term. One workgroup per token.
__global__ void __launch_bounds__(256) split_x_kernel(const float* X, int ldx, int K, uint16_t* T, uint32_t tstride,
                                                      uint32_t* flags) {
    const int m = blockIdx.x;
    const float* x = X + (size_t)m * ldx;
    uint16_t* t = T + (size_t)m * K;
    bool more = false;
    for (int k = threadIdx.x; k < K; k += 256) {
        const Split3 sp = split3(x[k]);
        const uint16_t b1 = __builtin_bit_cast(uint16_t, sp.p1), b2 = __builtin_bit_cast(uint16_t, sp.p2);
        t[k] = __builtin_bit_cast(uint16_t, sp.p0);
        t[k + tstride] = b1;
        t[(size_t)k + 2 * (size_t)tstride] = b2;
        more |= ((b1 | b2) & 0x7FFFu) != 0;
    }
    more = __syncthreads_or(more);
    if (threadIdx.x == 0) flags[m] = more ? 1u : 0u;
}

template <int NT, bool TILED, bool XF32, int TM>
hipError_t launch_gemm(const GemmArgs& a, dim3 grid, hipStream_t s) {
    const size_t lds = (size_t)2 * KP * (NT * TN + TM) * 8 * sizeof(uint16_t);
    static bool attr[64] = {};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    if (dev >= 64 || !attr[dev]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_q4_kernel<NT, TILED, XF32, TM>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        if (dev < 64) attr[dev] = true;
    }
    hipLaunchKernelGGL((gemm_q4_kernel<NT, TILED, XF32, TM>), grid, dim3(kGemmThreads), lds, s, a);
    return hipGetLastError();
}

template <int NT, bool TILED>
hipError_t launch_gemm_x(const GemmArgs& a, bool xf32, int tm, dim3 grid, hipStream_t s) {
    if (tm == 64)
        return xf32 ? launch_gemm<NT, TILED, true, 64>(a, grid, s) : launch_gemm<NT, TILED, false, 64>(a, grid, s);
    return xf32 ? launch_gemm<NT, TILED, true, 256>(a, grid, s) : launch_gemm<NT, TILED, false, 256>(a, grid, s);
}

}  // namespace

int launch_gemm_tiled(const GemvLaunch& L, hipStream_t s) {
    const uint64_t wbytes = L.tiled ? tile_bytes(L.N, L.K) : (uint64_t)L.N * (uint64_t)(L.K / 32) * kBlockBytes;
    // Lane offset + step offset of a load must not wrap 32 bits: weights below
    // 3.75 GiB, activations below 2 GiB.
    if (wbytes >= 0xF0000000ull) return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 3.75 GiB prefill range", (unsigned long long)wbytes);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    bool xf32 = L.Xb == nullptr;
    const void* x = xf32 ? static_cast<const void*>(L.X) : static_cast<const void*>(L.Xb);
    // 16-byte activation loads: 4-byte aligned rows for fp32; for bf16 (the FFN's
    // own activation buffer) 16-byte aligned rows.
    if (xf32 ? reinterpret_cast<uintptr_t>(x) % 4 != 0 : reinterpret_cast<uintptr_t>(x) % 16 != 0 || L.ldx % 8 != 0)
        return fail(ALV_ERR_ALIGN, "prefill activations are not aligned for 16-byte loads");
    uint64_t xbytes = ((uint64_t)(L.M - 1) * L.ldx + L.K) * (xf32 ? 4 : 2);
    if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activations of %llu bytes exceed the 2 GiB buffer range", (unsigned long long)xbytes);
    const int NT = L.glu ? 2 : 1;
    // Token tile: 64 for small batches (a quarter of the MFMA and LDS work per
    // weight tile of the 256-token tile), 256 above small_tile_max_m().
    const int TM = L.M <= small_tile_max_m() ? 64 : 256;
    const dim3 tiles((L.M + TM - 1) / TM, (L.N + TN - 1) / TN);
    const int ntiles = (int)(tiles.x * tiles.y);
    // Split K while the grid leaves CUs idle and each split keeps enough
    // steps: 256-token tiles aim at one workgroup per CU (16+ steps each);
    // 64-token tiles at ALV_GEMM_SMALL_WG_PER_CU workgroups per CU (default
    // 1; 2-4 measured no faster) with 8+ steps each.
    const int nsteps = (L.K + TK - 1) / TK;
    int ks = 1;
    const int wg_target = TM == 64 ? small_wg_per_cu() * device_cus() : device_cus();
    const int min_steps = TM == 64 ? 8 : 16;
    while (ntiles * ks * 2 <= wg_target && nsteps / (ks * 2) >= min_steps) ks *= 2;
    // Split-K arrival counters: the stream's dedicated counter words (zero
    // between launches, shared with the streaming kernel's split K), never
    // the scratch below, whose bytes hold other launches' flags and terms.
    Workspace ws{};
    if (ks > 1 && (ntiles > kSplitCounters || get_workspace(s, (size_t)ntiles, &ws))) {
        clear_error();
        ks = 1;
    }
    // Scratch: token flags and partial tiles, then the activation terms.
    const size_t flag_bytes = ((size_t)L.M * 4 + 255) & ~(size_t)255;
    const size_t tstride = (size_t)L.M * L.K;
    const size_t term_bytes = xf32 ? 3 * tstride * sizeof(uint16_t) : 0;
    void* scratch = nullptr;
    size_t part_bytes = 0;
    if (ks > 1 || xf32) {
        part_bytes = ks > 1 ? (size_t)ntiles * ks * NT * TM * TN * sizeof(float) : 0;
        if (6 * tstride >= 0x7FFFFF00ull || get_scratch(s, kScratchGemm, flag_bytes + part_bytes + term_bytes, &scratch)) {
            // No scratch (a graph capture that would have to grow it): one
            // launch over all of K, activations split inside the kernel.
            clear_error();
            scratch = nullptr;
            ks = 1;
            part_bytes = 0;
        }
    }
    uint8_t* sb = static_cast<uint8_t*>(scratch);
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
    a.ks = ks;
    if (sb) {
        a.cnt = ks > 1 ? ws.counters : nullptr;
        a.part = reinterpret_cast<float*>(sb + flag_bytes);
        if (xf32) {
            uint32_t* flags = reinterpret_cast<uint32_t*>(sb);
            uint16_t* terms = reinterpret_cast<uint16_t*>(sb + flag_bytes + part_bytes);
            hipLaunchKernelGGL(split_x_kernel, dim3(L.M), dim3(256), 0, s, L.X, L.ldx, L.K, terms, (uint32_t)tstride, flags);
            if (int rc = hip_check(hipGetLastError(), "split_x_kernel launch")) return rc;
            a.X = terms;
            a.ldx = L.K;
            a.tflags = L.parts == 3 ? flags : nullptr;
            a.tstride = (uint32_t)tstride;
            a.xbytes = (uint32_t)(3 * tstride * sizeof(uint16_t));
            xf32 = false;
        }
    }
    const dim3 grid(tiles.x, tiles.y, ks);
    hipError_t e;
    if (L.glu)
        e = L.tiled ? launch_gemm_x<2, true>(a, xf32, TM, grid, s) : launch_gemm_x<2, false>(a, xf32, TM, grid, s);
    else
        e = L.tiled ? launch_gemm_x<1, true>(a, xf32, TM, grid, s) : launch_gemm_x<1, false>(a, xf32, TM, grid, s);
    if (int rc = hip_check(e, "gemm_q4_kernel launch")) return rc;
    if (L.Nz > L.N) {
        const int64_t n = (int64_t)(L.Nz - L.N) * L.M;
        const int zg = (int)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 1024));
        hipLaunchKernelGGL(zero_rows_kernel, dim3(zg), dim3(256), 0, s, L.Y, L.Yb, L.ldy, L.M, L.N, L.Nz);
        return hip_check(hipGetLastError(), "zero_rows_kernel launch");
    }
    return ALV_OK;
}

}  // namespace alv
