// Streaming Q4 matrix-vector kernel for decode and small-M batches (gfx950):
// the M <= 16 path of alv_gemv_q, alv_gemv, alv_gemm_q and alv_ffn_fused.
//
// The kernel is HBM-bound by design: weights are read once with 16-byte
// loads, dequantized in registers (q4_device.h::dequant8, ~2.4 VALU ops per
// weight) and multiplied on the matrix cores. Doing the products on MFMA even
// at M = 1 keeps the VALU budget for the exact bf16 dequantization.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, D = A x B):
//   B columns = 16 weight rows (one row tile), B k = 32 weights;
//   A rows    = activation terms: token m contributes `parts` rows (its fp32
//               value split exactly into 3 bf16 terms, or 1 term when the
//               activation is bf16); rows >= parts*M are don't-care (their
//               lanes read a valid row; the D rows they feed are unused).
// Lane l = (j, g), j = l % 16, g = l / 16 owns weight row j and, within a
// super-step of 16 blocks (512 k), blocks 4g..4g+3 of that row: an 80-byte
// run held as five 16-byte pieces. The A operand for the same k comes from
// LDS, where the workgroup staged its K range in MFMA operand order.
//
// Work split: K is cut into KS chunks; workgroup b works on chunk b % KS and
// stages that chunk's activations once. Each of its waves then streams whole
// jobs -- one row tile over the chunk -- one super-step ("unit") at a time,
// with the weight loads of the next P units in flight while it computes the
// current one. The prefetch ring is unrolled so every buffer index is static
// and every iteration has the same loads outstanding. A finished job writes
// its rows (KS = 1) or a partial sum; the last chunk to arrive at a row tile
// (per-row-tile counter) adds the partials in chunk order, so results do not
// depend on scheduling.
//
// Weights come either in the combined layout (RAW: a lane's 80-byte run is
// contiguous, a wave's 16-byte loads touch 16 rows x 4 runs and lean on the
// caches to merge) or in the tiled layout (TILED, q4_device.h: every load
// instruction of a wave reads 1 KiB of contiguous memory, with the
// nontemporal hint since weights are read once). Out-of-range loads (buffer
// resource bounds) return zero, which is how tails are handled.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

struct StreamArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const void* X;   // fp32 (XB = false) or bf16 (XB = true) activations
    float* Y;        // fp32 output, or
    uint16_t* Yb;    // bf16 output (bit patterns)
    float* partial;
    uint32_t* counters;
    uint32_t wbytes;  // weight buffer range in bytes
    uint32_t xbytes;  // activation buffer range in bytes
    uint32_t rstride; // bytes per row (RAW) or per row tile (TILED)
    uint32_t xs_bytes;  // LDS bytes of the staged activations
    int ldx, ldy, M, N, K;
    int parts;  // activation terms per token (1 or 3)
    int R;      // parts * M, rows of A in use
    int nb, nss, ng_last, RT;
    int KS, nss_c;  // K chunks and super-steps per chunk
    int act;
};

constexpr int kStreamThreads = 512;  // at most 8 waves per workgroup (room for 256 VGPRs)

template <bool XB>
__device__ __forceinline__ void stage_octet(const u32x4 (&v)[2], __bf16* dst, int parts) {
    if constexpr (XB) {
        *reinterpret_cast<u32x4*>(dst) = v[0];
    } else {
        // Convert each element as a value: hipcc miscompiles __builtin_bit_cast
        // applied directly to a vector-element lvalue (it reads element 0).
        float f[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) f[4 * h + e] = __builtin_bit_cast(float, (uint32_t)v[h][e]);
        if (parts == 3) {
            bf16x8 p0, p1, p2;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const Split3 s = split3(f[e]);
                p0[e] = s.p0;
                p1[e] = s.p1;
                p2[e] = s.p2;
            }
            *reinterpret_cast<bf16x8*>(dst) = p0;
            *reinterpret_cast<bf16x8*>(dst + 8) = p1;
            *reinterpret_cast<bf16x8*>(dst + 16) = p2;
        } else {
            bf16x8 p0;
#pragma unroll
            for (int e = 0; e < 8; ++e) p0[e] = (__bf16)f[e];
            *reinterpret_cast<bf16x8*>(dst) = p0;
        }
    }
}

// P: units of prefetch; AT: 16-row A tiles; RC: rows of A known at compile
// time (1: one bf16 token, 3: one fp32 token; 0 = a.R at run time, which makes
// the LDS operand addresses run-time values).
template <int P, int AT, int RC, bool GLU, bool XB, bool TILED>
__global__ void __launch_bounds__(kStreamThreads) q4_stream_kernel(StreamArgs a) {
    constexpr int NT = GLU ? 2 : 1;
    constexpr int NB = P + 1;
    constexpr int ES = XB ? 2 : 4;  // activation element size
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int WPB = nthr >> 6;
    const int R = RC ? RC : a.R;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int chunk = blockIdx.x % a.KS;
    const int grp = blockIdx.x / a.KS;
    const int ngrp = gridDim.x / a.KS;
    const int ss0 = chunk * a.nss_c;             // first super-step of the chunk
    const int css = min(a.nss_c, a.nss - ss0);   // super-steps in the chunk
    float* scratch = reinterpret_cast<float*>(smem + a.xs_bytes) + wave * (NT * AT * 256);

    // Jobs of this wave: row tiles rt_first, rt_first + rt_step, ...
    const int rt_first = grp * WPB + wave;
    const int rt_step = ngrp * WPB;
    const int njobs = rt_first < a.RT ? (a.RT - rt_first + rt_step - 1) / rt_step : 0;
    const int U = njobs * css;

    // ---- weight loads of one unit ----------------------------------------------
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);
    // Lane offset (fixed) + unit offset (wave-uniform, in soffset). Invalid
    // units start at wbytes: every piece is out of range and reads zero.
    // Combined layout: lane (j, g) sits at row j, byte 80 g of the super-step;
    // rows past N fall past wbytes. Tiled layout: lane l at 16 l of each plane.
    const uint32_t voff = TILED ? 16u * (uint32_t)lane : (uint32_t)j * a.rstride + 80u * (uint32_t)g;
    auto issue = [&](u32x4 (&q)[NT][5], int rt, int s) {
        const int ss = ss0 + s;
        uint32_t soff = a.wbytes, step = 16;
        if constexpr (TILED) {
            step = ss == a.nss - 1 ? 256u * (uint32_t)a.ng_last : 1024u;
            if (rt < a.RT) soff = (uint32_t)rt * a.rstride + (uint32_t)ss * 5120u;
        } else {
            if (rt < a.RT) soff = (uint32_t)rt * 16u * a.rstride + (uint32_t)ss * 320u;
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            q[0][i] = buf_load16_so<TILED>(r0, voff, soff + step * i);
            if constexpr (GLU) q[1][i] = buf_load16_so<TILED>(r1, voff, soff + step * i);
        }
    };

    u32x4 buf[NB][NT][5];
    int prt = rt_first, ps = 0;  // prefetch cursor
    auto advance = [&](int& rt, int& s) {
        if (++s == css) {
            s = 0;
            rt += rt_step;
        }
    };
#pragma unroll
    for (int b = 0; b < P; ++b) {
        issue(buf[b], U > 0 ? prt : a.RT, ps);
        advance(prt, ps);
    }

    // ---- stage this chunk's activations (their waits cover the prefetch) ----
    // Octet o (8 consecutive k) of token m: k = ss0 * 512 + 8 o. It lives at
    // operand slot ((o / 64) * 16 + o % 16) * 4 + (o / 16) % 4, i.e. super-step
    // o / 64, block 4g + bl with g = (o / 16) % 4, bl = (o / 4) % 4, dword
    // t = o % 4: slot = (ss * 16 + bl * 4 + t) * 4 + g.
    {
        const int octs = css * 64;
        const int units = octs * a.M;
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);
        for (int u = tid; u < units; u += nthr) {
            int m = 0, o = u;
            if (a.M != 1) {
                m = u / octs;
                o = u - m * octs;
            }
            const int k = ss0 * 512 + o * 8;
            const uint32_t off = k < a.K ? (uint32_t)((m * a.ldx + k) * ES) : a.xbytes;
            u32x4 v[2];
            v[0] = buf_load16(rx, off);
            v[1] = XB ? u32x4{0u, 0u, 0u, 0u} : buf_load16(rx, off + 16);
            const int slot = ((o >> 6) * 16 + (o & 15)) * 4 + ((o >> 4) & 3);
            stage_octet<XB>(v, xs + ((size_t)slot * R + (size_t)m * a.parts) * 8, a.parts);
        }
    }
    __syncthreads();

    // ---- stream the units ----------------------------------------------------------
    const __bf16* xa[AT];  // operand base of this lane: slot g, row arow
#pragma unroll
    for (int at = 0; at < AT; ++at) xa[at] = xs + ((size_t)g * R + min(at * 16 + j, R - 1)) * 8;

    f32x4 acc[NT][AT][2];
    auto zero_acc = [&]() {
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int at = 0; at < AT; ++at) acc[n][at][0] = acc[n][at][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    zero_acc();

    auto compute = [&](const u32x4 (&q)[NT][5], int s) {
        const int sl_off = s * 64 * R * 8;  // this super-step's operands (bf16 elements)
        // Blocks of this lane that exist. Tiled: a lane past the last
        // super-step's ng reads the next plane's bytes; combined: blocks past
        // the row end read the next row's. Their scales are cleared (their
        // activations are zero), so the garbage dequantizes to zero.
        const int ss = ss0 + s;
        const int nvalid = TILED ? (ss != a.nss - 1 || g < a.ng_last ? 4 : 0) : a.nb - (ss * 16 + g * 4);
#pragma unroll
        for (int bl = 0; bl < 4; ++bl) {
            Scale sc[NT];
            uint32_t dw[NT][4];
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                // dwords 5*bl .. 5*bl+4 of the 80-byte run are this block.
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int w = 5 * bl + t;
                    dw[n][t] = q[n][w >> 2][w & 3];
                }
                const int w4 = 5 * bl + 4;
                const uint32_t sd = bl < nvalid ? (uint32_t)q[n][w4 >> 2][w4 & 3] : 0u;
                sc[n] = make_scale(scale_of(sd));
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int so = sl_off + (bl * 4 + t) * 4 * R * 8;
                bf16x8 av[AT];
#pragma unroll
                for (int at = 0; at < AT; ++at) av[at] = *reinterpret_cast<const bf16x8*>(xa[at] + so);
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const bf16x8 b = dequant8(dw[n][t], sc[n]);
#pragma unroll
                    for (int at = 0; at < AT; ++at)
                        acc[n][at][t & 1] = mfma16x16x32(av[at], b, acc[n][at][t & 1]);
                }
            }
        }
    };

    // Output (m, jj) of a finished job: y = sum over terms p (in order) of
    // D[m * parts + p][jj], read back through this wave's LDS scratch.
    const size_t plane = (size_t)a.M * a.N;
    auto finish = [&](int rt) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int at = 0; at < AT; ++at)
                *reinterpret_cast<f32x4*>(scratch + (n * AT + at) * 256 + lane * 4) = acc[n][at][0] + acc[n][at][1];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        auto term_sum = [&](int n, int m, int jj) {
            float y = 0.0f;
            for (int p = 0; p < a.parts; ++p) {
                const int i = m * a.parts + p;
                const int ii = i & 15;
                y += scratch[(n * AT + (i >> 4)) * 256 + (jj + 16 * (ii >> 2)) * 4 + (ii & 3)];
            }
            return y;
        };
        auto store = [&](int m, int row, float y0, float y1) {
            float out = y0;
            if constexpr (GLU) out = bf16_round(glu_act(bf16_round(y0), bf16_round(y1), a.act));
            if (a.Yb)
                a.Yb[(size_t)m * a.ldy + row] = __builtin_bit_cast(uint16_t, (__bf16)out);
            else
                a.Y[(size_t)m * a.ldy + row] = out;
        };
        if (a.KS == 1) {
            for (int idx = lane; idx < a.M * 16; idx += 64) {
                const int m = idx >> 4, jj = idx & 15, row = rt * 16 + jj;
                if (row < a.N) store(m, row, term_sum(0, m, jj), GLU ? term_sum(NT - 1, m, jj) : 0.0f);
            }
            return;
        }
        // Partial sums are written through to the device-coherent level (agent
        // scope atomic stores bypass this XCD's L2), the wave waits until they
        // have landed, then counts itself in; the last chunk reads them back
        // the same way. No L2-wide writeback or invalidate is needed.
        for (int idx = lane; idx < a.M * 16; idx += 64) {
            const int m = idx >> 4, jj = idx & 15, row = rt * 16 + jj;
            if (row < a.N)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    __hip_atomic_store(&a.partial[((size_t)chunk * NT + n) * plane + (size_t)m * a.N + row],
                                       term_sum(n, m, jj), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(&a.counters[rt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (prev != (uint32_t)(a.KS - 1)) return;
        for (int idx = lane; idx < a.M * 16; idx += 64) {
            const int m = idx >> 4, jj = idx & 15, row = rt * 16 + jj;
            if (row >= a.N) continue;
            float y[NT];
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                float sum = 0.0f;
                for (int c = 0; c < a.KS; ++c)
                    sum += __hip_atomic_load(&a.partial[((size_t)c * NT + n) * plane + (size_t)m * a.N + row],
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                y[n] = sum;
            }
            store(m, row, y[0], y[NT - 1]);
        }
        if (lane == 0) __hip_atomic_store(&a.counters[rt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    int crt = rt_first, cs = 0;  // compute cursor
    for (int u0 = 0; u0 < U; u0 += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(buf[(b + P) % NB], prt, ps);  // past the end: out of range, no traffic
            advance(prt, ps);
            if (u0 + b < U) {  // wave-uniform
                compute(buf[b], cs);
                if (cs == css - 1) {
                    finish(crt);
                    zero_acc();
                }
                advance(crt, cs);
            }
        }
    }
}

// ---- host side -----------------------------------------------------------------

namespace {

struct Plan {
    int P, WPB, KS, JPW;  // prefetch units, waves per workgroup, K chunks, jobs per wave
    int nss_c, groups;
    size_t xs_bytes, lds;
};

constexpr int kNumCU = 256;                 // MI355X
constexpr size_t kStageLds = 48 * 1024;    // activation staging budget per workgroup
constexpr size_t kMaxLds = 64 * 1024;      // staging + per-wave scratch

Plan plan_stream(const GemvLaunch& L, bool tiled) {
    const int NT = L.glu ? 2 : 1;
    const int nb = L.K / 32, nss = (nb + 15) / 16, RT = (L.N + 15) / 16;
    const int R = L.parts * L.M, AT = (R + 15) / 16;
    Plan p{};
    p.P = AT == 1 ? 2 : 1;
    p.WPB = 4;
    p.JPW = 1;
    // Fewest K chunks whose staged activations fit, then more chunks while the
    // chip has fewer than ~4 jobs per CU and chunks keep >= 2 super-steps.
    const size_t ss_bytes = (size_t)1024 * R;
    p.KS = (int)std::max<size_t>(1, ((size_t)nss * ss_bytes + kStageLds - 1) / kStageLds);
    while ((long)RT * p.KS < 4L * kNumCU && (nss + p.KS) / (p.KS + 1) >= 2) ++p.KS;
    const char* ev = L.glu ? "ALV_PLAN_GLU" : L.Xb ? "ALV_PLAN_BF16" : "ALV_PLAN_F32";
    if (const char* e = getenv(ev)) {  // tuning override: P,WPB,KS,JPW
        int pp, w, k, jp;
        if (sscanf(e, "%d,%d,%d,%d", &pp, &w, &k, &jp) == 4 && pp >= 1 && pp <= 3 && (AT == 1 || pp == 1) &&
            w >= 1 && w <= kStreamThreads / 64 && k >= 1 && k <= nss && jp >= 1 &&
            (size_t)((nss + k - 1) / k) * ss_bytes <= kStageLds) {
            p.P = pp;
            p.WPB = w;
            p.KS = k;
            p.JPW = jp;
        }
    }
    p.nss_c = (nss + p.KS - 1) / p.KS;
    p.KS = (nss + p.nss_c - 1) / p.nss_c;  // no empty chunks
    p.xs_bytes = (size_t)p.nss_c * ss_bytes;
    while (p.WPB > 1 && p.xs_bytes + (size_t)p.WPB * NT * AT * 1024 > kMaxLds) p.WPB /= 2;
    p.groups = (RT + p.WPB * p.JPW - 1) / (p.WPB * p.JPW);
    p.lds = p.xs_bytes + (size_t)p.WPB * NT * AT * 1024;
    (void)tiled;
    return p;
}

template <int P, int AT, int RC, bool GLU, bool XB, bool TILED>
hipError_t launch_one(const StreamArgs& a, const Plan& p, hipStream_t s) {
    hipLaunchKernelGGL((q4_stream_kernel<P, AT, RC, GLU, XB, TILED>), dim3(p.groups * p.KS), dim3(64 * p.WPB),
                       p.lds, s, a);
    return hipGetLastError();
}

// One token (R = 1 for bf16 activations, 3 for fp32) gets compile-time operand
// offsets; other token counts use the run-time row count.
template <int RC, bool GLU, bool XB, bool TILED>
hipError_t launch_p(const StreamArgs& a, const Plan& p, hipStream_t s) {
    if (p.P == 3) return launch_one<3, 1, RC, GLU, XB, TILED>(a, p, s);
    if (p.P == 2) return launch_one<2, 1, RC, GLU, XB, TILED>(a, p, s);
    return launch_one<1, 1, RC, GLU, XB, TILED>(a, p, s);
}

template <bool GLU, bool XB, bool TILED>
hipError_t launch_variant(const StreamArgs& a, const Plan& p, int AT, hipStream_t s) {
    constexpr int R1 = XB ? 1 : 3;
    if (AT == 1)
        return a.R == R1 ? launch_p<R1, GLU, XB, TILED>(a, p, s) : launch_p<0, GLU, XB, TILED>(a, p, s);
    if (AT == 2) return launch_one<1, 2, 0, GLU, XB, TILED>(a, p, s);
    return launch_one<1, 3, 0, GLU, XB, TILED>(a, p, s);
}

template <bool TILED>
hipError_t launch_layout(const StreamArgs& a, const Plan& p, const GemvLaunch& L, hipStream_t s) {
    const int AT = (a.R + 15) / 16;
    if (L.glu) return launch_variant<true, false, TILED>(a, p, AT, s);
    if (L.Xb) return launch_variant<false, true, TILED>(a, p, AT, s);
    return launch_variant<false, false, TILED>(a, p, AT, s);
}

}  // namespace

int launch_gemv(const GemvLaunch& L, hipStream_t s) {
    if (L.M < 1 || L.M > kGemvMaxM) return fail(ALV_ERR_ARG, "stream kernel takes 1 <= M <= %d (got %d)", kGemvMaxM, L.M);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    if (L.Xb && (L.parts != 1 || L.glu)) return fail(ALV_ERR_ARG, "bf16 activations take one term and no GLU");
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const uint64_t rs = (uint64_t)tg.nb * kBlockBytes;
    const uint64_t wbytes = L.tiled ? (uint64_t)RT * tg.rtb : (uint64_t)L.N * rs;
    if (wbytes >= 0xFFFFE000ull) return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    const uint64_t xbytes = ((uint64_t)(L.M - 1) * L.ldx + L.K) * (L.Xb ? 2 : 4);
    if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activation buffer exceeds the 2 GiB range");
    const Plan p = plan_stream(L, L.tiled);
    StreamArgs a{};
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = L.Xb ? (const void*)L.Xb : (const void*)L.X;
    a.Y = L.Y;
    a.Yb = L.Yb;
    a.wbytes = (uint32_t)wbytes;
    a.xbytes = (uint32_t)xbytes;
    a.rstride = L.tiled ? tg.rtb : (uint32_t)rs;
    a.xs_bytes = (uint32_t)p.xs_bytes;
    a.ldx = L.ldx;
    a.ldy = L.ldy;
    a.M = L.M;
    a.N = L.N;
    a.K = L.K;
    a.parts = L.parts;
    a.R = L.parts * L.M;
    a.nb = tg.nb;
    a.nss = tg.nss;
    a.ng_last = tg.ng_last;
    a.RT = RT;
    a.KS = p.KS;
    a.nss_c = p.nss_c;
    a.act = L.act;
    if (p.KS > 1) {
        Workspace ws;
        const int NT = L.glu ? 2 : 1;
        if (int rc = get_workspace(s, (size_t)p.KS * NT * L.M * L.N, (size_t)RT, &ws)) return rc;
        a.partial = ws.partial;
        a.counters = ws.counters;
    }
    const hipError_t e = L.tiled ? launch_layout<true>(a, p, L, s) : launch_layout<false>(a, p, L, s);
    return hip_check(e, "q4_stream_kernel launch");
}

}  // namespace alv
