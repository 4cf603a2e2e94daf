// One-shot Q4 matrix-vector kernel for a single op (decode and small-M
// batches, gfx950): the kernel behind alv_gemv_q, alv_gemv, alv_gemm_q
// (M < 32) and alv_ffn_fused (M < 32). Chains of ops run on the op-chain
// executor (stream_q.hip).
//
// HBM-bound by design: weights are read once with 16-byte loads, dequantized
// in registers (q4_device.h::dequant8) and multiplied on the matrix cores.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, D = A x B):
//   B columns = 16 weight rows (one row tile), B k = 32 weights;
//   A rows    = activation terms: token m contributes `parts` rows (its fp32
//               value split exactly into 3 bf16 terms, or 1 term when the
//               activation is bf16); rows >= parts*M are don't-care.
// Lane l = (j, g), j = l % 16, g = l / 16 owns weight row j and, within a
// super-step of 16 blocks (512 k), blocks 4g..4g+3 of that row: an 80-byte
// run held as five 16-byte pieces. The A operand comes from LDS, where the
// workgroup staged the activations in MFMA operand order.
//
// Work split: a workgroup holds RTW row tiles x KW waves per row tile; wave
// (rtl, kw) takes SPW consecutive super-steps of row tile rtl (2; 4 when K is
// longer than 16 x 2 super-steps), and the KW waves of a row tile cover K.
// Every weight load of a wave is issued when it starts, right after the
// activation loads, so staging waits only for the activations while the
// weights stream in; nothing else waits on memory.
// The waves of a row tile add their D tiles through LDS in a fixed order, so
// results do not depend on scheduling.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

struct OneShotArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const void* X;   // fp32 (XB = false) or bf16 (XB = true) activations
    float* Y;        // fp32 output, or
    uint16_t* Yb;    // bf16 output (bit patterns)
    uint32_t wbytes;   // weight buffer range
    uint32_t xbytes;   // activation buffer range
    uint32_t rstride;  // bytes per row (combined layout) or per row tile (tiled layout)
    int ldx, ldy, M, N, K;
    int parts;  // activation terms per token (1 or 3)
    int R;      // parts * M <= 16, rows of A in use
    int nb, nss, ng_last;
    int KW, RTW;
    int act;
};

constexpr int kOneShotMaxThreads = 1024;
constexpr int kXO = 2;  // activation octets per thread held in registers

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

// RC: rows of A in use when known at compile time (1: one bf16 token, 3: one
// fp32 token), 0 = a.R at run time; a compile-time row count turns every LDS
// operand address into an immediate offset.
template <int SPW, int RC, bool GLU, bool XB, bool TILED>
__global__ void __launch_bounds__(kOneShotMaxThreads) q4_oneshot_kernel(OneShotArgs a) {
    constexpr int NT = GLU ? 2 : 1;
    constexpr int ES = XB ? 2 : 4;  // activation element size
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KW = a.KW;
    const int rtl = wave / KW;
    const int kw = wave - rtl * KW;
    const int rt = blockIdx.x * a.RTW + rtl;
    const int RT = (a.N + 15) >> 4;
    const int R = RC ? RC : a.R;
    const int j = lane & 15;
    const int g = lane >> 4;

    // ---- 1. activation loads for staging (issued first) --------------------
    // Octet o (8 consecutive k) of token m: k = 8 o. It lives at operand slot
    // ((o / 64) * 16 + o % 16) * 4 + (o / 16) % 4, i.e. super-step o / 64,
    // block 4g + bl with g = (o / 16) % 4, bl = (o / 4) % 4, dword t = o % 4:
    // slot = (ss * 16 + bl * 4 + t) * 4 + g. Unit u = m * octs + o.
    const int octs = a.nss * 64;
    const int units = octs * a.M;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);
    auto split_unit = [&](int u, int& m, int& o) {
        if (a.M == 1) {
            m = 0;
            o = u;
        } else {
            m = u / octs;
            o = u - m * octs;
        }
    };
    auto x_off = [&](int u) -> uint32_t {
        int m, o;
        split_unit(u, m, o);
        const int k = o * 8;
        if (u >= units || k >= a.K) return a.xbytes;  // out of range: loads return 0
        return (uint32_t)((m * a.ldx + k) * ES);
    };
    auto slot_dst = [&](int u) -> __bf16* {
        int m, o;
        split_unit(u, m, o);
        const int slot = ((o >> 6) * 16 + (o & 15)) * 4 + ((o >> 4) & 3);
        return xs + ((size_t)slot * R + (size_t)m * a.parts) * 8;
    };
    // More octets than registers hold (large M x K): stage them all before any
    // weight load is in flight, so the waits here cost nothing later.
    const bool staged = units > kXO * nthr;  // workgroup-uniform
    if (staged) {
        for (int u = tid; u < units; u += nthr) {
            u32x4 v[2];
            const uint32_t off = x_off(u);
            v[0] = buf_load16(rx, off);
            v[1] = XB ? u32x4{0u, 0u, 0u, 0u} : buf_load16(rx, off + 16);
            stage_octet<XB>(v, slot_dst(u), a.parts);
        }
    }
    u32x4 xr[kXO][2];
#pragma unroll
    for (int i = 0; i < kXO; ++i) {
        const uint32_t off = staged ? a.xbytes : x_off(tid + i * nthr);
        xr[i][0] = buf_load16(rx, off);
        xr[i][1] = XB ? u32x4{0u, 0u, 0u, 0u} : buf_load16(rx, off + 16);
    }

    // ---- 2. weight loads: every super-step of this wave, up front ----------
    // Tiled layout: lane l at 16 l of each 256 * ng-byte plane of the
    // (row tile, super-step) tile; the last super-step has ng_last lanes of g
    // per row, so the lanes past it read the next plane's bytes and their
    // scales are cleared below. Combined layout: lane (j, g) reads the 80-byte
    // run of row j at block 16 ss + 4 g; a run passing the end of its row
    // reads the next row's bytes, whose scales are cleared likewise.
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);
    u32x4 q[NT][SPW][5];
    int nvalid[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const int ss = kw * SPW + s;
        const bool ok = rt < RT && ss < a.nss;
        uint32_t off = a.wbytes, step = 16;
        if constexpr (TILED) {
            nvalid[s] = ss != a.nss - 1 || g < a.ng_last ? 4 : 0;
            step = ss == a.nss - 1 ? 256u * (uint32_t)a.ng_last : 1024u;
            if (ok) off = (uint32_t)rt * a.rstride + (uint32_t)ss * 5120u + 16u * (uint32_t)lane;
        } else {
            const int blk0 = ss * 16 + g * 4;
            const int row = rt * 16 + j;
            nvalid[s] = a.nb - blk0;
            if (ok && row < a.N) off = (uint32_t)row * a.rstride + (uint32_t)blk0 * kBlockBytes;
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) q[0][s][i] = buf_load16_so<TILED>(r0, off, step * i);
        if constexpr (GLU) {
#pragma unroll
            for (int i = 0; i < 5; ++i) q[1][s][i] = buf_load16_so<TILED>(r1, off, step * i);
        }
    }

    // ---- 3. stage activation terms in MFMA operand order -------------------
    if (!staged) {
#pragma unroll
        for (int i = 0; i < kXO; ++i) {
            const int u = tid + i * nthr;
            if (u < units) stage_octet<XB>(xr[i], slot_dst(u), a.parts);
        }
    }
    __syncthreads();

    // ---- 4. dequantize + MFMA --------------------------------------------------
    f32x4 acc[NT][2];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n][0] = acc[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Lane base of the A operand: slot g of super-step kw * SPW, row j (rows
    // >= R read row R - 1; their D rows are never used).
    const __bf16* xa = xs + ((size_t)(kw * SPW * 64 + g) * R + min(j, R - 1)) * 8;

#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        if (kw * SPW + s >= a.nss) break;  // wave-uniform
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
                    dw[n][t] = q[n][s][w >> 2][w & 3];
                }
                const int w4 = 5 * bl + 4;
                const uint32_t sd = bl < nvalid[s] ? (uint32_t)q[n][s][w4 >> 2][w4 & 3] : 0u;
                sc[n] = make_scale(scale_of(sd));
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int so = (s * 16 + bl * 4 + t) * 4 * R * 8;  // slot offset in bf16
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(xa + so);
#pragma unroll
                for (int n = 0; n < NT; ++n) acc[n][t & 1] = mfma16x16x32(av, dequant8(dw[n][t], sc[n]), acc[n][t & 1]);
            }
        }
    }

    // ---- 5. reduce across the waves of each row tile ----------------------------
    __syncthreads();  // every wave is done with xs
    float* red = reinterpret_cast<float*>(smem);  // [wave][NT][64][4]
#pragma unroll
    for (int n = 0; n < NT; ++n)
        *reinterpret_cast<f32x4*>(red + (((size_t)wave * NT + n) * 64 + lane) * 4) = acc[n][0] + acc[n][1];
    __syncthreads();

    // Thread t < RTW * 16 owns output row (t / 16, t % 16) of the workgroup, for
    // every token: y = sum over terms p (in order) of the sum over the row
    // tile's waves (in order) of D[m * parts + p][jj].
    const int rt_l = tid >> 4, jj = tid & 15;
    const int orow = (blockIdx.x * a.RTW + rt_l) * 16 + jj;
    if (tid >= a.RTW * 16 || orow >= a.N) return;
    for (int m = 0; m < a.M; ++m) {
        float y[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float yt = 0.0f;
            for (int p = 0; p < a.parts; ++p) {
                const int i = m * a.parts + p;
                const float* src = red + ((size_t)(rt_l * KW) * NT + n) * 256 + (jj + 16 * (i >> 2)) * 4 + (i & 3);
                float s = 0.0f;
                for (int w = 0; w < KW; ++w) s += src[(size_t)w * NT * 256];
                yt += s;
            }
            y[n] = yt;
        }
        float out = y[0];
        if constexpr (GLU) out = bf16_round(glu_exact(bf16_round(y[0]), bf16_round(y[NT - 1]), a.act));
        if (a.Yb)
            a.Yb[(size_t)m * a.ldy + orow] = __builtin_bit_cast(uint16_t, (__bf16)out);
        else
            a.Y[(size_t)m * a.ldy + orow] = out;
    }
}

struct Plan {
    int SPW, KW, RTW;
    size_t lds;
};

constexpr int kMaxKW = 16;  // waves per row tile

// Waves of a row tile cover K with SPW super-steps each; row tiles per
// workgroup amortise nothing but launch count, so a workgroup takes as many
// as fit while the grid keeps at least one workgroup per CU.
bool plan_oneshot(const GemvLaunch& L, int cus, size_t lds_max, Plan* out) {
    const TileGeom tg = tile_geom(L.K);
    const int NT = L.glu ? 2 : 1;
    const int RT = (L.N + 15) / 16;
    const int R = L.parts * L.M;
    if (R > 16) return false;
    Plan p{};
    p.SPW = tg.nss >= 2 ? 2 : 1;
    p.KW = (tg.nss + p.SPW - 1) / p.SPW;
    if (p.KW > kMaxKW && !L.glu) {  // long K: four super-steps per wave
        p.SPW = 4;
        p.KW = (tg.nss + p.SPW - 1) / p.SPW;
    }
    if (p.KW > kMaxKW) return false;
    const size_t x_bytes = (size_t)tg.nss * 1024 * R;
    auto lds_of = [&](int rtw) { return std::max(x_bytes, (size_t)p.KW * rtw * NT * 1024); };
    if (lds_of(1) > lds_max) return false;
    p.RTW = 1;
    while (p.RTW * 2 * p.KW <= kMaxKW && p.RTW * 2 <= RT && (RT + p.RTW * 2 - 1) / (p.RTW * 2) >= cus &&
           lds_of(p.RTW * 2) <= lds_max)
        p.RTW *= 2;
    p.lds = lds_of(p.RTW);
    *out = p;
    return true;
}

template <int SPW, int RC, bool GLU, bool XB, bool TILED>
hipError_t launch_one(const OneShotArgs& a, const Plan& p, int groups, hipStream_t s) {
    auto k = q4_oneshot_kernel<SPW, RC, GLU, XB, TILED>;
    if (p.lds > 64 * 1024) {
        // Dynamic LDS above 64 KiB (gfx950 has 160 KiB per CU) is opted into.
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
    }
    hipLaunchKernelGGL(k, dim3(groups), dim3(64 * p.KW * p.RTW), p.lds, s, a);
    return hipGetLastError();
}

// One token (R = 1 for bf16 activations, 3 for fp32) gets compile-time operand
// offsets; other token counts use the run-time row count.
template <bool GLU, bool XB, bool TILED>
hipError_t launch_variant(const OneShotArgs& a, const Plan& p, int groups, hipStream_t s) {
    constexpr int R1 = XB ? 1 : 3;
    if constexpr (!GLU)
        if (p.SPW == 4) return launch_one<4, 0, GLU, XB, TILED>(a, p, groups, s);
    if (a.R == R1)
        return p.SPW == 2 ? launch_one<2, R1, GLU, XB, TILED>(a, p, groups, s)
                          : launch_one<1, R1, GLU, XB, TILED>(a, p, groups, s);
    return p.SPW == 2 ? launch_one<2, 0, GLU, XB, TILED>(a, p, groups, s)
                      : launch_one<1, 0, GLU, XB, TILED>(a, p, groups, s);
}

template <bool TILED>
hipError_t launch_tiled(const OneShotArgs& a, const GemvLaunch& L, const Plan& p, int groups, hipStream_t s) {
    if (L.glu) return launch_variant<true, false, TILED>(a, p, groups, s);
    if (L.Xb) return launch_variant<false, true, TILED>(a, p, groups, s);
    return launch_variant<false, false, TILED>(a, p, groups, s);
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cus[dev];
}

size_t device_lds() {
    static size_t lds[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    if (!lds[dev]) {
        int n = 0;
        lds[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && n > 0
                       ? (size_t)n
                       : 64 * 1024;
    }
    return lds[dev];
}

// One launch for tokens [0, L.M) (R <= 16 and the plan fits), else false.
int launch_oneshot(const GemvLaunch& L, hipStream_t s, bool* done) {
    *done = false;
    Plan p;
    if (!plan_oneshot(L, device_cus(), std::min<size_t>(device_lds(), 160 * 1024), &p)) return ALV_OK;
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const uint64_t rs = (uint64_t)tg.nb * kBlockBytes;
    const uint64_t wbytes = L.tiled ? (uint64_t)RT * tg.rtb : (uint64_t)L.N * rs;
    if (wbytes >= 0xFFFFE000ull)
        return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    const uint64_t xbytes = ((uint64_t)(L.M - 1) * L.ldx + L.K) * (L.Xb ? 2 : 4);
    if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activation buffer exceeds the 2 GiB range");
    OneShotArgs a{};
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = L.Xb ? (const void*)L.Xb : (const void*)L.X;
    a.Y = L.Y;
    a.Yb = L.Yb;
    a.wbytes = (uint32_t)wbytes;
    a.xbytes = (uint32_t)xbytes;
    a.rstride = L.tiled ? tg.rtb : (uint32_t)rs;
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
    a.KW = p.KW;
    a.RTW = p.RTW;
    a.act = L.act;
    const int groups = (RT + p.RTW - 1) / p.RTW;
    const hipError_t e = L.tiled ? launch_tiled<true>(a, L, p, groups, s) : launch_tiled<false>(a, L, p, groups, s);
    *done = true;
    return hip_check(e, "q4_oneshot_kernel launch");
}

}  // namespace

int launch_gemv(const GemvLaunch& L, hipStream_t s) {
    if (L.M < 1 || L.M > kGemvMaxM) return fail(ALV_ERR_ARG, "stream kernel takes 1 <= M <= %d (got %d)", kGemvMaxM, L.M);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    if (L.Xb && (L.parts != 1 || L.glu)) return fail(ALV_ERR_ARG, "bf16 activations take one term and no GLU");
    // Registered weights: the streaming kernel, up to 16 tokens per launch.
    if (gemv1_ok(L)) return launch_gemv1(L, s);
    // Token groups of at most 16 A rows whose activations (the whole K range
    // of every token of the group) fit the LDS; a shape the one-shot plan does
    // not cover (K above 16 waves x 4 super-steps, or one token's staging
    // beyond the LDS) runs on the executor.
    const size_t per_token = (size_t)tile_geom(L.K).nss * 1024 * L.parts;
    const size_t lds_max = std::min<size_t>(device_lds(), 160 * 1024);
    const int mc = std::max(1, std::min(16 / L.parts, (int)(lds_max / per_token)));
    for (int m0 = 0; m0 < L.M; m0 += mc) {
        GemvLaunch c = L;
        c.M = std::min(mc, L.M - m0);
        if (L.X) c.X = L.X + (size_t)m0 * L.ldx;
        if (L.Xb) c.Xb = L.Xb + (size_t)m0 * L.ldx;
        if (L.Y) c.Y = L.Y + (size_t)m0 * L.ldy;
        if (L.Yb) c.Yb = L.Yb + (size_t)m0 * L.ldy;
        bool done = false;
        if (int rc = launch_oneshot(c, s, &done)) return rc;
        if (!done) {
            ExecOp op;
            static_cast<GemvLaunch&>(op) = c;
            op.dep = -1;
            if (int rc = exec_chain(&op, 1, c.tiled, s)) return rc;
        }
    }
    return ALV_OK;
}

}  // namespace alv
