// Streaming Q4 matrix-vector kernel for decode and small-M batches (gfx950),
// the dequant test kernel, and the alv_gemv_q / alv_gemm_q / alv_dequant_q4
// entry points.
//
// The kernel is HBM-bound by design: weights are read once, straight from the
// combined layout, with 16-byte buffer loads; dequantization happens in
// registers (q4_device.h::dequant8, ~2.5 VALU ops per weight) and the dot
// product runs on the matrix cores. Doing the products on MFMA even at M = 1
// keeps the VALU budget for the exact bf16 dequantization: at 70% of 8 TB/s
// the chip must dequantize ~9e12 weights/s, ~4.4 VALU lane-ops per weight.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, D = A x B):
//   B columns = 16 weight rows (one "row tile"), B k = 32 weights = one block;
//   A rows    = activation terms: token m contributes `parts` rows (its fp32
//               value split exactly into 3 bf16 terms, or 1 term when the
//               activation is bf16-valued); rows >= parts*M are zero.
// Lane l = (j, g), j = l % 16, g = l / 16 owns weight row j and, within a
// super-step of 16 blocks (512 k), blocks 4g..4g+3 of that row: 80 contiguous
// bytes fetched as five 16-byte loads. The A operand for the same k comes from
// LDS, where the workgroup staged its K-chunk of activation terms in MFMA
// operand order.
//
// Work split: grid = (row tiles, K chunks); a workgroup of KW waves covers one
// row tile and one K chunk, wave w taking super-steps w, w + KW, ... Partial
// results are reduced across waves in LDS and, when a row tile spans several
// K chunks, across workgroups through a partial-sum buffer: the last
// workgroup to arrive (per-row-tile counter) adds the chunks in chunk order,
// so results do not depend on scheduling.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

struct GemvKArgs {
    const uint8_t* W0;
    const uint8_t* W1;
    const float* X;
    float* Y;
    float* partial;
    uint32_t* counters;
    uint32_t wbytes;  // N * row bytes (buffer range)
    int ldx, ldy, M, N, K;
    int parts;  // activation terms per token (1 or 3)
    int R;      // parts * M, rows of A in use
    int css;    // super-steps per K chunk
    int KS;     // K chunks
    int act;
};

// At most 16 waves per workgroup (8 with the gate/up pair, whose doubled
// register set would otherwise spill).
template <bool GLU>
constexpr int stream_max_threads() { return GLU ? 512 : 1024; }

template <int AT, bool GLU>
__global__ void __launch_bounds__(stream_max_threads<GLU>()) gemv_stream_kernel(GemvKArgs a) {
    constexpr int NT = GLU ? 2 : 1;
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int KW = blockDim.x >> 6;
    const int rt = blockIdx.x;
    const int chunk = blockIdx.y;
    const int nb = a.K >> 5;
    const uint32_t rs = (uint32_t)nb * kBlockBytes;
    const int nss = (nb + 15) >> 4;
    const int ss_begin = chunk * a.css;
    const int ss_count = min(a.css, nss - ss_begin);
    const int k0 = ss_begin * 512;
    const int R = a.R;

    // ---- 1. stage this chunk's activation terms in MFMA operand order -----
    // Octet (8 consecutive k) number o of the chunk lives at operand slot
    // ((ss * 16 + t) * 4 + g) with ss = o / 64, g = (o / 16) % 4, t = o % 16.
    {
        const int octs = ss_count * 64;
        const int units = octs * a.M;
        for (int u = tid; u < units; u += blockDim.x) {
            const int m = u / octs;
            const int o = u - m * octs;
            const int k = k0 + o * 8;
            float v[8];
            if (k < a.K) {
                const float* xp = a.X + (size_t)m * a.ldx + k;
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = xp[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = 0.0f;
            }
            const int slot = ((o >> 6) * 16 + (o & 15)) * 4 + ((o >> 4) & 3);
            __bf16* dst = xs + ((size_t)slot * R + (size_t)m * a.parts) * 8;
            if (a.parts == 3) {
                bf16x8 p0, p1, p2;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const Split3 s = split3(v[e]);
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
                for (int e = 0; e < 8; ++e) p0[e] = (__bf16)v[e];
                *reinterpret_cast<bf16x8*>(dst) = p0;
            }
        }
    }
    __syncthreads();

    // ---- 2. stream the weights -------------------------------------------
    const int j = lane & 15;
    const int g = lane >> 4;
    const int row = rt * 16 + j;
    const bool row_ok = row < a.N;
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);

    f32x4 acc[NT][AT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < AT; ++t) acc[n][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto load = [&](int ssl, u32x4 (&q)[NT][5]) {
        const int blk0 = (ss_begin + ssl) * 16 + g * 4;
        const uint32_t off = row_ok ? (uint32_t)row * rs + (uint32_t)blk0 * kBlockBytes : a.wbytes;
#pragma unroll
        for (int i = 0; i < 5; ++i) q[0][i] = buf_load16(r0, off + 16 * i);
        if constexpr (GLU) {
#pragma unroll
            for (int i = 0; i < 5; ++i) q[1][i] = buf_load16(r1, off + 16 * i);
        }
    };

    u32x4 cur[NT][5], nxt[NT][5];
    int ssl = wave;
    if (ssl < ss_count) load(ssl, cur);
    for (; ssl < ss_count; ssl += KW) {
        if (ssl + KW < ss_count) load(ssl + KW, nxt);
        const int blk0 = (ss_begin + ssl) * 16 + g * 4;
#pragma unroll
        for (int bl = 0; bl < 4; ++bl) {
            const bool blk_ok = blk0 + bl < nb;
            Scale sc[NT];
            uint32_t dw[NT][4];
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                // dwords 5*bl .. 5*bl+4 of the 80-byte run are this block.
                uint32_t d5[5];
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    const int w = 5 * bl + i;
                    d5[i] = cur[n][w >> 2][w & 3];
                }
                sc[n] = make_scale(blk_ok ? bf16_bits_to_f32(d5[4] & 0xFFFFu) : 0.0f);
#pragma unroll
                for (int t = 0; t < 4; ++t) dw[n][t] = d5[t];
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int slot = (ssl * 16 + bl * 4 + t) * 4 + g;
                bf16x8 av[AT];
#pragma unroll
                for (int at = 0; at < AT; ++at) {
                    const int arow = at * 16 + j;
                    av[at] = bf16x8{};
                    if (arow < R)
                        av[at] = *reinterpret_cast<const bf16x8*>(xs + ((size_t)slot * R + arow) * 8);
                }
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const bf16x8 b = dequant8(dw[n][t], sc[n]);
#pragma unroll
                    for (int at = 0; at < AT; ++at) acc[n][at] = mfma16x16x32(av[at], b, acc[n][at]);
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 5; ++i) cur[n][i] = nxt[n][i];
    }

    // ---- 3. reduce across waves --------------------------------------------
    __syncthreads();  // all waves are done with xs
    float* red = reinterpret_cast<float*>(smem);  // [KW][NT][AT][64][4]
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int at = 0; at < AT; ++at)
            *reinterpret_cast<f32x4*>(red + ((((size_t)wave * NT + n) * AT + at) * 64 + lane) * 4) =
                acc[n][at];
    __syncthreads();
    float* dsum = red + (size_t)KW * NT * AT * 256;  // [NT][R][16]
    for (int idx = tid; idx < NT * R * 16; idx += blockDim.x) {
        const int n = idx / (R * 16);
        const int i = (idx >> 4) % R;
        const int jj = idx & 15;
        const int at = i >> 4, ii = i & 15;
        const int l = jj + 16 * (ii >> 2), rr = ii & 3;
        float s = 0.0f;
        for (int w = 0; w < KW; ++w) s += red[((((size_t)w * NT + n) * AT + at) * 64 + l) * 4 + rr];
        dsum[idx] = s;
    }
    __syncthreads();

    // y[n][m][j] = sum over the token's activation terms, in term order.
    auto token_sum = [&](int n, int m, int jj) {
        float y = 0.0f;
        for (int p = 0; p < a.parts; ++p) y += dsum[(n * R + m * a.parts + p) * 16 + jj];
        return y;
    };
    auto epilogue_store = [&](int m, int jj, float y0, float y1) {
        const int orow = rt * 16 + jj;
        float out = y0;
        if constexpr (GLU) out = bf16_round(glu_act(bf16_round(y0), bf16_round(y1), a.act));
        a.Y[(size_t)m * a.ldy + orow] = out;
    };

    if (a.KS == 1) {
        for (int idx = tid; idx < a.M * 16; idx += blockDim.x) {
            const int m = idx >> 4, jj = idx & 15;
            if (rt * 16 + jj >= a.N) continue;
            epilogue_store(m, jj, token_sum(0, m, jj), GLU ? token_sum(NT - 1, m, jj) : 0.0f);
        }
        return;
    }

    // ---- 4. cross-workgroup split-K reduction --------------------------------
    const size_t plane = (size_t)a.M * a.N;
    for (int idx = tid; idx < NT * a.M * 16; idx += blockDim.x) {
        const int n = idx / (a.M * 16);
        const int m = (idx >> 4) % a.M, jj = idx & 15;
        const int orow = rt * 16 + jj;
        if (orow >= a.N) continue;
        a.partial[((size_t)chunk * NT + n) * plane + (size_t)m * a.N + orow] = token_sum(n, m, jj);
    }
    __threadfence();
    __syncthreads();
    __shared__ int is_last;
    if (tid == 0) is_last = atomicAdd(&a.counters[rt], 1u) == (uint32_t)(a.KS - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int idx = tid; idx < a.M * 16; idx += blockDim.x) {
        const int m = idx >> 4, jj = idx & 15;
        const int orow = rt * 16 + jj;
        if (orow >= a.N) continue;
        float y[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float s = 0.0f;
            for (int c = 0; c < a.KS; ++c)
                s += __builtin_nontemporal_load(&a.partial[((size_t)c * NT + n) * plane + (size_t)m * a.N + orow]);
            y[n] = s;
        }
        epilogue_store(m, jj, y[0], y[NT - 1]);
    }
    if (tid == 0) a.counters[rt] = 0u;
}

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

// ---- host side -----------------------------------------------------------------

namespace {

struct Plan {
    int KW, css, KS;
    size_t lds;
};

Plan plan_stream(int M, int N, int K, int parts, bool glu) {
    const int NT = glu ? 2 : 1;
    const int nb = K / 32, nss = (nb + 15) / 16, RT = (N + 15) / 16;
    const int R = parts * M, AT = (R + 15) / 16;
    const int css_lds = std::max(1, (64 * 1024) / (1024 * R));
    const int kw_cap = glu ? stream_max_threads<true>() / 64 : stream_max_threads<false>() / 64;
    const int kw_max = std::max(1, std::min(kw_cap, (64 * 1024 - NT * R * 64) / (NT * AT * 1024)));
    const double work = (double)RT * nss * NT;
    int sspw = (int)(work / 4096.0 + 0.5);
    sspw = std::max(1, std::min(4, sspw));
    const int css_max = std::max(1, std::min(css_lds, sspw * kw_max));
    const int KS = (nss + css_max - 1) / css_max;
    const int css = (nss + KS - 1) / KS;
    const int KW = std::max(1, std::min(kw_max, (css + sspw - 1) / sspw));
    const size_t xs_bytes = (size_t)css * 1024 * R;
    const size_t red_bytes = (size_t)KW * NT * AT * 1024 + (size_t)NT * R * 16 * 4;
    return Plan{KW, css, KS, std::max(xs_bytes, red_bytes)};
}

template <int AT, bool GLU>
hipError_t launch_at(const GemvKArgs& a, const Plan& p, int RT, hipStream_t s) {
    hipLaunchKernelGGL((gemv_stream_kernel<AT, GLU>), dim3(RT, p.KS), dim3(64 * p.KW), p.lds, s, a);
    return hipGetLastError();
}

}  // namespace

int launch_gemv(const GemvLaunch& L, hipStream_t s) {
    if (L.M < 1 || L.M > kGemvMaxM) return fail(ALV_ERR_ARG, "stream kernel takes 1 <= M <= %d (got %d)", kGemvMaxM, L.M);
    if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
    const uint64_t rs = (uint64_t)(L.K / 32) * kBlockBytes;
    const uint64_t wbytes = (uint64_t)L.N * rs;
    if (wbytes >= 0xFFFFFF00ull) return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    const Plan p = plan_stream(L.M, L.N, L.K, L.parts, L.glu);
    const int RT = (L.N + 15) / 16;
    GemvKArgs a{};
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = L.X;
    a.Y = L.Y;
    a.wbytes = (uint32_t)wbytes;
    a.ldx = L.ldx;
    a.ldy = L.ldy;
    a.M = L.M;
    a.N = L.N;
    a.K = L.K;
    a.parts = L.parts;
    a.R = L.parts * L.M;
    a.css = p.css;
    a.KS = p.KS;
    a.act = L.act;
    if (p.KS > 1) {
        Workspace ws;
        const int NT = L.glu ? 2 : 1;
        if (int rc = get_workspace(s, (size_t)p.KS * NT * L.M * L.N, (size_t)RT, &ws)) return rc;
        a.partial = ws.partial;
        a.counters = ws.counters;
    }
    const int AT = (a.R + 15) / 16;
    hipError_t e;
    if (L.glu) {
        e = AT == 1 ? launch_at<1, true>(a, p, RT, s) : AT == 2 ? launch_at<2, true>(a, p, RT, s) : launch_at<3, true>(a, p, RT, s);
    } else {
        e = AT == 1 ? launch_at<1, false>(a, p, RT, s) : AT == 2 ? launch_at<2, false>(a, p, RT, s) : launch_at<3, false>(a, p, RT, s);
    }
    return hip_check(e, "gemv_stream_kernel launch");
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
    if (M >= kTiledMinM) {
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

extern "C" int alv_dequant_q4(const uint8_t* W, uint16_t* out, int N, int K, void* stream) {
    if (int rc = check_common(W, out, out, N, K)) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 16) return fail(ALV_ERR_ALIGN, "out needs 16-byte alignment");
    const int64_t blocks = (int64_t)N * (K / 32);
    const int grid = (int)std::min<int64_t>((blocks + 255) / 256, 65535);
    hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, W, out, N, K);
    return hip_check(hipGetLastError(), "dequant_kernel launch");
}
