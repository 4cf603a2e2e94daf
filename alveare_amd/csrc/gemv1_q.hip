// Streaming Q4 GEMV on registered (tiled) weights for one to a few tokens,
// gfx950: the kernel behind alv_gemv_q / alv_gemv / alv_ffn_fused /
// alv_chain_run for M <= 16 (the decode step of runtime/py/model.py:632-818,
// where every projection and FFN half is a matrix-vector product, and the
// small-M batches of speculative verification), up to four tokens per launch.
//
// HBM-bound: every weight byte is read once per launch, with 16-byte
// nontemporal buffer loads, and dequantized in registers
// (q4_device.h::dequant8_mix) straight into the B operand of
// v_mfma_f32_16x16x32_bf16. The A operand holds the activations, each fp32
// value split exactly into three bf16 terms (one term for bf16 activations),
// token m in rows m * terms .. + terms - 1, staged once per workgroup in LDS in
// operand order; the tokens of a launch share every dequantized weight.
//
// Work split. A unit is one (row tile, super-step[, matrix]) tile of the
// registered layout: 16 rows x 512 columns, 5 KiB, read by one wave as five
// contiguous 1 KiB pieces. Workgroup b owns a contiguous run of row tiles;
// its units are numbered tile-major, then super-step, then matrix (gate/up).
// Wave w starts on units w, w + NW, ... (P of them, one per ring slot), so the
// waves of a workgroup read neighbouring 5 KiB pieces of HBM; after that a
// wave takes the next unit from a workgroup counter in LDS whenever it frees a
// ring slot, so waves whose loads come back late do fewer units.
//
// The workgroup stages the activation before it issues any weight load: an
// activation load queued behind the weight loads of every CU would wait for
// most of them (the L2 holds nothing from the previous launch).
//
// Each unit's 16 x (rows of A) partial product goes to its own LDS slot; after the
// last unit the workgroup sums each row's slots in a fixed order (super-steps
// ascending, terms ascending), so results are deterministic whichever wave
// computed which unit.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

struct Gemv1Args {
    const uint8_t* W0;
    const uint8_t* W1;  // up matrix of a GLU pair
    const void* X;      // fp32 (R = 3) or bf16 (R = 1) activations, token m at m * ldx
    float* Y;           // fp32 output, or
    uint16_t* Yb;       // bf16 output (bit patterns); token m at m * ldy
    uint32_t wbytes;    // bytes of one matrix (row tiles x rtb)
    uint32_t rtb;       // bytes per row tile
    uint32_t xbytes;    // activation buffer range
    int N, K, nss, ng_last;
    int ldx, ldy;
    int rt_q, rt_r;  // workgroup b owns rt_q + (b < rt_r) row tiles
    int act;
};

constexpr int kXO = 4;  // activation octets per thread and staging round

// Row tiles [rt0, rt0 + nt) of workgroup b.
__device__ __forceinline__ void wg_tiles(const Gemv1Args& a, int b, int& rt0, int& nt) {
    rt0 = b * a.rt_q + min(b, a.rt_r);
    nt = a.rt_q + (b < a.rt_r ? 1 : 0);
}

// Eight activations of one token as R bf16 terms at dst, dst + 8, dst + 16
// (R = 3: the exact split of fp32 values; R = 1: bf16 values as they are).
template <int R>
__device__ __forceinline__ void stage_octet(const u32x4 (&v)[2], __bf16* dst) {
    if constexpr (R == 1) {
        *reinterpret_cast<u32x4*>(dst) = v[0];
    } else {
        float f[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) f[4 * h + e] = __builtin_bit_cast(float, (uint32_t)v[h][e]);
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
    }
}

// Byte offset of unit u's tile in its matrix, the plane step of its pieces,
// its super-step and matrix index. Units of a workgroup: ((tl * nss) + ss) * NT + n.
template <int NT>
struct UnitPos {
    uint32_t off, step;
    int ss, n;
};

template <int NT>
__device__ __forceinline__ UnitPos<NT> unit_pos(const Gemv1Args& a, int rt0, int u) {
    UnitPos<NT> p;
    const int t = NT == 2 ? u >> 1 : u;
    p.n = NT == 2 ? u & 1 : 0;
    const int tl = t / a.nss;
    p.ss = t - tl * a.nss;
    p.off = (uint32_t)(rt0 + tl) * a.rtb + (uint32_t)p.ss * 5120u;
    p.step = p.ss == a.nss - 1 ? 256u * (uint32_t)a.ng_last : 1024u;
    return p;
}

// Rows of A in use (MT tokens x R terms, row m * R + p) and the lanes whose D
// output holds them (lane l holds D rows 4 (l / 16) .. + 3 of column l % 16).
template <int R, int MT>
struct ARows {
    static constexpr int RM = R * MT;
    static constexpr int DL = 16 * ((RM + 3) / 4);
};

template <int NW, int P, int R, bool GLU, int MT>
__global__ void __launch_bounds__(64 * NW) q4_gemv1_kernel(Gemv1Args a) {
    constexpr int NT = GLU ? 2 : 1;
    constexpr int ES = R == 3 ? 4 : 2;  // activation element size
    constexpr int RM = ARows<R, MT>::RM, DL = ARows<R, MT>::DL;
    static_assert(RM <= 16, "one MFMA row block");
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);
    f32x4* part = reinterpret_cast<f32x4*>(smem + (size_t)a.nss * 1024 * RM);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15;
    const int g = lane >> 4;
    int rt0, nt;
    wg_tiles(a, blockIdx.x, rt0, nt);
    const int U = nt * a.nss * NT;
    // Unit counter of the workgroup, after the unit slots: the first P * NW
    // units go to the waves statically, the rest to whichever wave frees a ring
    // slot first, so a wave whose loads come back late does fewer units.
    int* next = reinterpret_cast<int*>(part + (size_t)U * DL);
    if (tid == 0) *next = P * NW;

    // ---- 1. stage the activation terms before any weight load --------------------
    // Octet o (8 consecutive k) of token m sits at operand slot
    // ((o / 64) * 16 + o % 16) * 4 + (o / 16) % 4 -- super-step o / 64, block
    // 4 g + bl with g = (o / 16) % 4, bl = (o / 4) % 4, dword t = o % 4 of the
    // block -- rows m * R .. m * R + R - 1 of the slot's RM rows.
    const int octs = a.nss * 64;
    const int E = MT * octs;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);
    for (int e0 = 0; e0 < E; e0 += kXO * 64 * NW) {
        u32x4 xr[kXO][2];
#pragma unroll
        for (int i = 0; i < kXO; ++i) {
            const int e = e0 + tid + i * 64 * NW;
            const int m = MT == 1 ? 0 : e / octs;
            const int o = e - m * octs;
            const uint32_t off = e < E && o * 8 < a.K ? (uint32_t)((m * a.ldx + o * 8) * ES) : a.xbytes;  // past: zeros
            xr[i][0] = buf_load16(rx, off);
            xr[i][1] = R == 3 ? buf_load16(rx, off + 16) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < kXO; ++i) {
            const int e = e0 + tid + i * 64 * NW;
            const int m = MT == 1 ? 0 : e / octs;
            const int o = e - m * octs;
            if (e < E) {
                const int slot = ((o >> 6) * 16 + (o & 15)) * 4 + ((o >> 4) & 3);
                stage_octet<R>(xr[i], xs + ((size_t)slot * RM + m * R) * 8);
            }
        }
    }
    lds_barrier();

    // ---- 2. the first P units of this wave -----------------------------------------
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);
    const uint32_t voff = 16u * (uint32_t)lane;
    u32x4 q[P][5];
    auto issue = [&](u32x4 (&d)[5], int u) __attribute__((always_inline)) {
        uint32_t off = a.wbytes, step = 1024u;  // past the range: zeros, no memory traffic
        int n = 0;
        if (u < U) {
            const UnitPos<NT> p = unit_pos<NT>(a, rt0, u);
            off = p.off;
            step = p.step;
            n = p.n;
        }
        // Wave-uniform by construction; saying so keeps the loads out of
        // per-lane (waterfall) loops.
        off = __builtin_amdgcn_readfirstlane(off);
        step = __builtin_amdgcn_readfirstlane(step);
        const __amdgpu_buffer_rsrc_t r = (GLU && __builtin_amdgcn_readfirstlane(n)) ? r1 : r0;
#pragma unroll
        for (int i = 0; i < 5; ++i) d[i] = buf_load16_so<true>(r, voff, off + step * i);
    };
    int uk[P];  // the unit in each ring slot (>= U: none)
#pragma unroll
    for (int k = 0; k < P; ++k) {
        uk[k] = w + k * NW;
        issue(q[k], uk[k]);
    }

    // ---- 3. stream: dequantize + MFMA one unit, refill its ring slot ---------------
    // Lane base of the A operand: slot g, row j (rows >= RM read row RM - 1;
    // their D rows are never used).
    const __bf16* xa = xs + ((size_t)g * RM + min(j, RM - 1)) * 8;
    // Every pass refills every slot (past the last unit the loads read past the
    // buffer and return zeros), so the loads in flight per slot are the same on
    // every path and the compiler's wait counts keep P - 1 units in flight.
    for (bool live = true; live;) {
        live = false;
#pragma unroll
        for (int k = 0; k < P; ++k) {
            int un = 0;
            if (lane == 0) un = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            un = __builtin_amdgcn_readfirstlane(un);
            const int u = uk[k];
            if (u < U) {
                const UnitPos<NT> p = unit_pos<NT>(a, rt0, u);
                // The last super-step holds ng_last lanes of g per row; the
                // other lanes read the next plane's bytes: zero their scales.
                const bool valid = p.ss != a.nss - 1 || g < a.ng_last;
                const __bf16* xu = xa + (size_t)p.ss * 16 * 4 * RM * 8;
                f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int bl = 0; bl < 4; ++bl) {
                    const int w4 = 5 * bl + 4;
                    const uint32_t sd = valid ? (uint32_t)q[k][w4 >> 2][w4 & 3] : 0u;
                    const Scale2 sc = make_scale2(scale_of(sd));
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int wi = 5 * bl + t;
                        const bf16x8 av = *reinterpret_cast<const bf16x8*>(xu + (bl * 4 + t) * 4 * RM * 8);
                        const bf16x8 bv = dequant8_mix((uint32_t)q[k][wi >> 2][wi & 3], sc);
                        if (t & 1)
                            t1 = mfma16x16x32(av, bv, t1);
                        else
                            t0 = mfma16x16x32(av, bv, t0);
                    }
                }
                if (lane < DL) part[(size_t)u * DL + lane] = t0 + t1;
            }
            issue(q[k], un);
            uk[k] = un;
            live |= un < U;
        }
    }
    lds_barrier();

    // ---- 4. per row: sum the unit slots in a fixed order, epilogue, store ----------
    // D row m * R + p (token m, term p) of column jj sits in slot lane
    // 16 * (row / 4) + jj, element row % 4. Wave w takes rows 16 w .. 16 w + 15
    // of the workgroup (then 16 NW further on); four lanes share a row: lane c
    // sums super-steps c, c + 4, ... in ascending order, the four partial sums
    // combine in a fixed butterfly, so the result does not depend on timing,
    // and lane 0 of the four finishes the row -- the epilogue is spread over
    // nt waves.
    const int c = lane & 3;
    for (int r0 = w * 16; r0 < nt * 16; r0 += NW * 16) {
        const int rid = r0 + (lane >> 2);
        const int tl = rid >> 4, jj = rid & 15;
        float y[MT][NT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n) y[m][n] = 0.0f;
        for (int ss = c; ss < a.nss; ss += 4) {
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const f32x4* sl = part + ((size_t)(tl * a.nss + ss) * NT + n) * DL + jj;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float v = 0.0f;
#pragma unroll
                    for (int p = 0; p < R; ++p) {
                        const int row = m * R + p;
                        v += sl[(row >> 2) * 16][row & 3];
                    }
                    y[m][n] += v;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                y[m][n] += __shfl_xor(y[m][n], 1);
                y[m][n] += __shfl_xor(y[m][n], 2);
            }
        const int row = (rt0 + tl) * 16 + jj;
        if (c != 0 || row >= a.N) continue;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float out = y[m][0];
            if constexpr (GLU) out = bf16_round(glu_act(bf16_round(y[m][0]), bf16_round(y[m][NT - 1]), a.act));
            if (a.Yb)
                a.Yb[(size_t)m * a.ldy + row] = __builtin_bit_cast(uint16_t, (__bf16)out);
            else
                a.Y[(size_t)m * a.ldy + row] = out;
        }
    }
}

struct DevInfo {
    int cus = 0;
    size_t lds = 0;
};

const DevInfo& dev_info() {
    static DevInfo info[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    DevInfo& d = info[dev];
    if (!d.cus) {
        int n = 0, l = 0;
        d.lds = hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && l > 0
                    ? std::min<size_t>((size_t)l, 160 * 1024)
                    : 64 * 1024;
        d.cus = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return d;
}

constexpr int kNW = 16;

template <int P, int R, bool GLU, int MT>
hipError_t launch_k(const Gemv1Args& a, int groups, size_t lds, hipStream_t s) {
    auto k = q4_gemv1_kernel<kNW, P, R, GLU, MT>;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
    }
    hipLaunchKernelGGL(k, dim3(groups), dim3(64 * kNW), lds, s, a);
    return hipGetLastError();
}

template <int P, int R, bool GLU>
hipError_t launch_mt(const Gemv1Args& a, int mt, int groups, size_t lds, hipStream_t s) {
    switch (mt) {
        case 1: return launch_k<P, R, GLU, 1>(a, groups, lds, s);
        case 2: return launch_k<P, R, GLU, 2>(a, groups, lds, s);
        case 3: return launch_k<P, R, GLU, 3>(a, groups, lds, s);
        default: return launch_k<P, R, GLU, 4>(a, groups, lds, s);
    }
}

struct Gemv1Plan {
    int groups, rt_q, rt_r;
    size_t lds;
};

// Ring depth: one unit in flight per wave (16 per CU) measures faster than two
// on every decode shape -- a deeper ring only lengthens the memory queues.
constexpr int kP = 1;
// Tokens per launch: the activations of all of them sit in LDS with the unit
// slots, which bounds the count (4 at the 12B-class shapes).
constexpr int kMaxMT = 4;

bool plan_gemv1(const GemvLaunch& L, int mt, Gemv1Plan* out) {
    if (!L.tiled || L.parts != (L.Xb ? 1 : 3) || mt < 1 || mt > kMaxMT) return false;
    const DevInfo& d = dev_info();
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const int NT = L.glu ? 2 : 1;
    const int RM = L.parts * mt;
    Gemv1Plan p;
    p.groups = std::min(RT, d.cus);
    p.rt_q = RT / p.groups;
    p.rt_r = RT % p.groups;
    const int tiles = p.rt_q + (p.rt_r ? 1 : 0);
    const int units = tiles * tg.nss * NT;
    p.lds = (size_t)tg.nss * 1024 * RM + (size_t)units * 256 * ((RM + 3) / 4) + 16;
    if (p.lds > d.lds) return false;
    *out = p;
    return true;
}

// Most tokens one launch takes for this shape (0: none).
int max_mt(const GemvLaunch& L) {
    Gemv1Plan p;
    for (int mt = kMaxMT; mt >= 1; --mt)
        if (plan_gemv1(L, mt, &p)) return mt;
    return 0;
}

}  // namespace

bool gemv1_ok(const GemvLaunch& L) { return L.M >= 1 && max_mt(L) > 0; }

int launch_gemv1(const GemvLaunch& L, hipStream_t s) {
    const int mtmax = L.M >= 1 ? max_mt(L) : 0;
    if (!mtmax) return fail(ALV_ERR_ARG, "streaming GEMV: shape M=%d N=%d K=%d outside its plan", L.M, L.N, L.K);
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const uint64_t wbytes = (uint64_t)RT * tg.rtb;
    if (wbytes >= 0xFFFFE000ull)
        return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    const int ES = L.Xb ? 2 : 4;
    for (int m0 = 0; m0 < L.M; m0 += mtmax) {
        const int mt = std::min(mtmax, L.M - m0);
        Gemv1Plan p;
        if (!plan_gemv1(L, mt, &p)) return fail(ALV_ERR_ARG, "streaming GEMV: no plan for %d tokens", mt);
        const uint64_t xbytes = ((uint64_t)(mt - 1) * L.ldx + L.K) * ES;
        if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activation buffer exceeds the 2 GiB range");
        Gemv1Args a{};
        a.W0 = L.W0;
        a.W1 = L.W1;
        a.X = L.Xb ? (const void*)(L.Xb + (size_t)m0 * L.ldx) : (const void*)(L.X + (size_t)m0 * L.ldx);
        a.Y = L.Y ? L.Y + (size_t)m0 * L.ldy : nullptr;
        a.Yb = L.Yb ? L.Yb + (size_t)m0 * L.ldy : nullptr;
        a.wbytes = (uint32_t)wbytes;
        a.rtb = tg.rtb;
        a.xbytes = (uint32_t)xbytes;
        a.N = L.N;
        a.K = L.K;
        a.nss = tg.nss;
        a.ng_last = tg.ng_last;
        a.ldx = L.ldx;
        a.ldy = L.ldy;
        a.rt_q = p.rt_q;
        a.rt_r = p.rt_r;
        a.act = L.act;
        const hipError_t e = L.glu ? launch_mt<kP, 3, true>(a, mt, p.groups, p.lds, s)
                             : L.Xb ? launch_mt<kP, 1, false>(a, mt, p.groups, p.lds, s)
                                    : launch_mt<kP, 3, false>(a, mt, p.groups, p.lds, s);
        if (int rc = hip_check(e, "q4_gemv1_kernel launch")) return rc;
    }
    return ALV_OK;
}

}  // namespace alv
