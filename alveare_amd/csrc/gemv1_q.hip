// Streaming Q4 GEMV, gfx950: the one kernel behind alv_gemv_q / alv_gemm_q /
// alv_gemv / alv_ffn_fused / alv_chain_run for M <= 16 (the decode step of
// runtime/py/model.py:632-818, where every projection and FFN half is a
// matrix-vector product, and the small-M batches of speculative
// verification), up to 16 tokens per launch, on registered (tiled) weights or
// straight from the combined layout (per-call weights of alv_gemv_q).
//
// HBM-bound: every weight byte is read once per launch, with 16-byte
// nontemporal buffer loads, and dequantized in registers
// (q4_device.h::dequant8_mix) straight into the B operand of
// v_mfma_f32_16x16x32_bf16. The A operand holds the activations, each fp32
// value split exactly into three bf16 terms (one term for bf16 activations),
// token-major (token m in rows m * terms .. + terms - 1), in token quads
// (2 to 8 tokens) or term-major (9 to 16; see ARows), staged once per workgroup in LDS in operand
// order; the tokens of a launch share every dequantized weight. When a
// workgroup's activations outgrow the LDS, K is split over several workgroups
// per row-tile group (partial sums in a per-stream scratch, added in split
// order by the last workgroup of the group or, from 4 splits, by a second
// launch, split_fix_kernel).
//
// Work split. A unit is one (row tile, super-step[, matrix]) tile of the
// registered layout: 16 rows x 512 columns, 5 KiB, read by one wave as five
// contiguous 1 KiB pieces. Row tiles are dealt to the workgroups in turn
// (workgroup b: tiles b, b + G, ...), so the units in flight GPU-wide cover a
// contiguous window of each matrix; a workgroup's units are numbered
// tile-major, then super-step, then matrix (gate/up).
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
#include <atomic>
#include <cstdlib>

#include "q4_device.h"
#include "q4_host.h"
#include "row_norm.h"

namespace alv {

namespace {

struct Gemv1Args {
    const uint8_t* W0;  // tiled layout, or the combined layout (TL = false)
    const uint8_t* W1;  // up matrix of a GLU pair
    const void* X;      // fp32 or bf16 activations, token m at m * ldx
    float* Y;           // fp32 output, or
    uint16_t* Yb;       // bf16 output (bit patterns); token m at m * ldy
    float* part;        // split-K partial sums, [row][ks][token][matrix] (ks > 1)
    uint32_t pbytes;    // bytes of part
    uint32_t* cnt;      // split-K arrivals per tile group (zero between launches)
    uint32_t wbytes;    // bytes of one matrix (row tiles x rtb)
    uint32_t rtb;       // bytes per row tile (combined layout: 16 rows)
    uint32_t rs;        // combined layout: bytes per row
    uint32_t xbytes;    // activation buffer range (M tokens)
    int N, K, nb, nss, ng_last;
    int ldx, ldy, M;
    int ntg;         // tile groups: group t owns row tiles t, t + ntg, t + 2 ntg, ...
    int rt_q, rt_r;  // so group t owns rt_q + (t < rt_r) row tiles
    int ks;          // K splits: workgroup b is tile group b / ks, super-step range b % ks
    int act;
    int fix;         // split K: shares stored plainly, summed by a separate launch (split_fix_kernel)
    int Nz;          // output rows [N, Nz) of every token are written as zeros
    // Fused residual step (bf16 one-token launches; pr_r null: none).
    const uint16_t* pr_r;
    const uint16_t* pr_y;
    const float* pr_wy;
    const float* pr_wx;
    uint16_t* pr_s;
    float pr_scale, pr_eps;
    int pr_norm_y, pr_mode;
    int pr_k;  // width of the step's rows (K may differ: activation octets past both are zeros)
};

constexpr int kXO = 4;  // activation octets per thread and staging round

// Eight activations of one token as R bf16 terms at dst, dst + TS, dst + 2 TS:
// R = 3 is the exact split of fp32 values, R = 1 bf16 values as they are.
template <int R, int TS>
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
        *reinterpret_cast<bf16x8*>(dst + TS) = p1;
        *reinterpret_cast<bf16x8*>(dst + 2 * TS) = p2;
    }
}

// The work of workgroup b: row tiles tg, tg + ntg, ... (nt of them) x
// super-steps [s0, s0 + nsw). Row tiles are dealt to the tile groups in turn,
// so at any moment the workgroups stream neighbouring tiles: the bytes in
// flight GPU-wide form one contiguous window per matrix (DRAM pages are read
// whole while open), not one stream per workgroup.
struct WgWork {
    int tg, kq, ntg, nt, s0, nsw;
};

__device__ __forceinline__ WgWork wg_work(const Gemv1Args& a, int b) {
    WgWork w;
    w.tg = b / a.ks;
    w.kq = b - w.tg * a.ks;
    w.ntg = a.ntg;
    w.nt = a.rt_q + (w.tg < a.rt_r ? 1 : 0);
    w.s0 = w.kq * a.nss / a.ks;
    w.nsw = (w.kq + 1) * a.nss / a.ks - w.s0;
    return w;
}

// Row tile of the workgroup's local tile tl.
__device__ __forceinline__ int tile_row(const WgWork& wk, int tl) { return wk.tg + tl * wk.ntg; }

// Byte offset of unit u's tile in its matrix, the plane step of its pieces,
// its super-step (absolute) and matrix index. Units of a workgroup:
// ((tl * nsw) + ss - s0) * NT + n.
struct UnitPos {
    uint32_t off, step;
    int ss, n;
};

// Tiled layout: piece i of lane l at off + i * step + 16 l. Combined layout
// (TL = false): lane (g, j) reads row 16 rt + j at byte 80 g of the
// super-step's 320-byte run, piece i at + 16 i (lane_voff).
template <int NT, bool TL>
__device__ __forceinline__ UnitPos unit_pos(const Gemv1Args& a, const WgWork& wk, int u) {
    UnitPos p;
    const int t = NT == 2 ? u >> 1 : u;
    p.n = NT == 2 ? u & 1 : 0;
    const int tl = t / wk.nsw;
    p.ss = wk.s0 + t - tl * wk.nsw;
    p.off = (uint32_t)tile_row(wk, tl) * a.rtb + (uint32_t)p.ss * (TL ? 5120u : 320u);
    p.step = TL ? (p.ss == a.nss - 1 ? 256u * (uint32_t)a.ng_last : 1024u) : 16u;
    return p;
}

template <bool TL>
__device__ __forceinline__ uint32_t lane_voff(const Gemv1Args& a, int lane) {
    return TL ? 16u * (uint32_t)lane : (uint32_t)(lane & 15) * a.rs + 80u * (uint32_t)(lane >> 4);
}

// Activation rows of an operand slot (MT tokens x R terms) and how they meet
// the MFMA. Token-major (TB = false): one A block, row m * R + p, the terms
// added up per row at the end. Term-major (TB = true): R blocks of MT rows,
// block p = term p of every token, one MFMA per block into the same
// accumulator, so D row m is already token m's sum. Lane l holds D rows
// 4 (l / 16) .. + 3 of column l % 16; DL lanes hold the rows in use.
//
// Token quads (QUAD: 2, 4 or 8 fp32 tokens, token-major): A block b holds
// tokens 4b .. 4b + 3 at four rows each, the three terms and a zero row
// (tokens past MT: zero rows), so one lane group of the D tile holds one token
// and each lane adds its token's terms itself; a unit's slot holds the token
// sums, MT x 16 floats. For 8 tokens two MFMAs per weight octet (term-major
// would take three).
template <int R, int MT, bool TB>
struct ARows {
    static constexpr bool QUAD = !TB && R == 3 && (MT == 2 || MT == 4 || MT == 8);
    static constexpr int RM = R * MT;                          // rows per slot in LDS
    static constexpr int AR = QUAD ? 16 : (TB ? MT : RM);      // rows per A block
    static constexpr int DL = 16 * ((AR + 3) / 4);
    static constexpr int US = QUAD ? MT * 4 : DL;              // f32x4 per unit slot
};

// Operand geometry of one phase: MT tokens x R activation terms, one or two
// weight matrices (GLU: gate and up of the same rows).
template <int R, bool XB, bool GLU, int MT, bool TB>
struct PhaseT {
    static constexpr int NT = GLU ? 2 : 1;
    static constexpr int ES = XB ? 2 : 4;  // activation element size
    static constexpr int RM = ARows<R, MT, TB>::RM, AR = ARows<R, MT, TB>::AR, DL = ARows<R, MT, TB>::DL;
    static constexpr bool QUAD = ARows<R, MT, TB>::QUAD;
    static constexpr int US = ARows<R, MT, TB>::US;
    // Rows per operand slot in LDS: token quads add one zero row (row RM).
    // Term-major slots (48 rows) take no padding: slots a multiple of 256
    // bytes apart read conflict-free (measured; 784 bytes apart they conflict).
    static constexpr int SR = RM + (QUAD ? 1 : 0);
    static_assert(AR <= 16, "MFMA row block");
    static_assert(!XB || R == 1, "bf16 activations take one term");
};

// ---- 1. stage the activation terms of workgroup work wk into xs -------------------
// Octet o (8 consecutive k) of token m sits at operand slot
// ((o / 64 - s0) * 16 + o % 16) * 4 + (o / 16) % 4 -- super-step o / 64,
// block 4 g + bl with g = (o / 16) % 4, bl = (o / 4) % 4, dword t = o % 4
// of the block -- rows m * R + p (token-major) or p * MT + m (term-major)
// of the slot's RM rows. Tokens past M (a launch's last group) read zeros.
// Threads walk the slots in order (tokens fastest), so neighbouring lanes
// store neighbouring rows of LDS (slots in octet order would put them whole
// slots apart, on the same banks); the four lanes that load a cache line's
// four octets sit in one instruction, so the global loads stay whole-line.
template <int NW, int R, bool XB, int MT, bool TB>
__device__ __forceinline__ void stage_acts(const Gemv1Args& a, const WgWork& wk, __bf16* xs, int tid) {
    using Ph = PhaseT<R, XB, false, MT, TB>;
    const int octs = wk.nsw * 64;
    const int E = MT * octs;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, a.xbytes);
    for (int e0 = 0; e0 < E; e0 += kXO * 64 * NW) {
        u32x4 xr[kXO][2];
#pragma unroll
        for (int i = 0; i < kXO; ++i) {
            const int e = e0 + tid + i * 64 * NW;
            const int m = MT == 1 ? 0 : e % MT;
            const int sl = MT == 1 ? e : e / MT;  // slot, relative to super-step s0
            const int o = (sl >> 6) * 64 + (sl & 3) * 16 + ((sl >> 2) & 15);
            const int k = (wk.s0 * 64 + o) * 8;
            const uint32_t off =
                e < E && m < a.M && k < a.K ? (uint32_t)((m * a.ldx + k) * Ph::ES) : a.xbytes;  // past: zeros
            xr[i][0] = buf_load16(rx, off);
            xr[i][1] = XB ? u32x4{0u, 0u, 0u, 0u} : buf_load16(rx, off + 16);
        }
#pragma unroll
        for (int i = 0; i < kXO; ++i) {
            const int e = e0 + tid + i * 64 * NW;
            const int m = MT == 1 ? 0 : e % MT;
            const int sl = MT == 1 ? e : e / MT;
            if (e < E) stage_octet<R, TB ? MT * 8 : 8>(xr[i], xs + ((size_t)sl * Ph::SR + (TB ? m : m * R)) * 8);
        }
    }
    if constexpr (Ph::QUAD)
        for (int sl = tid; sl < wk.nsw * 64; sl += 64 * NW)
            *reinterpret_cast<u32x4*>(xs + ((size_t)sl * Ph::SR + Ph::RM) * 8) = u32x4{0u, 0u, 0u, 0u};
}

// ---- 1'. the activation from a fused residual step -----------------------------------
// Thread t owns octet t of the row (K <= 8 * threads, K % 8 == 0, one K split):
// it loads y, the residual and both norm weights at once, and the workgroup
// runs the layer's residual step exactly as alv_add_norm does -- s =
// resid_step(y, r) with y's norm when pr_norm_y, then x = bf16(rmsnorm(s) [*
// w_x]) -- in the float row `row` (LDS, K floats) with `red` (LDS, 128
// floats) for the pairwise sums. Workgroup 0 writes s to pr_s. Octet t of x
// goes to operand slot (t / 64) * 64 + (t % 16) * 4 + (t / 16) % 4 (the
// inverse of stage_acts' slot order); octets past K are zeros.
// The residual step of one octet with its flags as constants: resid_step's
// branches on runtime flags cost a scalar branch per value and flag.
template <bool NY, bool HW, int MODE>
__device__ __forceinline__ void resid_octet(float (&f)[8], const float (&rf)[8], const float (&wy)[8], float inv,
                                            float scale) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = resid_step(f[e], rf[e], wy[e], inv, NY, HW, MODE, scale);
}

__device__ __forceinline__ void resid_octet_any(const Gemv1Args& a, float (&f)[8], const float (&rf)[8],
                                                const float (&wy)[8], float inv) {
    const float sc = a.pr_scale;
    switch ((a.pr_norm_y ? 1 : 0) | (a.pr_wy ? 2 : 0) | (a.pr_mode << 2)) {
        case 0: resid_octet<false, false, 0>(f, rf, wy, inv, sc); break;
        case 1: resid_octet<true, false, 0>(f, rf, wy, inv, sc); break;
        case 2: resid_octet<false, true, 0>(f, rf, wy, inv, sc); break;
        case 3: resid_octet<true, true, 0>(f, rf, wy, inv, sc); break;
        case 4: resid_octet<false, false, 1>(f, rf, wy, inv, sc); break;
        case 5: resid_octet<true, false, 1>(f, rf, wy, inv, sc); break;
        case 6: resid_octet<false, true, 1>(f, rf, wy, inv, sc); break;
        case 7: resid_octet<true, true, 1>(f, rf, wy, inv, sc); break;
        case 8: resid_octet<false, false, 2>(f, rf, wy, inv, sc); break;
        case 9: resid_octet<true, false, 2>(f, rf, wy, inv, sc); break;
        case 10: resid_octet<false, true, 2>(f, rf, wy, inv, sc); break;
        default: resid_octet<true, true, 2>(f, rf, wy, inv, sc); break;
    }
}

// The rows are pr_k wide; the matmul's K may differ (a head registered K
// columns wider than the hidden size, or trimmed of all-zero columns):
// activation octets at or past either width are zeros. Without y (pr_y null)
// there is no residual step: s is resid as given (a first layer's input norm).
template <int NW>
__device__ void fused_resid_step(const Gemv1Args& a, const WgWork& wk, __bf16* xs, float* red, float* row, int tid) {
    constexpr int NT = 64 * NW;
    const int K = a.pr_k;
    const int v = tid;
    const bool in = 8 * v < K;
    const bool has_y = a.pr_y != nullptr;
    const uint4 yv = in && has_y ? reinterpret_cast<const uint4*>(a.pr_y)[v] : uint4{0u, 0u, 0u, 0u};
    const uint4 rv = in ? reinterpret_cast<const uint4*>(a.pr_r)[v] : uint4{0u, 0u, 0u, 0u};
    float wy[8], wx[8], f[8], rf[8];
    load_w8(in && has_y && a.pr_norm_y ? a.pr_wy : nullptr, v, wy);
    load_w8(in ? a.pr_wx : nullptr, v, wx);
    if (!a.pr_wx)  // t * 1 is t, bit for bit (NaN, signed zeros and subnormals included)
#pragma unroll
        for (int e = 0; e < 8; ++e) wx[e] = 1.0f;
    unpack8(yv, f);
    float inv = 1.0f;
    // Neither sum waits at its end: red is next written after the barrier
    // that follows the step, and nothing reads it after the second sum.
    if (has_y && a.pr_norm_y) {
        if (in)
#pragma unroll
            for (int e = 0; e < 8; ++e) row[8 * v + e] = f[e];
        __syncthreads();
        inv = rms_inv<NT, false>(row, K, a.pr_eps, red, tid);
    }
    if (in) {  // waves wholly past K skip the step
        unpack8(rv, rf);
        if (has_y) {
            resid_octet_any(a, f, rf, wy, inv);
            uint16_t b[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                b[e] = (uint16_t)(__builtin_bit_cast(uint32_t, f[e]) >> 16);  // f[e] holds a bf16 value
                row[8 * v + e] = f[e];
            }
            if (blockIdx.x == 0) reinterpret_cast<uint4*>(a.pr_s)[v] = pack8(b);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f[e] = rf[e];
                row[8 * v + e] = f[e];
            }
        }
    }
    __syncthreads();
    const float inv2 = rms_inv<NT, false>(row, K, a.pr_eps, red, tid);
    if (v < wk.nsw * 64) {
        uint16_t xb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (in && 8 * v < a.K)
#pragma unroll
            for (int e = 0; e < 8; ++e) xb[e] = bf16_rne_bits(mul_rn(mul_rn(f[e], inv2), wx[e]));
        const int sl = (v >> 6) * 64 + ((v & 15) << 2) + ((v >> 4) & 3);
        *reinterpret_cast<uint4*>(xs + (size_t)sl * 8) = pack8(xb);
    }
}

// The five 16-byte pieces of unit u (u >= U: past the range, zeros and no
// memory traffic). Offsets are wave-uniform by construction; saying so keeps
// the loads out of per-lane (waterfall) loops.
template <bool GLU, bool TL>
__device__ __forceinline__ void issue_unit(const Gemv1Args& a, const WgWork& wk, int U, __amdgpu_buffer_rsrc_t r0,
                                           __amdgpu_buffer_rsrc_t r1, uint32_t voff, u32x4 (&d)[5], int u) {
    constexpr int NT = GLU ? 2 : 1;
    uint32_t off = a.wbytes, step = 1024u;
    int n = 0;
    if (u < U) {
        const UnitPos p = unit_pos<NT, TL>(a, wk, u);
        off = p.off;
        step = p.step;
        n = p.n;
    }
    off = __builtin_amdgcn_readfirstlane(off);
    step = __builtin_amdgcn_readfirstlane(step);
    const __amdgpu_buffer_rsrc_t r = (GLU && __builtin_amdgcn_readfirstlane(n)) ? r1 : r0;
#pragma unroll
    for (int i = 0; i < 5; ++i) d[i] = buf_load16_so<true>(r, voff, off + step * i);
}

// ---- 3. dequantize + MFMA unit u (held in q) into its LDS slot ----------------------
// Lane base of the A operand: slot g, row j of the (first) block (rows >= AR
// read row AR - 1; their D rows are never used). A block past the row's end
// (the last super-step: the next plane's bytes, or the next row's in the
// combined layout) gets a zero scale, so its weights are zero.
// Unit u of super-step ss (nb: 32-column blocks of the matrix; s0: the
// workgroup's first super-step, whose activations sit first in xs).
template <int R, bool GLU, int MT, bool TB>
__device__ __forceinline__ void compute_unit_ss(int nb, int ss, int s0, const u32x4 (&q)[5], int u, const __bf16* xs,
                                                f32x4* part, int lane) {
    using Ph = PhaseT<R, false, GLU, MT, TB>;
    constexpr int SR = Ph::SR, AR = Ph::AR, DL = Ph::DL, RM = Ph::RM;
    constexpr bool QUAD = Ph::QUAD;
    constexpr int NB = TB ? R : (QUAD ? (MT + 3) / 4 : 1);  // A blocks per weight octet
    constexpr int ND = QUAD ? NB : 1;                 // D tiles
    const int j = lane & 15;
    const int g = lane >> 4;
    const int kb0 = ss * 16 + g * 4;
    const __bf16* xu = xs + (size_t)g * SR * 8 + (size_t)(ss - s0) * 16 * 4 * SR * 8;
    // This lane's A row in each block (rows >= AR read row AR - 1; their D rows
    // are never used; a token quad's fourth row reads the zero row).
    int arow[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
        arow[b] = QUAD ? ((j & 3) < 3 && 4 * b + (j >> 2) < MT ? (4 * b + (j >> 2)) * 3 + (j & 3) : RM)
                       : min(j, AR - 1) + (TB ? b * MT : 0);
    f32x4 t0[ND], t1[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) t0[d] = t1[d] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int bl = 0; bl < 4; ++bl) {
        const int w4 = 5 * bl + 4;
        const uint32_t sd = kb0 + bl < nb ? (uint32_t)q[w4 >> 2][w4 & 3] : 0u;
        const Scale2 sc = make_scale2(scale_of(sd));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int wi = 5 * bl + t;
            const bf16x8 bv = dequant8_mix((uint32_t)q[wi >> 2][wi & 3], sc);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int d = QUAD ? b : 0;
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(xu + ((bl * 4 + t) * 4 * SR + arow[b]) * 8);
                if (t & 1)
                    t1[d] = mfma16x16x32(av, bv, t1[d]);
                else
                    t0[d] = mfma16x16x32(av, bv, t0[d]);
            }
        }
    }
    if constexpr (QUAD) {
        // Lane (g, j) of tile b: token 4b + g, terms in elements 0..2.
        float* pf = reinterpret_cast<float*>(part + (size_t)u * Ph::US);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const f32x4 v = t0[b] + t1[b];
            if (4 * b + g < MT) pf[(4 * b + g) * 16 + j] = (v[0] + v[1]) + v[2];
        }
    } else {
        if (lane < DL) part[(size_t)u * DL + lane] = t0[0] + t1[0];
    }
}

template <int R, bool GLU, int MT, bool TB, bool TL>
__device__ __forceinline__ void compute_unit(const Gemv1Args& a, const WgWork& wk, const u32x4 (&q)[5], int u,
                                             const __bf16* xs, f32x4* part, int lane) {
    const UnitPos p = unit_pos<PhaseT<R, false, GLU, MT, TB>::NT, TL>(a, wk, u);
    compute_unit_ss<R, GLU, MT, TB>(a.nb, p.ss, wk.s0, q, u, xs, part, lane);
}

__device__ __forceinline__ void ystore(const Gemv1Args& a, int m, int row, float out) {
    if (a.Yb)
        a.Yb[(size_t)m * a.ldy + row] = __builtin_bit_cast(uint16_t, (__bf16)out);
    else
        a.Y[(size_t)m * a.ldy + row] = out;
}

// GLU of one output: the float64 arithmetic of the reference for one token
// (a few values per lane: a wave with any lane on the float64 path would run
// both), the float32 fast path with its float64 fallback for several.
template <int MT>
__device__ __forceinline__ float glu_out(float g, float u, int act) {
    return bf16_round(MT == 1 ? glu_exact(bf16_round(g), bf16_round(u), act) : glu_act(bf16_round(g), bf16_round(u), act));
}

// ---- 4. per row: sum the unit slots in a fixed order --------------------------------
// D row m * R + p (token m, term p; term-major: row m, terms summed) of
// column jj sits in slot lane 16 * (row / 4) + jj, element row % 4. One wave
// finishes the 16 rows of a row tile; four lanes share a row: lane c sums
// super-steps c, c + 4, ... in ascending order and the four partial sums
// combine in a fixed butterfly, so the result does not depend on timing;
// lane c of the four finishes tokens c, c + 4, ... Split K: this workgroup's
// shares go out instead, and the last workgroup of the tile group adds them
// (section 5).
template <int R, bool GLU, int MT, bool TB>
__device__ __forceinline__ void finish_tile(const Gemv1Args& a, const WgWork& wk, const f32x4* part, int tl,
                                            int lane) {
    using Ph = PhaseT<R, false, GLU, MT, TB>;
    constexpr int NT = Ph::NT, US = Ph::US;
    constexpr bool QUAD = Ph::QUAD;
    const int c = lane & 3;
    const int jj = lane >> 2;
    float y[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) y[m][n] = 0.0f;
    for (int ss = c; ss < wk.nsw; ss += 4) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const f32x4* sl = part + ((size_t)(tl * wk.nsw + ss) * NT + n) * US + (QUAD ? 0 : jj);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float v = 0.0f;
                if constexpr (QUAD) {
                    v = reinterpret_cast<const float*>(sl)[m * 16 + jj];
                } else {
#pragma unroll
                    for (int p = 0; p < (TB ? 1 : R); ++p) {
                        const int row = TB ? m : m * R + p;
                        v += sl[(row >> 2) * 16][row & 3];
                    }
                }
                y[m][n] += v;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            // lanes c ^ 1, then c ^ 2, of the row's four (DPP quad_perm moves)
            y[m][n] += dpp_f<0xB1>(y[m][n]);
            y[m][n] += dpp_f<0x4E>(y[m][n]);
        }
    const int row = tile_row(wk, tl) * 16 + jj;
    if (row >= a.N) return;
    if (a.ks > 1) {
        // This workgroup's share of K, written through (sc1 stores, as
        // agent-scope stores are) for the last of the ks workgroups of the
        // tile group to add up: the row's MT x NT floats are contiguous, and
        // its four lanes store them as whole 16-byte pieces, one line per row
        // (single-float write-through stores cost a partial-line write each).
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.part, a.pbytes);
        const uint32_t base = (uint32_t)((((size_t)row * a.ks + wk.kq) * MT) * NT * sizeof(float));
        constexpr int F = MT * NT;
        if constexpr (F % 4 == 0) {
#pragma unroll
            for (int ch = 0; ch < F / 4; ++ch) {
                if ((ch & 3) != c) continue;
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(uint32_t, y[(4 * ch + e) / NT][(4 * ch + e) % NT]);
                if (a.fix)
                    __builtin_amdgcn_raw_buffer_store_b128(v, rp, base + 16u * ch, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b128(v, rp, base + 16u * ch, 0, 16);
            }
        } else if (c == 0) {
#pragma unroll
            for (int f = 0; f < F; ++f) {
                const uint32_t v = __builtin_bit_cast(uint32_t, y[f / NT][f % NT]);
                if (a.fix)
                    __builtin_amdgcn_raw_buffer_store_b32(v, rp, base + 4u * f, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(v, rp, base + 4u * f, 0, 16);
            }
        }
        return;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if ((m & 3) != c || m >= a.M) continue;
        float out = y[m][0];
        if constexpr (GLU) out = glu_out<MT>(y[m][0], y[m][NT - 1], a.act);
        ystore(a, m, row, out);
    }
}

// ---- 5'. the split-K sum of rows row_of(0 .. nrow - 1) ---------------------------
// Each row's ks shares in split order (so the result does not depend on
// which workgroup wrote which share), then the epilogue: GLU or the plain
// output. SC1: the shares were written through by workgroups of this launch
// (the last arriver reads them past its XCD's L2); otherwise a launch before
// this one wrote them. flag[1] counts the GELU values the float32 path cannot
// settle, queued in `part` (part_n 16-byte entries) for a float64 pass.
template <int NW, bool GLU, int MT, bool SC1, class RowOf>
__device__ __forceinline__ void split_sum(const Gemv1Args& a, int nrow, RowOf row_of, f32x4* part, int part_n,
                                          int* flag, int tid) {
    constexpr int NT = GLU ? 2 : 1;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.part, a.pbytes);
    constexpr int F = MT * NT;
    if constexpr (F % 4 == 0) {
        // One (row, 16-byte piece) per thread: the piece of every split, in
        // split order, then the piece's tokens (two (gate, up) pairs, or four
        // outputs).
        for (int i = tid; i < nrow * (F / 4); i += 64 * NW) {
            const int r = i / (F / 4), ch = i - r * (F / 4);
            const int row = row_of(r);
            if (row >= a.N) continue;
            const uint32_t base = (uint32_t)(((size_t)row * a.ks * F + 4 * ch) * sizeof(float));
            float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
            for (int kq = 0; kq < a.ks; ++kq) {
                const u32x4 v = (SC1 ? buf_load16_sc1(rp, base + (uint32_t)((size_t)kq * F * sizeof(float)))
                                    : buf_load16(rp, base + (uint32_t)((size_t)kq * F * sizeof(float))));
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] += __builtin_bit_cast(float, (uint32_t)v[e]);
            }
#pragma unroll
            for (int e = 0; e < 4; e += NT) {
                const int m = (4 * ch + e) / NT;
                if (m >= a.M) continue;
                if constexpr (GLU) {
                    // GELU values the float32 path cannot settle wait in a
                    // queue in the (now unused) unit slots: about one in ten
                    // here, so nearly every wave would otherwise run the float64
                    // path for all its values.
                    const float gb = bf16_round(y[e]), ub = bf16_round(y[e + NT - 1]);
                    float v;
                    if (a.act != ALV_ACT_GELU_TANH) {
                        v = glu_exact(gb, ub, a.act);
                    } else if (!glu_fast(gb, ub, a.act, &v)) {
                        const int qi = __hip_atomic_fetch_add(&flag[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        if (qi < part_n) {
                            reinterpret_cast<u32x4*>(part)[qi] = u32x4{__builtin_bit_cast(uint32_t, gb),
                                                                       __builtin_bit_cast(uint32_t, ub), (uint32_t)m,
                                                                       (uint32_t)row};
                            continue;
                        }
                        v = glu_exact(gb, ub, a.act);
                    }
                    ystore(a, m, row, bf16_round(v));
                } else {
                    ystore(a, m, row, y[e]);
                }
            }
        }
        if constexpr (GLU) {
            __syncthreads();
            const int nq = min(flag[1], part_n);
            for (int i = tid; i < nq; i += 64 * NW) {
                // Elements through scalars: this clang lowers a bit cast of a
                // vector element to a read of element 0.
                const u32x4 q = reinterpret_cast<const u32x4*>(part)[i];
                const uint32_t gbits = q[0], ubits = q[1], m = q[2], row = q[3];
                ystore(a, (int)m, (int)row,
                       bf16_round(glu_exact(__builtin_bit_cast(float, gbits), __builtin_bit_cast(float, ubits), a.act)));
            }
        }
    } else {
        for (int i = tid; i < nrow * MT; i += 64 * NW) {  // one (row, token) per thread
            const int r = i / MT, m = i - r * MT;
            const int row = row_of(r);
            if (row >= a.N || m >= a.M) continue;
            const uint32_t base = (uint32_t)((((size_t)row * a.ks) * MT + m) * NT * sizeof(float));
            float y[NT];
#pragma unroll
            for (int n = 0; n < NT; ++n) y[n] = 0.0f;
#pragma unroll 4
            for (int kq = 0; kq < a.ks; ++kq)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    y[n] += __builtin_bit_cast(float, SC1 ? buf_load4_sc1(rp, base + (uint32_t)(((size_t)kq * MT * NT + n) * 4))
                                                          : buf_load4(rp, base + (uint32_t)(((size_t)kq * MT * NT + n) * 4)));
            float out = y[0];
            if constexpr (GLU) out = glu_out<MT>(y[0], y[NT - 1], a.act);
            ystore(a, m, row, out);
        }
    }
}

// Every tile of the workgroup (wave w: tiles w, w + NW, ...), then the split-K
// fixup (section 5). Split-K launches finish here, after all their units.
template <int NW, int R, bool GLU, int MT, bool TB>
__device__ __forceinline__ void finish_rows(const Gemv1Args& a, const WgWork& wk, f32x4* part, int part_n, int* flag,
                                            int tid) {
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool split = a.ks > 1;
    for (int tl = w; tl < wk.nt; tl += NW) finish_tile<R, GLU, MT, TB>(a, wk, part, tl, lane);
    if (!split || a.fix) return;

    // ---- 5. split K: the last workgroup of the tile group adds the shares ---------
    // The shares land before the workgroup counts itself in; the workgroup
    // that brings the count to ks reads all of them (sc1, past this XCD's L2)
    // and sums them in split order, so the result does not depend on which
    // workgroup came last; it then clears the count for the next launch.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.cnt[wk.tg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == (uint32_t)(a.ks - 1) ? 1 : 0;
        flag[1] = 0;
    }
    __syncthreads();
    if (!*flag) return;
    const int nrow = wk.nt * 16;
    split_sum<NW, GLU, MT, true>(a, nrow, [&](int r) { return tile_row(wk, r >> 4) * 16 + (r & 15); }, part, part_n, flag, tid);
    if (tid == 0) __hip_atomic_store(&a.cnt[wk.tg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ST: the workgroups compute their activation from a fused residual step
// (a.pr_r set). Those launches run a kernel of their own
// (q4_gemv1_step_kernel), so the one-token launches without a step (O, FFN
// down, the LM head) carry none of its code: decode-step rocprof on one box,
// O 5.84-5.92 against 6.00 µs, down 11.32-11.36 against 11.44, head
// 104.6-105.3 against 107.0-107.3.
template <int NW, int P, int R, bool XB, bool GLU, int MT, bool TB, bool TL, bool ST>
__device__ __forceinline__ void gemv1_body(const Gemv1Args& a) {
    using Ph = PhaseT<R, XB, GLU, MT, TB>;
    constexpr int NT = Ph::NT, SR = Ph::SR, US = Ph::US;
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const WgWork wk = wg_work(a, blockIdx.x);
    const int U = wk.nt * wk.nsw * NT;
    if (a.Nz > a.N) {
        // Trimmed all-zero rows: their outputs are zeros, spread over the grid.
        const int nz = a.Nz - a.N;
        for (int i = blockIdx.x * 64 * NW + tid; i < nz * a.M; i += gridDim.x * 64 * NW)
            ystore(a, i / nz, a.N + i % nz, 0.0f);
    }
    __bf16* xs = reinterpret_cast<__bf16*>(smem);
    f32x4* part = reinterpret_cast<f32x4*>(smem + (size_t)wk.nsw * 1024 * SR);
    // Unit counter of the workgroup, after the unit slots: the first P * NW
    // units go to the waves statically, the rest to whichever wave frees a ring
    // slot first, so a wave whose loads come back late does fewer units.
    int* next = reinterpret_cast<int*>(part + (size_t)U * US);
    if (tid == 0) *next = P * NW;

    // The activation is staged before any weight load: queued behind the
    // weight loads of every CU it would wait for (bytes in flight) / bandwidth
    // (issuing the first weight loads ahead of a fused residual step's
    // computation measured slower as well).
    bool fused = false;
    if constexpr (XB && MT == 1 && ST) {
        if (a.pr_r) {
            // The fused residual step's LDS follows the unit counter.
            float* red = reinterpret_cast<float*>(next + 4);
            fused_resid_step<NW>(a, wk, xs, red, red + 128, tid);
            fused = true;
        }
    }
    if (!fused) stage_acts<NW, R, XB, MT, TB>(a, wk, xs, tid);
    lds_barrier();

    // ---- 2. the first P units of this wave -----------------------------------------
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(GLU ? a.W1 : a.W0, a.wbytes);
    const uint32_t voff = lane_voff<TL>(a, lane);
    u32x4 q[P][5];
    int uk[P];  // the unit in each ring slot (>= U: none)
#pragma unroll
    for (int k = 0; k < P; ++k) {
        uk[k] = w + k * NW;
        issue_unit<GLU, TL>(a, wk, U, r0, r1, voff, q[k], uk[k]);
    }

    // ---- 3. stream: dequantize + MFMA one unit, refill its ring slot ---------------
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
            if (uk[k] < U) compute_unit<R, GLU, MT, TB, TL>(a, wk, q[k], uk[k], xs, part, lane);
            issue_unit<GLU, TL>(a, wk, U, r0, r1, voff, q[k], un);
            uk[k] = un;
            live |= un < U;
        }
    }
    lds_barrier();
    finish_rows<NW, R, GLU, MT, TB>(a, wk, part, U * US, next, tid);
}

template <int NW, int P, int R, bool XB, bool GLU, int MT, bool TB, bool TL>
__global__ void __launch_bounds__(64 * NW) q4_gemv1_kernel(Gemv1Args a) {
    gemv1_body<NW, P, R, XB, GLU, MT, TB, TL, false>(a);
}

template <int NW, int P, int R, bool XB, bool GLU, int MT, bool TB, bool TL>
__global__ void __launch_bounds__(64 * NW) q4_gemv1_step_kernel(Gemv1Args a) {
    gemv1_body<NW, P, R, XB, GLU, MT, TB, TL, true>(a);
}

// ---- One-token FFN in one launch (q4_ffn1_kernel) ------------------------------------
// The reference's NPU dataflow (kernels/ffn_fused/ffn_fused.py:28-328: each
// core owns a slice of the intermediate rows, computes gate, up and the
// activation for them and multiplies the slice's columns of the down matrix
// into a partial output; the host sums the partials, runtime/cpp/src/npu.cpp:
// 360-377), planned for the GPU. Workgroup b owns the 64 intermediate rows of
// row-tile pairs b and b + G (rows 32 b .. 32 b + 31 and 32 (b + G) .. + 31):
//   A. the gate/up units of its four row tiles against the staged activation,
//      then the GLU epilogue of those 64 rows into LDS (bf16 values, the
//      reference's rounding points) and into the handle's activation buffer;
//   B. the down units of its slice: the 64 down columns of those rows, from
//      a registration-time layout (ffn1_vdown_kernel) in which down unit u of
//      workgroup b (tile u G + b) is an ordinary 16-row x 512-column tile whose block
//      4 g + bl is the real block (row 128 u + 16 ((4 g + bl) >> 1) + j,
//      column block b + G ((4 g + bl) & 1)). Its A operand holds eight rows,
//      one per real row tile: row t carries the slice's activations in the
//      two blocks of tile t and zeros elsewhere, so D row t of the unit is
//      the partial output of rows 128 u + 16 t .. + 15 -- the eight-token
//      bf16 instance of compute_unit as it stands;
//   C. the 128 U partial outputs to part[b][.], summed over the workgroups
//      in a fixed order by ffn1_sum_kernel.
// No workgroup waits for another: the down weights of a slice stream behind
// its gate/up units in the same ring, and a wave that takes its first down
// unit issues the loads before the GLU epilogue runs.
struct Ffn1Args {
    Gemv1Args gu;       // the gate/up launch at one token (tiled gate W0 and up W1, X, act, nss, nb)
    const uint8_t* Wv;  // down slices, tiled layout of the (G U 16) x 512 matrix above
    uint32_t vbytes;
    float* part;   // G x He partial outputs
    uint16_t* act; // the bf16 activation of the I rows (token 0)
    int G, U, He;
};

constexpr int kFfn1Rows = 64;  // intermediate rows per workgroup

// Unit u of workgroup b: u < UA a gate/up unit, (local tile tl * nss + ss) * 2
// + matrix, local tile tl being row tile 2 (b + G (tl >> 1)) + (tl & 1);
// UA <= u < UE down unit u - UA; past UE nothing (loads past the range read
// zeros). Offsets and the descriptor are wave-uniform.
__device__ __forceinline__ void ffn1_issue(const Ffn1Args& f, int b, int UA, int UE, __amdgpu_buffer_rsrc_t r0,
                                           __amdgpu_buffer_rsrc_t r1, __amdgpu_buffer_rsrc_t rv, uint32_t voff,
                                           u32x4 (&d)[5], int u) {
    const int nss = f.gu.nss;
    uint32_t off = f.gu.wbytes, step = 1024u;
    int sel = 0;
    if (u < UA) {
        const int t = u >> 1, tl = t / nss, ss = t - tl * nss;
        const int rt = 2 * (b + f.G * (tl >> 1)) + (tl & 1);
        off = (uint32_t)rt * f.gu.rtb + (uint32_t)ss * 5120u;
        step = ss == nss - 1 ? 256u * (uint32_t)f.gu.ng_last : 1024u;
        sel = u & 1;
    } else if (u < UE) {
        off = (uint32_t)((u - UA) * f.G + b) * 5120u;  // unit-major: the workgroups' units u are neighbours
        sel = 2;
    }
    off = __builtin_amdgcn_readfirstlane(off);
    step = __builtin_amdgcn_readfirstlane(step);
    sel = __builtin_amdgcn_readfirstlane(sel);
    const __amdgpu_buffer_rsrc_t r = sel == 2 ? rv : (sel ? r1 : r0);
#pragma unroll
    for (int i = 0; i < 5; ++i) d[i] = buf_load16_so<true>(r, voff, off + step * i);
}

// ST: the activation comes from a fused residual step (a.pr_r set; bf16, one
// token), computed in phase B's LDS before that region is used.
template <int NW, int R, bool XB, bool ST>
__global__ void __launch_bounds__(64 * NW) q4_ffn1_kernel(Ffn1Args f) {
    using PA = PhaseT<R, XB, true, 1, false>;
    using PB = PhaseT<1, true, false, 8, false>;
    const Gemv1Args& a = f.gu;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x;
    const int nss = a.nss;
    const int UA = 4 * nss * 2;
    const int UE = UA + f.U;
    __bf16* xsA = reinterpret_cast<__bf16*>(smem);
    f32x4* partA = reinterpret_cast<f32x4*>(smem + (size_t)nss * 1024 * PA::SR);
    int* next = reinterpret_cast<int*>(partA + (size_t)UA * PA::US);
    float* aval = reinterpret_cast<float*>(next + 4);
    unsigned char* xsB_bytes = reinterpret_cast<unsigned char*>(aval + kFfn1Rows);
    __bf16* xsB = reinterpret_cast<__bf16*>(xsB_bytes);
    f32x4* partB = reinterpret_cast<f32x4*>(xsB_bytes + 1024 * PB::SR);

    WgWork wk;
    wk.tg = 0;
    wk.kq = 0;
    wk.ntg = 1;
    wk.nt = 4;
    wk.s0 = 0;
    wk.nsw = nss;
    bool fused = false;
    if constexpr (ST) {
        if (a.pr_r) {
            float* red = reinterpret_cast<float*>(xsB_bytes);  // 128 + K floats, free until the GLU epilogue
            fused_resid_step<NW>(a, wk, xsA, red, red + 128, tid);
            fused = true;
        }
    }
    if (!fused) stage_acts<NW, R, XB, 1, false>(a, wk, xsA, tid);
    if (tid == 0) *next = NW;
    lds_barrier();

    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.W0, a.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(a.W1, a.wbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(f.Wv, f.vbytes);
    const uint32_t voff = 16u * (uint32_t)lane;
    u32x4 q[5];
    int uk = w;
    ffn1_issue(f, b, UA, UE, r0, r1, rv, voff, q, uk);

    // ---- A: gate/up units; a wave leaves holding the loads of its first down unit
    for (;;) {
        int un = 0;
        if (lane == 0) un = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        un = __builtin_amdgcn_readfirstlane(un);
        const int t = uk >> 1;
        compute_unit_ss<R, true, 1, false>(a.nb, t % nss, 0, q, uk, xsA, partA, lane);
        ffn1_issue(f, b, UA, UE, r0, r1, rv, voff, q, un);
        uk = un;
        if (un >= UA) break;
    }
    lds_barrier();

    // GLU of local tile w (waves 0..3), as finish_tile sums and rounds it.
    if (w < 4) {
        const int c = lane & 3, jj = lane >> 2;
        float y[2] = {0.0f, 0.0f};
        for (int ss = c; ss < nss; ss += 4) {
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const f32x4* sl = partA + ((size_t)(w * nss + ss) * 2 + n) * PA::US + jj;
                float v = 0.0f;
#pragma unroll
                for (int p = 0; p < R; ++p) v += sl[(p >> 2) * 16][p & 3];
                y[n] += v;
            }
        }
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            y[n] += dpp_f<0xB1>(y[n]);
            y[n] += dpp_f<0x4E>(y[n]);
        }
        if (c == 0) {
            const float out = glu_out<1>(y[0], y[1], a.act);
            aval[16 * w + jj] = out;
            const int row = 16 * (2 * (b + f.G * (w >> 1)) + (w & 1)) + jj;
            f.act[row] = (uint16_t)(__builtin_bit_cast(uint32_t, out) >> 16);  // out holds a bf16 value
        }
    }
    lds_barrier();
    // The down units' A operand: slot (bl 4 + t) 4 + g of virtual block
    // vb = 4 g + bl, octet t; its row rr holds the slice's octet when the block
    // belongs to real row tile rr (vb >> 1 == rr), zeros otherwise.
    for (int e = tid; e < 64 * PB::SR; e += 64 * NW) {
        const int sl = e / PB::SR, rr = e - sl * PB::SR;
        const int g = sl & 3, bt = sl >> 2, bl = bt >> 2, t = bt & 3;
        const int vb = 4 * g + bl;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if ((vb >> 1) == rr) {
            const float* src = aval + 32 * (vb & 1) + 8 * t;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                v[h] = (__builtin_bit_cast(uint32_t, src[2 * h]) >> 16) | (__builtin_bit_cast(uint32_t, src[2 * h + 1]) & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x4*>(xsB + (size_t)e * 8) = v;
    }
    lds_barrier();

    // ---- B: down units -------------------------------------------------------------
    while (uk < UE) {
        int un = 0;
        if (lane == 0) un = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        un = __builtin_amdgcn_readfirstlane(un);
        compute_unit_ss<1, false, 8, false>(16, 0, 0, q, uk - UA, xsB, partB, lane);
        ffn1_issue(f, b, UA, UE, r0, r1, rv, voff, q, un);
        uk = un;
    }
    lds_barrier();

    // ---- C: this slice's partial outputs -------------------------------------------
    // D of down unit u: lane 16 g + j, element e = rows 128 u + 16 (4 g + e) + j.
    const float* pb = reinterpret_cast<const float*>(partB);
    for (int i = tid; i < f.U * 128; i += 64 * NW) {
        const int u = i >> 7, r = i & 127, tt = r >> 4, j = r & 15;
        f.part[(size_t)b * f.He + i] = pb[((size_t)u * 32 + (tt >> 2) * 16 + j) * 4 + (tt & 3)];
    }
}

// Output row r = the G partials in a fixed order: thread group q (of 32)
// adds workgroups q, q + 32, ... (its loads issued together), then the 32
// sums in order; rows [He, H) are zeros (trimmed all-zero rows).
constexpr int kFfn1SumRows = 32, kFfn1SumGroups = 32, kFfn1SumLoads = 8;  // G <= 256

__global__ void __launch_bounds__(kFfn1SumRows * kFfn1SumGroups) ffn1_sum_kernel(const float* part, int G, int He,
                                                                                 int H, float* Y, uint16_t* Yb) {
    __shared__ float red[kFfn1SumGroups][kFfn1SumRows + 1];
    const int r = threadIdx.x % kFfn1SumRows, qg = threadIdx.x / kFfn1SumRows;
    const int row = blockIdx.x * kFfn1SumRows + r;
    float v[kFfn1SumLoads];
#pragma unroll
    for (int i = 0; i < kFfn1SumLoads; ++i) {
        const int b = qg + i * kFfn1SumGroups;
        v[i] = row < He && b < G ? part[(size_t)b * He + row] : 0.0f;
    }
    float sacc = 0.0f;
#pragma unroll
    for (int i = 0; i < kFfn1SumLoads; ++i) sacc += v[i];
    red[qg][r] = sacc;
    __syncthreads();
    if (qg == 0 && row < H) {
        float y = 0.0f;
        if (row < He)
#pragma unroll
            for (int i = 0; i < kFfn1SumGroups; ++i) y += red[i][r];
        if (Yb)
            Yb[row] = __builtin_bit_cast(uint16_t, (__bf16)y);
        else
            Y[row] = y;
    }
}

// The split-K sums of a launch made with a.fix, after it: workgroup b adds
// the shares of rows [b rpw, b rpw + rpw), one (row, 16-byte piece) or one
// (row, token) per thread, in split order -- the arithmetic of the last
// arriver's sum, so both give the same bits.
constexpr int kFixThreads = 256;

template <bool GLU, int MT>
__global__ void __launch_bounds__(kFixThreads) split_fix_kernel(Gemv1Args a, int rpw) {
    __shared__ f32x4 queue[2 * kFixThreads];  // GELU values for the float64 pass
    __shared__ int flag[2];
    const int tid = threadIdx.x;
    if (tid == 0) flag[1] = 0;
    __syncthreads();
    const int r0 = blockIdx.x * rpw;
    split_sum<kFixThreads / 64, GLU, MT, false>(a, min(rpw, a.N - r0), [&](int r) { return r0 + r; }, queue,
                                                2 * kFixThreads, flag, tid);
}

// Rows per fixup workgroup: one 16-byte piece (or one token) per thread.
constexpr int fix_rows(bool glu, int mt) {
    return (mt * (glu ? 2 : 1)) % 4 == 0 ? kFixThreads / (mt * (glu ? 2 : 1) / 4) : kFixThreads / mt;
}

template <bool GLU>
hipError_t launch_fix_g(const Gemv1Args& a, int mt, hipStream_t s) {
    const int rpw = fix_rows(GLU, mt);
    const dim3 grid((a.N + rpw - 1) / rpw);
    switch (mt) {
        case 1: hipLaunchKernelGGL((split_fix_kernel<GLU, 1>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
        case 2: hipLaunchKernelGGL((split_fix_kernel<GLU, 2>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
        case 4: hipLaunchKernelGGL((split_fix_kernel<GLU, 4>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
        case 5: hipLaunchKernelGGL((split_fix_kernel<GLU, 5>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
        case 8: hipLaunchKernelGGL((split_fix_kernel<GLU, 8>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
        default: hipLaunchKernelGGL((split_fix_kernel<GLU, 16>), grid, dim3(kFixThreads), 0, s, a, rpw); break;
    }
    return hipGetLastError();
}

hipError_t launch_fix(const Gemv1Args& a, bool glu, int mt, hipStream_t s) {
    return glu ? launch_fix_g<true>(a, mt, s) : launch_fix_g<false>(a, mt, s);
}

// Whether a launch of ks K splits sums its shares in a launch of its own
// (split_fix_kernel) rather than in its last-arriving workgroups: from 4
// splits. Measured on the 12B-class FFN (3840 <-> 15360, 16 distinct layers,
// same box, bit-identical outputs), µs per call: 16 tokens (gate/up and down
// at 4 splits) 50.7 against 58.9 with the last arrivers; 8 tokens (2 splits)
// 43.9 against 43.0 -- there the second launch costs more than the shorter
// tail saves. The environment variable ALV_SPLIT_FIX (0: never, 1: every
// split launch), read at each call, overrides.
bool split_fix(int ks) {
    const char* e = getenv("ALV_SPLIT_FIX");
    if (e && *e) return ks > 1 && atoi(e) != 0;
    return ks >= 4;
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

// The dynamic-LDS limit of kernel k on the current device, raised to `lds`
// once per (kernel, device) rather than on every launch.
inline hipError_t ensure_lds(const void* k, std::atomic<int> (&set)[64], size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (set[dev].load(std::memory_order_relaxed) >= (int)lds) return hipSuccess;
    const int want = (int)dev_info().lds;  // the whole per-workgroup limit: one call per kernel and device
    const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return e;
    }
    set[dev].store(want, std::memory_order_relaxed);
    return hipSuccess;
}

template <int P, int R, bool XB, bool GLU, int MT, bool TB = false, bool TL = true, bool ST = false>
hipError_t launch_k(const Gemv1Args& a, int groups, size_t lds, hipStream_t s) {
    void (*k)(Gemv1Args);
    if constexpr (ST)
        k = q4_gemv1_step_kernel<kNW, P, R, XB, GLU, MT, TB, TL>;
    else
        k = q4_gemv1_kernel<kNW, P, R, XB, GLU, MT, TB, TL>;
    static std::atomic<int> set[64];
    if (const hipError_t e = ensure_lds(reinterpret_cast<const void*>(k), set, lds)) return e;
    hipLaunchKernelGGL(k, dim3(groups), dim3(64 * kNW), lds, s, a);
    return hipGetLastError();
}

// Ring depth: one unit in flight per wave (16 per CU) measures faster than two
// on every one-token shape -- a deeper ring only lengthens the memory queues.
// From 8 tokens a unit's compute (two or three MFMAs per weight octet) holds
// a wave long enough that a second unit in flight pays: 12B-class FFN at 8
// tokens 42.8 against 43.5 µs, at 16 tokens 50.2 against 50.8 (same box,
// bit-identical; no more VGPRs at 16 tokens).
constexpr int kP = 1;
constexpr int kPWide = 2;  // 8 and 16 tokens

// Token capacity of a launch, activation terms per token and row layout:
// fp32 activations take the exact three-term split: token quads for 2, 3-4
// and 6-8 tokens (one MFMA per weight octet up to 4 tokens, two for 8),
// token-major rows for 1 and 5 (3 and 15 A rows, one MFMA), term-major for
// 9-16 (three MFMAs that fill every A row; K splits until the 48 staged rows
// fit the LDS); bf16 activations one term, up to 16 tokens.
struct Shape {
    int mt, r;
    bool tb;
};

Shape shape_for(const GemvLaunch& L, int m) {
    if (L.Xb) {
        int mt = 1;
        while (mt < m && mt < 16) mt *= 2;
        return {mt, 1, false};
    }
    if (m <= 2) return {m, 3, false};
    if (m <= 4) return {4, 3, false};
    if (m <= 5) return {5, 3, false};
    if (m <= 8) return {8, 3, false};
    return {16, 3, true};
}

hipError_t launch_shape(const Gemv1Args& a, const GemvLaunch& L, Shape sh, int groups, size_t lds, hipStream_t s) {
    if (L.Xb && L.glu) {
        switch (sh.mt) {
            case 1:
                return a.pr_r ? launch_k<kP, 1, true, true, 1, false, true, true>(a, groups, lds, s)
                              : launch_k<kP, 1, true, true, 1>(a, groups, lds, s);
            case 2: return launch_k<kP, 1, true, true, 2>(a, groups, lds, s);
            case 4: return launch_k<kP, 1, true, true, 4>(a, groups, lds, s);
            case 8: return launch_k<kPWide, 1, true, true, 8>(a, groups, lds, s);
            default: return launch_k<kPWide, 1, true, true, 16>(a, groups, lds, s);
        }
    }
    if (L.Xb) {
        switch (sh.mt) {
            case 1:
                return a.pr_r ? launch_k<kP, 1, true, false, 1, false, true, true>(a, groups, lds, s)
                              : launch_k<kP, 1, true, false, 1>(a, groups, lds, s);
            case 2: return launch_k<kP, 1, true, false, 2>(a, groups, lds, s);
            case 4: return launch_k<kP, 1, true, false, 4>(a, groups, lds, s);
            case 8: return launch_k<kPWide, 1, true, false, 8>(a, groups, lds, s);
            default: return launch_k<kPWide, 1, true, false, 16>(a, groups, lds, s);
        }
    }
    if (L.glu) {
        switch (sh.mt) {
            case 1: return launch_k<kP, 3, false, true, 1>(a, groups, lds, s);
            case 2: return launch_k<kP, 3, false, true, 2>(a, groups, lds, s);
            case 4: return launch_k<kP, 3, false, true, 4>(a, groups, lds, s);
            case 5: return launch_k<kP, 3, false, true, 5>(a, groups, lds, s);
            case 8: return launch_k<kPWide, 3, false, true, 8>(a, groups, lds, s);
            default: return launch_k<kPWide, 3, false, true, 16, true>(a, groups, lds, s);
        }
    }
    if (!L.tiled) {
        switch (sh.mt) {
            case 1: return launch_k<kP, 3, false, false, 1, false, false>(a, groups, lds, s);
            case 2: return launch_k<kP, 3, false, false, 2, false, false>(a, groups, lds, s);
            case 4: return launch_k<kP, 3, false, false, 4, false, false>(a, groups, lds, s);
            case 5: return launch_k<kP, 3, false, false, 5, false, false>(a, groups, lds, s);
            case 8: return launch_k<kP, 3, false, false, 8, false, false>(a, groups, lds, s);
            default: return launch_k<kP, 3, false, false, 16, true, false>(a, groups, lds, s);
        }
    }
    switch (sh.mt) {
        case 1: return launch_k<kP, 3, false, false, 1>(a, groups, lds, s);
        case 2: return launch_k<kP, 3, false, false, 2>(a, groups, lds, s);
        case 4: return launch_k<kP, 3, false, false, 4>(a, groups, lds, s);
        case 5: return launch_k<kP, 3, false, false, 5>(a, groups, lds, s);
        case 8: return launch_k<kP, 3, false, false, 8>(a, groups, lds, s);
        default: return launch_k<kP, 3, false, false, 16, true>(a, groups, lds, s);
    }
}

struct Gemv1Plan {
    Shape sh;
    int tg, rt_q, rt_r, ks;
    size_t lds;
};

// K splits (1, 2, 4, ... up to 16 and the super-step count) until the
// workgroup's activations and unit slots fit the LDS and the split's partial
// sums fit their scratch. One split when it fits: no partial sums at all.
bool plan_gemv1(const GemvLaunch& L, int m, Gemv1Plan* out) {
    if (L.parts != (L.Xb ? 1 : 3) || m < 1) return false;
    if (!L.tiled && (L.Xb || L.glu)) return false;  // the combined layout serves alv_gemv_q / alv_gemm_q only
    const DevInfo& d = dev_info();
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const int NT = L.glu ? 2 : 1;
    Gemv1Plan p;
    p.sh = shape_for(L, m);
    const int RM = p.sh.mt * p.sh.r;
    const bool quad = !p.sh.tb && p.sh.r == 3 && (p.sh.mt == 2 || p.sh.mt == 4 || p.sh.mt == 8);  // ARows::QUAD
    const int AR = p.sh.tb ? p.sh.mt : RM;
    const int SR = RM + (quad ? 1 : 0);  // rows per LDS operand slot (PhaseT::SR)
    const size_t slot_bytes = quad ? (size_t)p.sh.mt * 64 : (size_t)256 * ((AR + 3) / 4);  // ARows::US * 16
    for (p.ks = 1; p.ks <= 16 && p.ks <= tg.nss; p.ks *= 2) {
        p.tg = std::min(RT, std::max(1, d.cus / p.ks));
        p.rt_q = RT / p.tg;
        p.rt_r = RT % p.tg;
        const int tiles = p.rt_q + (p.rt_r ? 1 : 0);
        const int nsw = (tg.nss + p.ks - 1) / p.ks;
        const int units = tiles * nsw * NT;
        p.lds = (size_t)nsw * 1024 * SR + (size_t)units * slot_bytes + 16;
        const size_t part = p.ks > 1 ? (size_t)RT * 16 * p.ks * p.sh.mt * NT * sizeof(float) : 0;
        if (p.lds <= d.lds && part <= kPartMax && (p.ks == 1 || p.tg <= kSplitCounters)) {
            *out = p;
            return true;
        }
    }
    return false;
}

// Most tokens one launch takes (0: the shape has no plan).
int max_tokens(const GemvLaunch& L) {
    Gemv1Plan p;
    for (int m : {16, 8, 5, 4, 2, 1})
        if (plan_gemv1(L, m, &p)) return m;
    return 0;
}

}  // namespace

namespace {

// Split-K partial sums of one launch of m tokens under plan p:
// [row][ks][token][matrix] floats.
size_t split_part_bytes(const GemvLaunch& L, const Gemv1Plan& p) {
    const int RT = (L.N + 15) / 16;
    return (size_t)RT * 16 * p.ks * p.sh.mt * (L.glu ? 2 : 1) * sizeof(float);
}

// Kernel arguments of tokens [m0, m0 + m) of L under plan p.
int fill_args(const GemvLaunch& L, const Gemv1Plan& p, int m0, int m, hipStream_t s, Gemv1Args* out) {
    const TileGeom tg = tile_geom(L.K);
    const int RT = (L.N + 15) / 16;
    const uint64_t rs = (uint64_t)tg.nb * kBlockBytes;
    const uint64_t wbytes = L.tiled ? (uint64_t)RT * tg.rtb : (uint64_t)L.N * rs;
    if (wbytes >= 0xFFFFE000ull)
        return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
    const int ES = L.Xb ? 2 : 4;
    const uint64_t xbytes = ((uint64_t)(m - 1) * L.ldx + L.K) * ES;
    if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activation buffer exceeds the 2 GiB range");
    Gemv1Args a{};
    if (p.ks > 1) {
        const size_t pb = split_part_bytes(L, p);
        if (L.split) {
            if (pb > L.split->part_bytes)
                return fail(ALV_ERR_RANGE, "split-K partial sums of %zu bytes exceed the %zu provided", pb,
                            L.split->part_bytes);
            a.cnt = L.split->counters;
            a.part = L.split->part;
        } else {
            Workspace ws;
            if (int rc = get_workspace(s, kSplitCounters, &ws)) return rc;
            a.cnt = ws.counters;
            void* part = nullptr;
            if (int rc = get_scratch(s, kScratchSplit, pb, &part)) return rc;
            a.part = static_cast<float*>(part);
        }
        a.pbytes = (uint32_t)pb;
    }
    a.W0 = L.W0;
    a.W1 = L.W1;
    a.X = L.Xb ? (const void*)(L.Xb + (size_t)m0 * L.ldx) : (const void*)(L.X + (size_t)m0 * L.ldx);
    a.Y = L.Y ? L.Y + (size_t)m0 * L.ldy : nullptr;
    a.Yb = L.Yb ? L.Yb + (size_t)m0 * L.ldy : nullptr;
    a.wbytes = (uint32_t)wbytes;
    a.rtb = L.tiled ? tg.rtb : (uint32_t)(16 * rs);
    a.rs = (uint32_t)rs;
    a.nb = tg.nb;
    a.xbytes = (uint32_t)xbytes;
    a.N = L.N;
    a.K = L.K;
    a.nss = tg.nss;
    a.ng_last = tg.ng_last;
    a.ldx = L.ldx;
    a.ldy = L.ldy;
    a.M = m;
    a.ntg = p.tg;
    a.rt_q = p.rt_q;
    a.rt_r = p.rt_r;
    a.ks = p.ks;
    a.act = L.act;
    a.fix = split_fix(p.ks) ? 1 : 0;
    a.Nz = L.Nz;
    if (const ResidStep* st = L.step) {
        a.pr_r = st->resid;
        a.pr_y = st->y;
        a.pr_wy = st->w_y;
        a.pr_wx = st->w_x;
        a.pr_s = st->sum_out;
        a.pr_scale = st->scale;
        a.pr_eps = st->eps;
        a.pr_norm_y = st->norm_y;
        a.pr_mode = st->scale_mode;
        a.pr_k = st->k ? st->k : L.K;
    }
    *out = a;
    return ALV_OK;
}

}  // namespace

// Token groups of a launch: as equal a size as the capacity allows (16 tokens
// at a capacity of 5: four groups of 4, not 5 + 5 + 5 + 1).
int64_t gemv_split_bytes(const GemvLaunch& L) {
    const int mmax = L.M >= 1 && L.M <= kGemvMaxM ? max_tokens(L) : 0;
    if (!mmax) return -1;
    const int ngroups = (L.M + mmax - 1) / mmax;
    const int gsize = (L.M + ngroups - 1) / ngroups;
    size_t most = 0;
    for (int m0 = 0; m0 < L.M; m0 += gsize) {
        Gemv1Plan p;
        if (!plan_gemv1(L, std::min(gsize, L.M - m0), &p)) return -1;
        if (p.ks > 1) most = std::max(most, split_part_bytes(L, p));
    }
    return (int64_t)most;
}

// A one-token launch whose workgroups compute their bf16 activation from a
// fused residual step (fused_resid_step): one K split, the float row and the
// pairwise-sum scratch after the unit counter.
namespace {

// The argument checks of a launch with a fused residual step.
int check_step(const GemvLaunch& L) {
    const ResidStep& st = *L.step;
    if (L.M != 1 || !L.Xb || !L.tiled || L.parts != 1)
        return fail(ALV_ERR_ARG, "a fused residual step takes one token of bf16 activations on registered weights");
    if (L.K % 8 || L.K > kResidStepMaxK)
        return fail(ALV_ERR_ARG, "a fused residual step takes K a multiple of 8 up to %d (got %d)", kResidStepMaxK, L.K);
    const int rk = st.k ? st.k : L.K;  // the rows' width
    if (rk < 8 || rk % 8 || rk > kResidStepMaxK)
        return fail(ALV_ERR_ARG, "a fused residual step takes rows a multiple of 8 up to %d wide (got %d)",
                    kResidStepMaxK, rk);
    if (!st.resid || (st.y && !st.sum_out)) return fail(ALV_ERR_ARG, "null residual-step pointer");
    if (st.scale_mode < 0 || st.scale_mode > 2) return fail(ALV_ERR_ARG, "bad scale_mode %d", st.scale_mode);
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!al(st.resid) || !al(st.y) || !al(st.sum_out) || !al(st.w_y) || !al(st.w_x))
        return fail(ALV_ERR_ALIGN, "residual-step rows and weights need 16-byte alignment");
    return ALV_OK;
}

}  // namespace

int launch_gemv_step(const GemvLaunch& L, hipStream_t s) {
    if (int rc = check_step(L)) return rc;
    const ResidStep& st = *L.step;
    const int rk = st.k ? st.k : L.K;
    Gemv1Plan p;
    if (!plan_gemv1(L, 1, &p)) return fail(ALV_ERR_RANGE, "streaming GEMV: no plan for N=%d K=%d", L.N, L.K);
    if (p.ks != 1) return fail(ALV_ERR_RANGE, "a fused residual step needs the whole of K in one workgroup (K=%d)", L.K);
    p.lds += 128 * sizeof(float) + (size_t)rk * sizeof(float);
    if (p.lds > dev_info().lds) return fail(ALV_ERR_RANGE, "a fused residual step at K=%d exceeds the LDS", L.K);
    Gemv1Args a;
    if (int rc = fill_args(L, p, 0, 1, s, &a)) return rc;
    return hip_check(launch_shape(a, L, p.sh, p.tg * p.ks, p.lds, s), "q4_gemv1_kernel launch");
}

int launch_gemv(const GemvLaunch& L, hipStream_t s) {
    if (L.step) return launch_gemv_step(L, s);
    if (L.M < 1 || L.M > kGemvMaxM) return fail(ALV_ERR_ARG, "streaming GEMV takes 1 <= M <= %d (got %d)", kGemvMaxM, L.M);
    if (L.parts != (L.Xb ? 1 : 3)) return fail(ALV_ERR_ARG, "fp32 activations take 3 terms, bf16 activations 1");
    const int mmax = max_tokens(L);
    if (!mmax) return fail(ALV_ERR_RANGE, "streaming GEMV: no launch plan for M=%d N=%d K=%d", L.M, L.N, L.K);
    // Groups of as equal a size as the capacity allows (16 tokens at a
    // capacity of 5: four groups of 4, not 5 + 5 + 5 + 1).
    const int ngroups = (L.M + mmax - 1) / mmax;
    const int gsize = (L.M + ngroups - 1) / ngroups;
    for (int m0 = 0; m0 < L.M; m0 += gsize) {
        const int m = std::min(gsize, L.M - m0);
        Gemv1Plan p;
        if (!plan_gemv1(L, m, &p)) return fail(ALV_ERR_ARG, "streaming GEMV: no plan for %d tokens", m);
        Gemv1Args a;
        if (int rc = fill_args(L, p, m0, m, s, &a)) return rc;
        const hipError_t e = launch_shape(a, L, p.sh, p.tg * p.ks, p.lds, s);
        if (int rc = hip_check(e, "q4_gemv1_kernel launch")) return rc;
        if (a.fix)
            if (int rc = hip_check(launch_fix(a, L.glu, p.sh.mt, s), "split_fix_kernel launch")) return rc;
    }
    return ALV_OK;
}


// LDS bytes of q4_ffn1_kernel at nss super-steps of the hidden size.
size_t ffn1_lds(int nss, int U, bool xb) {
    const int SRA = xb ? 1 : 3, USA = 16, SRB = 8, USB = 32;
    return (size_t)nss * 1024 * SRA + (size_t)8 * nss * USA * 16 + 16 + kFfn1Rows * 4 + 1024 * SRB +
           (size_t)U * USB * 16;
}

int launch_ffn1(const GemvLaunch& up, const uint8_t* Wv, uint64_t vbytes, float* part, uint16_t* act, int G, int U,
                int H, float* Y, uint16_t* Yb, hipStream_t s, bool sum) {
    if (up.step)
        if (int rc = check_step(up)) return rc;
    Gemv1Plan p;
    if (!plan_gemv1(up, 1, &p) || p.ks != 1) return fail(ALV_ERR_RANGE, "one-launch FFN: no one-token plan");
    Ffn1Args f{};
    if (int rc = fill_args(up, p, 0, 1, s, &f.gu)) return rc;
    const bool xb = up.Xb != nullptr;
    const size_t lds = ffn1_lds(f.gu.nss, U, xb);
    if (lds > dev_info().lds || 8 * f.gu.nss < 16 || vbytes >= 0xFFFFE000ull || G > kFfn1SumGroups * kFfn1SumLoads)
        return fail(ALV_ERR_RANGE, "one-launch FFN: shape outside the kernel's limits");
    f.Wv = Wv;
    f.vbytes = (uint32_t)vbytes;
    f.part = part;
    f.act = act;
    f.G = G;
    f.U = U;
    f.He = 128 * U;
    // The step's rows (128 + K floats) take phase B's region: 4 (128 + 128 U)
    // <= 8192 + 512 U bytes for every U, so the LDS size does not change.
    const int ki = up.step ? 2 : (xb ? 1 : 0);
    void (*k)(Ffn1Args) = ki == 2 ? q4_ffn1_kernel<kNW, 1, true, true>
                                  : (ki == 1 ? q4_ffn1_kernel<kNW, 1, true, false> : q4_ffn1_kernel<kNW, 3, false, false>);
    static std::atomic<int> set[3][64];
    if (int rc = hip_check(ensure_lds(reinterpret_cast<const void*>(k), set[ki], lds), "q4_ffn1_kernel LDS"))
        return rc;
    hipLaunchKernelGGL(k, dim3(G), dim3(64 * kNW), lds, s, f);
    if (int rc = hip_check(hipGetLastError(), "q4_ffn1_kernel launch")) return rc;
    if (!sum) return ALV_OK;
    hipLaunchKernelGGL(ffn1_sum_kernel, dim3((H + kFfn1SumRows - 1) / kFfn1SumRows), dim3(kFfn1SumRows * kFfn1SumGroups),
                       0, s, part, G, f.He, H, Y, Yb);
    return hip_check(hipGetLastError(), "ffn1_sum_kernel launch");
}
}  // namespace alv
