// Streaming Q4 executor for decode and small-M batches (gfx950): one launch
// runs a chain of up to kMaxOps matrix-vector ops -- a projection, or a
// gate/up pair with the GLU activation -- where an op may take its input from
// an earlier op of the chain: the kernel behind alv_chain_run, and behind
// single ops whose shape the one-shot kernel (oneshot_q.hip) does not cover.
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
// LDS, where the workgroup staged the whole K range in MFMA operand order.
//
// Work split: one workgroup of 16 waves per CU (the grid is exactly the
// resident capacity). A row tile's work is U units -- one super-step of one
// matrix (gate and up are separate units of a gate/up op) -- split evenly over
// a group of 16 / r waves; the r groups of a workgroup take different row
// tiles. Each round every group finishes one row tile: the waves leave their
// partial D tiles in LDS, and after a barrier the workgroup sums them per
// output in a fixed order (waves, then terms) and writes the outputs. No
// partial sum leaves the workgroup, so results do not depend on scheduling
// and no global-memory handshake sits inside an op.
//
// Streaming: every wave walks one sequence of steps across all ops of the
// chain and keeps the weight loads of the next P steps in flight while it
// computes the current one -- also across op boundaries, so the next op's
// weights stream in while the current op drains and while a workgroup waits
// for its input. The ring is unrolled (each op's step count per wave is padded
// to a multiple of P + 1), so every buffer index is static; all waves of a
// workgroup run the same number of steps per round, so every barrier is the
// same instruction for all of them.
//
// Dependencies: an op whose input is an earlier op's output waits, per
// workgroup, until every row tile of that op has been written. Outputs go
// through the device-coherent level (agent-scope stores), activation staging
// of a dependent op reads with sc1, so no L2-wide writeback or invalidate is
// needed. Waits are bounded (a timeout sets a flag the host reads through
// alv_check_async) and the last workgroup to leave resets the counters for the
// next launch.
//
// Weights come either in the combined layout (RAW, one-op chains: a lane's
// 80-byte run is contiguous, a wave's 16-byte loads touch 16 rows x 4 runs and
// lean on the caches to merge) or in the tiled layout (TILED, q4_device.h:
// every load instruction of a wave reads 1 KiB of contiguous memory, with the
// nontemporal hint since weights are read once). Out-of-range loads (buffer
// resource bounds) return zero, which is how tails and empty steps are handled.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

constexpr int kExecThreads = 1024;           // 16 waves: one workgroup per CU
constexpr int kWPB = kExecThreads / 64;
constexpr size_t kScratchBytes = kWPB * 2 * 1024;  // per wave: one 16x16 fp32 D tile per matrix

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

// Steps of one wave in one op (wave-uniform). Round i: the wave's group works
// on row tile worker0 + i * wstride; step k of the round is unit u0 + k when
// k < nu (steps nu..numax-1 are empty, so every wave of the workgroup runs
// numax steps per round).
struct WavePlan {
    int worker0, wstride;
    int u0, nu, numax;
    int nrounds;           // rounds of this workgroup (those of its group 0)
    int steps, steps_pad;  // nrounds * numax, padded to a multiple of the ring size
};

// No divisions: the scalar unit is shared by the CU's 16 waves, so per-op
// set-up work is kept to shifts and the host precomputes the rest.
template <int NB>
__device__ __forceinline__ WavePlan wave_plan(const OpDesc& d, int b, int G, int wave) {
    WavePlan p;
    const int q = wave >> d.gw_shift, wi = wave & ((1 << d.gw_shift) - 1);
    p.worker0 = q * G + b;
    p.wstride = d.wstride;
    p.u0 = (wi * d.U) >> d.gw_shift;
    p.nu = (((wi + 1) * d.U) >> d.gw_shift) - p.u0;
    p.numax = d.numax;
    p.nrounds = d.nr_full + (b < d.nr_rem ? 1 : 0);
    p.steps = p.nrounds * p.numax;
    p.steps_pad = (p.steps + NB - 1) / NB * NB;
    return p;
}

// Output (token m, row jj) of matrix n of group q, from the D tiles the
// group's GW waves left in LDS: the sum over the waves (in order) of the sum
// over the PARTS terms (in order) of D[m * PARTS + p][jj]. Straight-line code:
// every load issues before the first add.
template <int PARTS, int GW>
__device__ __forceinline__ float group_sum(const float* scr, int q, int n, int NT, int m, int jj) {
    int off[PARTS];
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
        const int i = m * PARTS + p;
        off[p] = (jj + 16 * (i >> 2)) * 4 + (i & 3);
    }
    constexpr int C = GW < 4 ? GW : 4;  // waves per batch of loads (bounds the registers held)
    float s = 0.0f;
#pragma unroll
    for (int w0 = 0; w0 < GW; w0 += C) {
        float v[C][PARTS];
#pragma unroll
        for (int w = 0; w < C; ++w)
#pragma unroll
            for (int p = 0; p < PARTS; ++p) v[w][p] = scr[((q * GW + w0 + w) * NT + n) * 256 + off[p]];
#pragma unroll
        for (int w = 0; w < C; ++w) {
            float ws = v[w][0];
#pragma unroll
            for (int p = 1; p < PARTS; ++p) ws += v[w][p];
            s += ws;
        }
    }
    return s;
}

template <int PARTS>
__device__ __forceinline__ float group_sum_gw(int gw, const float* scr, int q, int n, int NT, int m, int jj) {
    switch (gw) {
        case 1: return group_sum<PARTS, 1>(scr, q, n, NT, m, jj);
        case 2: return group_sum<PARTS, 2>(scr, q, n, NT, m, jj);
        case 4: return group_sum<PARTS, 4>(scr, q, n, NT, m, jj);
        case 8: return group_sum<PARTS, 8>(scr, q, n, NT, m, jj);
        default: return group_sum<PARTS, 16>(scr, q, n, NT, m, jj);
    }
}

// P: steps of prefetch.
template <int P, bool TILED>
__global__ void __launch_bounds__(kExecThreads) q4_exec_kernel(ExecArgs a) {
    constexpr int NB = P + 1;
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);
    float* scr = reinterpret_cast<float*>(smem + a.xs_bytes);

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = gridDim.x;
    const int blk = blockIdx.x;
    const int j = lane & 15;
    const int g = lane >> 4;

    // ---- weight loads of one step ----------------------------------------------
    // Lane offset (fixed) + step offset (wave-uniform, in soffset). An empty
    // step starts at wbytes: every piece is out of range and reads zero.
    // Combined layout (one-op chains): lane (j, g) sits at row j, byte 80 g of
    // the super-step; rows past N fall past wbytes. Tiled layout: lane l at
    // 16 l of each plane.
    const uint32_t voff = TILED ? 16u * (uint32_t)lane : (uint32_t)j * a.op[0].rstride + 80u * (uint32_t)g;
    // The stream parameters of the op the prefetch cursor is in, copied once
    // per op (kernel-argument loads are slow to come back and share a counter
    // with LDS reads).
    struct StreamOp {
        const uint8_t* W0;
        const uint8_t* W1;
        uint32_t wbytes, rstride;
        int nss, ng_last, RT;
    };
    auto stream_op = [&](int o) {
        const OpDesc& d = a.op[o];
        return StreamOp{d.W0, d.W1, d.wbytes, d.rstride, d.nss, d.ng_last, d.RT};
    };
    auto issue = [&](u32x4 (&q)[5], const StreamOp& d, int rt, int n, int ss, bool valid) {
        uint32_t soff = d.wbytes, step = 16;
        if constexpr (TILED) {
            step = ss == d.nss - 1 ? 256u * (uint32_t)d.ng_last : 1024u;
            if (valid) soff = (uint32_t)rt * d.rstride + (uint32_t)ss * 5120u;
        } else {
            if (valid) soff = (uint32_t)rt * 16u * d.rstride + (uint32_t)ss * 320u;
        }
        const __amdgpu_buffer_rsrc_t r = make_rsrc(n ? d.W1 : d.W0, d.wbytes);
#pragma unroll
        for (int i = 0; i < 5; ++i) q[i] = buf_load16_so<TILED>(r, voff, soff + step * i);
    };

    // ---- activation staging ------------------------------------------------------
    // Octet o8 (8 consecutive k) of token m: k = 8 o8. It lives at operand slot
    // ((o8 / 64) * 16 + o8 % 16) * 4 + (o8 / 16) % 4, i.e. super-step o8 / 64,
    // block 4g + bl with g = (o8 / 16) % 4, bl = (o8 / 4) % 4, dword t = o8 % 4:
    // slot = (ss * 16 + bl * 4 + t) * 4 + g. Staging unit u = m * octs + o8.
    // A dependent op's input was just written through by other workgroups:
    // those loads use sc1.
    auto stage_load = [&](const OpDesc& d, int u, u32x4 (&v)[2]) {
        const int ES = d.xb ? 2 : 4;
        const int octs = d.nss * 64;
        int m = 0, o8 = u;
        if (d.M != 1) {
            m = u / octs;
            o8 = u - m * octs;
        }
        const int k = o8 * 8;
        const uint32_t off = k < d.K && m < d.M ? (uint32_t)((m * d.ldx + k) * ES) : d.xbytes;
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(d.X, d.xbytes);
        if (d.dep >= 0) {
            v[0] = buf_load16_sc1(rx, off);
            v[1] = d.xb ? u32x4{0u, 0u, 0u, 0u} : buf_load16_sc1(rx, off + 16);
        } else {
            v[0] = buf_load16(rx, off);
            v[1] = d.xb ? u32x4{0u, 0u, 0u, 0u} : buf_load16(rx, off + 16);
        }
    };
    auto stage_store = [&](const OpDesc& d, int u, const u32x4 (&v)[2]) {
        const int octs = d.nss * 64;
        int m = 0, o8 = u;
        if (d.M != 1) {
            m = u / octs;
            o8 = u - m * octs;
        }
        const int slot = ((o8 >> 6) * 16 + (o8 & 15)) * 4 + ((o8 >> 4) & 3);
        __bf16* dst = xs + ((size_t)slot * d.R + (size_t)m * d.parts) * 8;
        if (d.xb)
            stage_octet<true>(v, dst, 1);
        else
            stage_octet<false>(v, dst, d.parts);
    };
    auto stage_all = [&](const OpDesc& d) {
        const int units = d.nss * 64 * d.M;
        for (int u = tid; u < units; u += nthr) {
            u32x4 v[2];
            stage_load(d, u, v);
            stage_store(d, u, v);
        }
    };
    // The first op's activations are staged before any weight load is issued:
    // issued together, the small activation reads queue behind the weight
    // stream (~3 us at full load) and every wave waits for them.
    const OpDesc& d0 = a.op[0];
    const int units0 = d0.nss * 64 * d0.M;
    const bool reg_stage = (a.flags & 1) && units0 <= 2 * nthr;
    u32x4 xv[2][2];
    if (reg_stage) {
#pragma unroll
        for (int i = 0; i < 2; ++i) stage_load(d0, min(tid + i * nthr, units0), xv[i]);
    } else {
        stage_all(d0);
    }

    // Prefetch cursor: op po, step pstep of this wave in that op, round pround,
    // step pk within the round.
    u32x4 buf[NB][5];
    int po = 0, pstep = 0, pround = 0, pk = 0;
    WavePlan pp = wave_plan<NB>(a.op[0], blk, G, wave);
    StreamOp ps = stream_op(0);
    auto skip_empty_ops = [&]() {
        while (po < a.nops && pstep >= pp.steps_pad) {
            if (++po < a.nops) {
                pp = wave_plan<NB>(a.op[po], blk, G, wave);
                ps = stream_op(po);
                pstep = pround = pk = 0;
            }
        }
    };
    skip_empty_ops();
    auto issue_next = [&](u32x4 (&q)[5]) {
        int rt = 0, n = 0, ss = 0;
        bool valid = false;
        if (po < a.nops) {
            rt = pp.worker0 + pround * pp.wstride;
            const int u = pp.u0 + pk;
            valid = pstep < pp.steps && pk < pp.nu && rt < ps.RT;
            n = u >= ps.nss ? 1 : 0;
            ss = u - n * ps.nss;
        }
        issue(q, ps, rt, n, ss, valid);
        if (po < a.nops) {
            ++pstep;
            if (++pk == pp.numax) {
                pk = 0;
                ++pround;
            }
            skip_empty_ops();
        }
    };
#pragma unroll
    for (int b = 0; b < P; ++b) issue_next(buf[b]);
    if (reg_stage) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (tid + i * nthr < units0) stage_store(d0, tid + i * nthr, xv[i]);
    }

    // ---- counters: the last workgroup past the chain's last wait resets them -------
    // Two-level count (same-address atomics serialise): workgroup blk into slot
    // blk % kSyncSlots; the workgroup that completes its slot counts the slot
    // into one word; the one that completes that word is the last. By then
    // every workgroup has passed every wait, and every count of a row tile done
    // came before its workgroup's last wait (a producer precedes its
    // consumer). Called by wave 0, which issued this workgroup's counts: they
    // complete first, so the reset cannot be overtaken by one of them.
    auto leave = [&]() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t last = 0;
        if (lane == 0) {
            const int slot = blk & (kSyncSlots - 1);
            const uint32_t in_slot = (uint32_t)(G / kSyncSlots + (slot < G % kSyncSlots ? 1 : 0));
            const uint32_t slots = (uint32_t)min(G, kSyncSlots);
            if (__hip_atomic_fetch_add(&a.sync[kSyncExit1 + slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                in_slot - 1)
                last = __hip_atomic_fetch_add(&a.sync[kSyncExit2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       slots - 1;
        }
        if (__builtin_amdgcn_readfirstlane(last)) {
            for (int i = lane; i < a.nops * kSyncSlots; i += 64)
                __hip_atomic_store(&a.sync[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int i = lane; i <= kSyncSlots; i += 64)
                __hip_atomic_store(&a.sync[kSyncExit1 + i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };

    f32x4 acc[2][2];
    auto zero_acc = [&]() {
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[n][0] = acc[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    for (int o = 0; o < a.nops; ++o) {
        const OpDesc& d = a.op[o];
        const WavePlan cp = wave_plan<NB>(d, blk, G, wave);
        const int R = d.R;
        const int NT = d.glu ? 2 : 1;

        // ---- op boundary: wait for the input, stage the activations -----------
        if (o > 0) {
            __syncthreads();  // every wave is done with the previous op's operands
            if (cp.nrounds > 0) {
                if (d.dep >= 0) {
                    // Wave 0 polls the producer's spread counters: one sc1 load
                    // per lane, summed across the wave.
                    if (wave == 0) {
                        const uint32_t target = (uint32_t)a.op[d.dep].RT;
                        uint32_t n = 0;
                        while (true) {
                            uint32_t v = __hip_atomic_load(&a.sync[d.dep * kSyncSlots + lane], __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
                            if (v >= target) break;
                            __builtin_amdgcn_s_sleep(2);
                            if (++n > a.spin_limit) {
                                if (lane == 0)
                                    __hip_atomic_store(&a.sync[kSyncError], 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                                break;
                            }
                        }
                    }
                    __syncthreads();
                }
                stage_all(d);
            }
            if (o == a.last_wait && wave == 0) leave();
        }
        __syncthreads();

        // ---- stream this op's steps ------------------------------------------------
        const __bf16* xa = xs + ((size_t)g * R + min(j, R - 1)) * 8;  // operand base: slot g, row j

        // One unit: super-step ss of one matrix, into ac.
        auto compute_into = [&](const u32x4 (&q)[5], int ss, f32x4 (&ac)[2]) {
            const int sl_off = ss * 64 * R * 8;  // this super-step's operands (bf16 elements)
            // Blocks of this lane that exist. Tiled: a lane past the last
            // super-step's ng reads the next plane's bytes; combined: blocks
            // past the row end read the next row's. Their scales are cleared
            // (their activations are zero), so they dequantize to zero.
            const int nvalid = TILED ? (ss != d.nss - 1 || g < d.ng_last ? 4 : 0) : d.nb - (ss * 16 + g * 4);
#pragma unroll
            for (int bl = 0; bl < 4; ++bl) {
                // dwords 5*bl .. 5*bl+4 of the 80-byte run are this block.
                uint32_t dw[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int w = 5 * bl + t;
                    dw[t] = q[w >> 2][w & 3];
                }
                const int w4 = 5 * bl + 4;
                const uint32_t sd = bl < nvalid ? (uint32_t)q[w4 >> 2][w4 & 3] : 0u;
                const Scale sc = make_scale(scale_of(sd));
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int so = sl_off + (bl * 4 + t) * 4 * R * 8;
                    const bf16x8 b = dequant8(dw[t], sc);
                    const bf16x8 av = *reinterpret_cast<const bf16x8*>(xa + so);
                    ac[t & 1] = mfma16x16x32(av, b, ac[t & 1]);
                }
            }
        };

        // End of a round: the waves' D tiles go to LDS; output (group q, token
        // m, row jj) = sum over the group's waves (in order) of the sum over
        // terms p (in order) of D[m * parts + p][jj].
        const int gw = 1 << d.gw_shift;
        auto round_end = [&](int round) {
#pragma unroll
            for (int n = 0; n < 2; ++n)
                if (n < NT)
                    *reinterpret_cast<f32x4*>(scr + (wave * NT + n) * 256 + lane * 4) = acc[n][0] + acc[n][1];
            zero_acc();
            __syncthreads();
            const int per_group = d.M * 16;
            const bool last = round == cp.nrounds - 1;
            for (int idx = tid; idx < d.r * per_group; idx += nthr) {
                const int q = idx / per_group, rem = idx - q * per_group;
                const int m = rem >> 4, jj = rem & 15;
                const int rt = q * G + blk + round * cp.wstride;
                const int row = rt * 16 + jj;
                if (rt >= d.RT || row >= d.N) continue;
                float y[2] = {0.0f, 0.0f};
#pragma unroll
                for (int n = 0; n < 2; ++n)
                    if (n < NT)
                        y[n] = d.parts == 3 ? group_sum_gw<3>(gw, scr, q, n, NT, m, jj)
                                            : group_sum_gw<1>(gw, scr, q, n, NT, m, jj);
                // Final values, written through (a later op may read them).
                float out = y[0];
                if (d.glu) out = bf16_round(glu_act(bf16_round(y[0]), bf16_round(y[1]), d.act));
                if (d.Yb)
                    __hip_atomic_store(&d.Yb[(size_t)m * d.ldy + row], __builtin_bit_cast(uint16_t, (__bf16)out),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    __hip_atomic_store(&d.Y[(size_t)m * d.ldy + row], out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // A later op reads this one: after the last round, the stores land
            // before the workgroup counts its row tiles done. Only the waves
            // that stored wait (the others keep their prefetch in flight).
            if (d.signal && last && wave * 64 < d.r * per_group) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (d.signal && last && tid == 0) {
                uint32_t done = 0;
                for (int q = 0; q < d.r; ++q)
                    for (int i = 0; i < cp.nrounds; ++i) done += q * G + blk + i * cp.wstride < d.RT ? 1u : 0u;
                __hip_atomic_fetch_add(&a.sync[o * kSyncSlots + (blk & (kSyncSlots - 1))], done, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        };

        zero_acc();
        int cround = 0, ck = 0;  // compute cursor
        for (int s0 = 0; s0 < cp.steps_pad; s0 += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                issue_next(buf[(b + P) % NB]);
                if (s0 + b < cp.steps) {  // workgroup-uniform
                    const int rt = cp.worker0 + cround * cp.wstride;
                    if (ck < cp.nu && rt < d.RT) {  // wave-uniform
                        const int u = cp.u0 + ck;
                        if (u >= d.nss)
                            compute_into(buf[b], u - d.nss, acc[1]);
                        else
                            compute_into(buf[b], u, acc[0]);
                    }
                    if (++ck == cp.numax) {
                        round_end(cround);
                        ck = 0;
                        ++cround;
                    }
                }
            }
        }
    }
}

// ---- host side -----------------------------------------------------------------

namespace {

template <int P, bool TILED>
hipError_t launch_one(const ExecArgs& a, int G, size_t lds, hipStream_t s) {
    static size_t allowed = 64 * 1024;
    if (lds > allowed) {
        // Dynamic LDS above 64 KiB (gfx950 has 160 KiB per CU) is opted into
        // per kernel.
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&q4_exec_kernel<P, TILED>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        allowed = lds;
    }
    hipLaunchKernelGGL((q4_exec_kernel<P, TILED>), dim3(G), dim3(kExecThreads), lds, s, a);
    return hipGetLastError();
}

template <int P, bool TILED>
int occupancy(size_t lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, q4_exec_kernel<P, TILED>, kExecThreads, lds) != hipSuccess)
        return 0;
    return nb;
}

struct DevInfo {
    int cus = 0;
    size_t lds = 0;
};

DevInfo dev_info() {
    static DevInfo info[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DevInfo{256, 64 * 1024};
    DevInfo& d = info[dev];
    if (!d.cus) {
        int n = 0, l = 0;
        d.lds = hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && l > 0
                    ? (size_t)l
                    : 64 * 1024;
        d.cus = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return d;
}

// Prefetch depth: P = 1 (one step in flight per wave while it computes
// another: 16 waves x 5 KiB per CU cover the HBM latency-bandwidth product, and
// the 128-VGPR budget of 16 waves per CU holds P = 1 without spills) unless
// overridden (tuning: ALV_EXEC_P=1|2).
int prefetch_depth() {
    static int p = 0;
    if (!p) {
        p = 1;
        if (const char* e = getenv("ALV_EXEC_P")) {
            const int v = atoi(e);
            if (v == 1 || v == 2) p = v;
        }
    }
    return p;
}

// Wave groups per workgroup (a power of two dividing the 16 waves): enough
// groups that one round covers every row tile (fewer rounds, fewer barriers;
// each wave then streams several units of its row tile), and at least as many
// as keep every wave busy with one unit.
int groups_for(int U, int RT, int G) {
    int r = 1;
    while (r < kWPB && U * r * 2 <= kWPB) r *= 2;
    while (r < kWPB && (long)G * r < RT) r *= 2;
    return r;
}

int launch_chunk(const ExecOp* ops, int nops, bool tiled, int m0, int M, hipStream_t s) {
    const int P = prefetch_depth();
    ExecArgs a{};
    a.nops = nops;
    size_t xs_bytes = 0;
    bool any_dep = false;
    for (int o = 0; o < nops; ++o) {
        const ExecOp& L = ops[o];
        const TileGeom tg = tile_geom(L.K);
        const int RT = (L.N + 15) / 16;
        OpDesc& d = a.op[o];
        const uint64_t rs = (uint64_t)tg.nb * kBlockBytes;
        const uint64_t wbytes = tiled ? (uint64_t)RT * tg.rtb : (uint64_t)L.N * rs;
        if (wbytes >= 0xFFFFE000ull)
            return fail(ALV_ERR_RANGE, "weight matrix of %llu bytes exceeds the 4 GiB buffer range", (unsigned long long)wbytes);
        const uint64_t xbytes = ((uint64_t)(M - 1) * L.ldx + L.K) * (L.Xb ? 2 : 4);
        if (xbytes >= 0x7FFFFF00ull) return fail(ALV_ERR_RANGE, "activation buffer exceeds the 2 GiB range");
        d.W0 = L.W0;
        d.W1 = L.W1;
        d.X = L.Xb ? (const void*)(L.Xb + (size_t)m0 * L.ldx) : (const void*)(L.X + (size_t)m0 * L.ldx);
        d.Y = L.Y ? L.Y + (size_t)m0 * L.ldy : nullptr;
        d.Yb = L.Yb ? L.Yb + (size_t)m0 * L.ldy : nullptr;
        d.wbytes = (uint32_t)wbytes;
        d.xbytes = (uint32_t)xbytes;
        d.rstride = tiled ? tg.rtb : (uint32_t)rs;
        d.ldx = L.ldx;
        d.ldy = L.ldy;
        d.M = M;
        d.N = L.N;
        d.K = L.K;
        d.parts = L.parts;
        d.R = L.parts * M;
        d.nb = tg.nb;
        d.nss = tg.nss;
        d.ng_last = tg.ng_last;
        d.RT = RT;
        d.U = tg.nss * (L.glu ? 2 : 1);
        d.act = L.act;
        d.glu = L.glu ? 1 : 0;
        d.xb = L.Xb != nullptr;
        d.dep = L.dep;
        d.signal = 0;
        any_dep |= L.dep >= 0;
        xs_bytes = std::max(xs_bytes, (size_t)tg.nss * 1024 * d.R);
    }
    a.last_wait = -1;
    a.flags = getenv("ALV_EXEC_FLAGS") ? atoi(getenv("ALV_EXEC_FLAGS")) : 0;
    for (int o = 0; o < nops; ++o)
        if (a.op[o].dep >= 0) {
            a.op[a.op[o].dep].signal = 1;
            a.last_wait = o;
        }
    const size_t lds = xs_bytes + kScratchBytes;
    const int per_cu = tiled ? (P == 1 ? occupancy<1, true>(lds) : occupancy<2, true>(lds))
                             : (P == 1 ? occupancy<1, false>(lds) : occupancy<2, false>(lds));
    if (per_cu < 1) return fail(ALV_ERR_HIP, "the executor kernel does not fit a CU with %zu bytes of LDS", lds);
    // Every workgroup of a chain must be resident at once (its waits rely on it).
    const int G = per_cu * dev_info().cus;
    for (int o = 0; o < nops; ++o) {
        OpDesc& d = a.op[o];
        d.r = groups_for(d.U, d.RT, G);
        const int gw = kWPB / d.r;
        d.gw_shift = __builtin_ctz(gw);
        d.numax = (d.U + gw - 1) / gw;
        d.wstride = G * d.r;
        d.nr_full = d.RT / d.wstride;
        d.nr_rem = d.RT % d.wstride;
    }
    Workspace ws;
    if (int rc = get_workspace(s, kSyncWords, &ws)) return rc;
    a.sync = ws.counters;
    a.xs_bytes = (uint32_t)xs_bytes;
    // Waits poll with s_sleep; 2^24 polls is far beyond any chain's run time.
    a.spin_limit = any_dep ? (1u << 24) : 0u;
    const hipError_t e = tiled ? (P == 1 ? launch_one<1, true>(a, G, lds, s) : launch_one<2, true>(a, G, lds, s))
                               : (P == 1 ? launch_one<1, false>(a, G, lds, s) : launch_one<2, false>(a, G, lds, s));
    return hip_check(e, "q4_exec_kernel launch");
}

}  // namespace

int exec_chain(const ExecOp* ops, int nops, bool tiled, hipStream_t s) {
    if (nops < 1 || nops > kMaxOps) return fail(ALV_ERR_ARG, "a chain holds 1..%d ops (got %d)", kMaxOps, nops);
    if (!tiled && nops != 1) return fail(ALV_ERR_ARG, "combined-layout weights run as one-op chains");
    const int M = ops[0].M;
    for (int o = 0; o < nops; ++o) {
        const ExecOp& L = ops[o];
        if (L.M != M) return fail(ALV_ERR_ARG, "ops of a chain share the token count");
        if (L.M < 1 || L.M > kGemvMaxM) return fail(ALV_ERR_ARG, "stream kernel takes 1 <= M <= %d (got %d)", kGemvMaxM, L.M);
        if (L.parts != 1 && L.parts != 3) return fail(ALV_ERR_ARG, "parts must be 1 or 3");
        if (L.Xb && (L.parts != 1 || L.glu)) return fail(ALV_ERR_ARG, "bf16 activations take one term and no GLU");
        if (L.dep >= o) return fail(ALV_ERR_ARG, "op %d depends on op %d, not an earlier one", o, L.dep);
    }
    // Tokens per launch: the A operand holds 16 rows (parts * tokens) and every
    // op's whole K range, for every token, is staged in LDS next to the
    // reduction scratch.
    const size_t lds_max = std::min<size_t>(dev_info().lds, 160 * 1024);
    int mc = M;
    for (int o = 0; o < nops; ++o) {
        const size_t per_token = (size_t)tile_geom(ops[o].K).nss * 1024 * ops[o].parts;
        const size_t fixed = kScratchBytes + 256;  // reduction scratch + static LDS
        const int fit = lds_max > fixed ? (int)((lds_max - fixed) / per_token) : 0;
        mc = std::min(mc, std::min(16 / ops[o].parts, fit));
    }
    if (mc < 1) return fail(ALV_ERR_RANGE, "K is too large for the executor's LDS staging");
    for (int m0 = 0; m0 < M; m0 += mc)
        if (int rc = launch_chunk(ops, nops, tiled, m0, std::min(mc, M - m0), s)) return rc;
    return ALV_OK;
}

int check_async(hipStream_t s) {
    if (int rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize")) return rc;
    Workspace ws;
    if (int rc = get_workspace(s, kSyncWords, &ws)) return rc;
    uint32_t flag = 0;
    if (int rc = hip_check(hipMemcpy(&flag, ws.counters + kSyncError, sizeof(flag), hipMemcpyDeviceToHost), "hipMemcpy")) return rc;
    if (!flag) return ALV_OK;
    const uint32_t zero = 0;
    (void)hipMemcpy(ws.counters + kSyncError, &zero, sizeof(zero), hipMemcpyHostToDevice);
    return fail(ALV_ERR_HIP, "a chained op timed out waiting for its input (not every workgroup was resident)");
}

}  // namespace alv
