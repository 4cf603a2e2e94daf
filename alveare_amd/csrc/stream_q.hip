// Persistent op-chain executor for decode and small-M batches (gfx950): one
// launch runs a chain of up to kMaxOps matrix-vector ops -- a projection, or a
// gate/up pair with the GLU activation -- where an op may take its input from
// an earlier op of the chain. It is the kernel behind alv_chain_run with
// ALV_CHAIN_FUSED=1, and behind single ops whose shape the one-shot kernel
// (oneshot_q.hip) does not cover.
//
// Each op is computed the way the one-shot kernel computes it -- MFMA
// v_mfma_f32_16x16x32_bf16 with B = 16 weight rows x 32 k and A = the
// activation terms staged in LDS in operand order; a row tile's K range split
// over the waves of one slot of a workgroup, whose D tiles are added through
// LDS in a fixed order -- but the grid is resident for the whole chain (one
// workgroup of 8 waves per CU; a wave holds up to 4 units -- 80 VGPRs -- of
// loads in flight) and walks the ops in order:
//
//   for each op: wait for its input (if it reads an earlier op's output),
//                stage the activations in LDS,
//     for each round: compute the wave's units (their weights are already in
//                flight), issue the weight loads of the NEXT round or op, add
//                the slot's D tiles, write the outputs.
//
// Issuing the next op's weights as soon as a wave's compute is done keeps HBM
// busy across op boundaries: while the workgroup reduces, writes, signals and
// waits for the next op's input, those loads are already in flight -- the
// bubble a separate launch pays (drain, launch, ramp-up) is covered.
//
// Dependencies: a workgroup counts the row tiles it wrote into one of
// kSyncSlots words per op once its stores have landed (same-address device
// atomics serialise, so the counts are spread); a consumer's wave 0 polls the
// words with one sc1 load per lane and a wave sum. Outputs are written with
// agent-scope stores and a dependent op's activations read with sc1, so no
// L2-wide writeback or invalidate is needed. Every workgroup of the grid is
// resident (the grid is the occupancy), waits are bounded (a timeout sets a
// flag the host reads through alv_check_async), and the last workgroup past
// the chain's last wait resets the words for the next launch.
//
// Weights come either in the combined layout (RAW, one-op chains) or in the
// tiled layout (TILED, q4_device.h: every 16-byte load instruction of a wave
// reads 1 KiB of contiguous memory, nontemporal). Out-of-range loads (buffer
// resource bounds) return zero, which is how tails and idle waves are handled.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

constexpr int kExecThreads = 512;  // 8 waves: one workgroup per CU, 256 VGPRs per wave
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


// Output (token m, row jj) of matrix n of the slot whose waves start at w0:
// the sum over the slot's KW waves (in order) of the sum over the PARTS terms
// (in order) of D[m * PARTS + p][jj]. Straight-line: the loads of a batch of
// waves issue before their adds.
template <int PARTS, int KW>
__device__ __forceinline__ float slot_sum(const float* scr, int w0, int n, int NT, int m, int jj) {
    int off[PARTS];
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
        const int i = m * PARTS + p;
        off[p] = (jj + 16 * (i >> 2)) * 4 + (i & 3);
    }
    constexpr int C = KW < 4 ? KW : 4;
    float s = 0.0f;
#pragma unroll
    for (int k0 = 0; k0 < KW; k0 += C) {
        float v[C][PARTS];
#pragma unroll
        for (int k = 0; k < C; ++k)
#pragma unroll
            for (int p = 0; p < PARTS; ++p) v[k][p] = scr[((w0 + k0 + k) * NT + n) * 256 + off[p]];
#pragma unroll
        for (int k = 0; k < C; ++k) {
            float ws = v[k][0];
#pragma unroll
            for (int p = 1; p < PARTS; ++p) ws += v[k][p];
            s += ws;
        }
    }
    return s;
}

template <int PARTS>
__device__ __forceinline__ float slot_sum_kw(int kw, const float* scr, int w0, int n, int NT, int m, int jj) {
    switch (kw) {
        case 1: return slot_sum<PARTS, 1>(scr, w0, n, NT, m, jj);
        case 2: return slot_sum<PARTS, 2>(scr, w0, n, NT, m, jj);
        case 4: return slot_sum<PARTS, 4>(scr, w0, n, NT, m, jj);
        default: return slot_sum<PARTS, 8>(scr, w0, n, NT, m, jj);
    }
}

using UnitBuf = u32x4[4][5];  // [unit][16-byte piece]; unit k = matrix * spw + super-step of the wave

// The weight loads of one round of op d for wave kw of a slot on row tile rt:
// units k < NT * spw, unit k = super-step kw * spw + k % spw of matrix k / spw.
// One code path for every split (unit indices are static, the unit count is a
// uniform run-time bound), so one kernel runs every op of a chain. Tiled: lane
// l at 16 l of each 256 * ng-byte plane of the (row tile, super-step) tile.
// Combined: lane (j, g) reads the 80-byte run of row j at block 16 ss + 4 g.
// Loads of a missing row tile, super-step or unit start past the buffer and
// read zero.
template <bool TILED>
__device__ __forceinline__ void issue_round(UnitBuf& q, const OpDesc& d, int rt, int kw, int lane, bool valid) {
    const int j = lane & 15, g = lane >> 4;
    const int spw = d.spw, units = (d.glu ? 2 : 1) * spw;
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(d.W0, d.wbytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(d.glu ? d.W1 : d.W0, d.wbytes);
    // Every unit issues its five loads on every path (a unit past the op's
    // count reads past the buffer, i.e. zero): the number of loads in flight
    // is a compile-time constant, so the compiler's waits for each unit (and
    // for activations loaded before it) count exactly, and compute starts on
    // the first unit while the rest are still arriving.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int n = k >= spw ? 1 : 0;
        const int ss = kw * spw + (k - n * spw);
        const bool ok = valid && k < units && ss < d.nss;
        uint32_t off = d.wbytes, step = 16;
        if constexpr (TILED) {
            step = ss == d.nss - 1 ? 256u * (uint32_t)d.ng_last : 1024u;
            if (ok) off = (uint32_t)rt * d.rstride + (uint32_t)ss * 5120u + 16u * (uint32_t)lane;
        } else {
            const int row = rt * 16 + j;
            if (ok && row < d.N) off = (uint32_t)row * d.rstride + (uint32_t)(ss * 16 + g * 4) * kBlockBytes;
        }
        const __amdgpu_buffer_rsrc_t r = n ? r1 : r0;
#pragma unroll
        for (int i = 0; i < 5; ++i) q[k][i] = buf_load16_so<TILED>(r, off, step * i);
    }
}

// Dequantize + MFMA of one round's units into acc[matrix]. Blocks past the end
// of a row (combined: the next row's bytes; tiled: lanes past the last
// super-step's ng) get their scale cleared, so they dequantize to zero (their
// activations are zero too).
template <bool TILED>
__device__ __forceinline__ void compute_round(const UnitBuf& q, const OpDesc& d, const __bf16* xs, int kw, int lane,
                                              f32x4 (&acc)[2][2]) {
    const int j = lane & 15, g = lane >> 4;
    const int R = d.R;
    const int spw = d.spw, units = (d.glu ? 2 : 1) * spw;
    const __bf16* xa = xs + ((size_t)(kw * spw * 64 + g) * R + min(j, R - 1)) * 8;
    const int tstride = 4 * R * 8;  // bf16 elements between consecutive operand slots of a lane
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k >= units) break;  // uniform
        const int n = k >= spw ? 1 : 0;
        const int s = k - n * spw;
        const int ss = kw * spw + s;
        if (ss >= d.nss) continue;  // uniform
        const int nvalid = TILED ? (ss != d.nss - 1 || g < d.ng_last ? 4 : 0) : d.nb - (ss * 16 + g * 4);
        const __bf16* xk = xa + s * 16 * tstride;
#pragma unroll
        for (int bl = 0; bl < 4; ++bl) {
            uint32_t dw[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int w = 5 * bl + t;
                dw[t] = q[k][w >> 2][w & 3];
            }
            const int w4 = 5 * bl + 4;
            const Scale sc = make_scale(scale_of(bl < nvalid ? (uint32_t)q[k][w4 >> 2][w4 & 3] : 0u));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(xk + (bl * 4 + t) * tstride);
                const bf16x8 b = dequant8(dw[t], sc);
                if (n)
                    acc[1][t & 1] = mfma16x16x32(av, b, acc[1][t & 1]);
                else
                    acc[0][t & 1] = mfma16x16x32(av, b, acc[0][t & 1]);
            }
        }
    }
}

template <bool TILED>
__global__ void __launch_bounds__(kExecThreads) q4_exec_kernel(ExecArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __bf16* xs = reinterpret_cast<__bf16*>(smem);
    float* scr = reinterpret_cast<float*>(smem + a.xs_bytes);

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = gridDim.x;
    const int blk = blockIdx.x;

    auto rounds_of = [&](const OpDesc& d) { return d.nr_full + (blk < d.nr_rem ? 1 : 0); };

    // ---- activations of op d into LDS, in MFMA operand order ---------------------
    // Octet o8 (8 consecutive k) of token m: k = 8 o8. It lives at operand slot
    // ((o8 / 64) * 16 + o8 % 16) * 4 + (o8 / 16) % 4, i.e. super-step o8 / 64,
    // block 4g + bl with g = (o8 / 16) % 4, bl = (o8 / 4) % 4, dword t = o8 % 4:
    // slot = (ss * 16 + bl * 4 + t) * 4 + g. A dependent op's input was just
    // written through by other workgroups: those loads use sc1.
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
        // Two loads on every path (the second is out of range for bf16 input)
        // so that the count of loads in flight stays a compile-time constant.
        const uint32_t off1 = d.xb ? d.xbytes : off + 16;
        if (d.dep >= 0) {
            v[0] = buf_load16_sc1(rx, off);
            v[1] = buf_load16_sc1(rx, off1);
        } else {
            v[0] = buf_load16(rx, off);
            v[1] = buf_load16(rx, off1);
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
    auto stage = [&](const OpDesc& d) {
        const int units = d.nss * 64 * d.M;
        for (int u = tid; u < units; u += nthr) {
            u32x4 v[2];
            stage_load(d, u, v);
            stage_store(d, u, v);
        }
    };

    // ---- the weights of round r of op o for this wave -----------------------------
    UnitBuf q;
    auto issue = [&](int o, int r) {
        const OpDesc& d = a.op[o];
        const int rtl = wave >> d.kw_shift, kw = wave & ((1 << d.kw_shift) - 1);
        const int rt = (r * d.rtw + rtl) * G + blk;
        issue_round<TILED>(q, d, rt, kw, lane, rtl < d.rtw && rt < d.RT);
    };
    f32x4 acc[2][2];
    auto zero_acc = [&]() {
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[n][0] = acc[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    auto compute = [&](const OpDesc& d, int kw) { compute_round<TILED>(q, d, xs, kw, lane, acc); };

    // ---- counters: the last workgroup past the chain's last wait resets them -------
    // Two-level count (same-address atomics serialise): workgroup blk into slot
    // blk % kSyncSlots; the workgroup that completes its slot counts the slot
    // into one word; the one that completes that word is the last. By then
    // every workgroup has passed every wait, and every count of a row tile done
    // came before its workgroup's last wait (a producer precedes its consumer).
    // Called by wave 0, which issues this workgroup's counts: they complete
    // first, so the reset cannot be overtaken by one of them.
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

    // The round after (o, r) that this workgroup runs, or o = nops.
    auto next_round = [&](int& o, int& r) {
        if (++r < rounds_of(a.op[o])) return;
        r = 0;
        while (++o < a.nops && rounds_of(a.op[o]) == 0) {
        }
    };

    bool loaded = false;  // q holds the weights of the round about to run
    for (int o = 0; o < a.nops; ++o) {
        const OpDesc& d = a.op[o];
        const int nr = rounds_of(d);
        if (nr == 0) {
            if (o == a.last_wait && wave == 0) leave();
            continue;
        }
        const int NT = d.glu ? 2 : 1;
        const int KW = 1 << d.kw_shift;
        const int rtl = wave >> d.kw_shift, kw = wave & (KW - 1);
        const bool active = rtl < d.rtw;

        // ---- op boundary: wait for the input, stage it --------------------------------
        __syncthreads();  // the previous op is done with the LDS
        if (d.dep >= 0) {
            // Wave 0 polls the producer's spread counters: one sc1 load per
            // lane, summed across the wave.
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
                            __hip_atomic_store(&a.sync[kSyncError], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __syncthreads();
        }
        if (o == a.last_wait && wave == 0) leave();
        const int xunits = d.nss * 64 * d.M;
        if (!loaded && xunits <= 2 * nthr) {
            // No weights in flight yet: the activation loads go out first, the
            // weights right behind them, and the staging waits only for the
            // activations (loads complete in order).
            u32x4 xv[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) stage_load(d, min(tid + i * nthr, xunits), xv[i]);
            issue(o, 0);
            loaded = true;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (tid + i * nthr < xunits) stage_store(d, tid + i * nthr, xv[i]);
        } else {
            // Weights already in flight (issued during the previous op), or
            // more activations than registers hold: stage, then load.
            stage(d);
            if (!loaded) {
                issue(o, 0);
                loaded = true;
            }
        }
        __syncthreads();

        for (int r = 0; r < nr; ++r) {
            if (!loaded) issue(o, r);
            zero_acc();
            if (active) compute(d, kw);
            loaded = false;
            // The next round's (or op's) weights go out now, so they stream
            // while this round is reduced and written and the next input is
            // awaited. A wave that stores outputs a later op waits for issues
            // them after its signal: its wait for the stores would also wait
            // for them.
            int no = o, nrr = r;
            next_round(no, nrr);
            const bool last = r == nr - 1;
            const int outs = d.rtw * d.M * 16;
            const bool storer = wave * 64 < outs;
            const bool defer = storer && d.signal && last;
            if (no < a.nops && !defer) {
                issue(no, nrr);
                loaded = true;
            }
            // ---- add the slot's D tiles, write the outputs ------------------------
#pragma unroll
            for (int n = 0; n < 2; ++n)
                if (n < NT) *reinterpret_cast<f32x4*>(scr + (wave * NT + n) * 256 + lane * 4) = acc[n][0] + acc[n][1];
            __syncthreads();
            for (int idx = tid; idx < outs; idx += nthr) {
                const int per = d.M * 16;
                const int sl = idx / per, rem = idx - sl * per;
                const int m = rem >> 4, jj = rem & 15;
                const int rt = (r * d.rtw + sl) * G + blk;
                const int row = rt * 16 + jj;
                if (rt >= d.RT || row >= d.N) continue;
                float y[2] = {0.0f, 0.0f};
#pragma unroll
                for (int n = 0; n < 2; ++n)
                    if (n < NT)
                        y[n] = d.parts == 3 ? slot_sum_kw<3>(KW, scr, sl * KW, n, NT, m, jj)
                                            : slot_sum_kw<1>(KW, scr, sl * KW, n, NT, m, jj);
                // Final values, written through (a later op may read them).
                float out = y[0];
                if (d.glu) out = bf16_round(glu_exact(bf16_round(y[0]), bf16_round(y[1]), d.act));
                if (d.Yb)
                    __hip_atomic_store(&d.Yb[(size_t)m * d.ldy + row], __builtin_bit_cast(uint16_t, (__bf16)out),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    __hip_atomic_store(&d.Y[(size_t)m * d.ldy + row], out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (d.signal && last) {
                // The stores land before the workgroup counts its row tiles done.
                if (storer) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                if (tid == 0) {
                    uint32_t done = 0;
                    for (int rr = 0; rr < nr; ++rr)
                        for (int sl = 0; sl < d.rtw; ++sl) done += (rr * d.rtw + sl) * G + blk < d.RT ? 1u : 0u;
                    __hip_atomic_fetch_add(&a.sync[o * kSyncSlots + (blk & (kSyncSlots - 1))], done, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (no < a.nops && defer) {
                issue(no, nrr);
                loaded = true;
            }
            if (!last) __syncthreads();  // scratch reuse by the next round
        }
    }
}

// ---- host side -----------------------------------------------------------------

namespace {

template <bool TILED>
hipError_t launch_one(const ExecArgs& a, int G, size_t lds, hipStream_t s) {
    static size_t allowed = 64 * 1024;
    if (lds > allowed) {
        // Dynamic LDS above 64 KiB (gfx950 has 160 KiB per CU) is opted into
        // per kernel.
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&q4_exec_kernel<TILED>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        allowed = lds;
    }
    hipLaunchKernelGGL((q4_exec_kernel<TILED>), dim3(G), dim3(kExecThreads), lds, s, a);
    return hipGetLastError();
}

template <bool TILED>
int occupancy(size_t lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, q4_exec_kernel<TILED>, kExecThreads, lds) != hipSuccess)
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

// Work split of one op over G workgroups of 16 waves: super-steps per wave
// (spw), waves per row-tile slot (a power of two), slots per workgroup. The
// fewest rounds win (each round's loads all go out at once); on a tie the
// smaller spw (more waves, fewer registers held). False when K is too long.
bool plan_op(OpDesc& d, int G) {
    const int NT = d.glu ? 2 : 1;
    int best_rounds = 0;
    bool found = false;
    for (int spw : {1, 2, 4}) {
        if (spw * NT > 4) break;
        const int kw = (d.nss + spw - 1) / spw;
        if (kw > kWPB) continue;
        int KW = 1;
        while (KW < kw) KW *= 2;
        const int rtw = kWPB / KW;
        const long per_round = (long)G * rtw;
        const int rounds = (int)((d.RT + per_round - 1) / per_round);
        if (!found || rounds < best_rounds) {
            found = true;
            best_rounds = rounds;
            d.spw = spw;
            d.kw_shift = __builtin_ctz(KW);
            d.rtw = rtw;
            d.nr_full = (int)(d.RT / per_round);
            d.nr_rem = (int)(d.RT % per_round);
        }
    }
    return found;
}

int launch_chunk(const ExecOp* ops, int nops, bool tiled, int m0, int M, hipStream_t s) {
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
        d.act = L.act;
        d.glu = L.glu ? 1 : 0;
        d.xb = L.Xb != nullptr;
        d.dep = L.dep;
        d.signal = 0;
        any_dep |= L.dep >= 0;
        xs_bytes = std::max(xs_bytes, (size_t)tg.nss * 1024 * d.R);
    }
    a.last_wait = -1;
    for (int o = 0; o < nops; ++o)
        if (a.op[o].dep >= 0) {
            a.op[a.op[o].dep].signal = 1;
            a.last_wait = o;
        }
    const size_t lds = xs_bytes + kScratchBytes;
    const int per_cu = tiled ? occupancy<true>(lds) : occupancy<false>(lds);
    if (per_cu < 1) return fail(ALV_ERR_HIP, "the executor kernel does not fit a CU with %zu bytes of LDS", lds);
    // Every workgroup of a chain must be resident at once (its waits rely on it).
    const int G = per_cu * dev_info().cus;
    for (int o = 0; o < nops; ++o)
        if (!plan_op(a.op[o], G))
            return fail(ALV_ERR_RANGE, "op %d: K=%d is beyond what the executor splits over one workgroup", o, a.op[o].K);
    Workspace ws;
    if (int rc = get_workspace(s, kSyncWords, &ws)) return rc;
    a.sync = ws.counters;
    a.xs_bytes = (uint32_t)xs_bytes;
    // Waits poll with s_sleep; 2^24 polls is far beyond any chain's run time.
    a.spin_limit = any_dep ? (1u << 24) : 0u;
    const hipError_t e = tiled ? launch_one<true>(a, G, lds, s) : launch_one<false>(a, G, lds, s);
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
