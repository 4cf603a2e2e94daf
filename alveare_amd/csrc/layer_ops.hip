// Host ops of a decode layer on gfx950: the work the reference runs on the
// CPU between its NPU matmuls (runtime/py/model.py:522-628, :705-790;
// runtime/cpp/src/model.cpp:127-262, :314-420).
//
//   alv_rmsnorm      rows of bf16 -> bf16(x / sqrt(mean(x^2) + eps) * w)
//   alv_qkv_post     per-head q/k/v norms, RoPE of q and k, K/V cache insert
//   alv_attention    one token's attention over the cache (GQA, optional
//                    sliding window), float32 softmax, bf16 out
//   alv_add_norm     residual add of a (normalised) branch, output scale, and
//                    the next norm, in one pass
//   alv_embed        token embedding row (fp16 table) scaled to bf16, the token
//                    read from device memory
//
// Bit-exact parts. The reference computes with numpy in float32 on bf16
// arrays. Every elementwise step here is the same float32 operation with the
// same rounding (floating-point contraction is off in this file: nothing
// fuses a product and a sum into one FMA), and the one reduction whose order matters at
// bf16 output precision -- np.mean(x ** 2) of RMSNorm -- is numpy's own
// summation order (row_norm.h).
//
// Attention is not bit-exact: the reference's scores and weighted sums are
// BLAS dot products (np.dot) whose order is the library's. Here the positions
// are split into chunks of 64: a workgroup per (chunk, kv head, group of up
// to 4 q heads) writes the chunk's max, exp-sum and weighted V sum to the
// stream's scratch, and a second launch merges the chunks of every (head,
// column) in chunk order (deterministic).
//
// Row kernels run 256 threads per row: 16-byte loads and stores, and the
// pairwise sum with 8 lanes per leaf (lane j holds the leaf's accumulator
// r[j]; three xor shuffles combine them in numpy's order).
//
// Decode position `pos` is read from device memory (pos_dev), so a captured
// graph replays for every token; positions at or past the cache length write
// nothing and leave the outputs unchanged.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "q4_device.h"
#include "q4_host.h"
#include "row_norm.h"

#pragma clang fp contract(off)


namespace alv {

namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxRowK = 32768;  // 128 KiB of float32 row in LDS

// Rows of up to 8 * kRegOct * kRowThreads values (4096: every hidden size of
// the reference's models) keep their octets in registers, thread t holding
// octets t and t + kRowThreads, and issue every load of the row -- values,
// residual, norm weights -- before the first wait: one memory round trip per
// kernel instead of one per step.
constexpr int kRegOct = 2;

__device__ __forceinline__ bool reg_row(int K, int pad) {
    return K % 8 == 0 && pad % 8 == 0 && pad <= 8 * kRegOct * kRowThreads;
}

// xs[0, K) = float(x[0, K)); all threads, then a barrier.
__device__ void stage_row(const uint16_t* x, float* xs, int K, int tid) {
    if (al16(x) && K % 8 == 0) {
        for (int v = tid; v < K / 8; v += kRowThreads) {
            float f[8];
            unpack8(reinterpret_cast<const uint4*>(x)[v], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) xs[8 * v + e] = f[e];
        }
    } else {
        for (int i = tid; i < K; i += kRowThreads) xs[i] = bf16_bits_to_f32(x[i]);
    }
    __syncthreads();
}

// out[0, pad) = bf16(xs * inv * w) for i < K (w may be null), 0 past K.
__device__ void write_norm(const float* xs, int K, int pad, float inv, const float* w, uint16_t* out, int tid) {
    if (al16(out) && al16(w) && K % 8 == 0 && pad % 8 == 0) {
        for (int v = tid; v < pad / 8; v += kRowThreads) {
            uint16_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (8 * v < K) {
                float wf[8];
                if (w) {
                    const float4 w0 = reinterpret_cast<const float4*>(w)[2 * v];
                    const float4 w1 = reinterpret_cast<const float4*>(w)[2 * v + 1];
                    wf[0] = w0.x; wf[1] = w0.y; wf[2] = w0.z; wf[3] = w0.w;
                    wf[4] = w1.x; wf[5] = w1.y; wf[6] = w1.z; wf[7] = w1.w;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float t = mul_rn(xs[8 * v + e], inv);
                    b[e] = bf16_rne_bits(w ? mul_rn(t, wf[e]) : t);
                }
            }
            reinterpret_cast<uint4*>(out)[v] = pack8(b);
        }
    } else {
        for (int i = tid; i < pad; i += kRowThreads) {
            uint16_t b = 0;
            if (i < K) {
                const float t = mul_rn(xs[i], inv);
                b = bf16_rne_bits(w ? mul_rn(t, w[i]) : t);
            }
            out[i] = b;
        }
    }
}

// ---- alv_rmsnorm ---------------------------------------------------------------

__global__ void __launch_bounds__(kRowThreads) rmsnorm_kernel(const uint16_t* x, int ldx, const float* w, uint16_t* out,
                                                              int ldo, int K, int pad, float eps) {
    extern __shared__ __align__(16) float lds[];
    float* red = lds;
    float* xs = lds + 128;
    const int tid = threadIdx.x;
    const size_t row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    uint16_t* o = out + row * ldo;
    if (reg_row(K, pad) && al16(xr) && al16(w) && al16(o)) {
        uint4 xv[kRegOct];
        float wv[kRegOct][8], f[kRegOct][8];
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            const bool in = 8 * v < K;
            xv[i] = in ? reinterpret_cast<const uint4*>(xr)[v] : uint4{0u, 0u, 0u, 0u};
            load_w8(in ? w : nullptr, v, wv[i]);
        }
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            unpack8(xv[i], f[i]);
            if (8 * v < K)
#pragma unroll
                for (int e = 0; e < 8; ++e) xs[8 * v + e] = f[i][e];
        }
        __syncthreads();
        const float inv = rms_inv<kRowThreads>(xs, K, eps, red, tid);
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            if (8 * v >= pad) continue;
            uint16_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (8 * v < K)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float t = mul_rn(f[i][e], inv);
                    b[e] = bf16_rne_bits(w ? mul_rn(t, wv[i][e]) : t);
                }
            reinterpret_cast<uint4*>(o)[v] = pack8(b);
        }
        return;
    }
    stage_row(xr, xs, K, tid);
    const float inv = rms_inv<kRowThreads>(xs, K, eps, red, tid);
    write_norm(xs, K, pad, inv, w, o, tid);
}

// ---- alv_qkv_post --------------------------------------------------------------

struct QkvPostArgs {
    const uint16_t* qkv;  // [q | k | v] bf16
    int k_off, v_off;     // element offsets of k and v (v_off < 0: v is the raw k)
    int heads, kv_heads, D;
    const float* q_w;     // per-dim norm weights (null: no weight)
    const float* k_w;
    int norm_q, norm_k, norm_v;
    float eps;
    const uint16_t* rope;  // bf16 table rows (null: no rotation)
    int rope_stride, cos_off, sin_off, half;
    const int* pos;
    int max_seq;
    uint16_t* q_out;
    uint16_t* kcache;  // [kv_heads][max_seq][D]
    uint16_t* vcache;
};

// Block b: q head b, k head b - heads, or v head b - heads - kv_heads.
__global__ void __launch_bounds__(kRowThreads) qkv_post_kernel(QkvPostArgs a) {
    extern __shared__ __align__(16) float lds[];
    float* red = lds;
    float* xs = lds + 128;
    const int D = a.D;
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) return;
    const int role = b < a.heads ? 0 : (b < a.heads + a.kv_heads ? 1 : 2);
    const int h = role == 0 ? b : (role == 1 ? b - a.heads : b - a.heads - a.kv_heads);
    const int src = role == 0 ? h * D : (role == 1 || a.v_off < 0 ? a.k_off + h * D : a.v_off + h * D);
    const int norm = role == 0 ? a.norm_q : (role == 1 ? a.norm_k : a.norm_v);
    const float* w = role == 0 ? a.q_w : (role == 1 ? a.k_w : nullptr);
    const bool rot = role < 2 && a.rope;
    const uint16_t* rrow = rot ? a.rope + (size_t)pos * a.rope_stride : nullptr;
    // Heads of up to 2 x kRowThreads columns: this thread's norm weights and
    // rotation values are loaded before the head is staged, so one memory
    // round trip serves them all.
    const bool pre = D <= 2 * kRowThreads;
    float wv[2] = {0.0f, 0.0f}, cv = 0.0f, sv = 0.0f;
    if (pre) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (norm && w && tid + j * kRowThreads < D) wv[j] = w[tid + j * kRowThreads];
        if (rot && tid < a.half) {
            cv = bf16_bits_to_f32(rrow[a.cos_off + tid]);
            sv = bf16_bits_to_f32(rrow[a.sin_off + tid]);
        }
    }
    stage_row(a.qkv + src, xs, D, tid);
    if (norm) {
        const float inv = rms_inv<kRowThreads>(xs, D, a.eps, red, tid);
        if (pre) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int i = tid + j * kRowThreads;
                if (i >= D) continue;
                const float t = mul_rn(xs[i], inv);
                xs[i] = bf16r(w ? mul_rn(t, wv[j]) : t);
            }
        } else {
            for (int i = tid; i < D; i += kRowThreads) {
                const float t = mul_rn(xs[i], inv);
                xs[i] = bf16r(w ? mul_rn(t, w[i]) : t);
            }
        }
        __syncthreads();
    }
    uint16_t* dst = role == 0 ? a.q_out + (size_t)h * D
                              : (role == 1 ? a.kcache : a.vcache) + ((size_t)h * a.max_seq + pos) * D;
    if (rot) {
        // run_rope_cpu_gemma (model.py:549-575): y1 = x1 c - x2 s, y2 = x2 c + x1 s.
        for (int i = tid; i < a.half; i += kRowThreads) {
            const float c = pre ? cv : bf16_bits_to_f32(rrow[a.cos_off + i]);
            const float s = pre ? sv : bf16_bits_to_f32(rrow[a.sin_off + i]);
            const float x1 = xs[i], x2 = xs[i + a.half];
            dst[i] = bf16_rne_bits(sub_rn(mul_rn(x1, c), mul_rn(x2, s)));
            dst[i + a.half] = bf16_rne_bits(add_rn(mul_rn(x2, c), mul_rn(x1, s)));
        }
        for (int i = 2 * a.half + tid; i < D; i += kRowThreads) dst[i] = bf16_rne_bits(xs[i]);
    } else {
        for (int i = tid; i < D; i += kRowThreads) dst[i] = bf16_rne_bits(xs[i]);
    }
}

// ---- alv_attention -------------------------------------------------------------

constexpr int kAttnChunk = 64;    // cache positions per workgroup
constexpr int kAttnThreads = 256;
constexpr int kAttnHeads = 4;     // q heads per workgroup
constexpr int kAttnMaxChunks = 1024;

struct AttnArgs {
    const uint16_t* q;  // [heads][D]
    const uint16_t* kcache;
    const uint16_t* vcache;
    uint16_t* out;      // [heads][D]
    int heads, kv_heads, D, max_seq, window, hg;
    float scale;
    const int* pos;
    int nchunk;          // grid.x: chunks the largest window can need
    float* part;         // [kv_heads][nchunk][g][D + 2]: weighted V sums, max, exp-sum
    // Fused q/k/v post-processing (alv_qkv_attention): the QKV projection's
    // output in place of q, and alv_qkv_post's parameters.
    QkvPostArgs post;
};

struct AttnSpan {
    int start, W, nch;
};

__device__ __forceinline__ AttnSpan attn_span(const AttnArgs& a, int pos) {
    const int seq = pos + 1;
    const int start = a.window > 0 && seq > a.window ? seq - a.window : 0;
    const int W = seq - start;
    return {start, W, (W + kAttnChunk - 1) / kAttnChunk};
}

// Chunk c of kv head blockIdx.y for q heads [HG * blockIdx.z, + HG) of its
// group. D and HG are template parameters so that every thread issues all of
// its K and V loads (D/32 16-byte pieces each) before it needs any of them, and
// the per-head loops carry no branches (a branch per head around each
// multiply-add serialises its LDS read).
// FQ: the q/k/v post-processing of alv_qkv_post runs here, per workgroup,
// while the chunk's K and V loads are in flight: every workgroup normalises
// and rotates its HG q heads from the QKV output (each wave a row, the
// pairwise sums wave-wide), and the workgroups of the chunk that holds pos
// also the kv head's k and v rows, which they use in place of the cache row
// they loaded (workgroup z = 0 writes them into the caches; chunk 0 writes
// the rotated q). Bit for bit alv_qkv_post's arithmetic.
template <int D, int HG, bool FQ>
__global__ void __launch_bounds__(kAttnThreads) attn_partial_kernel(AttnArgs a) {
    constexpr int QD = D / 4;                // score slice per thread (4 threads per position)
    constexpr int NK = QD / 8;               // its 16-byte K pieces
    constexpr int DV = D / 8;                // 16-byte column pieces of a V row
    constexpr int PG = kAttnThreads / DV;    // position groups of the V sum
    constexpr int NV = kAttnChunk / PG;      // positions per thread in the V sum
    // q in LDS, each head's quarters 4 floats apart so that the four threads
    // of a position read different banks.
    constexpr int QQ = QD + 4, QS = 4 * QQ;
    __shared__ __align__(16) float qs[HG * QS];
    __shared__ float es[HG][kAttnChunk];
    __shared__ float ms[HG], ls[HG];
    __shared__ __align__(16) float red[PG * HG * D];  // [pg][head][D]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int g = a.heads / a.kv_heads;
    const int h0 = blockIdx.z * HG;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) return;
    const AttnSpan sp = attn_span(a, pos);
    if (c >= sp.nch) return;
    const int p0 = c * kAttnChunk;
    const int np = min(kAttnChunk, sp.W - p0);
    const size_t row0 = (size_t)kvh * a.max_seq + sp.start + p0;

    // Fused post-processing: the rows this workgroup normalises, loaded
    // before the K and V loads (a wait for them then waits for nothing else).
    constexpr int RW = D / 64;  // row elements per lane, lane l: [RW l, RW l + RW)
    const bool lastc = c == sp.nch - 1;
    const int nrows = FQ ? HG + (lastc ? 2 : 0) : 0;
    __shared__ __align__(16) uint16_t kvn[2][D];  // the new k and v rows (bf16)
    // Raw bits only: every load unconditional (addresses of unused values
    // clamped to valid memory) and nothing converted until the K and V loads
    // are issued, so that no wait for these loads comes before them.
    uint32_t xraw[2][RW], wraw[2][RW], craw[2][RW], sraw[2][RW];
    int role[2], hrow[2];
    if constexpr (FQ) {
        const QkvPostArgs& pa = a.post;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int r = wave + 4 * t;
            // role 0: q head kvh g + h0 + r; 1: k of kv head kvh; 2: v (raw k when v_off < 0)
            role[t] = r < HG ? 0 : (r == HG ? 1 : 2);
            hrow[t] = role[t] == 0 ? kvh * g + h0 + r : kvh;
            const int src = role[t] == 0 ? hrow[t] * D
                                         : (role[t] == 1 || pa.v_off < 0 ? pa.k_off + kvh * D : pa.v_off + kvh * D);
            const float* w = role[t] == 0 ? pa.q_w : (role[t] == 1 ? pa.k_w : nullptr);
            const uint32_t* wp = w ? reinterpret_cast<const uint32_t*>(w) : reinterpret_cast<const uint32_t*>(pa.qkv);
            const uint16_t* rr = pa.rope ? pa.rope + (size_t)pos * pa.rope_stride : pa.qkv;
            const int co = pa.rope ? pa.cos_off : 0, so = pa.rope ? pa.sin_off : 0, hf = pa.rope ? pa.half : 1;
#pragma unroll
            for (int e = 0; e < RW; ++e) {
                const int d = RW * lane + e;
                const int i = d % hf;
                xraw[t][e] = pa.qkv[src + d];
                wraw[t][e] = wp[w ? d : 0];
                craw[t][e] = rr[co + i];
                sraw[t][e] = rr[so + i];
            }
        }
        asm volatile("" ::: "memory");  // these loads go out before the K and V loads
    }

    // Every load of the workgroup up front: K slices, V pieces, q.
    const int p = tid >> 2, part = tid & 3;
    const int dv = tid % DV, pg = tid / DV;
    uint4 kreg[NK], vreg[NV];
    {
        const uint4* kr = reinterpret_cast<const uint4*>(a.kcache + (row0 + min(p, np - 1)) * D + part * QD);
#pragma unroll
        for (int i = 0; i < NK; ++i) kreg[i] = kr[i];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int pp = min(pg + j * PG, np - 1);
            vreg[j] = reinterpret_cast<const uint4*>(a.vcache + (row0 + pp) * D)[dv];
        }
    }
    if constexpr (FQ) {
        // Each wave its rows: the float row in LDS (red is free until the V
        // sum), the wave-wide pairwise sum, the norm, RoPE from the row.
        const QkvPostArgs& pa = a.post;
        float* rowb = red + wave * D;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (wave + 4 * t >= nrows) break;
            const int norm = role[t] == 0 ? pa.norm_q : (role[t] == 1 ? pa.norm_k : pa.norm_v);
            const bool hasw = role[t] == 0 ? pa.q_w != nullptr : (role[t] == 1 ? pa.k_w != nullptr : false);
            float xrow[RW], crow[RW], srow[RW];
#pragma unroll
            for (int e = 0; e < RW; ++e) {
                xrow[e] = bf16_bits_to_f32(xraw[t][e]);
                crow[e] = bf16_bits_to_f32(craw[t][e]);
                srow[e] = bf16_bits_to_f32(sraw[t][e]);
                rowb[RW * lane + e] = xrow[e];
            }
            if (norm) {
                const float inv = rms_inv_wave(rowb, D, pa.eps, lane);
#pragma unroll
                for (int e = 0; e < RW; ++e) {
                    const float tt = mul_rn(xrow[e], inv);
                    rowb[RW * lane + e] = bf16r(hasw ? mul_rn(tt, __builtin_bit_cast(float, wraw[t][e])) : tt);
                }
            }
            uint16_t ob[RW];
            const bool rot = role[t] < 2 && pa.rope;
#pragma unroll
            for (int e = 0; e < RW; ++e) {
                const int d = RW * lane + e;
                float y = rowb[d];
                if (rot && d < 2 * pa.half) {
                    // run_rope_cpu_gemma (model.py:549-575): y1 = x1 c - x2 s, y2 = x2 c + x1 s.
                    const int i = d < pa.half ? d : d - pa.half;
                    y = d < pa.half ? sub_rn(mul_rn(rowb[i], crow[e]), mul_rn(rowb[i + pa.half], srow[e]))
                                    : add_rn(mul_rn(rowb[d], crow[e]), mul_rn(rowb[i], srow[e]));
                }
                ob[e] = bf16_rne_bits(y);
            }
#pragma unroll
            for (int e = 0; e < RW; ++e) {
                const int d = RW * lane + e;
                if (role[t] == 0) {
                    const int hl = hrow[t] - kvh * g - h0;
                    qs[hl * QS + (d / QD) * QQ + d % QD] = bf16_bits_to_f32(ob[e]);
                    if (c == 0 && pa.q_out) pa.q_out[(size_t)hrow[t] * D + d] = ob[e];
                } else {
                    kvn[role[t] - 1][d] = ob[e];
                    if (blockIdx.z == 0)
                        (role[t] == 1 ? pa.kcache : pa.vcache)[((size_t)kvh * a.max_seq + pos) * D + d] = ob[e];
                }
            }
        }
    } else {
        const uint4* qv = reinterpret_cast<const uint4*>(a.q + ((size_t)kvh * g + h0) * D);
        for (int i = tid; i < HG * DV; i += kAttnThreads) {
            float f[8];
            unpack8(qv[i], f);
            const int h = i / DV, d = (i - h * DV) * 8;
            float4* dst = reinterpret_cast<float4*>(qs + h * QS + (d / QD) * QQ + d % QD);
            dst[0] = float4{f[0], f[1], f[2], f[3]};
            dst[1] = float4{f[4], f[5], f[6], f[7]};
        }
    }
    __syncthreads();
    if constexpr (FQ) {
        // The chunk that holds pos: its last row (and every clamped load of
        // it) is the new k and v, not what the cache held.
        if (lastc) {
            if (p >= np - 1)
#pragma unroll
                for (int i = 0; i < NK; ++i) kreg[i] = reinterpret_cast<const uint4*>(kvn[0] + part * QD)[i];
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (pg + j * PG >= np - 1) vreg[j] = reinterpret_cast<const uint4*>(kvn[1])[dv];
        }
    }

    // Scores: 4 threads per position, each a quarter of the row.
    {
        float acc[HG];
#pragma unroll
        for (int h = 0; h < HG; ++h) acc[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            float kf[8];
            unpack8(kreg[i], kf);
#pragma unroll
            for (int h = 0; h < HG; ++h) {
                const float4* qp = reinterpret_cast<const float4*>(qs + h * QS + part * QQ + i * 8);
                const float4 q0 = qp[0], q1 = qp[1];
                const float qf[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h] = fmaf(kf[e], qf[e], acc[h]);
            }
        }
#pragma unroll
        for (int h = 0; h < HG; ++h) {
            float v = acc[h];
            v += __shfl_xor(v, 1);
            v += __shfl_xor(v, 2);
            if (part == 0) es[h][p] = p < np ? v * a.scale : -__builtin_inff();
        }
    }
    __syncthreads();

    // The chunk's softmax pieces: one wave per head; positions past the
    // chunk's end weigh zero.
    if (wave < HG) {
        const int h = wave;
        const float s = es[h][lane];
        float m = s;
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float e = lane < np ? expf(s - m) : 0.0f;
        float l = e;
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
        es[h][lane] = e;
        if (lane == 0) {
            ms[h] = m;
            ls[h] = l;
        }
    }
    __syncthreads();

    // Weighted V sum: thread (pg, dv) over positions pg, pg + PG, ... (those
    // past the chunk's end weigh zero and read a valid row); the PG partial
    // sums then added in order.
    {
        float acc[HG][8];
#pragma unroll
        for (int h = 0; h < HG; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int pp = pg + j * PG;
            float vf[8];
            unpack8(vreg[j], vf);
#pragma unroll
            for (int h = 0; h < HG; ++h) {
                const float w = es[h][pp];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(w, vf[e], acc[h][e]);
            }
        }
#pragma unroll
        for (int h = 0; h < HG; ++h) {
            float4* dst = reinterpret_cast<float4*>(red + ((size_t)pg * HG + h) * D + dv * 8);
            dst[0] = float4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
            dst[1] = float4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
        }
    }
    __syncthreads();
    constexpr int gstride = D + 2;
    float* out = a.part + (((size_t)kvh * a.nchunk + c) * g + h0) * gstride;
    for (int i = tid; i < HG * D; i += kAttnThreads) {
        const int h = i / D, d = i - h * D;
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < PG; ++q) o += red[((size_t)q * HG + h) * D + d];
        out[(size_t)h * gstride + d] = o;
    }
    if (tid < HG) {
        out[(size_t)tid * gstride + D] = ms[tid];
        out[(size_t)tid * gstride + D + 1] = ls[tid];
    }
}

// Head blockIdx.x, columns [256 blockIdx.y, + 256): the chunks merged in order,
// out = sum_c o_c f_c / sum_c l_c f_c with f_c = exp(m_c - max_c m_c).
__global__ void __launch_bounds__(kAttnThreads) attn_merge_kernel(AttnArgs a) {
    __shared__ float fs[kAttnMaxChunks], lsum[kAttnMaxChunks];
    __shared__ float Ls;
    const int tid = threadIdx.x;
    const int hq = blockIdx.x;
    const int g = a.heads / a.kv_heads, kvh = hq / g, hl = hq - kvh * g;
    const int D = a.D, gstride = D + 2;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) return;
    const int nch = attn_span(a, pos).nch;
    const float* base = a.part + ((size_t)kvh * a.nchunk * g + hl) * gstride;  // chunk q at + q * g * gstride
    for (int q = tid; q < nch; q += kAttnThreads) {
        fs[q] = base[(size_t)q * g * gstride + D];
        lsum[q] = base[(size_t)q * g * gstride + D + 1];
    }
    __syncthreads();
    if (tid == 0) {
        float M = -__builtin_inff();
        for (int q = 0; q < nch; ++q) M = fmaxf(M, fs[q]);
        float L = 0.0f;
        for (int q = 0; q < nch; ++q) {
            const float f = expf(fs[q] - M);
            L = fmaf(lsum[q], f, L);
            fs[q] = f;
        }
        Ls = L;
    }
    __syncthreads();
    const int d = blockIdx.y * kAttnThreads + tid;
    if (d >= D) return;
    float O = 0.0f;
#pragma unroll 8
    for (int q = 0; q < nch; ++q) O = fmaf(base[(size_t)q * g * gstride + d], fs[q], O);
    a.out[(size_t)hq * D + d] = bf16_rne_bits(__fdiv_rn(O, Ls));
}

// ---- alv_add_norm --------------------------------------------------------------

struct AddNormArgs {
    const uint16_t* resid;
    const uint16_t* y;
    int ldr, ldy;
    const float* w_y;
    int norm_y;
    float scale;
    int scale_mode;  // 0 none; 1 bf16(bf16(r + t) * scale); 2 bf16((r + t) * scale)
    uint16_t* sum_out;
    int ld_sum;
    const float* w_out;
    uint16_t* norm_out;
    int ldn, K, pad;
    float eps;
};

__global__ void __launch_bounds__(kRowThreads) add_norm_kernel(AddNormArgs a) {
    extern __shared__ __align__(16) float lds[];
    float* red = lds;
    float* xs = lds + 128;
    const int K = a.K;
    const int tid = threadIdx.x;
    const size_t row = blockIdx.x;
    const uint16_t* yr = a.y + row * a.ldy;
    const uint16_t* r = a.resid + row * a.ldr;
    uint16_t* so = a.sum_out + row * a.ld_sum;
    uint16_t* no = a.norm_out ? a.norm_out + row * a.ldn : nullptr;
    float inv = 1.0f;  // 1 / rms of y when it is normalised
    // s = bf16(r + t) (scaled), t = bf16(y * inv * w_y) or y.
    auto step = [&](float x, float rv, float w) -> float {
        return resid_step(x, rv, w, inv, a.norm_y, a.w_y != nullptr, a.scale_mode, a.scale);
    };
    if (reg_row(K, a.pad) && al16(yr) && al16(r) && al16(so) && al16(a.w_y) && al16(a.w_out) && al16(no)) {
        uint4 yv[kRegOct], rv[kRegOct];
        float wy[kRegOct][8], wo[kRegOct][8], f[kRegOct][8];
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            const bool in = 8 * v < K;
            yv[i] = in ? reinterpret_cast<const uint4*>(yr)[v] : uint4{0u, 0u, 0u, 0u};
            rv[i] = in ? reinterpret_cast<const uint4*>(r)[v] : uint4{0u, 0u, 0u, 0u};
            load_w8(in && a.norm_y ? a.w_y : nullptr, v, wy[i]);
            load_w8(in && no ? a.w_out : nullptr, v, wo[i]);
        }
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            unpack8(yv[i], f[i]);
            if (a.norm_y && 8 * v < K)
#pragma unroll
                for (int e = 0; e < 8; ++e) xs[8 * v + e] = f[i][e];
        }
        if (a.norm_y) {
            __syncthreads();
            inv = rms_inv<kRowThreads>(xs, K, a.eps, red, tid);
        }
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            if (8 * v >= K) continue;
            float rf[8];
            unpack8(rv[i], rf);
            uint16_t b[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f[i][e] = step(f[i][e], rf[e], wy[i][e]);
                b[e] = bf16_rne_bits(f[i][e]);
                if (no) xs[8 * v + e] = f[i][e];
            }
            reinterpret_cast<uint4*>(so)[v] = pack8(b);
        }
        if (!no) return;
        __syncthreads();
        const float inv2 = rms_inv<kRowThreads>(xs, K, a.eps, red, tid);
#pragma unroll
        for (int i = 0; i < kRegOct; ++i) {
            const int v = tid + i * kRowThreads;
            if (8 * v >= a.pad) continue;
            uint16_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (8 * v < K)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float t = mul_rn(f[i][e], inv2);
                    b[e] = bf16_rne_bits(a.w_out ? mul_rn(t, wo[i][e]) : t);
                }
            reinterpret_cast<uint4*>(no)[v] = pack8(b);
        }
        return;
    }
    stage_row(yr, xs, K, tid);
    if (a.norm_y) inv = rms_inv<kRowThreads>(xs, K, a.eps, red, tid);
    if (al16(r) && al16(so) && al16(a.w_y) && K % 8 == 0) {
        for (int v = tid; v < K / 8; v += kRowThreads) {
            float rf[8], wf[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            unpack8(reinterpret_cast<const uint4*>(r)[v], rf);
            if (a.norm_y && a.w_y) {
                const float4 w0 = reinterpret_cast<const float4*>(a.w_y)[2 * v];
                const float4 w1 = reinterpret_cast<const float4*>(a.w_y)[2 * v + 1];
                wf[0] = w0.x; wf[1] = w0.y; wf[2] = w0.z; wf[3] = w0.w;
                wf[4] = w1.x; wf[5] = w1.y; wf[6] = w1.z; wf[7] = w1.w;
            }
            uint16_t b[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v2 = step(xs[8 * v + e], rf[e], wf[e]);
                b[e] = bf16_rne_bits(v2);
                xs[8 * v + e] = v2;
            }
            reinterpret_cast<uint4*>(so)[v] = pack8(b);
        }
    } else {
        for (int i = tid; i < K; i += kRowThreads) {
            const float v2 = step(xs[i], bf16_bits_to_f32(r[i]), a.norm_y && a.w_y ? a.w_y[i] : 0.0f);
            so[i] = bf16_rne_bits(v2);
            xs[i] = v2;
        }
    }
    __syncthreads();
    if (!no) return;
    const float inv2 = rms_inv<kRowThreads>(xs, K, a.eps, red, tid);
    write_norm(xs, K, a.pad, inv2, a.w_out, no, tid);
}

// ---- alv_embed -------------------------------------------------------------------

// out = bf16(float(double(table[token]) * scale)): the reference's lookup
// (token_embd[token_id].astype(np.float32) * np.sqrt(hidden_size) is a float64
// product, cast to bf16 through float32, runtime/py/model.py:891). A token
// outside the table writes zeros.
__global__ void __launch_bounds__(256) embed_kernel(const uint16_t* table, int vocab, int H, const int32_t* token,
                                                    double scale, uint16_t* out) {
    const int t = *token;
    const bool ok = t >= 0 && t < vocab;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) {
        uint16_t b = 0;
        if (ok) {
            const float e = (float)__builtin_bit_cast(_Float16, table[(size_t)t * H + i]);
            b = bf16_rne_bits((float)__dmul_rn((double)e, scale));
        }
        out[i] = b;
    }
}

size_t row_lds(int K) { return (size_t)(128 + ((K + 3) & ~3)) * sizeof(float); }

hipError_t set_lds(const void* k, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

}  // namespace

}  // namespace alv

using namespace alv;

extern "C" int alv_rmsnorm(const uint16_t* x, const float* w, uint16_t* out, int rows, int K, int ldx, int ldo,
                           int pad, float eps, void* stream) {
    if (!x || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (rows < 1 || K < 1 || K > kMaxRowK || ldx < K || pad < K || ldo < pad)
        return fail(ALV_ERR_ARG, "bad rmsnorm shape rows=%d K=%d ldx=%d pad=%d ldo=%d (K <= %d)", rows, K, ldx, pad, ldo,
                    kMaxRowK);
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(out) % 2 || reinterpret_cast<uintptr_t>(w) % 4)
        return fail(ALV_ERR_ALIGN, "x and out need 2-byte, w 4-byte alignment");
    const size_t lds = row_lds(K);
    if (int rc = hip_check(set_lds(reinterpret_cast<const void*>(&rmsnorm_kernel), lds), "hipFuncSetAttribute")) return rc;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kRowThreads), lds, (hipStream_t)stream, x, ldx, w, out, ldo, K,
                       pad, eps);
    return hip_check(hipGetLastError(), "rmsnorm_kernel launch");
}

extern "C" int alv_qkv_post(const uint16_t* qkv, int k_off, int v_off, int heads, int kv_heads, int D,
                            const float* q_w, const float* k_w, int norm_q, int norm_k, int norm_v, float eps,
                            const uint16_t* rope, int rope_stride, int cos_off, int sin_off, int half,
                            const int* pos_dev, int max_seq, uint16_t* q_out, uint16_t* kcache, uint16_t* vcache,
                            void* stream) {
    if (!qkv || !pos_dev || !q_out || !kcache || !vcache) return fail(ALV_ERR_ARG, "null pointer");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || D < 1 || D > kMaxRowK || max_seq < 1 || k_off < heads * D ||
        (v_off >= 0 && v_off < k_off + kv_heads * D))
        return fail(ALV_ERR_ARG, "bad qkv layout heads=%d kv_heads=%d D=%d k_off=%d v_off=%d", heads, kv_heads, D, k_off,
                    v_off);
    if (rope && (half < 1 || 2 * half > D || rope_stride < 1 || cos_off < 0 || sin_off < 0 ||
                 cos_off + half > rope_stride || sin_off + half > rope_stride))
        return fail(ALV_ERR_ARG, "bad rope table layout stride=%d cos_off=%d sin_off=%d half=%d for D=%d", rope_stride,
                    cos_off, sin_off, half, D);
    QkvPostArgs a{qkv, k_off, v_off, heads, kv_heads, D, q_w, k_w, norm_q, norm_k, norm_v, eps,
                  rope, rope_stride, cos_off, sin_off, half, pos_dev, max_seq, q_out, kcache, vcache};
    const size_t lds = row_lds(D);
    if (int rc = hip_check(set_lds(reinterpret_cast<const void*>(&qkv_post_kernel), lds), "hipFuncSetAttribute")) return rc;
    hipLaunchKernelGGL(qkv_post_kernel, dim3(heads + 2 * kv_heads), dim3(kRowThreads), lds, (hipStream_t)stream, a);
    return hip_check(hipGetLastError(), "qkv_post_kernel launch");
}

namespace alv {
namespace {

// The attention launches for args a (q or the fused post-processing already
// set): the head group, the partial kernel, the merge.
int launch_attention(AttnArgs& a, bool fused, hipStream_t s) {
    const int heads = a.heads, kv_heads = a.kv_heads, D = a.D;
    const int span = a.window > 0 ? std::min(a.window, a.max_seq) : a.max_seq;
    const int nchunk = (span + kAttnChunk - 1) / kAttnChunk;
    if (nchunk > kAttnMaxChunks)
        return fail(ALV_ERR_RANGE, "a span of %d positions exceeds the %d the merge takes", span, kAttnMaxChunks * kAttnChunk);
    const int g = heads / kv_heads;
    // q heads per workgroup: the divisor of g (1, 2 or 4) whose grid at the
    // longest span comes closest to one workgroup per CU (measured: 16 heads
    // on one kv head of 512, 2048 positions: 13.5 us at 2 heads per
    // workgroup, 14.6 at 1, 21.7 at 4; 8 kv heads of 256, window 1024: 10.3
    // at 1, 11.1 at 2).
    // (At D = 512 at most 2: four heads' accumulators beside every K and V
    // load of the chunk would spill.)
    const int cus = device_cus();
    const int max_hg = D == 512 ? 2 : kAttnHeads;
    int hg = 1;
    for (int c = 2; c <= max_hg; c *= 2) {
        if (g % c) break;
        const long grid_c = (long)nchunk * kv_heads * (g / c), grid_h = (long)nchunk * kv_heads * (g / hg);
        if (std::labs(grid_c - cus) <= std::labs(grid_h - cus)) hg = c;
    }
    const size_t part_bytes = (size_t)kv_heads * nchunk * g * (D + 2) * sizeof(float);
    void* sc = nullptr;
    if (int rc = get_scratch(s, kScratchAttn, part_bytes, &sc)) return rc;
    a.hg = hg;
    a.nchunk = nchunk;
    a.part = static_cast<float*>(sc);
    const dim3 grid(nchunk, kv_heads, g / hg);
    const void* k = nullptr;
    auto pick = [&](auto d, auto f) {
        constexpr int DD = decltype(d)::value;
        constexpr bool FQ = decltype(f)::value;
        if constexpr (DD < 512) {
            if (hg == 4) {
                k = reinterpret_cast<const void*>(&attn_partial_kernel<DD, 4, FQ>);
                return;
            }
        }
        k = hg == 2 ? reinterpret_cast<const void*>(&attn_partial_kernel<DD, 2, FQ>)
                    : reinterpret_cast<const void*>(&attn_partial_kernel<DD, 1, FQ>);
    };
    auto pick_d = [&](auto f) {
        switch (D) {
            case 64: pick(std::integral_constant<int, 64>{}, f); break;
            case 128: pick(std::integral_constant<int, 128>{}, f); break;
            case 256: pick(std::integral_constant<int, 256>{}, f); break;
            default: pick(std::integral_constant<int, 512>{}, f); break;
        }
    };
    if (fused)
        pick_d(std::true_type{});
    else
        pick_d(std::false_type{});
    void* kargs[] = {&a};
    if (int rc = hip_check(hipLaunchKernel(k, grid, dim3(kAttnThreads), kargs, 0, s), "attn_partial_kernel launch"))
        return rc;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(heads, (D + kAttnThreads - 1) / kAttnThreads), dim3(kAttnThreads), 0, s, a);
    return hip_check(hipGetLastError(), "attn_merge_kernel launch");
}

int attn_shape_check(int heads, int kv_heads, int D, int max_seq, int window) {
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || (D != 64 && D != 128 && D != 256 && D != 512) ||
        max_seq < 1 || window < 0)
        return fail(ALV_ERR_ARG, "bad attention shape heads=%d kv_heads=%d D=%d max_seq=%d window=%d "
                    "(D one of 64, 128, 256, 512)", heads, kv_heads, D, max_seq, window);
    return ALV_OK;
}

}  // namespace
}  // namespace alv

extern "C" int alv_attention(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, uint16_t* out,
                             int heads, int kv_heads, int D, int max_seq, int window, float scale, const int* pos_dev,
                             void* stream) {
    if (!q || !kcache || !vcache || !out || !pos_dev) return fail(ALV_ERR_ARG, "null pointer");
    if (int rc = attn_shape_check(heads, kv_heads, D, max_seq, window)) return rc;
    if (reinterpret_cast<uintptr_t>(kcache) % 16 || reinterpret_cast<uintptr_t>(vcache) % 16 ||
        reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(out) % 2)
        return fail(ALV_ERR_ALIGN, "q, kcache and vcache need 16-byte alignment");
    AttnArgs a{};
    a.q = q;
    a.kcache = kcache;
    a.vcache = vcache;
    a.out = out;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.D = D;
    a.max_seq = max_seq;
    a.window = window;
    a.scale = scale;
    a.pos = pos_dev;
    return launch_attention(a, false, (hipStream_t)stream);
}

extern "C" int alv_qkv_attention(const uint16_t* qkv, int k_off, int v_off, int heads, int kv_heads, int D,
                                 const float* q_w, const float* k_w, int norm_q, int norm_k, int norm_v, float eps,
                                 const uint16_t* rope, int rope_stride, int cos_off, int sin_off, int half,
                                 const int* pos_dev, int max_seq, uint16_t* q_out, uint16_t* kcache, uint16_t* vcache,
                                 int window, float scale, uint16_t* out, void* stream) {
    if (!qkv || !pos_dev || !kcache || !vcache || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (int rc = attn_shape_check(heads, kv_heads, D, max_seq, window)) return rc;
    if (k_off < heads * D || (v_off >= 0 && v_off < k_off + kv_heads * D))
        return fail(ALV_ERR_ARG, "bad qkv layout heads=%d kv_heads=%d D=%d k_off=%d v_off=%d", heads, kv_heads, D, k_off,
                    v_off);
    if (rope && (half < 1 || 2 * half > D || rope_stride < 1 || cos_off < 0 || sin_off < 0 ||
                 cos_off + half > rope_stride || sin_off + half > rope_stride))
        return fail(ALV_ERR_ARG, "bad rope table layout stride=%d cos_off=%d sin_off=%d half=%d for D=%d", rope_stride,
                    cos_off, sin_off, half, D);
    if (reinterpret_cast<uintptr_t>(kcache) % 16 || reinterpret_cast<uintptr_t>(vcache) % 16 ||
        reinterpret_cast<uintptr_t>(out) % 2)
        return fail(ALV_ERR_ALIGN, "kcache and vcache need 16-byte alignment");
    AttnArgs a{};
    a.kcache = kcache;
    a.vcache = vcache;
    a.out = out;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.D = D;
    a.max_seq = max_seq;
    a.window = window;
    a.scale = scale;
    a.pos = pos_dev;
    a.post = QkvPostArgs{qkv, k_off, v_off, heads, kv_heads, D, q_w, k_w, norm_q, norm_k, norm_v, eps,
                         rope, rope_stride, cos_off, sin_off, half, pos_dev, max_seq, q_out, kcache, vcache};
    return launch_attention(a, true, (hipStream_t)stream);
}

extern "C" int alv_add_norm(const uint16_t* resid, int ldr, const uint16_t* y, int ldy, const float* w_y, int norm_y,
                            float scale, int scale_mode, uint16_t* sum_out, int ld_sum, const float* w_out,
                            uint16_t* norm_out, int ld_norm, int rows, int K, int pad, float eps, void* stream) {
    if (!resid || !y || !sum_out) return fail(ALV_ERR_ARG, "null pointer");
    if (rows < 1 || K < 1 || K > kMaxRowK || ldr < K || ldy < K || ld_sum < K || scale_mode < 0 || scale_mode > 2 ||
        (norm_out && (pad < K || ld_norm < pad)))
        return fail(ALV_ERR_ARG, "bad add_norm shape rows=%d K=%d pad=%d scale_mode=%d", rows, K, pad, scale_mode);
    AddNormArgs a{resid, y, ldr, ldy, w_y, norm_y, scale, scale_mode, sum_out, ld_sum, w_out, norm_out, ld_norm,
                  K, norm_out ? pad : K, eps};
    const size_t lds = row_lds(K);
    if (int rc = hip_check(set_lds(reinterpret_cast<const void*>(&add_norm_kernel), lds), "hipFuncSetAttribute")) return rc;
    hipLaunchKernelGGL(add_norm_kernel, dim3(rows), dim3(kRowThreads), lds, (hipStream_t)stream, a);
    return hip_check(hipGetLastError(), "add_norm_kernel launch");
}

extern "C" int alv_embed(const uint16_t* table_f16, int vocab, int H, const int32_t* token_dev, double scale,
                         uint16_t* out, void* stream) {
    if (!table_f16 || !token_dev || !out) return fail(ALV_ERR_ARG, "null pointer");
    if (vocab < 1 || H < 1) return fail(ALV_ERR_ARG, "bad embedding shape vocab=%d H=%d", vocab, H);
    hipLaunchKernelGGL(embed_kernel, dim3(std::min((H + 255) / 256, 64)), dim3(256), 0, (hipStream_t)stream,
                       table_f16, vocab, H, token_dev, scale, out);
    return hip_check(hipGetLastError(), "embed_kernel launch");
}
