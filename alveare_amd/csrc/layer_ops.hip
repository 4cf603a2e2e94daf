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
//
// Bit-exact parts. The reference computes with numpy in float32 on bf16
// arrays. Every elementwise step here is the same float32 operation with the
// same rounding (products and sums written with the _rn intrinsics so that
// nothing contracts into an FMA), and the one reduction whose order matters at
// bf16 output precision -- np.mean(x ** 2) of RMSNorm -- is numpy's own
// summation order: np.add.reduce over a contiguous float32 array is numpy's
// pairwise_sum (numpy/_core/src/umath/loops_utils.h.src): fewer than 8 values
// summed in order from 0; up to 128 values in eight interleaved accumulators
// r[j] += a[8i + j], combined ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)),
// then the n % 8 tail in order; more values split at n2 = n/2 - (n/2) % 8 with
// the two halves' sums added; arrays longer than numpy's 8192-element buffer
// are summed per buffer and the buffer sums added in order. For every row
// width whose splits are exact
// halvings (3840, 4096, 2048, 1152, 256, 512, ...) the leaves are summed one
// per lane and the halves combined across lanes in the recursion's own tree;
// other widths follow the recursion on one lane. numpy >= 2 evaluates the
// scalar steps (mean = sum / n, 1 / sqrt(var + eps)) in float32, as here.
//
// Attention is not bit-exact: the reference's scores and weighted sums are
// BLAS dot products (np.dot) whose order is the library's. Here the positions
// are split into chunks of 64 (workgroup per (kv head, chunk)); each chunk's
// max, exp-sum and weighted V sum go to the stream's scratch and the last
// workgroup of a kv head merges them in chunk order (deterministic).
//
// Decode position `pos` is read from device memory (pos_dev), so a captured
// graph replays for every token; positions at or past the cache length write
// nothing and leave the outputs unchanged.
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace alv {

namespace {

__device__ __forceinline__ uint16_t bf16_rne_bits(float v) {
    if (v != v) return 0x7FC0u;
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(bf16_rne_bits(v)); }

// ---- numpy's pairwise float32 sum ------------------------------------------------

// The leaf rule over a[0, n), n <= 128 (a 16-byte aligned when n >= 8).
__device__ float pw_leaf(const float* a, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r = __fadd_rn(r, a[i]);
        return r;
    }
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i = 8;
    for (; i < n - (n % 8); i += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = __fadd_rn(r[j], a[i + j]);
    }
    float res = __fadd_rn(__fadd_rn(__fadd_rn(r[0], r[1]), __fadd_rn(r[2], r[3])),
                          __fadd_rn(__fadd_rn(r[4], r[5]), __fadd_rn(r[6], r[7])));
    for (; i < n; ++i) res = __fadd_rn(res, a[i]);
    return res;
}

// The full recursion on one lane (row widths whose splits are not halvings).
__device__ float pw_serial(const float* a, int n) {
    struct Frame {
        int off, n, stage;
        float left;
    };
    Frame st[32];
    int sp = 0;
    st[0] = {0, n, 0, 0.0f};
    float ret = 0.0f;
    while (sp >= 0) {
        Frame& f = st[sp];
        if (f.n <= 128) {
            ret = pw_leaf(a + f.off, f.n);
            --sp;
            continue;
        }
        int n2 = f.n / 2;
        n2 -= n2 % 8;
        if (f.stage == 0) {
            f.stage = 1;
            st[sp + 1] = {f.off, n2, 0, 0.0f};
            ++sp;
        } else if (f.stage == 1) {
            f.left = ret;
            f.stage = 2;
            st[sp + 1] = {f.off + n2, f.n - n2, 0, 0.0f};
            ++sp;
        } else {
            ret = __fadd_rn(f.left, ret);
            --sp;
        }
    }
    return ret;
}

// The pairwise sum of a[0, n), n <= 8192, for the calling wave (all 64
// lanes; a in LDS, 16-byte aligned). Returned in every lane.
__device__ float pw_chunk_wave(const float* a, int n, int lane) {
    int leaf = n, leaves = 1;
    bool halving = true;
    while (leaf > 128) {
        if ((leaf & 1) || ((leaf / 2) % 8)) {
            halving = false;
            break;
        }
        leaf /= 2;
        leaves *= 2;
    }
    if (halving && leaves <= 64) {
        float v = lane < leaves ? pw_leaf(a + (size_t)lane * leaf, leaf) : 0.0f;
        for (int s = 1; s < leaves; s *= 2) {
            const float o = __shfl_down(v, s);
            if ((lane & (2 * s - 1)) == 0) v = __fadd_rn(v, o);
        }
        return __shfl(v, 0);
    }
    float r = 0.0f;
    if (lane == 0) r = pw_serial(a, n);
    return __shfl(r, 0);
}

// np.add.reduce(a[0, n)): numpy's reduction loop takes the array in buffers
// of 8192 elements (np.getbufsize()), sums each pairwise and adds the buffer
// sums in order.
__device__ float pw_sum_wave(const float* a, int n, int lane) {
    constexpr int kBuf = 8192;
    float r = pw_chunk_wave(a, min(n, kBuf), lane);
    for (int off = kBuf; off < n; off += kBuf) r = __fadd_rn(r, pw_chunk_wave(a + off, min(n - off, kBuf), lane));
    return r;
}

// 1 / sqrt(mean(x^2) + eps) of the K float32 values xs (LDS) in numpy's
// float32 arithmetic; sq is K floats of LDS scratch. One wave (the workgroup).
__device__ float rms_inv(const float* xs, float* sq, int K, float eps, int lane) {
    for (int i = lane; i < K; i += 64) sq[i] = __fmul_rn(xs[i], xs[i]);
    __syncthreads();
    const float s = pw_sum_wave(sq, K, lane);
    __syncthreads();
    const float var = __fdiv_rn(s, (float)K);
    // sqrtf is the correctly rounded square root here (v_sqrt_f32 plus a
    // neighbour test); __fsqrt_rn compiles to the bare 1-ulp v_sqrt_f32.
    return __fdiv_rn(1.0f, sqrtf(__fadd_rn(var, eps)));
}

__device__ __forceinline__ void stage_bf16(const uint16_t* x, float* xs, int K, int lane) {
    for (int i = lane; i < K; i += 64) xs[i] = bf16_bits_to_f32(x[i]);
    __syncthreads();
}

// bf16(x * inv * w) (w may be null), in place.
__device__ __forceinline__ void norm_apply(float* xs, int K, float inv, const float* w, int lane) {
    for (int i = lane; i < K; i += 64) {
        const float t = __fmul_rn(xs[i], inv);
        xs[i] = bf16r(w ? __fmul_rn(t, w[i]) : t);
    }
    __syncthreads();
}

// ---- alv_rmsnorm ---------------------------------------------------------------

__global__ void __launch_bounds__(64) rmsnorm_kernel(const uint16_t* x, int ldx, const float* w, uint16_t* out,
                                                     int ldo, int K, int pad, float eps) {
    extern __shared__ __align__(16) float lds[];
    float* xs = lds;
    float* sq = lds + ((K + 3) & ~3);
    const int lane = threadIdx.x;
    const size_t row = blockIdx.x;
    stage_bf16(x + row * ldx, xs, K, lane);
    const float inv = rms_inv(xs, sq, K, eps, lane);
    uint16_t* o = out + row * ldo;
    for (int i = lane; i < pad; i += 64) {
        uint16_t b = 0;
        if (i < K) {
            const float t = __fmul_rn(xs[i], inv);
            b = bf16_rne_bits(w ? __fmul_rn(t, w[i]) : t);
        }
        o[i] = b;
    }
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
__global__ void __launch_bounds__(64) qkv_post_kernel(QkvPostArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int D = a.D;
    float* xs = lds;
    float* sq = lds + ((D + 3) & ~3);
    const int lane = threadIdx.x;
    const int b = blockIdx.x;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) return;
    const int role = b < a.heads ? 0 : (b < a.heads + a.kv_heads ? 1 : 2);
    const int h = role == 0 ? b : (role == 1 ? b - a.heads : b - a.heads - a.kv_heads);
    const int src = role == 0 ? h * D : (role == 1 || a.v_off < 0 ? a.k_off + h * D : a.v_off + h * D);
    stage_bf16(a.qkv + src, xs, D, lane);
    const int norm = role == 0 ? a.norm_q : (role == 1 ? a.norm_k : a.norm_v);
    if (norm) {
        const float inv = rms_inv(xs, sq, D, a.eps, lane);
        norm_apply(xs, D, inv, role == 0 ? a.q_w : (role == 1 ? a.k_w : nullptr), lane);
    }
    uint16_t* dst = role == 0 ? a.q_out + (size_t)h * D
                              : (role == 1 ? a.kcache : a.vcache) + ((size_t)h * a.max_seq + pos) * D;
    if (role < 2 && a.rope) {
        // run_rope_cpu_gemma (model.py:549-575): y1 = x1 c - x2 s, y2 = x2 c + x1 s.
        const uint16_t* row = a.rope + (size_t)pos * a.rope_stride;
        for (int i = lane; i < a.half; i += 64) {
            const float c = bf16_bits_to_f32(row[a.cos_off + i]);
            const float s = bf16_bits_to_f32(row[a.sin_off + i]);
            const float x1 = xs[i], x2 = xs[i + a.half];
            dst[i] = bf16_rne_bits(__fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s)));
            dst[i + a.half] = bf16_rne_bits(__fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s)));
        }
        for (int i = 2 * a.half + lane; i < D; i += 64) dst[i] = bf16_rne_bits(xs[i]);
    } else {
        for (int i = lane; i < D; i += 64) dst[i] = bf16_rne_bits(xs[i]);
    }
}

// ---- alv_attention -------------------------------------------------------------

constexpr int kAttnChunk = 64;     // cache positions per workgroup
constexpr int kAttnThreads = 256;
constexpr int kAttnMaxGroup = 16;  // q heads per kv head
constexpr int kAttnMaxD = 512;

struct AttnArgs {
    const uint16_t* q;  // [heads][D]
    const uint16_t* kcache;
    const uint16_t* vcache;
    uint16_t* out;      // [heads][D]
    int heads, kv_heads, D, max_seq, window;
    float scale;
    const int* pos;
    int nchunk;          // grid.x: chunks the largest window can need
    float* part;         // [kv_heads][nchunk][g][D + 2]
    uint32_t* cnt;       // [kv_heads]
};

__global__ void __launch_bounds__(kAttnThreads) attention_kernel(AttnArgs a) {
    __shared__ __align__(16) float qs[kAttnMaxGroup * kAttnMaxD];
    __shared__ float es[kAttnMaxGroup][kAttnChunk];
    __shared__ float ms[kAttnMaxGroup], ls[kAttnMaxGroup];
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int D = a.D, g = a.heads / a.kv_heads;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) return;
    const int seq = pos + 1;
    const int start = a.window > 0 && seq > a.window ? seq - a.window : 0;
    const int W = seq - start;
    const int nch = (W + kAttnChunk - 1) / kAttnChunk;
    if (c >= nch) return;
    const int p0 = c * kAttnChunk;
    const int np = min(kAttnChunk, W - p0);

    // q of the group's heads, float32.
    for (int i = tid; i < g * D; i += kAttnThreads) qs[i] = bf16_bits_to_f32(a.q[(size_t)kvh * g * D + i]);
    __syncthreads();

    // Scores: 4 threads per position, each a quarter of the row (D % 32 == 0:
    // the quarter is whole 16-byte pieces).
    {
        const int p = tid >> 2, part = tid & 3;
        const int qd = D / 4;
        float acc[kAttnMaxGroup];
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) acc[h] = 0.0f;
        if (p < np) {
            const uint4* kr = reinterpret_cast<const uint4*>(
                a.kcache + ((size_t)kvh * a.max_seq + start + p0 + p) * D + part * qd);
            const float* qp = qs + part * qd;
            for (int c8 = 0; c8 < qd / 8; ++c8) {
                const uint4 v = kr[c8];
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float kv = bf16_bits_to_f32(e & 1 ? w4[e >> 1] >> 16 : w4[e >> 1] & 0xFFFFu);
#pragma unroll
                    for (int h = 0; h < kAttnMaxGroup; ++h)
                        if (h < g) acc[h] = fmaf(kv, qp[h * D + c8 * 8 + e], acc[h]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) {
            float v = acc[h];
            v += __shfl_xor(v, 1);
            v += __shfl_xor(v, 2);
            if (h < g && part == 0) es[h][p] = p < np ? v * a.scale : -__builtin_inff();
        }
    }
    __syncthreads();

    // Chunk softmax pieces: one wave per head.
    for (int h = wave; h < g; h += kAttnThreads / 64) {
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

    // Weighted V sum of the chunk, then the chunk's partial to scratch.
    const int gstride = D + 2;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.part, (uint32_t)((size_t)a.kv_heads * a.nchunk * g * gstride * 4));
    const uint32_t mybase = (uint32_t)((((size_t)kvh * a.nchunk + c) * g) * gstride * 4);
    for (int d = tid; d < D; d += kAttnThreads) {
        float o[kAttnMaxGroup];
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) o[h] = 0.0f;
        const uint16_t* vr = a.vcache + ((size_t)kvh * a.max_seq + start + p0) * D + d;
        for (int p = 0; p < np; ++p) {
            const float vv = bf16_bits_to_f32(vr[(size_t)p * D]);
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < g) o[h] = fmaf(es[h][p], vv, o[h]);
        }
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) {
            if (h < g)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o[h]), rp,
                                                  mybase + (uint32_t)((h * gstride + d) * 4), 0, 16);
        }
    }
    if (tid < g) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ms[tid]), rp,
                                              mybase + (uint32_t)((tid * gstride + D) * 4), 0, 16);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ls[tid]), rp,
                                              mybase + (uint32_t)((tid * gstride + D + 1) * 4), 0, 16);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&a.cnt[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(nch - 1);
    __syncthreads();
    if (!last) return;

    // Last workgroup of this kv head: merge the chunks. Per head, the chunk
    // maxima give M, the weights f_c = exp(m_c - M) go to LDS (the q slots,
    // free now) and L = sum l_c f_c; then O[d] = sum o_c[d] f_c and out = O / L.
    // Fixed lane assignment and reduction order: deterministic.
    const uint32_t hbase = (uint32_t)(((size_t)kvh * a.nchunk * g) * gstride * 4);
    float* fs = qs;  // [g][nch]
    for (int h = wave; h < g; h += kAttnThreads / 64) {
        float M = -__builtin_inff();
        for (int q = lane; q < nch; q += 64)
            M = fmaxf(M, __builtin_bit_cast(float, buf_load4_sc1(rp, hbase + (uint32_t)(((q * g + h) * gstride + D) * 4))));
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
        float L = 0.0f;
        for (int q = lane; q < nch; q += 64) {
            const uint32_t b0 = hbase + (uint32_t)(((q * g + h) * gstride + D) * 4);
            const float m = __builtin_bit_cast(float, buf_load4_sc1(rp, b0));
            const float l = __builtin_bit_cast(float, buf_load4_sc1(rp, b0 + 4u));
            const float f = expf(m - M);
            fs[h * nch + q] = f;
            L = fmaf(l, f, L);
        }
        for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o);
        if (lane == 0) ls[h] = L;
    }
    __syncthreads();
    for (int i = tid; i < g * D; i += kAttnThreads) {
        const int h = i / D, d = i - h * D;
        float O = 0.0f;
#pragma unroll 8
        for (int q = 0; q < nch; ++q)
            O = fmaf(__builtin_bit_cast(float, buf_load4_sc1(rp, hbase + (uint32_t)(((q * g + h) * gstride + d) * 4))),
                     fs[h * nch + q], O);
        a.out[((size_t)kvh * g + h) * D + d] = bf16_rne_bits(__fdiv_rn(O, ls[h]));
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

__global__ void __launch_bounds__(64) add_norm_kernel(AddNormArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int K = a.K;
    float* xs = lds;
    float* sq = lds + ((K + 3) & ~3);
    const int lane = threadIdx.x;
    const size_t row = blockIdx.x;
    stage_bf16(a.y + row * a.ldy, xs, K, lane);
    if (a.norm_y) {
        const float inv = rms_inv(xs, sq, K, a.eps, lane);
        norm_apply(xs, K, inv, a.w_y, lane);
    }
    const uint16_t* r = a.resid + row * a.ldr;
    uint16_t* so = a.sum_out + row * a.ld_sum;
    for (int i = lane; i < K; i += 64) {
        const float sum = __fadd_rn(bf16_bits_to_f32(r[i]), xs[i]);
        float v;
        if (a.scale_mode == 1)
            v = bf16r(__fmul_rn(bf16r(sum), a.scale));
        else if (a.scale_mode == 2)
            v = bf16r(__fmul_rn(sum, a.scale));
        else
            v = bf16r(sum);
        so[i] = bf16_rne_bits(v);
        xs[i] = v;
    }
    __syncthreads();
    if (!a.norm_out) return;
    const float inv = rms_inv(xs, sq, K, a.eps, lane);
    uint16_t* no = a.norm_out + row * a.ldn;
    for (int i = lane; i < a.pad; i += 64) {
        uint16_t b = 0;
        if (i < K) {
            const float t = __fmul_rn(xs[i], inv);
            b = bf16_rne_bits(a.w_out ? __fmul_rn(t, a.w_out[i]) : t);
        }
        no[i] = b;
    }
}

size_t row_lds(int K) { return (size_t)2 * ((K + 3) & ~3) * sizeof(float); }

hipError_t set_lds(const void* k, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

constexpr int kMaxRowK = 20480;  // 2 x 80 KiB of LDS per row

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
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(64), lds, (hipStream_t)stream, x, ldx, w, out, ldo, K, pad, eps);
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
    hipLaunchKernelGGL(qkv_post_kernel, dim3(heads + 2 * kv_heads), dim3(64), lds, (hipStream_t)stream, a);
    return hip_check(hipGetLastError(), "qkv_post_kernel launch");
}

extern "C" int alv_attention(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, uint16_t* out,
                             int heads, int kv_heads, int D, int max_seq, int window, float scale, const int* pos_dev,
                             void* stream) {
    if (!q || !kcache || !vcache || !out || !pos_dev) return fail(ALV_ERR_ARG, "null pointer");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || heads / kv_heads > kAttnMaxGroup || D < 32 || D % 32 ||
        D > kAttnMaxD || max_seq < 1 || window < 0)
        return fail(ALV_ERR_ARG, "bad attention shape heads=%d kv_heads=%d D=%d max_seq=%d window=%d "
                    "(group <= %d, D a multiple of 32 up to %d)", heads, kv_heads, D, max_seq, window, kAttnMaxGroup, kAttnMaxD);
    if (reinterpret_cast<uintptr_t>(kcache) % 16 || reinterpret_cast<uintptr_t>(q) % 2 ||
        reinterpret_cast<uintptr_t>(vcache) % 2 || reinterpret_cast<uintptr_t>(out) % 2)
        return fail(ALV_ERR_ALIGN, "kcache needs 16-byte alignment");
    hipStream_t s = (hipStream_t)stream;
    const int span = window > 0 ? std::min(window, max_seq) : max_seq;
    const int nchunk = (span + kAttnChunk - 1) / kAttnChunk;
    const int g = heads / kv_heads;
    if ((size_t)g * nchunk > (size_t)kAttnMaxGroup * kAttnMaxD)
        return fail(ALV_ERR_RANGE, "a span of %d positions in %d-head groups exceeds the merge's %d chunk weights", span, g,
                    kAttnMaxGroup * kAttnMaxD);
    const size_t part_bytes = (size_t)kv_heads * nchunk * g * (D + 2) * sizeof(float);
    if (part_bytes >= 0xFFFFF000ull) return fail(ALV_ERR_RANGE, "attention partials exceed the 4 GiB buffer range");
    const size_t cnt_bytes = ((size_t)kv_heads * sizeof(uint32_t) + 255) & ~(size_t)255;
    void* sc = nullptr;
    if (int rc = get_scratch(s, kScratchAttn, cnt_bytes + part_bytes, &sc)) return rc;
    AttnArgs a{q, kcache, vcache, out, heads, kv_heads, D, max_seq, window, scale, pos_dev, nchunk,
               reinterpret_cast<float*>(static_cast<uint8_t*>(sc) + cnt_bytes), static_cast<uint32_t*>(sc)};
    hipLaunchKernelGGL(attention_kernel, dim3(nchunk, kv_heads), dim3(kAttnThreads), 0, s, a);
    return hip_check(hipGetLastError(), "attention_kernel launch");
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
    hipLaunchKernelGGL(add_norm_kernel, dim3(rows), dim3(64), lds, (hipStream_t)stream, a);
    return hip_check(hipGetLastError(), "add_norm_kernel launch");
}
