// Row arithmetic shared by the host-op kernels and the streaming GEMV's
// fused residual step: bf16 rounding as the reference's astype(bfloat16),
// numpy's pairwise float32 sum of squares (the order np.mean(x ** 2) uses) and
// 1 / sqrt(mean + eps) in numpy's float32 steps, 16-byte row pieces.
//
// np.add.reduce over a contiguous float32 array is numpy's pairwise_sum
// (numpy/_core/src/umath/loops_utils.h.src): fewer than 8 values summed in
// order from 0; up to 128 values in eight interleaved accumulators
// r[j] += a[8i + j], combined ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)),
// then the n % 8 tail in order; more values split at n2 = n/2 - (n/2) % 8 with
// the two halves' sums added; arrays longer than numpy's 8192-element buffer
// are summed per buffer and the buffer sums added in order. For every row
// width whose splits are exact halvings (3840, 4096, 2048, 1152, 256, 512, ...)
// the leaves are summed with 8 lanes each and the halves combined across lanes
// in the recursion's own tree; other widths follow the recursion on one lane.
// numpy >= 2 evaluates the scalar steps (mean = sum / n, 1 / sqrt(var + eps))
// in float32, as here. Every product and sum goes through add_rn / mul_rn,
// which no FMA contraction can fuse (one rounding where numpy makes two).
#pragma once

#include "q4_device.h"

namespace alv {
namespace {

// float32 +, -, * rounded on their own: compiled with contraction off, so
// that no product and sum that use them fuse into one FMA (HIP's
// __fmul_rn / __fadd_rn are plain operators that do fuse).
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}

// Round to nearest even: v_cvt_pk_bf16_f32 (the round-to-nearest-even
// conversion, float32 denormals kept), NaN as 0x7FC0 -- two instructions
// where the integer form (u + 0x7FFF + lsb) >> 16 takes six.
__device__ __forceinline__ uint16_t bf16_rne_bits(float v) {
    const uint16_t h = __builtin_bit_cast(uint16_t, (__bf16)v);
    return v != v ? (uint16_t)0x7FC0u : h;
}

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(bf16_rne_bits(v)); }

__device__ __forceinline__ float sqv(const float* a, int i) { return mul_rn(a[i], a[i]); }

// ---- numpy's pairwise float32 sum of squares ---------------------------------------

// The leaf rule over the squares of a[0, n), n <= 128, on one lane.
__device__ float pw_leaf_sq(const float* a, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r = add_rn(r, sqv(a, i));
        return r;
    }
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = sqv(a, j);
    int i = 8;
    for (; i < n - (n % 8); i += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = add_rn(r[j], sqv(a, i + j));
    }
    float res = add_rn(add_rn(add_rn(r[0], r[1]), add_rn(r[2], r[3])),
                       add_rn(add_rn(r[4], r[5]), add_rn(r[6], r[7])));
    for (; i < n; ++i) res = add_rn(res, sqv(a, i));
    return res;
}

// The full recursion on one lane (widths whose splits are not halvings), its
// frames in LDS (st: 16 frames, 256 bytes; n <= 8192 nests at most 8 deep): a
// private array would give every launch of the kernel a scratch segment.
struct PwFrame {
    int off, n, stage;
    float left;
};

__device__ float pw_serial_sq(const float* a, int n, PwFrame* st) {
    int sp = 0;
    st[0] = {0, n, 0, 0.0f};
    float ret = 0.0f;
    while (sp >= 0) {
        PwFrame& f = st[sp];
        if (f.n <= 128) {
            ret = pw_leaf_sq(a + f.off, f.n);
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
            ret = add_rn(f.left, ret);
            --sp;
        }
    }
    return ret;
}

// ---- lane moves ----------------------------------------------------------------------
// DPP moves within rows of 16 lanes: quad_perm [1,0,3,2] (0xB1) and [2,3,0,1]
// (0x4E) pair lanes 1 and 2 apart, row_half_mirror (0x141) lane i with 7 - i,
// row_mirror (0x140) lane i with 15 - i. Every source lane must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// The sum of the squares of one leaf p[0, leaf), 8 <= leaf <= 128, by the
// leaf's 8 lanes (an 8-aligned group, j = lane % 8, all active): lane j sums
// r[j] = p[j]^2 + p[8 + j]^2 + ... in order (all loads issued at once), two
// quad_perm moves and a half mirror combine ((r0 + r1) + (r2 + r3)) +
// ((r4 + r5) + (r6 + r7)) on every lane (fadd is commutative, so both lanes of
// a pair hold the same bits), then the leaf % 8 tail is added in order.
__device__ __forceinline__ float leaf8_sq(const float* p, int leaf, int j) {
    const int m8 = leaf - leaf % 8;
    float sq[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) sq[q] = sqv(p, 8 * q + j < m8 ? 8 * q + j : j);
    float r = sq[0];
#pragma unroll
    for (int q = 1; q < 16; ++q) {
        const float t = add_rn(r, sq[q]);
        r = 8 * q + j < m8 ? t : r;
    }
    r = add_rn(r, dpp_f<0xB1>(r));
    r = add_rn(r, dpp_f<0x4E>(r));
    r = add_rn(r, dpp_f<0x141>(r));
    for (int i = m8; i < leaf; ++i) r = add_rn(r, sqv(p, i));
    return r;
}

// leaf8_sq for leaf = 8 N8 (every leaf of a halving row wider than 128): the
// loads at constant offsets from the lane's first value, no per-lane bounds.
template <int N8>
__device__ __forceinline__ float leaf8_sq_n(const float* p, int j) {
    const float* pj = p + j;
    float sq[N8];
#pragma unroll
    for (int q = 0; q < N8; ++q) sq[q] = mul_rn(pj[8 * q], pj[8 * q]);
    float r = sq[0];
#pragma unroll
    for (int q = 1; q < N8; ++q) r = add_rn(r, sq[q]);
    r = add_rn(r, dpp_f<0xB1>(r));
    r = add_rn(r, dpp_f<0x4E>(r));
    return add_rn(r, dpp_f<0x141>(r));
}

// A leaf's sum by its 8 lanes (leaf uniform across the wave).
__device__ __forceinline__ float leaf_sq(const float* p, int leaf, int j) {
    switch (leaf) {
        case 72: return leaf8_sq_n<9>(p, j);
        case 80: return leaf8_sq_n<10>(p, j);
        case 88: return leaf8_sq_n<11>(p, j);
        case 96: return leaf8_sq_n<12>(p, j);
        case 104: return leaf8_sq_n<13>(p, j);
        case 112: return leaf8_sq_n<14>(p, j);
        case 120: return leaf8_sq_n<15>(p, j);
        case 128: return leaf8_sq_n<16>(p, j);
        default: return leaf8_sq(p, leaf, j);
    }
}

// The recursion's tree over `count` (a power of two <= 64) values held by
// the wave's lanes 0, g, 2g, ... (g = 1: one per lane; g = 8: one per 8-lane
// group, each group's lanes holding the same bits), returned to every lane:
// DPP moves pair neighbours within rows of 16 lanes, readlane the rows.
// Every lane of the wave must be active.
__device__ __forceinline__ float fold_tree(float v, int count, int g) {
    int c = count;
    if (g == 1) {
        if (c > 1) v = add_rn(v, dpp_f<0xB1>(v));
        if (c > 2) v = add_rn(v, dpp_f<0x4E>(v));
        if (c > 4) v = add_rn(v, dpp_f<0x141>(v));
        c = c > 8 ? c / 8 : 1;  // groups of 8 lanes left to pair
    }
    if (c > 1) v = add_rn(v, dpp_f<0x140>(v));
    if (c > 4) return add_rn(add_rn(lane_f(v, 0), lane_f(v, 16)), add_rn(lane_f(v, 32), lane_f(v, 48)));
    if (c > 2) return add_rn(lane_f(v, 0), lane_f(v, 16));
    return lane_f(v, 0);
}

// Pairwise sum of the squares of a[0, n), n <= 8192, by the workgroup
// (NT threads; a and red in LDS, red >= 65 floats, 16-byte aligned: the
// one-lane recursion keeps its frames in red[0, 64)). Returned to all. SYNC:
// a closing barrier, so that the caller may write red (and a) at once; without
// it, red must not be written again before the caller's next barrier.
template <int NT, bool SYNC = true>
__device__ __forceinline__ float pw_chunk_sq(const float* a, int n, float* red, int tid) {
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
    if (!halving || leaf < 8 || leaves > 64) {
        if (tid == 0) red[64] = pw_serial_sq(a, n, reinterpret_cast<PwFrame*>(red));
        __syncthreads();
        const float r = red[64];
        if (SYNC) __syncthreads();  // red is reused by the next call
        return r;
    }
    // 8 lanes per leaf, leaf sums to red[lf]; every wave then folds them.
    for (int base = 0; base < leaves; base += NT / 8) {
        const int lf = base + (tid >> 3);
        if (lf < leaves) {
            const float r = leaf_sq(a + (size_t)lf * leaf, leaf, tid & 7);
            if ((tid & 7) == 0) red[lf] = r;
        }
    }
    __syncthreads();
    const int lane = tid & 63;
    const float r = fold_tree(red[lane < leaves ? lane : 0], leaves, 1);
    if (SYNC) __syncthreads();  // red is reused by the next call
    return r;
}

// 1 / sqrt(mean(x^2) + eps) of the K values xs (LDS) in numpy's float32
// arithmetic: np.add.reduce takes the array in buffers of 8192 elements
// (np.getbufsize()), sums each pairwise and adds the buffer sums in order.
template <int NT, bool SYNC = true>
__device__ __forceinline__ float rms_inv(const float* xs, int K, float eps, float* red, int tid) {
    constexpr int kBuf = 8192;
    if (!SYNC && K > kBuf) return rms_inv<NT, true>(xs, K, eps, red, tid);  // buffers reuse red in turn
    float s = pw_chunk_sq<NT, SYNC>(xs, min(K, kBuf), red, tid);
    for (int off = kBuf; off < K; off += kBuf)
        s = add_rn(s, pw_chunk_sq<NT, SYNC>(xs + off, min(K - off, kBuf), red, tid));
    const float var = __fdiv_rn(s, (float)K);
    // sqrtf is the correctly rounded square root here (v_sqrt_f32 plus a
    // neighbour test); __fsqrt_rn compiles to the bare 1-ulp v_sqrt_f32.
    return __fdiv_rn(1.0f, sqrtf(add_rn(var, eps)));
}

// The same pairwise sum by one wave, for rows whose splits are halvings down
// to at most 8 leaves (n <= 1024; every head width 64 ... 512): 8 lanes per
// leaf (leaf8_sq), then the leaves paired in the recursion's tree
// (fold_tree). No barrier; every lane returns the sum (all lanes of the wave
// must be active).
__device__ __forceinline__ float pw_wave_sq(const float* a, int n, int lane) {
    int leaf = n, leaves = 1;
    while (leaf > 128) {
        leaf /= 2;
        leaves *= 2;
    }
    if (leaf < 8) {
        float r = 0.0f;
        for (int i = 0; i < leaf; ++i) r = add_rn(r, sqv(a, i));
        return lane_f(r, 0);
    }
    // Lanes past the last leaf sum leaf 0 again; the tree reads only lanes
    // of real leaves.
    const int lf = lane >> 3;
    const float r = leaf_sq(a + (size_t)(lf < leaves ? lf : 0) * leaf, leaf, lane & 7);
    return fold_tree(r, leaves, 8);
}

// 1 / sqrt(mean(x^2) + eps) of a row of n <= 1024 halving width by one wave.
__device__ __forceinline__ float rms_inv_wave(const float* xs, int n, float eps, int lane) {
    const float var = __fdiv_rn(pw_wave_sq(xs, n, lane), (float)n);
    return __fdiv_rn(1.0f, sqrtf(add_rn(var, eps)));
}

__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = bf16_bits_to_f32(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu);
}

__device__ __forceinline__ uint4 pack8(const uint16_t (&b)[8]) {
    return uint4{b[0] | ((uint32_t)b[1] << 16), b[2] | ((uint32_t)b[3] << 16), b[4] | ((uint32_t)b[5] << 16),
                 b[6] | ((uint32_t)b[7] << 16)};
}

__device__ __forceinline__ bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Eight float32 weights w[8 v, 8 v + 8), or zeros for a null w.
__device__ __forceinline__ void load_w8(const float* w, int v, float (&f)[8]) {
    if (!w) {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = 0.0f;
        return;
    }
    const float4 w0 = reinterpret_cast<const float4*>(w)[2 * v];
    const float4 w1 = reinterpret_cast<const float4*>(w)[2 * v + 1];
    f[0] = w0.x; f[1] = w0.y; f[2] = w0.z; f[3] = w0.w;
    f[4] = w1.x; f[5] = w1.y; f[6] = w1.z; f[7] = w1.w;
}

// The residual step of a decode layer (runtime/py/model.py:775-788): the
// branch output x, normalised when norm_y (t = bf16(x * inv [* w])), added to
// the residual r, then scaled: scale_mode 1 bf16(bf16(r + t) * scale) (the
// Python runtime), 2 bf16((r + t) * scale) (the C++ runtime), 0 bf16(r + t).
__device__ __forceinline__ float resid_step(float x, float r, float w, float inv, int norm_y, bool has_w,
                                            int scale_mode, float scale) {
    float t = x;
    if (norm_y) {
        t = mul_rn(t, inv);
        t = bf16r(has_w ? mul_rn(t, w) : t);
    }
    const float sum = add_rn(r, t);
    if (scale_mode == 1) return bf16r(mul_rn(bf16r(sum), scale));
    if (scale_mode == 2) return bf16r(mul_rn(sum, scale));
    return bf16r(sum);
}

}  // namespace
}  // namespace alv
