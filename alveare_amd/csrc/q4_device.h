// Device-side building blocks shared by the gfx950 Q4 kernels.
//
// Q4 combined layout (tools/convert/gemv_q_convert.py:53-85): per row, K/32
// blocks of 20 bytes = 16 bytes of nibbles (byte i holds column 2i in the low
// nibble and 2i+1 in the high nibble, two's complement), a little-endian bf16
// scale at bytes 16-17, and 2 zero bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/alveare_q4.h"

namespace alv {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef float f32x2 __attribute__((__vector_size__(2 * sizeof(float))));
typedef uint32_t u32x4 __attribute__((__vector_size__(4 * sizeof(uint32_t))));

constexpr int kBlockBytes = 20;  // bytes per 32 weights
constexpr int kBlockK = 32;      // weights per block

// Tiled Q4 layout (the kernels' registration-time layout; a byte permutation
// of the combined layout, zero-padded to whole 128-column runs):
//   row tile rt = 16 rows; super-step ss = 16 blocks (512 columns); within a
//   row tile, lane (g, j), g = 0..3, j = 0..15, owns the 80-byte run of row
//   16 rt + j covering blocks 16 ss + 4 g .. 16 ss + 4 g + 3.
//   Tile (rt, ss) stores those runs as 5 planes of 16-byte pieces: piece i of
//   lane l = 16 g + j sits at tile + i * 256 * ng + 16 * l, where ng = 4 for
//   every super-step but the last, which holds ng = ceil(blocks left / 4)
//   lanes of g. Tiles follow each other in (rt, ss) order, so row tile rt
//   starts at rt * tile_row_bytes(K) and super-step ss at + ss * 5120.
//   Blocks past K and rows past N are zero (they dequantize to zero).
// A wave reading piece i of every lane reads 1 KiB of contiguous memory.
struct TileGeom {
    int nb;           // blocks per row
    int nss;          // super-steps per row
    int ng_last;      // lanes of g in the last super-step
    uint32_t rtb;     // bytes per row tile
};

// Byte offset in the tiled layout of byte x (0..19) of block kb of row `row`.
__host__ __device__ inline uint32_t tiled_offset(const TileGeom& t, int row, int kb, int x) {
    const int ss = kb >> 4, g = (kb >> 2) & 3, bl = kb & 3;
    const int rb = 20 * bl + x;
    const uint32_t ng = ss == t.nss - 1 ? (uint32_t)t.ng_last : 4u;
    return (uint32_t)(row >> 4) * t.rtb + (uint32_t)ss * 5120u + (uint32_t)(rb >> 4) * 256u * ng +
           (uint32_t)(g * 16 + (row & 15)) * 16u + (uint32_t)(rb & 15);
}

__host__ __device__ inline TileGeom tile_geom(int K) {
    TileGeom t;
    t.nb = K / kBlockK;
    t.nss = (t.nb + 15) / 16;
    t.ng_last = (t.nb - 16 * (t.nss - 1) + 3) / 4;
    t.rtb = (uint32_t)(t.nss - 1) * 5120u + 1280u * (uint32_t)t.ng_last;
    return t;
}

// Buffer resource over [base, base + bytes): loads past the end return 0
// instead of faulting. dword3 = 0x00020000 is the raw 32-bit data format on gfx9.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Read a loaded vector's elements through a scalar, `(uint32_t)v[e]`: this
// clang lowers __builtin_bit_cast(float, v[e]) on a vector element to a read
// of element 0.
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Streaming (nontemporal) variant for weights, which are read exactly once:
// aux bit 1 sets the `nt` cache policy on gfx950.
__device__ __forceinline__ u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}

// Loads addressed by a per-lane voffset that stays fixed and a wave-uniform
// soffset (an SGPR) that carries the moving part of the address, so a
// prefetch never writes a VGPR that an in-flight load may still target.
template <bool NT>
__device__ __forceinline__ u32x4 buf_load16_so(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, NT ? 2 : 0);
}

// Load that bypasses this XCD's L2 (sc1): sees data another workgroup wrote
// through with agent-scope stores.
__device__ __forceinline__ u32x4 buf_load16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}

__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint32_t buf_load4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) {
    return __builtin_bit_cast(float, h16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950), returned
// as the fp32 value it represents.
__device__ __forceinline__ float bf16_round(float v) {
    __bf16 h = (__bf16)v;
    return (float)h;
}

// Per-block scale constants for dequant8: s512 = 512*s, sm8 = -8*s. Both are
// exact (power-of-two multiples) for |s| < 2^118.
struct Scale {
    float s512, sm8;
};

__device__ __forceinline__ Scale make_scale(float s) { return Scale{s * 512.0f, s * -8.0f}; }

// The block scale from the dword holding block bytes 16..19: the bf16 at bytes
// 16-17 moved to the high half (one byte permute; bytes 18-19 are dropped).
__device__ __forceinline__ float scale_of(uint32_t d) {
    return __builtin_bit_cast(float, __builtin_amdgcn_perm(d, d, 0x01000C0Cu));
}

// Eight weights from one dword of nibbles, exactly as the reference dequantizes
// them: w = bf16_RNE(f32(q) * f32(s)) (tools/ref/gemv_q.py:19-37).
//
// XOR 0x8 turns each two's-complement nibble q into q + 8 in [0, 15]. A byte
// 0x0u read as OCP FP8 E4M3 is exactly u * 2^-9 (exponent field 0 is the
// subnormal range, 1 the first normal binade, both at step 2^-9), so
// v_cvt_pk_f32_fp8 yields (q + 8) * 2^-9 for two weights per instruction, and
// fma((q+8) 2^-9, 512 s, -8 s) is q*s with a single rounding of an exactly
// representable value, i.e. exact. The bf16 conversion then rounds to nearest
// even like the reference's astype(bfloat16).
//
// The nibble split is one v_bitop3 per half: (d & 0x0F0F0F0F) ^ 0x08080808
// (truth table 0x6A for S0 & S1 ^ S2).
//
// Output element e is column 8*t + e of the block when d is the block's
// dword t (natural column order).
__device__ __forceinline__ bf16x8 dequant8(uint32_t d, Scale s) {
    const uint32_t lo = __builtin_amdgcn_bitop3_b32(d, 0x0F0F0F0Fu, 0x08080808u, 0x6A);       // cols 0,2,4,6
    const uint32_t hi = __builtin_amdgcn_bitop3_b32(d >> 4, 0x0F0F0F0Fu, 0x08080808u, 0x6A);  // cols 1,3,5,7
    const f32x2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f32x2 l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    bf16x8 r;
    r[0] = (__bf16)__builtin_fmaf(l01[0], s.s512, s.sm8);
    r[1] = (__bf16)__builtin_fmaf(h01[0], s.s512, s.sm8);
    r[2] = (__bf16)__builtin_fmaf(l01[1], s.s512, s.sm8);
    r[3] = (__bf16)__builtin_fmaf(h01[1], s.s512, s.sm8);
    r[4] = (__bf16)__builtin_fmaf(l23[0], s.s512, s.sm8);
    r[5] = (__bf16)__builtin_fmaf(h23[0], s.s512, s.sm8);
    r[6] = (__bf16)__builtin_fmaf(l23[1], s.s512, s.sm8);
    r[7] = (__bf16)__builtin_fmaf(h23[1], s.s512, s.sm8);
    return r;
}

// The same eight weights with fewer instructions (the streaming kernel's and
// the prefill GEMM's form; v_cvt_pk_f32_fp8 issues at a quarter of the fp32 rate). One v_bitop3
// builds two fp16 values at once, 1.0 with mantissa bits [p, p + 4) = q + 8 in
// each half (p = 0 or 4), i.e. a = 1 + (q + 8) 2^(p - 10), and v_fma_mix_f32
// widens a half exactly inside fma(a, S_p, C_p) with S_p = s 2^(10 - p),
// C_p = -(S_p + 8 s) = -s (2^(10 - p) + 8): the product a S_p is exact inside
// the fma, C_p has at most 16 significant bits (exact), and the exact sum
// (q + 8) s - 8 s = q s has at most 11, so the one rounding changes nothing.
// Then RNE to bf16 as the reference does. 17 instructions per eight weights.
// Valid for |s| < 2^112 (S_0 and C_0 must not overflow), which every
// quantization scale is; the dequant parity entry point keeps dequant8.
struct Scale2 {
    float s0, s4, c0, c4;
};

__device__ __forceinline__ Scale2 make_scale2(float s) {
    Scale2 r;
    r.s0 = s * 1024.0f;  // 2^10
    r.s4 = s * 64.0f;    // 2^6
    r.c0 = __builtin_fmaf(s, -8.0f, -r.s0);
    r.c4 = __builtin_fmaf(s, -8.0f, -r.s4);
    return r;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp16 1.0 + ((x >> p) & 15 ^ 8) 2^(p - 10), one per 16-bit half;
// mask = 15 << p in each half, c = 0x3C00 | 8 << p in each half.
__device__ __forceinline__ f16x2 nib_f16x2(uint32_t x, uint32_t mask, uint32_t c) {
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_bitop3_b32(x, mask, c, 0x6A));
}

__device__ __forceinline__ bf16x8 dequant8_mix(uint32_t d, const Scale2& s) {
    const uint32_t d8 = d >> 8;                                  // nibbles 2, 3 / 6, 7 at bits 0, 4 / 16, 20
    const f16x2 a = nib_f16x2(d, 0x000F000Fu, 0x3C083C08u);   // nibbles 0, 4 (p = 0)
    const f16x2 b = nib_f16x2(d, 0x00F000F0u, 0x3C803C80u);   // nibbles 1, 5 (p = 4)
    const f16x2 c = nib_f16x2(d8, 0x000F000Fu, 0x3C083C08u);  // nibbles 2, 6
    const f16x2 e = nib_f16x2(d8, 0x00F000F0u, 0x3C803C80u);  // nibbles 3, 7
    float w[8];
    w[0] = __builtin_fmaf((float)a[0], s.s0, s.c0);
    w[1] = __builtin_fmaf((float)b[0], s.s4, s.c4);
    w[2] = __builtin_fmaf((float)c[0], s.s0, s.c0);
    w[3] = __builtin_fmaf((float)e[0], s.s4, s.c4);
    w[4] = __builtin_fmaf((float)a[1], s.s0, s.c0);
    w[5] = __builtin_fmaf((float)b[1], s.s4, s.c4);
    w[6] = __builtin_fmaf((float)c[1], s.s0, s.c0);
    w[7] = __builtin_fmaf((float)e[1], s.s4, s.c4);
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)w[i];
    return r;
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// traffic, not for its global loads, so weight loads stay in flight across
// it (__syncthreads would drain them).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Exact split of an fp32 value into three bf16 terms, x == p0 + p1 + p2 for
// every finite x whose low part does not underflow: p0 = RNE(x) leaves a
// residual with at most 16 significant bits, p1 = RNE(residual) leaves at most
// 8, which p2 holds exactly. Products p_i * w (bf16 * bf16) are exact in fp32,
// so an MFMA over the three terms is an fp32 dot product with the exact x.
struct Split3 {
    __bf16 p0, p1, p2;
};

__device__ __forceinline__ Split3 split3(float x) {
    Split3 s;
    s.p0 = (__bf16)x;
    const float r1 = x - (float)s.p0;  // exact
    s.p1 = (__bf16)r1;
    const float r2 = r1 - (float)s.p1;  // exact
    s.p2 = (__bf16)r2;
    return s;
}

// D(16x16, fp32) += A(16x32, bf16) * B(32x16, bf16). Lane l supplies row l%16
// of A and column l%16 of B for k-group l/16 (8 elements each); the result
// lane l holds D[4*(l/16) + r][l%16], r = 0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// GeGLU / SwiGLU of one element with the reference CPU path's dtype flow
// (runtime/py/model.py:800-803 under NumPy >= 2 promotion; :856 for SiLU):
// the cubic and the inner sum are fp32 (python floats are weak scalars),
// np.sqrt(2/np.pi) is a float64 scalar so tanh and the two products are
// float64, and the result reaches bf16 through fp32 (the caller rounds).
// Contraction is off so every fp32 operation rounds where numpy's does.
//
// GELU fast path, for results that reach the same bf16 value: with
// z = sqrt(2/pi) * inner rounded to fp32, 1 + tanh(z) = 2 / (1 + e^(-2z)) has
// no cancellation, and for z >= -11 (|2z| <= 22 where it matters) the fp32
// value v = (0.5 g) * that * u is within 34 * 2^-24 |V| of the reference's V:
// z's rounding 22 * 2^-24 through the exponential, expf 2 ulps (4 * 2^-24),
// the add, the divide and two products 2^-24 each, and the reference's own
// float64 1 + t, which loses at most 2^-53 / (1 + tanh(-11)) < 4 * 2^-24
// there (t within an ulp of tanh). That is at most 34 fp32 ulps of v, so when
// v's bits are more than 64 ulps from the bf16 rounding midpoint of its
// binade (low half 0x8000) and v is normal, bf16(f32(V)) = bf16(v).
// Anything else -- z < -11, NaN, zero, tiny or huge v, near a midpoint (about
// 0.2 % of values) -- takes the float64 path, which is the reference's.
// The reference's arithmetic, float64 tanh and all.
__device__ __forceinline__ float glu_exact(float g, float u, int act) {
#pragma clang fp contract(off)
    if (act == ALV_ACT_GELU_TANH) {
        const float g3 = (g * g) * g;
        const float inner = g + 0.044715f * g3;
        const double t = tanh(0.7978845608028654 * (double)inner);
        const double gl = (double)(0.5f * g) * (1.0 + t);
        return (float)(gl * (double)u);
    }
    // SiLU all in fp32 as numpy does it; exp(-g) correctly rounded to fp32
    // (through float64) as the CPU's libm expf gives it, where the device's
    // fp32 expf can be an ulp off.
    const float e = (float)exp(-(double)g);
    const float r = 1.0f / (1.0f + e);
    return (g * r) * u;
}

// The GELU fast path above: true (and *out) when v reaches the reference's
// bf16 value; false for SiLU and for every case the float64 path must settle.
__device__ __forceinline__ bool glu_fast(float g, float u, int act, float* out) {
#pragma clang fp contract(off)
    if (act != ALV_ACT_GELU_TANH) return false;
    const float g3 = (g * g) * g;
    const float inner = g + 0.044715f * g3;
    const double zd = 0.7978845608028654 * (double)inner;
    if (!(zd >= -11.0)) return false;
    const float z = (float)zd;
    const float v = ((0.5f * g) * (2.0f / (1.0f + expf(-2.0f * z)))) * u;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t mag = b & 0x7FFFFFFFu;
    *out = v;
    return mag >= 0x04000000u && mag < 0x7E800000u && (b & 0xFFFFu) - 0x7FC0u > 0x80u;
}

// Fast path, else the float64 one: the prefill GEMM's epilogue (64 values
// per lane) and alv_glu. The decode kernels evaluate a few values per lane,
// where a wave that has any lane on the float64 path runs both paths, so they
// call glu_exact directly (measured 1-4 % faster there).
__device__ __forceinline__ float glu_act(float g, float u, int act) {
    float v;
    return glu_fast(g, u, act, &v) ? v : glu_exact(g, u, act);
}

}  // namespace alv
