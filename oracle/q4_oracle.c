/*
 * CPU oracle for the Alveare Q4 decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's fp32 CPU path. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as
 * the checker (or as the timed CPU baseline); the product never does.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). Contraction is
 * off so that every fp32 operation rounds exactly where numpy's does.
 *
 * What pins each function (tests/test_oracle.py):
 *   orc_bf16_from_f32  exhaustive over all 2^32 fp32 patterns against the
 *                      reference's own runtime/cpp/src/bf16.cpp compiled into
 *                      oracle/_ref, and against torch's float->bfloat16 cast.
 *   orc_unpack_q4      exhaustive over all 256 byte values against the
 *                      closed form of tools/ref/gemv_q.py:19-28, and a
 *                      pack->unpack round trip over all 256 (q0, q1) pairs.
 *   orc_dequant_q4     exhaustive over 16 codes x 65536 bf16 scales against
 *                      torch (fp32 multiply then bf16 cast) and, where the
 *                      code is a power of two, the exact product.
 *   orc_gemv_q         fp64 brute force with the gamma_K bound; one-hot x
 *                      selects a dequantized column exactly; zero-scale rows
 *                      give 0; the numpy restatement (W.astype(f32) @ x).
 *   orc_glu / orc_ffn  the reference's own numpy expression evaluated by
 *                      numpy (oracle/q4_numpy.py), tanh vs long-double tanhl,
 *                      g=0 / u=0 special cases, fp64 brute force.
 *   orc_gemm_q         every row equals orc_gemv_q (runtime/cpp/src/main.cpp:98-108).
 *   orc_quantize_q4_0  hand-computed blocks (ties to even, clipping, zero
 *                      block -> scale 1.0), |dequant(quant(W)) - W| <= s/2, and
 *                      byte equality with the reference's numpy expressions
 *                      (oracle/q4_numpy.py) on random, tie, subnormal, NaN
 *                      and inf blocks.
 */
#include "q4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 (runtime/cpp/src/bf16.cpp:7-27) -------------------------------- */

uint16_t orc_bf16_from_f32(float f) {
    /* bf16.cpp:8-11: NaN becomes the quiet NaN 0x7FC0. */
    if (f != f) return 0x7FC0;
    uint32_t u;
    memcpy(&u, &f, 4);
    /* bf16.cpp:15-18: round to nearest even by adding 0x7FFF + lsb. */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f32_from_bf16(uint16_t h) {
    uint32_t u = (uint32_t)h << 16; /* bf16.cpp:22-27 */
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_bf16_from_f32_n(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(in[i]);
}

static inline float bf16_round(float f) { return orc_f32_from_bf16(orc_bf16_from_f32(f)); }

uint64_t orc_bf16_sweep(uint16_t (*other)(float), uint32_t* first_bad) {
    /* Exhaustive comparison over all 2^32 fp32 bit patterns. */
    uint64_t bad = 0;
    uint32_t first = 0xFFFFFFFFu;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(min : first)
    for (int64_t i = 0; i < (int64_t)1 << 32; ++i) {
        uint32_t u = (uint32_t)i;
        float f;
        memcpy(&f, &u, 4);
        if (orc_bf16_from_f32(f) != other(f)) {
            ++bad;
            if (u < first) first = u;
        }
    }
    if (first_bad) *first_bad = first;
    return bad;
}

/* ---- layout -------------------------------------------------------------- */

/* Two's-complement 4-bit sign extension: tools/ref/gemv_q.py:23-25
 * (q[q >= 8] -= 16). */
static inline int sext4(unsigned v) { return v >= 8 ? (int)v - 16 : (int)v; }

void orc_unpack_q4(const uint8_t* W, int64_t N, int64_t K, int8_t* q) {
    const int64_t nb = K / 32, rs = nb * 20;
    for (int64_t r = 0; r < N; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = W + r * rs + b * 20; /* gemv_q.py:55-57 */
            for (int i = 0; i < 16; ++i) {
                /* gemv_q.py:19-31: low nibble -> even column, high -> odd. */
                q[r * K + b * 32 + 2 * i] = (int8_t)sext4(blk[i] & 0x0F);
                q[r * K + b * 32 + 2 * i + 1] = (int8_t)sext4((blk[i] >> 4) & 0x0F);
            }
        }
}

void orc_scales_q4(const uint8_t* W, int64_t N, int64_t K, uint16_t* s) {
    const int64_t nb = K / 32, rs = nb * 20;
    for (int64_t r = 0; r < N; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = W + r * rs + b * 20;
            /* gemv_q.py:58-60: little-endian bf16 in bytes 16-17. */
            s[r * nb + b] = (uint16_t)(blk[16] | (blk[17] << 8));
        }
}

/* One dequantized row as fp32 values of bf16 numbers:
 * w = bf16_RNE(f32(q) * f32(scale)) (gemv_q.py:33-37). */
static void dequant_row_f32(const uint8_t* row, int64_t K, float* w) {
    const int64_t nb = K / 32;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = row + b * 20;
        const float s = orc_f32_from_bf16((uint16_t)(blk[16] | (blk[17] << 8)));
        for (int i = 0; i < 16; ++i) {
            w[b * 32 + 2 * i] = bf16_round((float)sext4(blk[i] & 0x0F) * s);
            w[b * 32 + 2 * i + 1] = bf16_round((float)sext4((blk[i] >> 4) & 0x0F) * s);
        }
    }
}

void orc_dequant_q4(const uint8_t* W, int64_t N, int64_t K, uint16_t* out) {
    const int64_t rs = (K / 32) * 20;
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
    for (int64_t r = 0; r < N; ++r) {
        dequant_row_f32(W + r * rs, K, w);
        for (int64_t k = 0; k < K; ++k) out[r * K + k] = orc_bf16_from_f32(w[k]);
    }
    free(w);
}

/* ---- matvec -------------------------------------------------------------- */

/* fp32 dot product with 8 striped partial sums combined pairwise, the order a
 * SIMD BLAS sgemv uses; numpy's exact BLAS order is not reproducible here
 * (gemv_q.py:79 runs `W.astype(np.float32) @ x.astype(np.float32)`). */
static float dot_f32(const float* w, const float* x, int64_t K) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= K; k += 8)
        for (int j = 0; j < 8; ++j) acc[j] += w[k + j] * x[k + j];
    for (; k < K; ++k) acc[k & 7] += w[k] * x[k];
    float a0 = acc[0] + acc[4], a1 = acc[1] + acc[5], a2 = acc[2] + acc[6], a3 = acc[3] + acc[7];
    return (a0 + a2) + (a1 + a3);
}

void orc_gemv_q(const uint8_t* W, const float* x, float* y, int64_t N, int64_t K,
                int threads) {
    const int64_t rs = (K / 32) * 20;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float* w = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < N; ++r) {
            dequant_row_f32(W + r * rs, K, w);
            y[r] = dot_f32(w, x, K);
        }
        free(w);
    }
}

void orc_gemv_q_f64(const uint8_t* W, const float* x, double* y, int64_t N, int64_t K,
                    int threads) {
    const int64_t rs = (K / 32) * 20;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float* w = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < N; ++r) {
            dequant_row_f32(W + r * rs, K, w);
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)w[k] * (double)x[k];
            y[r] = acc;
        }
        free(w);
    }
}

void orc_gemm_q(const uint8_t* W, const float* X, float* Y, int64_t M, int64_t N,
                int64_t K, int threads) {
    /* model.py:1049-1111: each token row is an independent GEMV. */
    for (int64_t m = 0; m < M; ++m) orc_gemv_q(W, X + m * K, Y + m * N, N, K, threads);
}

/* ---- activation ---------------------------------------------------------- */

/* GeGLU of one element with the dtype flow of runtime/py/model.py:800-803 under
 * NumPy >= 2 promotion: the cubic and the inner sum are float32 (python floats
 * are weak scalars), np.sqrt(2/np.pi) is a float64 scalar so the tanh argument,
 * tanh, the product with 0.5*g and with u are float64; `.astype(bfloat16)`
 * converts float64 -> float32 -> bf16 (ml_dtypes casts through float).
 * NumPy's float32 `g ** 3` is a SIMD routine not correctly rounded to the ulp;
 * g*g*g is used here (parity unpinned at that ulp). */
static float gelu_mul(float g, float u) {
    const double c = sqrt(2.0 / M_PI);
    float g2 = g * g;
    float g3 = g2 * g;
    float t32 = 0.044715f * g3;
    float inner = g + t32;
    double t = tanh(c * (double)inner);
    double gl = (double)(0.5f * g) * (1.0 + t);
    return (float)(gl * (double)u);
}

/* SiLU of one element, all float32 (model.py:856: python scalars are weak). */
static float silu_mul(float g, float u) {
    float e = expf(-g);
    float d = 1.0f + e;
    float r = 1.0f / d;
    float s = g * r;
    return s * u;
}

void orc_glu(const float* g, const float* u, float* a, int64_t n, int act) {
    for (int64_t i = 0; i < n; ++i)
        a[i] = bf16_round(act == 0 ? gelu_mul(g[i], u[i]) : silu_mul(g[i], u[i]));
}

void orc_ffn(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, const float* X,
             float* Y, int64_t M, int64_t H, int64_t I, int act, int threads) {
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* a = (float*)malloc(sizeof(float) * (size_t)I);
    for (int64_t m = 0; m < M; ++m) {
        /* model.py:798-799: gate/up matvec, each cast to bf16. */
        orc_gemv_q(Wg, X + m * H, g, I, H, threads);
        orc_gemv_q(Wu, X + m * H, u, I, H, threads);
        for (int64_t i = 0; i < I; ++i) {
            g[i] = bf16_round(g[i]);
            u[i] = bf16_round(u[i]);
        }
        orc_glu(g, u, a, I, act); /* model.py:800-803 */
        orc_gemv_q(Wd, a, Y + m * H, H, I, threads); /* model.py:806 before the cast */
    }
    free(g);
    free(u);
    free(a);
}

void orc_ffn_f64(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, const float* x,
                 double* y, int64_t H, int64_t I, int act) {
    double* gd = (double*)malloc(sizeof(double) * (size_t)I);
    double* ud = (double*)malloc(sizeof(double) * (size_t)I);
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* a = (float*)malloc(sizeof(float) * (size_t)I);
    orc_gemv_q_f64(Wg, x, gd, I, H, 1);
    orc_gemv_q_f64(Wu, x, ud, I, H, 1);
    for (int64_t i = 0; i < I; ++i) {
        g[i] = bf16_round((float)gd[i]);
        u[i] = bf16_round((float)ud[i]);
    }
    orc_glu(g, u, a, I, act);
    orc_gemv_q_f64(Wd, a, y, H, I, 1);
    free(gd);
    free(ud);
    free(g);
    free(u);
    free(a);
}

/* ---- quantizer (tools/convert/gemv_q_convert.py:5-85) --------------------- */

void orc_quantize_q4_0(const float* Wf, int64_t N, int64_t K, uint8_t* out) {
    const int64_t nb = K / 32, rs = nb * 20;
    for (int64_t r = 0; r < N; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float* w = Wf + r * K + b * 32;
            /* :24-25: scale = max|w| / 7 in float32; np.max propagates NaN. */
            float mx = 0.0f;
            int nan = 0;
            for (int i = 0; i < 32; ++i) {
                float a = fabsf(w[i]);
                if (a != a) nan = 1;
                if (a > mx) mx = a;
            }
            float s = nan ? NAN : mx / 7.0f;
            if (s == 0.0f) s = 1.0f; /* :28 */
            int q[32];
            for (int i = 0; i < 32; ++i) {
                /* :34-37: np.round (half to even) of a float32 quotient,
                 * astype(int32), clip. A NaN quotient (a NaN block, or inf / inf)
                 * converts to INT32_MIN on x86-64 (cvttss2si) and clips to -8. */
                float v = rintf(w[i] / s);
                int qi = v != v ? -8 : (int)v;
                q[i] = qi < -8 ? -8 : (qi > 7 ? 7 : qi);
            }
            uint8_t* blk = out + r * rs + b * 20;
            for (int i = 0; i < 16; ++i) /* :46-48 */
                blk[i] = (uint8_t)((q[2 * i] & 0x0F) | ((q[2 * i + 1] & 0x0F) << 4));
            uint16_t sb = orc_bf16_from_f32(s); /* :51 bf16 scales, :75-81 LE bytes */
            blk[16] = (uint8_t)(sb & 0xFF);
            blk[17] = (uint8_t)(sb >> 8);
            blk[18] = 0; /* :83 zero padding */
            blk[19] = 0;
        }
}

/* ---- seeded synthetic inputs --------------------------------------------- */

uint64_t orc_splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* 24-bit uniform in [0, 1). */
static inline float u01(uint64_t z) { return (float)(z >> 40) * (1.0f / 16777216.0f); }

void orc_synth_q4(uint8_t* W, int64_t N, int64_t K, uint64_t seed, float smin, float smax) {
    /* Codes: the 16 code bytes of each block are uniform random bytes, i.e.
     * i.i.d. uniform nibbles in [-8, 7]. Scales: fp32 ~U(smin, smax), rounded
     * to bf16 at pack time as the on-disk format requires. */
    const int64_t nb = K / 32, rs = nb * 20;
    const uint64_t seed_s = seed ^ 0x5CA1E5CA1E5CA1E5ull;
    for (int64_t r = 0; r < N; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint64_t blk_id = (uint64_t)(r * nb + b);
            uint8_t* blk = W + r * rs + b * 20;
            uint64_t z0 = orc_splitmix64_at(seed, 2 * blk_id);
            uint64_t z1 = orc_splitmix64_at(seed, 2 * blk_id + 1);
            for (int i = 0; i < 8; ++i) {
                blk[i] = (uint8_t)(z0 >> (8 * i));
                blk[8 + i] = (uint8_t)(z1 >> (8 * i));
            }
            float span = smax - smin;
            float s = smin + span * u01(orc_splitmix64_at(seed_s, blk_id));
            uint16_t sb = orc_bf16_from_f32(s);
            blk[16] = (uint8_t)(sb & 0xFF);
            blk[17] = (uint8_t)(sb >> 8);
            blk[18] = 0;
            blk[19] = 0;
        }
}

void orc_synth_uniform(float* x, int64_t n, uint64_t seed, float lo, float hi) {
    float span = hi - lo;
    for (int64_t i = 0; i < n; ++i) x[i] = lo + span * u01(orc_splitmix64_at(seed, (uint64_t)i));
}

void orc_synth_normal(float* x, int64_t n, uint64_t seed) {
    /* Box-Muller in fp64 on two consecutive counter values, rounded to fp32. */
    for (int64_t i = 0; i < n; ++i) {
        uint64_t a = orc_splitmix64_at(seed, 2 * (uint64_t)i);
        uint64_t b = orc_splitmix64_at(seed, 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        x[i] = (float)(sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2));
    }
}

/* ---- CPU-baseline timing ------------------------------------------------- */

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* The reference's per-call work (gemv_q.py:73-80): materialize the dequantized
 * matrix as fp32 (bf16-rounded values), then an fp32 matvec. */
static void gemv_faithful_once(const uint8_t* W, const float* x, float* y, float* wbuf,
                               int64_t N, int64_t K, int threads) {
    const int64_t rs = (K / 32) * 20;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t r = 0; r < N; ++r) dequant_row_f32(W + r * rs, K, wbuf + r * K);
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t r = 0; r < N; ++r) y[r] = dot_f32(wbuf + r * K, x, K);
}

double orc_time_gemv_faithful(const uint8_t* W, const float* x, float* y, int64_t N,
                              int64_t K, int iters, int threads) {
    float* wbuf = (float*)malloc(sizeof(float) * (size_t)(N * K));
    if (!wbuf) return -1.0;
    double t0 = now_s();
    for (int it = 0; it < iters; ++it) gemv_faithful_once(W, x, y, wbuf, N, K, threads);
    double t = now_s() - t0;
    free(wbuf);
    return t;
}

double orc_time_gemv_predequant(const uint8_t* W, const float* x, float* y, int64_t N,
                                int64_t K, int iters, int threads) {
    float* wbuf = (float*)malloc(sizeof(float) * (size_t)(N * K));
    if (!wbuf) return -1.0;
    const int64_t rs = (K / 32) * 20;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t r = 0; r < N; ++r) dequant_row_f32(W + r * rs, K, wbuf + r * K);
    double t0 = now_s();
    for (int it = 0; it < iters; ++it) {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int64_t r = 0; r < N; ++r) y[r] = dot_f32(wbuf + r * K, x, K);
    }
    double t = now_s() - t0;
    free(wbuf);
    return t;
}

double orc_time_ffn_faithful(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                             const float* x, float* y, int64_t H, int64_t I, int iters,
                             int threads) {
    /* model.py:727-737 dequantizes each projection per call, then :797-806. */
    float* wbuf = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* a = (float*)malloc(sizeof(float) * (size_t)I);
    if (!wbuf || !g || !u || !a) return -1.0;
    double t0 = now_s();
    for (int it = 0; it < iters; ++it) {
        gemv_faithful_once(Wg, x, g, wbuf, I, H, threads);
        gemv_faithful_once(Wu, x, u, wbuf, I, H, threads);
        for (int64_t i = 0; i < I; ++i) {
            g[i] = bf16_round(g[i]);
            u[i] = bf16_round(u[i]);
        }
        orc_glu(g, u, a, I, 0);
        gemv_faithful_once(Wd, a, y, wbuf, H, I, threads);
    }
    double t = now_s() - t0;
    free(wbuf);
    free(g);
    free(u);
    free(a);
    return t;
}

/* The pre-dequantized FFN (runtime/py/model.py:134-145 keeps small models'
 * matrices dequantized at load): per call only the fp32 matvecs and the
 * activation's rounding points (:797-806). The dequantization is outside
 * the timed region. */
double orc_time_ffn_predequant(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                               const float* x, float* y, int64_t H, int64_t I, int iters,
                               int threads) {
    float* wg = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wu = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wd = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* a = (float*)malloc(sizeof(float) * (size_t)I);
    if (!wg || !wu || !wd || !g || !u || !a) return -1.0;
    const int64_t rh = (H / 32) * 20, ri = (I / 32) * 20;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t r = 0; r < I; ++r) {
        dequant_row_f32(Wg + r * rh, H, wg + r * H);
        dequant_row_f32(Wu + r * rh, H, wu + r * H);
    }
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t r = 0; r < H; ++r) dequant_row_f32(Wd + r * ri, I, wd + r * I);
    double t0 = now_s();
    for (int it = 0; it < iters; ++it) {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int64_t r = 0; r < I; ++r) {
            g[r] = bf16_round(dot_f32(wg + r * H, x, H));
            u[r] = bf16_round(dot_f32(wu + r * H, x, H));
        }
        orc_glu(g, u, a, I, 0);
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int64_t r = 0; r < H; ++r) y[r] = dot_f32(wd + r * I, a, I);
    }
    double t = now_s() - t0;
    free(wg);
    free(wu);
    free(wd);
    free(g);
    free(u);
    free(a);
    return t;
}
