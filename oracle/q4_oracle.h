/*
 * CPU oracle for the Alveare Q4 decode path (gemv_q, ffn_fused, gemm_q).
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * fp32 CPU path, used by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg as the checker. The product (alveare_amd/) never links or
 * calls it.
 *
 * Every function cites the reference file:line it restates. Parity of each
 * function is pinned by tests/test_oracle.py (exhaustive tables, the
 * reference's own bf16.cpp built into oracle/_ref, torch's bf16 cast, fp64
 * brute force, closed forms); see the header comment of q4_oracle.c for the
 * pin of each function.
 */
#ifndef ALV_Q4_ORACLE_H
#define ALV_Q4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> fp32 (runtime/cpp/src/bf16.cpp:7-27). */
uint16_t orc_bf16_from_f32(float f);
float orc_f32_from_bf16(uint16_t h);
void orc_bf16_from_f32_n(const float* in, uint16_t* out, int64_t n);
/* Compare orc_bf16_from_f32 with `other` over all 2^32 fp32 patterns; returns
 * the number of mismatches and the lowest mismatching pattern. */
uint64_t orc_bf16_sweep(uint16_t (*other)(float), uint32_t* first_bad);

/* Q4 combined layout: 20 bytes per 32 weights along K
 * (tools/convert/gemv_q_convert.py:53-85, kernels/gemv_q/README.md:13-23). */
void orc_unpack_q4(const uint8_t* W, int64_t N, int64_t K, int8_t* q);
void orc_scales_q4(const uint8_t* W, int64_t N, int64_t K, uint16_t* s);
void orc_dequant_q4(const uint8_t* W, int64_t N, int64_t K, uint16_t* out);

/* y = fp32(dequant(W)) @ fp32(x), the value before the final bf16 cast
 * (tools/ref/gemv_q.py:73-80). */
void orc_gemv_q(const uint8_t* W, const float* x, float* y, int64_t N, int64_t K,
                int threads);
/* Same product accumulated in fp64 (error analysis only). */
void orc_gemv_q_f64(const uint8_t* W, const float* x, double* y, int64_t N, int64_t K,
                    int threads);
/* Y[M,N] = X[M,K] @ dequant(W)^T (runtime/py/model.py:1049-1111). */
void orc_gemm_q(const uint8_t* W, const float* X, float* Y, int64_t M, int64_t N,
                int64_t K, int threads);

/* GeGLU / SwiGLU activation with the reference's rounding points
 * (runtime/py/model.py:797-804 gelu; :853-858 silu). g, u are the already
 * bf16-rounded gate/up values; a receives bf16-valued floats. */
void orc_glu(const float* g, const float* u, float* a, int64_t n, int act);
/* Whole FFN for M tokens (runtime/py/model.py:797-806, :853-860). */
void orc_ffn(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, const float* X,
             float* Y, int64_t M, int64_t H, int64_t I, int act, int threads);
/* FFN with fp64 accumulation of the three matvecs; the bf16 rounding points
 * are kept (error analysis only). */
void orc_ffn_f64(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, const float* x,
                 double* y, int64_t H, int64_t I, int act);

/* quantize_to_q4_0 + pack_to_combined (tools/convert/gemv_q_convert.py:5-85). */
void orc_quantize_q4_0(const float* Wf, int64_t N, int64_t K, uint8_t* out);

/* Seeded synthetic inputs (counter-based SplitMix64). */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t i);
void orc_synth_q4(uint8_t* W, int64_t N, int64_t K, uint64_t seed, float smin, float smax);
void orc_synth_uniform(float* x, int64_t n, uint64_t seed, float lo, float hi);
void orc_synth_normal(float* x, int64_t n, uint64_t seed);

/* CPU-baseline timing helpers: the reference's per-call work (dequantize the
 * whole matrix to fp32, then matvec) and its pre-dequantized variant
 * (runtime/py/model.py:134-145). Return seconds for `iters` calls. */
double orc_time_gemv_faithful(const uint8_t* W, const float* x, float* y, int64_t N,
                              int64_t K, int iters, int threads);
double orc_time_gemv_predequant(const uint8_t* W, const float* x, float* y, int64_t N,
                                int64_t K, int iters, int threads);
double orc_time_ffn_faithful(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                             const float* x, float* y, int64_t H, int64_t I, int iters,
                             int threads);
double orc_time_ffn_predequant(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                               const float* x, float* y, int64_t H, int64_t I, int iters,
                               int threads);
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
