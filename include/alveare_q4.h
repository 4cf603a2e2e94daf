/*
 * alveare_q4 -- C ABI of the MI355X (gfx950) Q4 decode hot path.
 *
 * Drop-in for the three quantized-matmul backends of Alveare's runtime:
 * gemv_q, ffn_fused and gemm_q. Weights are in the layout `alveare quantize`
 * emits: per row, K/32 blocks of 20 bytes (16 bytes of two's-complement
 * nibbles, low nibble = even column; a little-endian bf16 scale; 2 zero
 * bytes), i.e. uint8 (N, K/32*20) row-major (tools/convert/gemv_q_convert.py:53-85,
 * kernels/gemv_q/README.md:13-23).
 *
 * Numerics are those of the reference's fp32 CPU path
 * (tools/ref/gemv_q.py:73-80, runtime/py/model.py:797-806):
 *   w = bf16_RNE(f32(q) * f32(scale)),  y = sum_k w[k] * x[k] in fp32.
 * Outputs are the fp32 values before the reference's final `.astype(bfloat16)`;
 * a caller that wants the reference's bf16 result rounds them to nearest even.
 *
 * Conventions:
 *  - All pointers are device pointers (hipMalloc / torch tensors), except where
 *    noted. `stream` is a hipStream_t (NULL = the null stream). Work is
 *    enqueued asynchronously on it; nothing blocks the host.
 *  - Every entry point returns ALV_OK (0) or a negative ALV_ERR_* status and
 *    never throws. alv_last_error() returns a message for the calling thread's
 *    last failure.
 *  - K must be a positive multiple of 32; N, M, H, I positive. Activations are
 *    dense fp32, row-major, with the given leading dimensions (in elements).
 *  - Calls on different streams may run concurrently; calls that share an FFN
 *    handle must be serialised on one stream (the handle owns its decode
 *    activation buffer).
 *  - Temporaries that grow with a call's shape (split-K partial sums and
 *    arrival counters of multi-token decode launches, prefill activations and
 *    partial tiles) live in buffers the library keeps per (device, stream).
 *    A call that fits what its stream already holds allocates nothing; one
 *    that does not allocates a larger buffer and keeps the old one allocated
 *    (a HIP graph captured earlier may still use it). Allocation cannot
 *    happen during HIP graph capture (ALV_ERR_ARG): run one call of each
 *    shape on the stream before capturing. Up to 64 streams per device.
 *    A captured graph uses the buffers of the stream it was captured on.
 */
#ifndef ALVEARE_Q4_H
#define ALVEARE_Q4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ALV_OK 0
#define ALV_ERR_ARG (-1)      /* null pointer, bad shape, bad activation id */
#define ALV_ERR_ALIGN (-2)    /* pointer alignment the kernels need is not met */
#define ALV_ERR_HANDLE (-3)   /* invalid or mismatched FFN handle */
#define ALV_ERR_HIP (-4)      /* a HIP runtime call failed */
#define ALV_ERR_RANGE (-5)    /* a size exceeds what the kernels address */

#define ALV_ACT_GELU_TANH 0   /* Gemma: gelu_pytorch_tanh (runtime/py/model.py:802) */
#define ALV_ACT_SILU 1        /* Llama: x*sigmoid(x) (runtime/py/model.py:856) */

typedef struct alv_ffn* alv_ffn_t;
typedef struct alv_weight* alv_weight_t;

/* Message for the calling thread's last failed call ("" if none). */
const char* alv_last_error(void);

/* Library version, e.g. "alveare_q4 1.0 gfx950". */
const char* alv_version(void);

/*
 * y[N] = dequant(W)[N,K] @ x[K].
 * Replaces the gemv_q NPU op: IRON `gemv_q_npu(W, X, Y, *, N, K, m, k_tile)`
 * (kernels/gemv_q/gemv_q.py:33-42) and NpuRegistry::run_gemv
 * (runtime/cpp/include/alveare/npu.h:78-80, runtime/cpp/src/npu.cpp:269-288).
 * W needs 4-byte alignment; x and y 4-byte alignment.
 */
int alv_gemv_q(const uint8_t* W, const float* x, float* y, int N, int K, void* stream);

/*
 * Y[M,N] = X[M,K] @ dequant(W)^T, rows of X/Y at leading dimensions ldx/ldy.
 * Replaces IRON `gemm_q_npu(W, X, Y, *, B, N, K, m, k_tile)`
 * (kernels/gemm_q/gemm_q.py:28-39) and NpuRegistry::run_gemm
 * (runtime/cpp/include/alveare/npu.h:82-87, runtime/cpp/src/npu.cpp:290-310).
 * M is any positive token count (the reference's B=16 chunking is not needed).
 * M <= 32 runs the streaming GEMV kernel (16 tokens per launch), M >= 33 the
 * MFMA tiled kernel, both reading the combined layout directly.
 */
int alv_gemm_q(const uint8_t* W, const float* X, float* Y, int M, int N, int K,
               int ldx, int ldy, void* stream);

/*
 * Register one projection: W is (N, K/32*20) in the combined Q4 layout on the
 * device. The handle keeps its own device copy in the kernels' tiled layout
 * (the caller may free W after the call returns). Synchronises `stream`.
 * Replaces NpuRegistry::create_gemv_weight (runtime/cpp/include/alveare/npu.h:68-69,
 * runtime/cpp/src/npu.cpp:241-253); the reference also registers weights once
 * and keeps them device-resident (runtime/py/model.py:31-35 ResidentWeight).
 * Trailing rows and 32-column blocks whose weights are all zero (the zero
 * padding of the reference's Gemma-4 shapes: K 3840 stored as 4096,
 * tools/quantize_gemma4.py:145-187; the sliding O projection padded to 8192
 * rows, runtime/cpp/src/weights.cpp:318-327) are not copied: calls stream the
 * nonzero part and write exact zeros to the trimmed output rows, the
 * reference's values there up to the sign of zero.
 */
int alv_weight_register(const uint8_t* W, int N, int K, alv_weight_t* out, void* stream);

/* Shape of a registered projection as registered (either pointer may be NULL). */
int alv_weight_shape(alv_weight_t w, int* N, int* K);

/* Shape a registered projection executes at: its rows and columns up to the
 * last nonzero weight (rounded up to a 32-column block). No reference
 * counterpart: it reports what alv_weight_register trimmed. */
int alv_weight_exec_shape(alv_weight_t w, int* N, int* K);

/*
 * Y[M,N] = X[M,K] @ dequant(W)^T with W registered; rows of X/Y at leading
 * dimensions ldx/ldy. M = 1 is the decode GEMV, small M the streaming kernel,
 * M >= 33 the MFMA tiled kernel (ALV_TILED_MIN_M overrides the threshold).
 * Replaces NpuRegistry::run_gemv / run_gemm (runtime/cpp/include/alveare/npu.h:78-87,
 * runtime/cpp/src/npu.cpp:269-310).
 */
int alv_gemv(alv_weight_t w, const float* X, float* Y, int M, int ldx, int ldy, void* stream);

/*
 * alv_gemv with bf16 activations and outputs (bit patterns): Y = bf16(X W^T),
 * the reference's run_gemv(N, K, w, x_bf16, y_bf16) contract
 * (runtime/cpp/include/alveare/npu.h:78-87; runtime/py/model.py:283-362
 * run_gemv_npu returns bf16). X rows 16-byte aligned (ldx a multiple of 8).
 * bf16 activations take the MFMA tiled kernel from M = 17 (one term per
 * activation on both kernels moves the crossover down; ALV_TILED_MIN_M
 * overrides it).
 */
int alv_gemv_bf16(alv_weight_t w, const uint16_t* X, uint16_t* Y, int M, int ldx, int ldy, void* stream);

/* Free a handle from alv_weight_register (NULL is a no-op). Synchronises the
 * device before freeing. */
void alv_weight_release(alv_weight_t w);

/*
 * LM head of a decode step on a registered projection w (N rows >= vocab,
 * K columns): logits[i] = softcap * tanh(bf16(W x)[i] / softcap) in float32
 * for i < vocab (softcap = 0: the bf16 logits themselves), and *argmax = the
 * first index of the largest logit, NaN counting as largest (np.argmax).
 * x is K fp32 values; logits (vocab floats) and argmax (one int32) are device
 * memory. Replaces the head GEMV chunks of Generator::run_lm_head
 * (runtime/cpp/src/generator.cpp:28-52, weights uploaded at
 * runtime/cpp/src/weights.cpp:198-224) with Generator::sample's greedy pick
 * (generator.cpp:15-26), and the Python head with its softcap
 * (runtime/py/model.py:904-916) and sampler (runtime/py/sampler.py:9).
 */
int alv_lm_head(alv_weight_t w, const float* x, float* logits, int vocab, float softcap, int32_t* argmax,
                void* stream);

/*
 * alv_lm_head with x as K bf16 values (bit patterns, 16-byte aligned), the
 * head's input as the reference produces it (the final norm's bf16 output,
 * runtime/py/model.py:907-912): one MFMA term per value where alv_lm_head
 * splits its fp32 x into three; the same logits and token as alv_lm_head on
 * the bf16 values widened to fp32, bit for bit. pos_dev (optional, device
 * int32; NULL: none) is a decode position the call also advances: the token
 * is written as -1 when *pos_dev >= max_pos, then *pos_dev += 1 -- the
 * bookkeeping of a device-resident decode step (alveare_amd.layer.Gemma4Decoder)
 * inside the head's last launch. No counterpart in the reference for pos_dev.
 */
int alv_lm_head_bf16(alv_weight_t w, const uint16_t* x, float* logits, int vocab, float softcap, int32_t* argmax,
                     int32_t* pos_dev, int max_pos, void* stream);

/*
 * alv_lm_head_bf16 on the final norm of the last layer's residual step, the
 * step inside the head GEMV's launch (as alv_gemv_bf16_addnorm): s =
 * resid_step(y, resid) -> sum_out, x = bf16(rmsnorm(s) * w_x) over the
 * first `hidden` values, zero-padded to the head's K -- the same bits as
 * alv_add_norm (pad = K) followed by alv_lm_head_bf16 on its norm_out
 * (runtime/py/model.py:783-788, then :907-916 with the final norm;
 * model.cpp:409-420 and generator.cpp:28-52). hidden <= K, a multiple of 8
 * up to 8192; y may be NULL (no step: x is the norm of resid itself).
 */
int alv_lm_head_bf16_addnorm(alv_weight_t w, const uint16_t* resid, const uint16_t* y, const float* w_y, int norm_y,
                             float scale, int scale_mode, uint16_t* sum_out, const float* w_x, float eps, int hidden,
                             float* logits, int vocab, float softcap, int32_t* argmax, int32_t* pos_dev, int max_pos,
                             void* stream);

/*
 * Quantize float32 weights to the Q4 combined layout on the GPU:
 * quantize_to_q4_0 + pack_to_combined (tools/convert/gemv_q_convert.py:5-85)
 * with the zero padding of quantize_and_pack_tensor
 * (tools/quantize_gemma4.py:26-41). W holds n_src rows of ldw floats (the
 * first k_src of each are read); out receives the (N, K/32*20) combined
 * matrix, N >= n_src, K >= k_src, K a multiple of 32, weights past the source
 * quantized as zeros. Per block: scale = max|w| / 7 (float32; 0 -> 1.0; NaN
 * if the block holds a NaN), codes clip(round-half-even(w / scale), -8, 7)
 * with a NaN quotient -> -8 (numpy on x86-64), bf16 scale round-to-nearest-even.
 * W and out need 4-byte alignment. Asynchronous on `stream`.
 */
int alv_quantize_q4(const float* W, int n_src, int k_src, int ldw, uint8_t* out, int N, int K, void* stream);

/*
 * alv_quantize_q4 straight into a registered projection (the kernels' tiled
 * layout; a temporary combined copy is allocated and freed). The counterpart
 * of quantizing on the host and registering with create_gemv_weight
 * (runtime/cpp/src/weights.cpp:192-330). Synchronises `stream`.
 */
int alv_weight_quantize(const float* W, int n_src, int k_src, int ldw, int N, int K, alv_weight_t* out,
                        void* stream);

/*
 * The kernels' tiled layout of a combined-layout matrix: byte size (0 for a
 * bad shape) and the repack itself into `out` (device, alv_q4_tiled_bytes
 * bytes). Test / parity entry points: registration performs this repack, the
 * counterpart of the reference's registration-time repack of FFN weights
 * (runtime/cpp/src/weights.cpp:94-190). W and out need 4-byte alignment.
 */
uint64_t alv_q4_tiled_bytes(int N, int K);
int alv_q4_tile(const uint8_t* W, uint8_t* out, int N, int K, void* stream);

/*
 * Register one FFN layer: Wg, Wu are (I, H/32*20), Wd is (H, I/32*20), all in
 * the combined Q4 layout, on the device. The handle keeps its own device copy
 * in the kernels' layout (the caller may free its buffers after the call
 * returns) plus scratch for the activation. act is ALV_ACT_*.
 * Replaces NpuRegistry::create_ffn_fused_weight (npu.h:70-71, npu.cpp:255-267)
 * together with the registration-time repack pack_ffn_fused_weights
 * (runtime/cpp/src/weights.cpp:94-190; kernels/ffn_fused/ffn_fused.py:330-395).
 * Trailing all-zero hidden / intermediate rows and columns (the reference's
 * 15360 x 3840 FFN stored as 16384 x 4096, tools/quantize_gemma4.py:177-187)
 * are trimmed as in alv_weight_register: their activations and outputs are
 * exact zeros. Synchronises `stream` before returning.
 */
int alv_ffn_register(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, int H, int I,
                     int act, alv_ffn_t* out, void* stream);

/* The (H, I) a registered FFN executes at after trimming (either pointer may
 * be NULL). No reference counterpart. */
int alv_ffn_exec_shape(alv_ffn_t w, int* H, int* I);

/*
 * Y[M,H] = down(GLU(gate X, up X)) with the reference CPU path's bf16 rounding
 * points: g = bf16(Wg x), u = bf16(Wu x), a = bf16(act(g) * u), y = Wd a (fp32).
 * Replaces IRON `ffn_fused_npu(W_fused, X, Y_partial, *, H, I, m_I, k_tile,
 * activation)` (kernels/ffn_fused/ffn_fused.py:28-39) plus the host sum of
 * the per-core partials (runtime/cpp/src/npu.cpp:340-378,
 * runtime/py/model.py:363-397); the sum is done on the device.
 * X and Y are (M, H) row-major with leading dimensions ldx, ldy.
 */
int alv_ffn_fused(alv_ffn_t w, const float* X, float* Y, int M, int ldx, int ldy,
                  void* stream);

/*
 * alv_ffn_fused with bf16 activations and outputs (bit patterns): the
 * reference's run_ffn_fused(H, I, act, w, x_bf16, y_bf16)
 * (runtime/cpp/include/alveare/npu.h:90-97, runtime/cpp/src/npu.cpp:340-378:
 * partials summed in float32, then bf16). Same rounding points as
 * alv_ffn_fused; Y = bf16(down). X rows 16-byte aligned (ldx a multiple of 8).
 * Tiled (MFMA) kernels from M = 17, as for alv_gemv_bf16.
 */
int alv_ffn_fused_bf16(alv_ffn_t w, const uint16_t* X, uint16_t* Y, int M, int ldx, int ldy, void* stream);

/*
 * alv_ffn_fused for M <= 16 tokens (decode and small-M verification) that
 * allocates nothing: the split-K partial sums and arrival counters of its
 * launches (gate/up and down, each followed by a summing launch when it splits
 * K four ways or more) live in a fixed 16 MiB + 4 KiB array in device memory, one per GPU
 * the library runs on, held until the process ends; X, Y and the handle are
 * the caller's as in alv_ffn_fused. Calls no hipMalloc / hipFree, so it may run
 * under HIP graph capture, inside tight serving loops and in harnesses that
 * forbid allocation. Results are bit-identical to alv_ffn_fused. A shape whose
 * partial sums exceed 16 MiB is rejected with ALV_ERR_RANGE before anything is
 * enqueued; M > 16 is ALV_ERR_ARG. Every call on one GPU shares that array:
 * calls that overlap on one GPU (concurrent streams, or replays of graphs that
 * captured this call while other such calls run) race and must be serialised.
 * No counterpart in the reference: it exists for callers that cannot allocate.
 */
int alv_ffn_fused_noalloc(alv_ffn_t w, const float* X, float* Y, int M, int ldx, int ldy, void* stream);

/*
 * out[M, I] = the activation a = bf16(act(g) * u) of the handle's last
 * alv_ffn_fused call (fp32 holding bf16 values), for M up to that call's
 * token count (all tokens when it had M <= 16 or ran the tiled kernel, M >= 33
 * for fp32 activations and M >= 17 for bf16; otherwise the last 16-token
 * chunk). Test / parity entry point: lets a checker separate the
 * bf16 rounding points from the down projection.
 */
int alv_ffn_activation(alv_ffn_t w, float* out, int M, void* stream);

/*
 * The first of alv_ffn_fused's two launches alone: a = bf16(act(g) * u) for
 * M <= 16 tokens into the handle's scratch (read it with alv_ffn_activation).
 * Measurement / parity entry point: it times and checks the gate/up kernel by
 * itself. The reference runs both phases inside one NPU kernel
 * (kernels/ffn_fused/ffn_fused.py:28-39).
 */
int alv_ffn_gate_up(alv_ffn_t w, const float* X, int M, int ldx, void* stream);

/*
 * The first of the one-token FFN's two launches alone (alv_ffn_fused at M = 1
 * runs it, then sums): each of the G = I / 64 workgroups computes gate, up
 * and the activation of its 64 intermediate rows and multiplies the matching
 * 64 columns of the down matrix into a partial output, P[b * H' + r] for
 * b < G, r < H' (H' = the executed hidden size, alv_ffn_exec_shape; P NULL:
 * the handle's buffer). Replaces the reference's ffn_fused_npu with its
 * Y_partial output of one row per core (kernels/ffn_fused/ffn_fused.py:28-328),
 * which the reference's host sums (runtime/cpp/src/npu.cpp:360-377). *slices
 * (if not NULL) receives G. One fp32 token; ALV_ERR_ARG for a registration
 * without the one-launch form (I not a multiple of 64, H not a multiple of
 * 128 above 512). The activation is readable with alv_ffn_activation.
 */
int alv_ffn_partials(alv_ffn_t w, const float* X, float* P, int* slices, void* stream);

/* Shape of a registered FFN (any output pointer may be NULL). *//* Shape of a registered FFN (any output pointer may be NULL). */
int alv_ffn_shape(alv_ffn_t w, int* H, int* I, int* act);

/* Free a handle from alv_ffn_register (NULL is a no-op). Synchronises the
 * device before freeing. */
void alv_ffn_release(alv_ffn_t w);

/*
 * ---- host ops of a decode layer (bf16 tensors as uint16 bit patterns) ----------
 * The work the reference does on the CPU between its matmuls
 * (runtime/py/model.py:522-628, :705-790; runtime/cpp/src/model.cpp:127-262,
 * :314-420). Elementwise steps and RMSNorm are bit-exact with the reference's
 * numpy float32 arithmetic (numpy >= 2; RMSNorm's mean uses numpy's pairwise
 * summation order); attention is float32 with its own summation order.
 * `pos_dev` is a device int holding the decode position, so captured graphs
 * replay for every token. All asynchronous on `stream`.
 */

/*
 * out[r, :K] = bf16(x * (1 / sqrt(mean(x^2) + eps)) * w) for rows r < rows
 * (w NULL: no weight), out[r, K:pad] = 0 (the reference pads 3840 -> 4096,
 * runtime/cpp/src/model.cpp:334-336). run_rmsnorm_cpu (runtime/py/model.py:522-531;
 * model.cpp:127-141). K <= 20480.
 */
int alv_rmsnorm(const uint16_t* x, const float* w, uint16_t* out, int rows, int K, int ldx, int ldo, int pad,
                float eps, void* stream);

/*
 * After the QKV projection: per-head RMSNorm of q (weights q_w), k (k_w) and,
 * when norm_v, of v without weights (Gemma-4); RoPE of q and k with the bf16
 * table row `rope + pos * rope_stride` (cos at cos_off, sin at sin_off, pairs
 * (i, i + half)); q to q_out [heads][D]; k and v into the caches at pos
 * ([kv_heads][max_seq][D]). qkv holds q at 0, k at k_off and v at v_off
 * (v_off < 0: v is the un-normalised k, Gemma-4 global layers). rope NULL: no
 * rotation; otherwise the table holds max_seq rows of rope_stride values.
 * model.py:742-770; model.cpp:357-404.
 */
int alv_qkv_post(const uint16_t* qkv, int k_off, int v_off, int heads, int kv_heads, int D, const float* q_w,
                 const float* k_w, int norm_q, int norm_k, int norm_v, float eps, const uint16_t* rope,
                 int rope_stride, int cos_off, int sin_off, int half, const int* pos_dev, int max_seq,
                 uint16_t* q_out, uint16_t* kcache, uint16_t* vcache, void* stream);

/*
 * out[h] = softmax(scale * K q[h]) V over cache positions [start, pos] of kv
 * head h / (heads / kv_heads), start = pos + 1 - window for a sliding layer
 * (window > 0), else 0; float32 scores and softmax, bf16 out [heads][D].
 * run_attention_host (runtime/py/model.py:577-628; model.cpp:185-262). D one
 * of 64, 128, 256, 512; q, kcache and vcache 16-byte aligned; at most 65536
 * positions in the window. Two launches (chunk partials, then their merge);
 * uses per-stream scratch (grown outside graph capture).
 */
int alv_attention(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, uint16_t* out, int heads,
                  int kv_heads, int D, int max_seq, int window, float scale, const int* pos_dev, void* stream);

/*
 * alv_qkv_post followed by alv_attention in the attention's launches: the
 * attention workgroups normalise and rotate q, k and v from the QKV output
 * themselves (alv_qkv_post's arithmetic, bit for bit) while their K/V loads
 * are in flight, insert k and v at pos into the caches and use them in place
 * of the rows the caches held; q_out (optional) receives the rotated q.
 * Arguments as the two calls'; the reference runs the same two steps one
 * after the other (runtime/py/model.py:742-770 then :577-628).
 */
int alv_qkv_attention(const uint16_t* qkv, int k_off, int v_off, int heads, int kv_heads, int D, const float* q_w,
                      const float* k_w, int norm_q, int norm_k, int norm_v, float eps, const uint16_t* rope,
                      int rope_stride, int cos_off, int sin_off, int half, const int* pos_dev, int max_seq,
                      uint16_t* q_out, uint16_t* kcache, uint16_t* vcache, int window, float scale, uint16_t* out,
                      void* stream);

/*
 * Residual step of a layer, per row: t = norm_y ? bf16(rmsnorm(y) * w_y) : y;
 * s = bf16(resid + t), then scale_mode 1: s = bf16(s * scale) (the Python
 * runtime's two roundings, model.py:783-788), 2: s = bf16((resid + t) * scale)
 * (the C++ runtime's one rounding, model.cpp:410-416), 0: no scale; sum_out = s;
 * norm_out (optional) = bf16(rmsnorm(s) * w_out) zero-padded to pad.
 * model.py:775-788; model.cpp:409-420.
 */
int alv_add_norm(const uint16_t* resid, int ldr, const uint16_t* y, int ldy, const float* w_y, int norm_y,
                 float scale, int scale_mode, uint16_t* sum_out, int ld_sum, const float* w_out, uint16_t* norm_out,
                 int ld_norm, int rows, int K, int pad, float eps, void* stream);

/*
 * The residual step fused into the next one-token matmul: alv_add_norm of one
 * row (resid, y, w_y, norm_y, scale, scale_mode -> sum_out; w_x the next
 * norm's weights, pad = K) followed by alv_gemv_bf16 / alv_ffn_fused_bf16 of
 * that norm at M = 1, in the matmul's own launch -- its workgroups compute the
 * normalised activation themselves (the same float32 steps and numpy
 * summation order, so every output bit equals the two-call sequence); no
 * launch, and no activation round trip through memory, sits between them.
 * This is how a decode layer moves from its attention output into the FFN
 * (runtime/py/model.py:775-788 then :797-806; model.cpp:409-420 then the FFN)
 * and from the FFN into the next layer's QKV (:783-788 then :705-713).
 * K = the weight's K (the FFN's H), a multiple of 8 up to 8192; rows and
 * weights 16-byte aligned; sum_out must not alias resid or y. y NULL: no
 * residual step, the activation is bf16(rmsnorm(resid) * w_x) as alv_rmsnorm
 * writes it (a first layer's input norm) and sum_out is not written.
 */
int alv_gemv_bf16_addnorm(alv_weight_t w, const uint16_t* resid, const uint16_t* y, const float* w_y, int norm_y,
                          float scale, int scale_mode, uint16_t* sum_out, const float* w_x, float eps, uint16_t* Y,
                          void* stream);
int alv_ffn_fused_bf16_addnorm(alv_ffn_t w, const uint16_t* resid, const uint16_t* y, const float* w_y, int norm_y,
                               float scale, int scale_mode, uint16_t* sum_out, const float* w_x, float eps,
                               uint16_t* Y, void* stream);

/*
 * out[:H] = bf16(float(double(table_f16[*token_dev]) * scale)), the Gemma-4
 * embedding lookup with scale = sqrt(hidden_size) (runtime/py/model.py:889-891:
 * a float64 product cast to bf16 through float32). The token is read from
 * device memory (the previous step's argmax); a token outside [0, vocab)
 * writes zeros.
 */
int alv_embed(const uint16_t* table_f16, int vocab, int H, const int32_t* token_dev, double scale, uint16_t* out,
              void* stream);

/*
 * One op of a chain: a registered projection (y = W x) or a registered FFN
 * layer (y = ffn(x)); exactly one of `weight` and `ffn` is set. x and y are
 * device fp32 buffers of M rows (leading dimension K, resp. N or H). dep is
 * the index of an earlier op whose output this op reads (its x points into
 * that op's y), or -1 when x is ready before the call.
 */
typedef struct {
    alv_weight_t weight;
    alv_ffn_t ffn;
    const float* x;
    float* y;
    int dep;
} alv_chain_op;

/*
 * Run ops[0..n) in order on `stream`, enqueued by one call with no host
 * waits between them (stream order satisfies each dep). Results equal
 * running the ops one after another through alv_gemv / alv_ffn_fused. M is
 * the token count (1..16). An FFN handle may appear more than once.
 * Device-side counterpart of the reference's per-layer dispatch, which calls
 * NpuRegistry::run_gemv / run_ffn_fused one after another
 * (runtime/cpp/src/model.cpp:265-420, runtime/py/model.py:632-818).
 */
int alv_chain_run(const alv_chain_op* ops, int n, int M, void* stream);

/*
 * out[N,K] = bf16 bit patterns of dequant(W). Test / parity entry point: the
 * reference materialises this matrix in dequantize_combined
 * (tools/ref/gemv_q.py:39-62).
 */
int alv_dequant_q4(const uint8_t* W, uint16_t* out, int N, int K, void* stream);

/*
 * out[i] = bf16(act(g[i]) * u[i]) (as fp32) with the arithmetic of the FFN
 * epilogue, act = ALV_ACT_GELU_TANH or ALV_ACT_SILU. Test / parity entry
 * point: the reference evaluates this elementwise on the CPU
 * (runtime/py/model.py:800-803 for GeGLU, :856 for SiLU).
 */
int alv_glu(const float* g, const float* u, float* out, int64_t n, int act, void* stream);


#ifdef __cplusplus
}
#endif
#endif /* ALVEARE_Q4_H */
