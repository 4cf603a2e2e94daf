// Host-side internals of libalveare_q4: error reporting, per-stream
// workspace, and the launch plan of the streaming GEMV kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/alveare_q4.h"

namespace alv {

// Record a failure for alv_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
int hip_check(hipError_t e, const char* what);

// Per-(device, stream) arrival counters of the streaming GEMV's split-K
// launches. They are zero when a launch starts and every launch leaves them
// zero. A device's counters (a set for each of up to 64 streams) are
// allocated at its first call, which synchronises the device; later calls, a
// stream's first included, allocate nothing.
struct Workspace {
    uint32_t* counters = nullptr;
    size_t counter_count = 0;
};
int get_workspace(hipStream_t s, size_t counters, Workspace* out);

// Per-(device, stream, slot) scratch of at least `bytes`, zeroed when
// allocated, for launches whose temporaries grow with their shape: slot 0 the
// prefill GEMM's (token flags, partial tiles, activation terms), slot 1 the
// streaming GEMV's split-K partial sums (rewritten by every such launch before
// it is read), slot 2 the FFN activation of prefill-sized calls, slot 3 the
// LM head's argmax pairs, slot 4 attention's chunk partials. No slot holds
// arrival counters: a slot's layout changes with the shape, so bytes one call
// leaves behind sit where another call would count (get_workspace holds them).
// A call that
// fits what the slot holds allocates nothing. Growing allocates a new block
// (at least twice the old capacity) and keeps the old one allocated for the
// life of the process, since a HIP graph captured earlier may still use it;
// growth is refused during graph capture. A graph captured on a stream uses
// that stream's blocks, so its replays must not overlap other calls on it.
constexpr int kScratchGemm = 0;
constexpr int kScratchSplit = 1;
constexpr int kScratchAct = 2;
constexpr int kScratchHead = 3;  // the LM head's per-workgroup argmax pairs
constexpr int kScratchAttn = 4;  // attention's chunk partials
int get_scratch(hipStream_t s, int slot, size_t bytes, void** out);
// Largest split-K partial-sum block of one streaming GEMV launch.
constexpr size_t kPartMax = 256u << 20;

// Split-K temporaries a caller provides in place of the per-stream ones:
// kSplitCounters arrival counters (zero between launches; every launch leaves
// them zero) and `part_bytes` of partial sums. A launch whose partial sums do
// not fit fails with ALV_ERR_RANGE before anything is enqueued.
struct SplitBuf {
    uint32_t* counters = nullptr;
    float* part = nullptr;
    size_t part_bytes = 0;
};

// One product on the streaming kernel (gemv1_q.hip), M <= kGemvMaxM tokens:
//   out[m, n] = sum_k X[m, k] * dequant(W0)[n, k]            (glu == false)
//   out[m, n] = act(bf16(X W0^T), bf16(X W1^T)) rounded to bf16 (glu == true)
// parts = 3 splits fp32 X exactly into three bf16 terms; parts = 1 requires X
// to hold bf16 values (the FFN's activation does). The activations are either
// fp32 (X) or bf16 bit patterns (Xb, parts = 1, no GLU); the output is fp32
// (Y) or bf16 bit patterns (Yb). Weights in the tiled layout (q4_device.h) or,
// for fp32 activations without a GLU, the combined layout.
// A decode layer's residual step fused ahead of a one-token bf16 GEMV: the
// workgroups compute the activation x = bf16(rmsnorm(s) [* w_x]) themselves
// from s = resid_step(y, resid) (row_norm.h), workgroup 0 also writing s to
// sum_out, so the separate alv_add_norm launch and its output round trip go.
// y null: no step, s = resid (the input norm alone; sum_out is not written).
struct ResidStep {
    const uint16_t* resid = nullptr;
    const uint16_t* y = nullptr;
    const float* w_y = nullptr;  // null: y's norm has no weight
    int norm_y = 1;
    float scale = 1.0f;
    int scale_mode = 0;
    uint16_t* sum_out = nullptr;
    const float* w_x = nullptr;  // null: the activation's norm has no weight
    float eps = 1e-6f;
    int k = 0;  // width of resid / y / sum_out / w_x (0: the matmul's K); activation values past it are zeros
};
// Widest row a fused residual step takes (one octet per thread of the
// 1024-thread workgroup, the float row in LDS).
constexpr int kResidStepMaxK = 8192;

struct GemvLaunch {
    const uint8_t* W0 = nullptr;
    const uint8_t* W1 = nullptr;
    const float* X = nullptr;
    const uint16_t* Xb = nullptr;
    int ldx = 0;
    float* Y = nullptr;
    uint16_t* Yb = nullptr;
    int ldy = 0;
    int M = 0, N = 0, K = 0;
    int parts = 3;
    bool glu = false;
    bool tiled = false;  // weights in the tiled layout (q4_device.h) instead of the combined one
    int act = ALV_ACT_GELU_TANH;
    const SplitBuf* split = nullptr;  // caller's split-K temporaries (nullptr: the stream's)
    const ResidStep* step = nullptr;  // fused residual step (M = 1, bf16 activation; nullptr: X / Xb as given)
    // Output rows [N, Nz) of every token are written as zeros (the all-zero
    // trailing rows a registration trimmed off, see weight_extent); Nz <= N: none.
    int Nz = 0;
};
int launch_gemv(const GemvLaunch& L, hipStream_t s);
// The split-K partial-sum bytes launch_gemv(L) needs (0: no launch splits K),
// or -1 when the shape has no launch plan.
int64_t gemv_split_bytes(const GemvLaunch& L);

// Arrival counters per stream: one per tile group of a split-K launch.
constexpr int kSplitCounters = 1024;

// Repack W (combined layout, N x K, rows `rs` bytes apart; 0: K / 32 * 20)
// into the tiled layout at `out` (tile_bytes(N, K) bytes), on `s` (tile_q.hip).
int launch_tile(const uint8_t* W, uint8_t* out, int N, int K, hipStream_t s, uint32_t rs = 0);
uint64_t tile_bytes(int N, int K);

// The part of a combined-layout matrix (N x K, rows `rs` bytes apart) that
// holds nonzero weights: ext[0] = 1 + its last row with a nonzero weight,
// ext[1] = 1 + its last 32-column block with one (0 and 0 when every weight
// is zero). A block's 32 weights bf16(q * s) are all zero exactly when its
// scale is +-0, or its codes are all zero and its scale is finite. Enqueued
// on `s`, then synchronised (tile_q.hip).
int weight_extent(const uint8_t* W, int N, int K, uint32_t rs, hipStream_t s, int ext[2]);

// Largest M the streaming kernel takes in one launch (3 * 16 = 48 A rows).
constexpr int kGemvMaxM = 16;

// MFMA tiled kernel for prefill-sized M (gemm_q.hip). Same contract as
// GemvLaunch (glu pairs W0/W1 into the activation).
int launch_gemm_tiled(const GemvLaunch& L, hipStream_t s);

// M at and above which the tiled kernel runs a product (below it the
// streaming kernel, 16 tokens per launch), by activation type: bf16
// activations (one term on both kernels) kTiledMinMBf16, fp32 ones (three
// terms on both unless bf16-valued) kTiledMinMF32; the positive value of the
// environment variable ALV_TILED_MIN_M, read at each call, overrides both (a
// tuning knob; the benchmark times both kernels at small M with it).
// Measured on the 12B-class FFN (3840 <-> 15360), 16 distinct layers, µs
// per call: streaming 53-56 at 16 tokens and 82-84 at 17 (two launches);
// tiled with 64-token tiles 78-80 for any M up to 64 with bf16-valued
// activations and 133-138 with fp32 ones; so from 17 tokens the tiled kernel
// wins for bf16 (78 against 82), and from 33 for fp32 (streaming 106 at 32,
// 148 at 40, against 135-138).
constexpr int kTiledMinMBf16 = 17;
constexpr int kTiledMinMF32 = 33;
int tiled_min_m(bool fp32_x);
// Largest M the prefill GEMM runs with 64-token tiles (256-token tiles above);
// ALV_GEMM_SMALL_TILE_MAX_M overrides.
constexpr int kSmallTileMaxM = 128;
int small_tile_max_m();
// Workgroups per CU the 64-token prefill tiles aim at when splitting K
// (default 1); ALV_GEMM_SMALL_WG_PER_CU overrides.
int small_wg_per_cu();
// Compute units of the current device (cached per device).
int device_cus();

// The two launches of one FFN call on handle w (ffn_fused.hip): gate/up with
// the GLU epilogue into the bf16 activation `act`, then down from it.
void ffn_ops(alv_ffn_t w, uint16_t* act, const float* X, int ldx, float* Y, int ldy, int M, GemvLaunch (&op)[2]);

// The one-token FFN in one launch (gemv1_q.hip, q4_ffn1_kernel, then the
// partials' sum): `up` is the gate/up launch of ffn_ops at M = 1; Wv the
// down slices (vbytes), part G x 128 U floats, act the handle's activation;
// the output (Y fp32 or Yb bf16) has H rows, zeros past 128 U. sum = false:
// the partials only (alv_ffn_partials).
int launch_ffn1(const GemvLaunch& up, const uint8_t* Wv, uint64_t vbytes, float* part, uint16_t* act, int G, int U,
                int H, float* Y, uint16_t* Yb, hipStream_t s, bool sum = true);

// The launch of registered matrix w (tile_q.hip): weights, executed shape and
// the zero rows up to its logical N; the caller adds activations and M.
void weight_launch(const struct alv_weight* w, GemvLaunch& L);

}  // namespace alv

namespace alv {
constexpr uint32_t kWeightMagic = 0xA1E4B0B5u;  // live alv_weight
constexpr uint32_t kFfnMagic = 0xA1FEED42u;     // live alv_ffn
}  // namespace alv

// Registered projection (tile_q.hip).
// Registration keeps the nonzero part of a matrix only: a padded matrix (the
// reference quantizer zero-pads Gemma-4's K to 4096 and its FFN to 16384 x
// 4096, tools/quantize_gemma4.py:145-187; its runtime pads the sliding O
// projection to 8192 rows, runtime/cpp/src/weights.cpp:318-327) is streamed
// at the executed shape Ne x Ke, and the trimmed rows [Ne, N) are written as
// exact zeros -- the value the reference computes there up to the sign of
// zero. N and K stay the caller's (logical) shape for every argument check.
struct alv_weight {
    uint32_t magic;
    int device;
    int N, K;
    int Ne, Ke;  // executed shape: the leading Ne rows and Ke columns
    uint8_t* w;  // tiled copy, tile_bytes(Ne, Ke)
};

// Registered FFN layer (ffn_fused.hip).
struct alv_ffn {
    uint32_t magic;
    int device;
    int H, I, act;
    int He, Ie;  // executed shape (trailing all-zero rows and columns trimmed, as for alv_weight)
    uint8_t* w;  // one allocation: gate | up | down, tiled layout (q4_device.h)
    size_t gate_bytes, down_bytes;
    uint16_t* a;  // decode activation (bf16 bit patterns), kGemvMaxM x I, fixed for the handle's life
    size_t a_cap;
    const uint16_t* last_a;  // activation of the last call: `a`, or the stream's prefill scratch
    int a_rows;              // tokens held at last_a after the last call
    // One-token FFN in one launch (q4_ffn1_kernel; null vdown: the shape does
    // not take it): the down matrix again in slice order, and G x He partials.
    uint8_t* vdown;
    uint64_t vdown_bytes;
    float* part1;
    int G1, U1;
};

