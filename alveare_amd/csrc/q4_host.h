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

// Per-(device, stream) synchronisation words of the op-chain executor. They
// are zero when a launch starts and every launch leaves them zero. A device's
// words (a set for each of up to 64 streams) are allocated at its first call,
// which synchronises the device; later calls, a stream's first included,
// allocate nothing.
struct Workspace {
    uint32_t* counters = nullptr;
    size_t counter_count = 0;
};
int get_workspace(hipStream_t s, size_t counters, Workspace* out);

// Per-(device, stream, slot) scratch of at least `bytes`, zeroed when
// allocated, for launches whose temporaries grow with their shape: slot 0 the
// prefill GEMM's (counters, partial tiles, activation terms), slot 1 the
// streaming GEMV's split-K partial sums (rewritten by every such launch before
// it is read). Growing synchronises the stream and reallocates, so it cannot
// happen during graph capture (an error then); a call that fits what the slot
// already holds allocates nothing.
constexpr int kScratchGemm = 0;
constexpr int kScratchSplit = 1;
int get_scratch(hipStream_t s, int slot, size_t bytes, void** out);
// Largest split-K partial-sum block of one streaming GEMV launch.
constexpr size_t kPartMax = 256u << 20;

// One launch of the streaming kernel (stream_q.hip):
//   out[m, n] = sum_k X[m, k] * dequant(W0)[n, k]            (glu == false)
//   out[m, n] = act(bf16(X W0^T), bf16(X W1^T)) rounded to bf16 (glu == true)
// parts = 3 splits fp32 X exactly into three bf16 terms; parts = 1 requires X
// to hold bf16 values (the FFN's activation does). The activations are either
// fp32 (X) or bf16 bit patterns (Xb, parts = 1, no GLU); the output is fp32
// (Y) or bf16 bit patterns (Yb).
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
};
int launch_gemv(const GemvLaunch& L, hipStream_t s);

// ---- op chains (stream_q.hip) --------------------------------------------------
// One op of a chain: a GemvLaunch plus the index of the earlier op whose output
// is its input (-1: the input is ready when the launch starts).
struct ExecOp : GemvLaunch {
    int dep = -1;
};
constexpr int kMaxOps = 16;
// Synchronisation words of a chain launch. Same-address device atomics
// serialise (~8 ns each), so counters that many workgroups bump are spread over
// kSyncSlots words: per op, "row tiles done" (workgroup b counts into slot
// b % kSyncSlots); a two-level exit count (workgroup b into slot
// b % kSyncSlots, the slot that completes into one word); and a sticky error
// flag set when a wait timed out.
constexpr int kSyncSlots = 64;
constexpr int kSyncExit1 = kMaxOps * kSyncSlots;
constexpr int kSyncExit2 = kSyncExit1 + kSyncSlots;
constexpr int kSyncError = kSyncExit2 + 1;
constexpr int kSyncWords = kSyncError + 1;
// Split-K arrival counters of the streaming GEMV, after the executor's words
// (one per tile group of a launch).
constexpr int kSplitCounters = 1024;
// Words of a stream's set: the executor's, then the split-K counters.
constexpr int kWsWords = kSyncWords + kSplitCounters;

// Device-side descriptor of one op (kernel argument; every field is
// wave-uniform). Work split: a workgroup of 16 waves holds rtw row-tile slots
// of (1 << kw_shift) waves each; wave kw of a slot takes super-steps
// [kw * spw, kw * spw + spw) of its row tile, for each of the op's one or two
// matrices. Round r, slot s of workgroup b is row tile (r * rtw + s) * grid + b;
// workgroup b runs nr_full + (b < nr_rem) rounds.
struct OpDesc {
    const uint8_t* W0;
    const uint8_t* W1;
    const void* X;
    float* Y;
    uint16_t* Yb;
    uint32_t wbytes, xbytes, rstride;
    int ldx, ldy, M, N, K, parts, R, nb, nss, ng_last, RT, act;
    int glu, xb, dep, signal;
    int spw, kw_shift, rtw, nr_full, nr_rem;
};
struct ExecArgs {
    OpDesc op[kMaxOps];
    int nops;
    uint32_t xs_bytes;  // LDS bytes of the staged activations (the reduction scratch follows)
    uint32_t spin_limit;
    int last_wait;  // the last op that waits for an earlier one (-1: none, no counters are used)
    uint32_t* sync;
};
// Run ops[0..nops) on `s`: one launch per group of tokens that fits the LDS
// (every op of a launch sees the same tokens). tiled: weights in the tiled
// layout (required for chains longer than one op).
int exec_chain(const ExecOp* ops, int nops, bool tiled, hipStream_t s);
// Report (and clear) a timed-out chain wait on stream `s` (synchronises it).
int check_async(hipStream_t s);

// ---- streaming GEMV for few tokens (gemv1_q.hip) -----------------------------------
// L on registered weights as launches of the streaming kernel, up to four
// tokens each; gemv1_ok: the shape's activations and unit slots fit the LDS
// for one token at least.
bool gemv1_ok(const GemvLaunch& L);
int launch_gemv1(const GemvLaunch& L, hipStream_t s);

// Repack W (combined layout, N x K) into the tiled layout at `out`
// (tile_bytes(N, K) bytes), on `s` (tile_q.hip).
int launch_tile(const uint8_t* W, uint8_t* out, int N, int K, hipStream_t s);
uint64_t tile_bytes(int N, int K);

// Largest M the streaming kernel takes in one launch (3 * 16 = 48 A rows).
constexpr int kGemvMaxM = 16;

// MFMA tiled kernel for prefill-sized M (gemm_q.hip). Same contract as
// GemvLaunch (glu pairs W0/W1 into the activation).
int launch_gemm_tiled(const GemvLaunch& L, hipStream_t s);

// M at and above which alv_gemm_q uses the tiled kernel.
constexpr int kTiledMinM = 32;

// The two ops of one FFN call on handle w (ffn_fused.hip).
void ffn_ops(alv_ffn_t w, const float* X, int ldx, float* Y, int ldy, int M, ExecOp (&op)[2]);

}  // namespace alv

namespace alv {
constexpr uint32_t kWeightMagic = 0xA1E4B0B5u;  // live alv_weight
constexpr uint32_t kFfnMagic = 0xA1FEED42u;     // live alv_ffn
}  // namespace alv

// Registered projection (tile_q.hip).
struct alv_weight {
    uint32_t magic;
    int device;
    int N, K;
    uint8_t* w;  // tiled copy, tile_bytes(N, K)
};

// Registered FFN layer (ffn_fused.hip).
struct alv_ffn {
    uint32_t magic;
    int device;
    int H, I, act;
    uint8_t* w;  // one allocation: gate | up | down, tiled layout (q4_device.h)
    size_t gate_bytes, down_bytes;
    uint16_t* a;  // activation scratch (bf16 bit patterns), a_cap elements
    size_t a_cap;
    int a_rows;  // tokens held in `a` after the last call
};

