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

// Per-(device, stream) scratch for cross-workgroup split-K reduction:
// fp32 partial sums and per-row-tile arrival counters. Counters are zero when
// a kernel starts and every kernel leaves them zero. Grown on demand (the
// growth synchronises the device); steady-state calls allocate nothing.
struct Workspace {
    float* partial = nullptr;
    size_t partial_floats = 0;
    uint32_t* counters = nullptr;
    size_t counter_count = 0;
};
int get_workspace(hipStream_t s, size_t partial_floats, size_t counters, Workspace* out);

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

}  // namespace alv
