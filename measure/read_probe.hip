// libalveare_probe.so: a plain streaming read, the practical HBM ceiling for
// a launch of a given size on this device. A measurement aid the benchmark
// sets beside the Q4 kernels (no reference counterpart); it is not part of
// libalveare_q4.so's ABI.
//
// DEPTH 16-byte nontemporal loads per thread and pass (all issued before the
// first is used), grid-stride over the buffer, `wg_per_cu` 256-thread
// workgroups per CU; the benchmark's default is depth 4 at four workgroups
// per CU (the shape that measured fastest for 10-1000 MB reads). Each workgroup
// folds what it read into word 32 (b % 64) of `sink` with an atomic XOR, so
// the loads cannot be elided (device atomics on one address serialise:
// spread over 64 lines, the folding stays far below the read time).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>

namespace {

typedef uint32_t u32x4 __attribute__((__vector_size__(4 * sizeof(uint32_t))));

thread_local char g_err[256] = "";

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return 1;
}

int cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        n = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                    hipSuccess && v > 0 ? v : 256;
    }
    return n;
}

template <int DEPTH>
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 256 * DEPTH;
    for (size_t i = (size_t)blockIdx.x * 256 * DEPTH + threadIdx.x; i < n16; i += stride) {
        u32x4 v[DEPTH];
#pragma unroll
        for (int u = 0; u < DEPTH; ++u)
            v[u] = i + (size_t)u * 256 < n16 ? __builtin_nontemporal_load(p + i + (size_t)u * 256) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) atomicXor(sink + (blockIdx.x % 64) * 32, red[0] ^ red[1] ^ red[2] ^ red[3]);
}

}  // namespace

extern "C" const char* alvprobe_last_error(void) { return g_err; }

// Read `bytes` at `buf` once, XOR-folding them into sink[0], sink[32], ...,
// sink[32 * 63] (2048 words of device memory): `wg_per_cu` 256-thread
// workgroups per CU (1-8), `depth` 16-byte loads in flight per thread (2, 4,
// 8 or 16). Returns 0, or 1 with a message in alvprobe_last_error().
extern "C" int alvprobe_stream_read(const void* buf, size_t bytes, uint32_t* sink, int wg_per_cu, int depth,
                                    void* stream) {
    if (!buf || !sink) return fail("null pointer");
    if (reinterpret_cast<uintptr_t>(buf) % 16 || bytes % 16) return fail("the buffer and its size need 16-byte alignment");
    if (wg_per_cu < 1 || wg_per_cu > 8 || (depth != 2 && depth != 4 && depth != 8 && depth != 16))
        return fail("bad read shape wg_per_cu=%d depth=%d (1-8 workgroups per CU; depth 2, 4, 8 or 16)", wg_per_cu, depth);
    if (bytes == 0) return 0;
    const size_t n16 = bytes / 16;
    const size_t per_wg = (size_t)256 * depth;
    const int grid = (int)std::max<size_t>(1, std::min<size_t>((size_t)wg_per_cu * cus(), (n16 + per_wg - 1) / per_wg));
    const u32x4* p = reinterpret_cast<const u32x4*>(buf);
    const hipStream_t s = (hipStream_t)stream;
    switch (depth) {
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        default: hipLaunchKernelGGL(stream_read_kernel<16>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail("stream_read_kernel launch: %s", hipGetErrorString(e));
}
