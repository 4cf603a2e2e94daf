// alv_stream_read: a plain streaming read, the practical HBM ceiling for a
// launch of a given size on this device (no reference counterpart; a
// measurement aid the benchmark sets beside the Q4 kernels).
//
// DEPTH 16-byte nontemporal loads per thread and pass (all issued before the
// first is used), grid-stride over the buffer, `wg_per_cu` 256-thread
// workgroups per CU; alv_stream_read is depth 4 at four workgroups per CU
// (the shape that measured fastest for 10-1000 MB reads). Each workgroup
// folds what it read into word 32 (b % 64) of `sink` with an atomic XOR, so
// the loads cannot be elided (device atomics on one address serialise:
// spread over 64 lines, the folding stays far below the read time).
#include <algorithm>

#include "q4_device.h"
#include "q4_host.h"

namespace {

using alv::u32x4;

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

extern "C" int alv_stream_read_shape(const void* buf, size_t bytes, uint32_t* sink, int wg_per_cu, int depth,
                                     void* stream) {
    using namespace alv;
    if (!buf || !sink) return fail(ALV_ERR_ARG, "null pointer");
    if (reinterpret_cast<uintptr_t>(buf) % 16 || bytes % 16)
        return fail(ALV_ERR_ALIGN, "the buffer and its size need 16-byte alignment");
    if (wg_per_cu < 1 || wg_per_cu > 8 || (depth != 2 && depth != 4 && depth != 8 && depth != 16))
        return fail(ALV_ERR_ARG, "bad read shape wg_per_cu=%d depth=%d (1-8 workgroups per CU; depth 2, 4, 8 or 16)",
                    wg_per_cu, depth);
    if (bytes == 0) return ALV_OK;
    const size_t n16 = bytes / 16;
    const size_t per_wg = (size_t)256 * depth;
    const int grid = (int)std::max<size_t>(1, std::min<size_t>((size_t)wg_per_cu * device_cus(), (n16 + per_wg - 1) / per_wg));
    const u32x4* p = reinterpret_cast<const u32x4*>(buf);
    const hipStream_t s = (hipStream_t)stream;
    switch (depth) {
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
        default: hipLaunchKernelGGL(stream_read_kernel<16>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    }
    return hip_check(hipGetLastError(), "stream_read_kernel launch");
}

extern "C" int alv_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
    return alv_stream_read_shape(buf, bytes, sink, 4, 4, stream);
}
