// alveare::NpuRegistry for MI355X: the reference runtime's matmul registry
// (runtime/cpp/include/alveare/npu.h:44-115) with the same public interface,
// backed by the gfx950 Q4 kernels of libalveare_q4.so instead of XDNA2 AOT
// kernels. The reference's C++ runtime (runtime/cpp/src/model.cpp,
// weights.cpp, generator.cpp, main.cpp) compiles against this header and
// links libalveare_npu.so in place of npu.cpp + XRT, unchanged.
//
// Semantics kept from the reference (runtime/cpp/src/npu.cpp):
//   * weights are uploaded once and stay device-resident behind a handle;
//     the caller keeps ownership of its host bytes (npu.cpp:241-267);
//   * run_* take and return bf16 on the host, synchronously (npu.cpp:269-378);
//     y = bf16 of the float32 sum, the FFN's partials summed in float32;
//   * errors are std::runtime_error (invalid handle, shape mismatch, a
//     failing device call).
// Differences that follow from the hardware:
//   * no per-shape kernels are compiled: every shape with K (and H, I) a
//     multiple of 32 has a kernel, so has_* answer by shape and the context
//     budget / pinning calls do nothing. The manifest, when the file exists,
//     is read for "model_type" and its "kernels" list, which kernels()
//     returns (so drivers that walk it, runtime/cpp/test/parity_test.cpp,
//     exercise its shapes);
//   * create_ffn_fused_weight takes the reference's packed blob
//     (pack_ffn_fused_weights, runtime/cpp/src/weights.cpp:94-190) and
//     unpacks it to gate / up / down before registering. Its m_I and k_tile
//     come from set_ffn_packing, else the manifest's ffn_fused kernel of the
//     same (H, I, activation), else the reference loader's rule (m_I = 32,
//     k_tile = 128 for H = 1152, else 256).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace alveare {

// One kernel of the reference's AOT manifest (kernels/build/manifest.json),
// as kernels() lists it from the manifest file.
struct KernelSpec {
    std::string kind;
    int N = 0;
    int K = 0;
    int B = 0;
    int H = 0;
    int I = 0;
    std::string activation;
    int m = 0;
    int k_tile = 0;
    int n_cores = 0;
    std::string xclbin;
    std::string insts;
};

// Opaque handle to a resident device weight owned by the registry.
using WeightHandle = uint32_t;
inline constexpr WeightHandle kInvalidWeight = 0xFFFFFFFFu;

class NpuRegistry {
public:
    // manifest_path: the reference's manifest, optional here (see above).
    // device_index: the HIP device; max_contexts is accepted and unused.
    explicit NpuRegistry(const std::string& manifest_path, unsigned device_index = 0, int max_contexts = 8);
    ~NpuRegistry();

    NpuRegistry(const NpuRegistry&) = delete;
    NpuRegistry& operator=(const NpuRegistry&) = delete;

    const std::vector<KernelSpec>& kernels() const;
    const std::string& model_type() const;

    bool has_gemv(int N, int K) const;
    bool has_gemm(int B, int N, int K) const;
    bool has_ffn_fused(int H, int I, const std::string& activation) const;

    // packed: (N, K/32*20) uint8 Q4 (the combined layout), nbytes >= N*K/32*20.
    WeightHandle create_gemv_weight(int N, int K, const void* packed, size_t nbytes);

    // packed: pack_ffn_fused_weights(gate, up, down, H, I, m_I, k_tile).
    WeightHandle create_ffn_fused_weight(int H, int I, const std::string& activation, const void* packed,
                                         size_t nbytes);

    // y_bf16[N] = bf16(W x), x_bf16[K]; host buffers.
    void run_gemv(int N, int K, WeightHandle w, const void* x_bf16, void* y_bf16);

    // Y[B, N] = bf16(X[B, K] W^T) on a gemv weight of the same (N, K).
    void run_gemm(int B, int N, int K, WeightHandle w, const void* x_bf16, void* y_bf16);

    // run_gemm on a weight passed per call from host memory (not registered).
    void run_gemm_streamed(int B, int N, int K, const void* packed, size_t nbytes, const void* x_bf16,
                           void* y_bf16);

    // y_bf16[H] = bf16(down(GLU(gate x, up x))), x_bf16[H]; activation "gelu" or "silu".
    void run_ffn_fused(int H, int I, const std::string& activation, WeightHandle w, const void* x_bf16,
                       void* y_bf16);

    void pin_gemv(int N, int K);
    void pin_ffn_fused(int H, int I, const std::string& activation);

    // Distinct shapes used so far (the reference counts loaded hardware contexts).
    int loaded_contexts() const;

    // Wall time (seconds) of run_gemv + run_ffn_fused calls, of run_ffn_fused
    // alone, and their count; reset_profile() zeroes them.
    double npu_seconds() const;
    double ffn_seconds() const;
    long npu_calls() const;
    void reset_profile();

    // Packing parameters of the FFN blobs create_ffn_fused_weight accepts
    // (0: the reference loader's rule, m_I = 32, k_tile = H == 1152 ? 128 : 256).
    void set_ffn_packing(int m_I, int k_tile);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace alveare

// Inverse of the reference's pack_ffn_fused_weights (weights.cpp:94-190):
// gate, up (I x H/32*20) and down (H x I/32*20) from the packed blob.
// Returns 0, or -1 with a message in alvnpu_last_error() when the blob size
// does not match or the packing drops rows (its four down passes of
// (H / k_tile) / 4 tiles cover all of H only when 4 divides H / k_tile).
extern "C" int alvnpu_unpack_ffn(const uint8_t* packed, size_t nbytes, int H, int I, int m_I, int k_tile,
                                 uint8_t* gate, uint8_t* up, uint8_t* down);
extern "C" const char* alvnpu_last_error(void);
