// Drives alveare::NpuRegistry (alveare_amd/cpp/alveare/npu.h) the way the
// reference runtime's main.cpp and weights.cpp drive theirs: register a
// weight, run it on host bf16 buffers. Inputs and outputs are raw files.
//
//   npu_registry_check gemv N K W x y
//   npu_registry_check gemm B N K W x y
//   npu_registry_check gemm_streamed B N K W x y
//   npu_registry_check ffn H I act packed x y [m_I k_tile]
//   npu_registry_check errors N K W
//   npu_registry_check manifest out.txt      (kernels() of $NPU_MANIFEST as text)
// NPU_MANIFEST, when set, is the manifest the registry reads.
// Prints "ok" and exits 0, or prints the exception and exits 1.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "alveare/npu.h"

static std::vector<char> slurp(const char* path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error(std::string("cannot read ") + path);
    return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static void spit(const char* path, const void* p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(p), (std::streamsize)n);
    if (!f) throw std::runtime_error(std::string("cannot write ") + path);
}

int main(int argc, char** argv) {
    try {
        if (argc < 2) throw std::runtime_error("usage: npu_registry_check <mode> ...");
        const std::string mode = argv[1];
        // NPU_MANIFEST names a manifest for the registry to read (none by default).
        const char* mf = getenv("NPU_MANIFEST");
        alveare::NpuRegistry reg(mf ? mf : "/nonexistent/manifest.json");
        if (mode == "manifest" && argc == 3) {
            // kernels() as text, one kernel a line, into argv[2]
            std::string out = "model_type " + reg.model_type() + "\n";
            for (const alveare::KernelSpec& k : reg.kernels())
                out += k.kind + " " + std::to_string(k.N) + " " + std::to_string(k.K) + " " + std::to_string(k.B) +
                       " " + std::to_string(k.H) + " " + std::to_string(k.I) + " " + k.activation + " " +
                       std::to_string(k.m) + " " + std::to_string(k.k_tile) + " " + std::to_string(k.n_cores) + " " +
                       k.xclbin + "\n";
            spit(argv[2], out.data(), out.size());
            printf("ok\n");
            return 0;
        }
        if (mode == "gemv" && argc == 7) {
            const int N = atoi(argv[2]), K = atoi(argv[3]);
            auto W = slurp(argv[4]);
            auto x = slurp(argv[5]);
            std::vector<uint16_t> y(N);
            if (!reg.has_gemv(N, K)) throw std::runtime_error("has_gemv false");
            const alveare::WeightHandle w = reg.create_gemv_weight(N, K, W.data(), W.size());
            reg.run_gemv(N, K, w, x.data(), y.data());
            reg.run_gemv(N, K, w, x.data(), y.data());  // a second call on the same buffers
            if (reg.npu_calls() != 2 || reg.loaded_contexts() != 1) throw std::runtime_error("profile counters");
            spit(argv[6], y.data(), y.size() * 2);
        } else if ((mode == "gemm" || mode == "gemm_streamed") && argc == 8) {
            const int B = atoi(argv[2]), N = atoi(argv[3]), K = atoi(argv[4]);
            auto W = slurp(argv[5]);
            auto x = slurp(argv[6]);
            std::vector<uint16_t> y((size_t)B * N);
            if (mode == "gemm") {
                const alveare::WeightHandle w = reg.create_gemv_weight(N, K, W.data(), W.size());
                reg.run_gemm(B, N, K, w, x.data(), y.data());
            } else {
                reg.run_gemm_streamed(B, N, K, W.data(), W.size(), x.data(), y.data());
            }
            spit(argv[7], y.data(), y.size() * 2);
        } else if (mode == "ffn" && (argc == 8 || argc == 10)) {
            const int H = atoi(argv[2]), I = atoi(argv[3]);
            const std::string act = argv[4];
            if (argc == 10) reg.set_ffn_packing(atoi(argv[8]), atoi(argv[9]));
            auto P = slurp(argv[5]);
            auto x = slurp(argv[6]);
            std::vector<uint16_t> y(H);
            const alveare::WeightHandle w = reg.create_ffn_fused_weight(H, I, act, P.data(), P.size());
            reg.run_ffn_fused(H, I, act, w, x.data(), y.data());
            if (reg.npu_calls() != 1 || reg.ffn_seconds() <= 0.0) throw std::runtime_error("profile counters");
            spit(argv[7], y.data(), y.size() * 2);
        } else if (mode == "errors" && argc == 5) {
            const int N = atoi(argv[2]), K = atoi(argv[3]);
            auto W = slurp(argv[4]);
            std::vector<uint16_t> x(K), y(N);
            const alveare::WeightHandle w = reg.create_gemv_weight(N, K, W.data(), W.size());
            int thrown = 0;
            try {
                reg.run_gemv(N, K, w + 7, x.data(), y.data());
            } catch (const std::runtime_error&) {
                ++thrown;
            }
            try {
                reg.run_gemv(N + 32, K, w, x.data(), y.data());
            } catch (const std::runtime_error&) {
                ++thrown;
            }
            try {
                reg.run_ffn_fused(N, K, "gelu", w, x.data(), y.data());
            } catch (const std::runtime_error&) {
                ++thrown;
            }
            try {
                reg.create_gemv_weight(N, K, W.data(), W.size() / 2);
            } catch (const std::runtime_error&) {
                ++thrown;
            }
            if (thrown != 4) throw std::runtime_error("expected 4 exceptions, got " + std::to_string(thrown));
        } else {
            throw std::runtime_error("bad arguments for mode " + mode);
        }
        printf("ok\n");
        return 0;
    } catch (const std::exception& e) {
        printf("error: %s\n", e.what());
        return 1;
    }
}
