// alveare::NpuRegistry over the gfx950 Q4 kernels (libalveare_q4.so): the
// reference runtime's registry interface (runtime/cpp/include/alveare/npu.h,
// runtime/cpp/src/npu.cpp) with device-resident weights on one HIP device and
// host bf16 activations, synchronous per call.
#include "alveare/npu.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <tuple>

#include "alveare_q4.h"

namespace {

thread_local char g_unpack_err[512] = "";

int unpack_fail(const char* fmt, int a, int b, int c, int d) {
    snprintf(g_unpack_err, sizeof g_unpack_err, fmt, a, b, c, d);
    return -1;
}

// bf16 round to nearest even with NaN -> 0x7FC0 (runtime/cpp/src/bf16.cpp:7-25).
uint16_t bf16_bits(float f) {
    if (f != f) return 0x7FC0u;
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float bf16_value(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("npu (hip): ") + what + ": " + hipGetErrorString(e));
}

void alv_ok(int rc, const char* what) {
    if (rc != ALV_OK) throw std::runtime_error(std::string("npu (alveare): ") + what + ": " + alv_last_error());
}

int act_id(const std::string& a) {
    if (a == "gelu" || a == "gelu_tanh") return ALV_ACT_GELU_TANH;
    if (a == "silu") return ALV_ACT_SILU;
    throw std::runtime_error("npu: unknown activation " + a);
}

// A device buffer that only grows (the registry runs no graphs).
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    void* get(size_t bytes) {
        if (bytes > cap) {
            if (p) (void)hipFree(p);
            p = nullptr;
            cap = 0;
            hip_ok(hipMalloc(&p, bytes), "hipMalloc");
            cap = bytes;
        }
        return p;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

// ---- the kernel manifest (kernels/build/manifest.json) -----------------------
// A small JSON reader for the manifest the reference registry loads
// (runtime/cpp/src/npu.cpp:186-216): "model_type" and the "kernels" array of
// objects with string and integer fields. Anything else is skipped.
struct Json {
    const std::string& s;
    size_t i = 0;
    explicit Json(const std::string& t) : s(t) {}
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    bool eat(char c) {
        ws();
        if (i < s.size() && s[i] == c) {
            ++i;
            return true;
        }
        return false;
    }
    void need(char c) {
        if (!eat(c)) throw std::runtime_error(std::string("npu: manifest: expected '") + c + "'");
    }
    std::string str() {
        need('"');
        std::string out;
        while (i < s.size() && s[i] != '"') {
            char c = s[i++];
            if (c == '\\' && i < s.size()) {
                const char e = s[i++];
                c = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
                if (e == 'u') {  // \uXXXX: kept as '?' (no manifest field needs it)
                    i = std::min(s.size(), i + 4);
                    c = '?';
                }
            }
            out += c;
        }
        need('"');
        return out;
    }
    // Skip one value of any kind; returns it as text for scalars.
    std::string value() {
        ws();
        if (i >= s.size()) throw std::runtime_error("npu: manifest: unexpected end");
        if (s[i] == '"') return str();
        if (s[i] == '{' || s[i] == '[') {
            const char open = s[i], close = open == '{' ? '}' : ']';
            ++i;
            if (eat(close)) return "";
            do {
                if (open == '{') {
                    str();
                    need(':');
                }
                value();
            } while (eat(','));
            need(close);
            return "";
        }
        const size_t b = i;
        while (i < s.size() && s[i] != ',' && s[i] != '}' && s[i] != ']' && s[i] != ' ' && s[i] != '\n' &&
               s[i] != '\r' && s[i] != '\t')
            ++i;
        return s.substr(b, i - b);
    }
};

int json_int(const std::string& v) {
    try {
        return v.empty() ? 0 : (int)std::stod(v);
    } catch (const std::exception&) {
        return 0;
    }
}

// model_type and the kernel list of a manifest's text.
void parse_manifest(const std::string& text, std::string* model_type, std::vector<alveare::KernelSpec>* specs) {
    Json j(text);
    j.need('{');
    if (j.eat('}')) return;
    do {
        const std::string key = j.str();
        j.need(':');
        if (key == "model_type") {
            *model_type = j.value();
        } else if (key == "kernels") {
            j.need('[');
            if (j.eat(']')) continue;
            do {
                alveare::KernelSpec k;
                j.need('{');
                if (!j.eat('}')) {
                    do {
                        const std::string f = j.str();
                        j.need(':');
                        const std::string v = j.value();
                        if (f == "kind") k.kind = v;
                        else if (f == "N") k.N = json_int(v);
                        else if (f == "K") k.K = json_int(v);
                        else if (f == "B") k.B = json_int(v);
                        else if (f == "H") k.H = json_int(v);
                        else if (f == "I") k.I = json_int(v);
                        else if (f == "activation") k.activation = v;
                        else if (f == "m") k.m = json_int(v);
                        else if (f == "k_tile") k.k_tile = json_int(v);
                        else if (f == "n_cores") k.n_cores = json_int(v);
                        else if (f == "xclbin") k.xclbin = v;
                        else if (f == "insts") k.insts = v;
                    } while (j.eat(','));
                    j.need('}');
                }
                specs->push_back(std::move(k));
            } while (j.eat(','));
            j.need(']');
        } else {
            j.value();
        }
    } while (j.eat(','));
    j.need('}');
}

}  // namespace

extern "C" const char* alvnpu_last_error(void) { return g_unpack_err; }

// The walk of pack_ffn_fused_weights (runtime/cpp/src/weights.cpp:94-190)
// run backwards: the same core split, tile order and (for 16 or 32 cores) the
// same column interleave, copying each tile from the blob to its rows.
extern "C" int alvnpu_unpack_ffn(const uint8_t* packed, size_t nbytes, int H, int I, int m_I, int k_tile,
                                 uint8_t* gate, uint8_t* up, uint8_t* down) {
    if (!packed || !gate || !up || !down) {
        snprintf(g_unpack_err, sizeof g_unpack_err, "null pointer");
        return -1;
    }
    if (H < 32 || I < 32 || H % 32 || I % 32 || m_I < 32 || m_I % 32 || k_tile < 32 || k_tile % 32)
        return unpack_fail("bad shape H=%d I=%d m_I=%d k_tile=%d", H, I, m_I, k_tile);
    int n_cores = 1;
    for (int c : {32, 16, 8, 4, 2})
        if (I % (c * m_I) == 0) {
            n_cores = c;
            break;
        }
    const int I_div = I / n_cores;
    const int nb_I = I_div / m_I;
    const int cpg = k_tile / 32;
    const int n_passes = 4;
    const int m_H = k_tile;
    const int dtpp = (H / m_H) / n_passes;
    if (H % k_tile || I_div % m_I || (H / m_H) % n_passes)
        return unpack_fail("H=%d I=%d m_I=%d k_tile=%d: the packing leaves out rows of the FFN", H, I, m_I, k_tile);
    const size_t gu_stride = (size_t)H / 32 * 20, d_stride = (size_t)I / 32 * 20;
    const size_t tile = (size_t)m_I * cpg * 20;
    const size_t per_core = tile * ((size_t)2 * nb_I * (H / k_tile) + (size_t)n_passes * nb_I * dtpp);
    if (nbytes != per_core * n_cores) {
        snprintf(g_unpack_err, sizeof g_unpack_err, "packed FFN of %zu bytes, expected %zu for H=%d I=%d", nbytes,
                 per_core * n_cores, H, I);
        return -1;
    }
    const int rows_per_col = n_cores >= 16 ? n_cores / 8 : 0;
    const size_t n_tiles = per_core / tile;
    // Byte `off` of core c's stream within the blob.
    auto at = [&](int c, size_t off) -> const uint8_t* {
        if (!rows_per_col) return packed + (size_t)c * per_core + off;
        const size_t t = off / tile, in = off % tile;
        const int col = c / rows_per_col, r = c % rows_per_col;
        return packed + (((size_t)col * n_tiles + t) * rows_per_col + r) * tile + in;
    };
    for (int c = 0; c < n_cores; ++c) {
        size_t off = 0;
        const int start_I = c * I_div;
        auto take = [&](uint8_t* w, int r0, int r1, size_t b0, size_t b1, size_t stride) {
            for (int r = r0; r < r1; ++r) {
                // a tile never crosses a tile boundary of the stream, so one
                // row's bytes are contiguous in the blob
                memcpy(w + (size_t)r * stride + b0, at(c, off), b1 - b0);
                off += b1 - b0;
            }
        };
        for (int b = 0; b < nb_I; ++b) {
            const int r0 = start_I + b * m_I;
            for (int hb = 0; hb < H / k_tile; ++hb) {
                const size_t c0 = (size_t)hb * cpg * 20, c1 = (size_t)(hb + 1) * cpg * 20;
                take(gate, r0, r0 + m_I, c0, c1, gu_stride);
                take(up, r0, r0 + m_I, c0, c1, gu_stride);
            }
        }
        for (int p = 0; p < n_passes; ++p)
            for (int b = 0; b < nb_I; ++b) {
                const size_t c0 = (size_t)(start_I / 32) * 20 + (size_t)b * (m_I / 32) * 20;
                const size_t c1 = c0 + (size_t)(m_I / 32) * 20;
                for (int hd = p * dtpp; hd < (p + 1) * dtpp; ++hd) take(down, hd * m_H, (hd + 1) * m_H, c0, c1, d_stride);
            }
    }
    return 0;
}

namespace alveare {

struct NpuRegistry::Impl {
    struct Entry {
        bool ffn = false;
        int N = 0, K = 0;  // gemv (N, K); ffn (H, I)
        int act = 0;
        alv_weight_t w = nullptr;
        alv_ffn_t f = nullptr;
    };
    int device = 0;
    hipStream_t stream = nullptr;
    std::string model_type;
    std::vector<KernelSpec> kernels;
    std::vector<Entry> weights;
    std::set<std::tuple<int, int, int, int>> shapes;
    DevBuf x, y, wtmp, xf, yf;
    std::mutex mu;
    int m_I = 0, k_tile = 0;
    double npu_s = 0, ffn_s = 0;
    long calls = 0;

    void enter() { hip_ok(hipSetDevice(device), "hipSetDevice"); }
    void sync() { hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize"); }

    const Entry& entry(WeightHandle w, bool ffn) {
        if (w >= weights.size() || weights[w].ffn != ffn || (ffn ? !weights[w].f : !weights[w].w))
            throw std::runtime_error("npu: invalid weight handle");
        return weights[w];
    }

    // Y[M, N] = bf16(X W^T) on a registered weight, host bf16 in and out.
    void gemv(const Entry& e, int M, const void* xh, void* yh) {
        const size_t xb = (size_t)M * e.K * 2, yb = (size_t)M * e.N * 2;
        void* xd = x.get(xb);
        void* yd = y.get(yb);
        hip_ok(hipMemcpyAsync(xd, xh, xb, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(x)");
        alv_ok(alv_gemv_bf16(e.w, static_cast<const uint16_t*>(xd), static_cast<uint16_t*>(yd), M, e.K, e.N, stream),
               "alv_gemv_bf16");
        hip_ok(hipMemcpyAsync(yh, yd, yb, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(y)");
        sync();
    }
};

NpuRegistry::NpuRegistry(const std::string& manifest_path, unsigned device_index, int /*max_contexts*/)
    : impl_(new Impl) {
    impl_->device = (int)device_index;
    impl_->enter();
    hip_ok(hipStreamCreate(&impl_->stream), "hipStreamCreate");
    std::ifstream f(manifest_path);
    if (f) {
        std::stringstream ss;
        ss << f.rdbuf();
        parse_manifest(ss.str(), &impl_->model_type, &impl_->kernels);
    }
}

NpuRegistry::~NpuRegistry() {
    if (!impl_) return;
    (void)hipSetDevice(impl_->device);
    for (auto& e : impl_->weights) {
        if (e.w) alv_weight_release(e.w);
        if (e.f) alv_ffn_release(e.f);
    }
    if (impl_->stream) (void)hipStreamDestroy(impl_->stream);
}

const std::vector<KernelSpec>& NpuRegistry::kernels() const { return impl_->kernels; }
const std::string& NpuRegistry::model_type() const { return impl_->model_type; }

bool NpuRegistry::has_gemv(int N, int K) const { return N >= 1 && K >= 32 && K % 32 == 0; }
bool NpuRegistry::has_gemm(int B, int N, int K) const { return B >= 1 && has_gemv(N, K); }
bool NpuRegistry::has_ffn_fused(int H, int I, const std::string& activation) const {
    return H >= 32 && I >= 32 && H % 32 == 0 && I % 32 == 0 && (activation == "gelu" || activation == "silu");
}

WeightHandle NpuRegistry::create_gemv_weight(int N, int K, const void* packed, size_t nbytes) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    impl_->enter();
    if (!has_gemv(N, K)) throw std::runtime_error("npu: no kernel for gemv " + std::to_string(N) + "x" + std::to_string(K));
    const size_t need = (size_t)N * (K / 32) * 20;
    if (!packed || nbytes < need) throw std::runtime_error("npu: packed weight smaller than (N, K/32*20)");
    void* d = impl_->wtmp.get(need);
    hip_ok(hipMemcpyAsync(d, packed, need, hipMemcpyHostToDevice, impl_->stream), "hipMemcpyAsync(weights)");
    Impl::Entry e;
    e.N = N;
    e.K = K;
    alv_ok(alv_weight_register(static_cast<const uint8_t*>(d), N, K, &e.w, impl_->stream), "alv_weight_register");
    impl_->weights.push_back(e);
    impl_->shapes.insert({0, N, K, 0});
    return (WeightHandle)(impl_->weights.size() - 1);
}

WeightHandle NpuRegistry::create_ffn_fused_weight(int H, int I, const std::string& activation, const void* packed,
                                                  size_t nbytes) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    impl_->enter();
    const int act = act_id(activation);
    // The blob's packing: set_ffn_packing's, else the manifest's ffn_fused
    // kernel of this shape (its m and k_tile, npu.cpp:211-213), else the
    // reference loader's rule (weights.cpp:364-365).
    int m_I = 32, k_tile = H == 1152 ? 128 : 256;
    for (const KernelSpec& k : impl_->kernels)
        if (k.kind == "ffn_fused" && k.H == H && k.I == I && act_id(k.activation.empty() ? "gelu" : k.activation) == act) {
            if (k.m > 0) m_I = k.m;
            if (k.k_tile > 0) k_tile = k.k_tile;
            break;
        }
    if (impl_->m_I) m_I = impl_->m_I;
    if (impl_->k_tile) k_tile = impl_->k_tile;
    const size_t gb = (size_t)I * (H / 32) * 20, db = (size_t)H * (I / 32) * 20;
    std::vector<uint8_t> host(2 * gb + db);
    if (alvnpu_unpack_ffn(static_cast<const uint8_t*>(packed), nbytes, H, I, m_I, k_tile, host.data(),
                          host.data() + gb, host.data() + 2 * gb))
        throw std::runtime_error(std::string("npu: ") + alvnpu_last_error());
    uint8_t* d = static_cast<uint8_t*>(impl_->wtmp.get(host.size()));
    hip_ok(hipMemcpyAsync(d, host.data(), host.size(), hipMemcpyHostToDevice, impl_->stream), "hipMemcpyAsync(ffn)");
    Impl::Entry e;
    e.ffn = true;
    e.N = H;
    e.K = I;
    e.act = act;
    alv_ok(alv_ffn_register(d, d + gb, d + 2 * gb, H, I, act, &e.f, impl_->stream), "alv_ffn_register");
    impl_->weights.push_back(e);
    impl_->shapes.insert({1, H, I, act});
    return (WeightHandle)(impl_->weights.size() - 1);
}

void NpuRegistry::run_gemv(int N, int K, WeightHandle w, const void* x_bf16, void* y_bf16) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    const auto t0 = std::chrono::steady_clock::now();
    impl_->enter();
    const Impl::Entry& e = impl_->entry(w, false);
    if (e.N != N || e.K != K)
        throw std::runtime_error("npu: weight/shape mismatch in run_gemv: expected (" + std::to_string(e.N) + ", " +
                                 std::to_string(e.K) + "), got (" + std::to_string(N) + ", " + std::to_string(K) + ")");
    impl_->gemv(e, 1, x_bf16, y_bf16);
    impl_->npu_s += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    ++impl_->calls;
}

void NpuRegistry::run_gemm(int B, int N, int K, WeightHandle w, const void* x_bf16, void* y_bf16) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    impl_->enter();
    const Impl::Entry& e = impl_->entry(w, false);
    if (B < 1 || e.N != N || e.K != K)
        throw std::runtime_error("npu: weight/shape mismatch in run_gemm: expected (" + std::to_string(e.N) + ", " +
                                 std::to_string(e.K) + "), got (" + std::to_string(N) + ", " + std::to_string(K) + ")");
    impl_->gemv(e, B, x_bf16, y_bf16);
}

void NpuRegistry::run_gemm_streamed(int B, int N, int K, const void* packed, size_t nbytes, const void* x_bf16,
                                    void* y_bf16) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    impl_->enter();
    if (B < 1 || !has_gemv(N, K)) throw std::runtime_error("npu: bad run_gemm_streamed shape");
    const size_t need = (size_t)N * (K / 32) * 20;
    if (!packed || nbytes < need) throw std::runtime_error("npu: packed weight smaller than (N, K/32*20)");
    // The weight goes up per call in the combined layout; activations cross as
    // float32 (bf16-valued) and the float32 result is rounded to bf16 here.
    std::vector<float> xf((size_t)B * K), yf((size_t)B * N);
    const uint16_t* xb = static_cast<const uint16_t*>(x_bf16);
    for (size_t i = 0; i < xf.size(); ++i) xf[i] = bf16_value(xb[i]);
    void* wd = impl_->wtmp.get(need);
    float* xd = static_cast<float*>(impl_->xf.get(xf.size() * 4));
    float* yd = static_cast<float*>(impl_->yf.get(yf.size() * 4));
    hip_ok(hipMemcpyAsync(wd, packed, need, hipMemcpyHostToDevice, impl_->stream), "hipMemcpyAsync(weights)");
    hip_ok(hipMemcpyAsync(xd, xf.data(), xf.size() * 4, hipMemcpyHostToDevice, impl_->stream), "hipMemcpyAsync(x)");
    alv_ok(alv_gemm_q(static_cast<const uint8_t*>(wd), xd, yd, B, N, K, K, N, impl_->stream), "alv_gemm_q");
    hip_ok(hipMemcpyAsync(yf.data(), yd, yf.size() * 4, hipMemcpyDeviceToHost, impl_->stream), "hipMemcpyAsync(y)");
    impl_->sync();
    uint16_t* yb = static_cast<uint16_t*>(y_bf16);
    for (size_t i = 0; i < yf.size(); ++i) yb[i] = bf16_bits(yf[i]);
}

void NpuRegistry::run_ffn_fused(int H, int I, const std::string& activation, WeightHandle w, const void* x_bf16,
                                void* y_bf16) {
    std::lock_guard<std::mutex> lk(impl_->mu);
    const auto t0 = std::chrono::steady_clock::now();
    impl_->enter();
    const Impl::Entry& e = impl_->entry(w, true);
    if (e.N != H || e.K != I || e.act != act_id(activation))
        throw std::runtime_error("npu: weight/shape mismatch in run_ffn_fused");
    void* xd = impl_->x.get((size_t)H * 2);
    void* yd = impl_->y.get((size_t)H * 2);
    hip_ok(hipMemcpyAsync(xd, x_bf16, (size_t)H * 2, hipMemcpyHostToDevice, impl_->stream), "hipMemcpyAsync(x)");
    alv_ok(alv_ffn_fused_bf16(e.f, static_cast<const uint16_t*>(xd), static_cast<uint16_t*>(yd), 1, H, H, impl_->stream),
           "alv_ffn_fused_bf16");
    hip_ok(hipMemcpyAsync(y_bf16, yd, (size_t)H * 2, hipMemcpyDeviceToHost, impl_->stream), "hipMemcpyAsync(y)");
    impl_->sync();
    const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    impl_->npu_s += dt;
    impl_->ffn_s += dt;
    ++impl_->calls;
}

void NpuRegistry::pin_gemv(int, int) {}
void NpuRegistry::pin_ffn_fused(int, int, const std::string&) {}

int NpuRegistry::loaded_contexts() const { return (int)impl_->shapes.size(); }

double NpuRegistry::npu_seconds() const { return impl_->npu_s; }
double NpuRegistry::ffn_seconds() const { return impl_->ffn_s; }
long NpuRegistry::npu_calls() const { return impl_->calls; }
void NpuRegistry::reset_profile() {
    impl_->npu_s = 0;
    impl_->ffn_s = 0;
    impl_->calls = 0;
}

void NpuRegistry::set_ffn_packing(int m_I, int k_tile) {
    impl_->m_I = m_I;
    impl_->k_tile = k_tile;
}

}  // namespace alveare
