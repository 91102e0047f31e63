// GPU test of the C++ host layer (chimere_amd/host/ggml_gpu.hpp): the
// reference's V3 launch sequence through the mirrored wrappers gives the
// same bits as the fused entry point (routing and output), for Q4_0 and
// IQ3_S experts, gated and ungated shared experts and a routing bias; the
// host expert path routes identically and lands within the Q8_K activation
// bound; the f32 GEMV wrapper equals quantize + Q8_1 GEMV; rejected calls
// throw.  Prints "host mirror ok" on success (run by tests/test_gpu_host_mirror.py).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../chimere_amd/host/ggml_gpu.hpp"

using namespace chimere::host;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
float urand() {   // xorshift64*, uniform in [-1, 1)
    g_state ^= g_state >> 12; g_state ^= g_state << 25; g_state ^= g_state >> 27;
    return (float)((g_state * 2685821657736338717ull) >> 40) / (float)(1 << 23) - 1.0f;
}

int fails = 0;
#define EXPECT(c, ...)                                                  \
    do {                                                                \
        if (!(c)) { std::printf("FAIL %s:%d ", __FILE__, __LINE__); std::printf(__VA_ARGS__); std::printf("\n"); ++fails; } \
    } while (0)

size_t rbytes(int t, int n) { return t == 2 ? n / 32 * 18 : (t == 8 ? n / 32 * 34 : n / 256 * 110); }

// n rows x cols of N(0, ~scale) quantized to type t on the device
DeviceBuffer<uint8_t> qmat(int t, int rows, int cols, float scale, hipStream_t s) {
    std::vector<float> h((size_t)rows * cols);
    for (auto& v : h) v = scale * (urand() + urand() + urand());
    DeviceBuffer<float> d(h.size());
    hip_check(hipMemcpy(d.get(), h.data(), h.size() * 4, hipMemcpyHostToDevice), "h2d");
    DeviceBuffer<uint8_t> q((size_t)rows * rbytes(t, cols));
    chimere_quantize_weights(t, d.get(), q.get(), (int64_t)h.size(), s);
    check();
    hip_check(hipStreamSynchronize(s), "sync");
    return q;
}

DeviceBuffer<float> fvec(size_t n, float scale) {
    std::vector<float> h(n);
    for (auto& v : h) v = scale * urand();
    DeviceBuffer<float> d(n);
    hip_check(hipMemcpy(d.get(), h.data(), n * 4, hipMemcpyHostToDevice), "h2d");
    return d;
}

template <typename T>
std::vector<T> host(const DeviceBuffer<T>& d, size_t n) {
    std::vector<T> h(n);
    hip_check(hipMemcpy(h.data(), d.get(), n * sizeof(T), hipMemcpyDeviceToHost), "d2h");
    return h;
}

void layer_case(const char* name, int et, int st, int H, int F, int E, int K, bool gate_vec, bool bias, bool ncmoe) {
    hipStream_t s = nullptr;
    auto router = fvec((size_t)E * H, 0.05f);
    auto gate = qmat(et, E * F, H, 0.02f, s), up = qmat(et, E * F, H, 0.02f, s), down = qmat(et, E * H, F, 0.02f, s);
    DeviceBuffer<uint8_t> sg, su, sd;
    if (st >= 0) { sg = qmat(st, F, H, 0.02f, s); su = qmat(st, F, H, 0.02f, s); sd = qmat(st, H, F, 0.02f, s); }
    auto gw = fvec((size_t)H, 0.05f);
    auto lb = fvec((size_t)E, 0.5f);
    chimere_moe_layer c{};
    c.hidden = H; c.ffn = F; c.n_experts = E; c.top_k = K; c.expert_type = et; c.shared_type = st;
    c.router_w = router.get(); c.logit_bias = bias ? lb.get() : nullptr;
    c.gate_exps = gate.get(); c.up_exps = up.get(); c.down_exps = down.get();
    c.gate_stride = (int64_t)(F * rbytes(et, H)); c.up_stride = c.gate_stride; c.down_stride = (int64_t)(H * rbytes(et, F));
    c.sh_gate = st >= 0 ? sg.get() : nullptr; c.sh_up = st >= 0 ? su.get() : nullptr; c.sh_down = st >= 0 ? sd.get() : nullptr;
    c.sh_gate_w = gate_vec ? gw.get() : nullptr;
    MoeLayer L(c, 8, s);
    DeviceBuffer<float> o1(H), o2(H), o3(H), ws(K), ws2(K), ws3(K);
    DeviceBuffer<int> i1(K), i2(K), i3(K);
    std::vector<uint8_t> hg, hu, hd;
    if (ncmoe) {
        hg = host(gate, gate.size()); hu = host(up, up.size()); hd = host(down, down.size());
        L.attach_cpu_experts(hg.data(), hu.data(), hd.data());
    }
    for (int rep = 0; rep < 3; rep++) {
        auto x = fvec((size_t)H, 1.5f);
        L.forward(x.get(), o1.get(), 1, i1.get(), ws.get(), s);
        L.forward_v3(x.get(), o2.get(), i2.get(), ws2.get(), s);
        hip_check(hipStreamSynchronize(s), "sync");
        auto a = host(o1, H), b = host(o2, H);
        auto ia = host(i1, K), ib = host(i2, K);
        auto wa = host(ws, K), wb = host(ws2, K);
        EXPECT(ia == ib, "%s rep %d: routing indices differ", name, rep);
        EXPECT(std::memcmp(wa.data(), wb.data(), 4 * K) == 0, "%s rep %d: routing weights differ", name, rep);
        EXPECT(std::memcmp(a.data(), b.data(), 4 * H) == 0, "%s rep %d: V3 output differs from the fused layer", name, rep);
        if (ncmoe) {
            L.forward_ncmoe(x.get(), o3.get(), i3.get(), ws3.get(), 4, s);
            auto c3 = host(o3, H);
            EXPECT(host(i3, K) == ia, "%s rep %d: ncmoe routing differs", name, rep);
            double num = 0, den = 0;
            for (int i = 0; i < H; i++) { num += (c3[i] - a[i]) * (double)(c3[i] - a[i]); den += (double)a[i] * a[i]; }
            EXPECT(std::sqrt(num) <= 0.03 * std::sqrt(den), "%s rep %d: ncmoe output off by %g", name, rep,
                   std::sqrt(num / (den + 1e-30)));
        }
    }
}

}  // namespace

int main() {
    try {
        layer_case("q4_0 gated", 2, 2, 1024, 256, 32, 4, true, false, false);
        layer_case("q4_0 ungated bias", 2, 8, 1024, 512, 64, 8, false, true, false);
        layer_case("iq3s q8_0 shared", 21, 8, 2048, 512, 64, 8, false, false, true);
        layer_case("iq3s no shared", 21, -1, 512, 256, 16, 4, false, true, true);
        // the fused f32 GEMV wrapper = quantize + Q8_1 GEMV
        {
            hipStream_t s = nullptr;
            const int R = 300, C = 2048;
            auto W = qmat(8, R, C, 0.02f, s);
            auto x = fvec(C, 1.0f);
            DeviceBuffer<uint8_t> q8(q8_1_row_bytes(C)), q8b(q8_1_row_bytes(C));
            DeviceBuffer<float> y1(R), y2(R);
            ggml_gpu_gemv_q8_0_f32(W.get(), x.get(), y1.get(), q8.get(), R, C, s);
            ggml_gpu_quantize_q8_1(x.get(), q8b.get(), C, s);
            ggml_gpu_gemv_q8_0_q8(W.get(), q8b.get(), y2.get(), R, C, s);
            hip_check(hipStreamSynchronize(s), "sync");
            auto a = host(y1, R), b = host(y2, R);
            EXPECT(std::memcmp(a.data(), b.data(), 4 * R) == 0, "f32 GEMV wrapper differs from quantize + GEMV");
        }
        // a rejected call throws
        {
            bool threw = false;
            try {
                ggml_gpu_gemv_q4_0_q8(nullptr, nullptr, nullptr, 16, 2048, nullptr);
            } catch (const Error& e) {
                threw = e.code == CHIMERE_ERR_ARG;
            }
            EXPECT(threw, "a null-pointer GEMV did not throw");
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    if (fails) return 1;
    std::printf("host mirror ok\n");
    return 0;
}
