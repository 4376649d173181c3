// host_test.cpp -- tests of the C++ host mirror (gonn_amd/host) of GoNN's
// attention seam, checked against the fp64 oracle (oracle/liboracle.so, the
// test-only C restatement of GoNN's CPU attention).
//
//   host_test cpu   argument checks, shape ops, Linear vs the oracle, the
//                   no-device error path (no GPU calls)
//   host_test gpu   MultiHeadAttention (config C1 and a D = 128 variant)
//                   Forward / ForwardFused vs the oracle's MHA, fusedAttnDiff's
//                   backward vs the oracle's autograd, in both MFMA modes
//
// Mirrors the reference's checks: benchmark/mha/main.go:55-73 (ForwardFused
// vs Forward), nn/attention_test.go (shape panics), benchmark/flashbwd
// (gradients). Tolerances: fp32-MFMA max-abs 1e-4; bf16-MFMA
// |got - ref| <= 2e-2 + 1e-2 |ref|. Exit status 0 = all passed.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "gonn_hip.h"
#include "gonn_host.hpp"

extern "C" {
int oracle_attn_fwd(const double* Q, const double* K, const double* V, double* O, double* LSE,
                    int BH, int H, int Sq, int Sk, int D, double scale, int causal,
                    const int* kv_len, const int* rows, int nrows);
int oracle_attn_bwd_autograd(const double* Q, const double* K, const double* V, const double* dO,
                             double* dQ, double* dK, double* dV, int BH, int S, int D,
                             double scale, int causal);
int oracle_attn_fwd_ex(const double* Q, const double* K, const double* V, double* O,
                       double* LSE, int BH, int H, int Sq, int Sk, int D, double scale,
                       int causal, const int* kv_len, const double* amask, long mask_sb,
                       long mask_sh, const int* rows, int nrows);
int oracle_attn_bwd_autograd_ex(const double* Q, const double* K, const double* V,
                                const double* dO, double* dQ, double* dK, double* dV, int BH,
                                int H, int S, int D, double scale, int causal, const int* kv_len,
                                const double* amask, long mask_sb, long mask_sh);
int oracle_attn_bwd_autograd_x(const double* Q, const double* K, const double* V,
                               const double* dO, double* dQ, double* dK, double* dV, int BH,
                               int H, int Sq, int Sk, int D, double scale, int causal,
                               const int* kv_len, const double* amask, long mask_sb,
                               long mask_sh);
int oracle_linear(const double* x, const double* W, const double* b, double* y, int N, int in,
                  int out);
void oracle_heads(const double* in, double* out, int B, int T, int H, int D, int dir);
}

using gonn::nn::Linear;
using gonn::nn::MultiHeadAttention;
using gonn::nn::Tensor;

static int g_fail = 0;

#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                     \
            std::printf("\n");                            \
            g_fail++;                                     \
        }                                                 \
    } while (0)

// splitmix64 -> Box-Muller N(0,1), a documented deterministic stream.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    double normal() {
        const double u = uniform(), v = uniform();
        return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
    }
    std::vector<double> normals(size_t n, double mul = 1.0) {
        std::vector<double> x(n);
        for (auto& e : x) e = normal() * mul;
        return x;
    }
};

template <typename F>
static bool throws_invalid(F f) {
    try {
        f();
    } catch (const std::invalid_argument&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

// max |got - ref| and whether every element is within atol + rtol |ref|.
static bool close(const std::vector<double>& got, const std::vector<double>& ref, double atol,
                  double rtol, const char* what) {
    if (got.size() != ref.size()) {
        std::printf("[%s] size %zu vs %zu\n", what, got.size(), ref.size());
        return false;
    }
    double mx = 0.0;
    bool ok = true;
    for (size_t i = 0; i < got.size(); i++) {
        const double e = std::fabs(got[i] - ref[i]);
        if (!(e <= atol + rtol * std::fabs(ref[i]))) ok = false;
        if (e > mx || std::isnan(e)) mx = e;
    }
    std::printf("[%s] max_abs %.3e (atol %.0e rtol %.0e)\n", what, mx, atol, rtol);
    return ok;
}

static Linear make_linear(Rng& r, int out, int in) {
    Linear l;
    l.W = Tensor::New(r.normals((size_t)out * in, 1.0 / std::sqrt((double)in)), {out, in});
    l.B = r.normals(out, 0.1);
    return l;
}

// The oracle's MHA forward: projections, split heads, core, merge, output;
// Tq and Tk may differ, kvLen (empty = none) is a prefix key-padding mask.
static std::vector<double> oracle_mha(const MultiHeadAttention& m, const Tensor& q,
                                      const Tensor& k, const Tensor& v, bool causal,
                                      const std::vector<int>& kvLen = {},
                                      const std::vector<double>& maskBQK = {}) {
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1], E = m.EmbedDim, H = m.NumHeads,
              D = m.HeadDim;
    auto lin = [](const Linear& l, const Tensor& x) {
        const int out = l.W.Shape[0], in = l.W.Shape[1], N = (int)(x.Numel() / in);
        std::vector<double> y((size_t)N * out);
        oracle_linear(x.Data.data(), l.W.Data.data(), l.B.data(), y.data(), N, in, out);
        return y;
    };
    std::vector<double> qp = lin(m.QProj, q), kp = lin(m.KProj, k), vp = lin(m.VProj, v);
    std::vector<double> qh(qp.size()), kh(kp.size()), vh(vp.size()), o(qp.size()), ctx(qp.size());
    oracle_heads(qp.data(), qh.data(), B, Tq, H, D, 0);
    oracle_heads(kp.data(), kh.data(), B, Tk, H, D, 0);
    oracle_heads(vp.data(), vh.data(), B, Tk, H, D, 0);
    // maskBQK: an optional (B, Tq, Tk) additive mask
    oracle_attn_fwd_ex(qh.data(), kh.data(), vh.data(), o.data(), nullptr, B * H, H, Tq, Tk, D,
                       1.0 / std::sqrt((double)D), causal ? 1 : 0,
                       kvLen.empty() ? nullptr : kvLen.data(),
                       maskBQK.empty() ? nullptr : maskBQK.data(), (long)Tq * Tk, 0, nullptr, 0);
    oracle_heads(o.data(), ctx.data(), B, Tq, H, D, 1);
    Tensor c = Tensor::New(ctx, {B, Tq, E});
    return lin(m.OutProj, c);
}

// op(X) materialised by explicit transposition, then the textbook triple
// loop: the brute-force check of the backends' strided GEMM.
static std::vector<double> naive_gemm(const std::vector<double>& a, const std::vector<double>& b,
                                      int batch, int m, int k, int n, bool ta, bool tb) {
    std::vector<double> c((size_t)batch * m * n);
    std::vector<double> A((size_t)m * k), B((size_t)k * n);
    for (int z = 0; z < batch; z++) {
        for (int i = 0; i < m; i++)
            for (int p = 0; p < k; p++)
                A[(size_t)i * k + p] = ta ? a[(size_t)z * m * k + (size_t)p * m + i]
                                          : a[(size_t)z * m * k + (size_t)i * k + p];
        for (int p = 0; p < k; p++)
            for (int j = 0; j < n; j++)
                B[(size_t)p * n + j] = tb ? b[(size_t)z * k * n + (size_t)j * k + p]
                                          : b[(size_t)z * k * n + (size_t)p * n + j];
        for (int i = 0; i < m; i++)
            for (int j = 0; j < n; j++) {
                double s = 0.0;
                for (int p = 0; p < k; p++) s += A[(size_t)i * k + p] * B[(size_t)p * n + j];
                c[(size_t)z * m * n + (size_t)i * n + j] = s;
            }
    }
    return c;
}

struct GemmCase {
    int batch, m, k, n;
    bool ta, tb;
};
// backend/backend_test.go:54-66, plus a transA-only batched case.
static const GemmCase kGemmCases[] = {{1, 3, 4, 5, false, false}, {1, 3, 4, 5, true, false},
                                      {1, 3, 4, 5, false, true},  {1, 3, 4, 5, true, true},
                                      {4, 2, 3, 2, false, false}, {4, 2, 3, 2, true, true},
                                      {2, 1, 1, 1, false, false}, {3, 5, 2, 4, false, true},
                                      {3, 5, 7, 4, true, false}};

static void test_backend_cpu(Rng& r) {
    namespace be = gonn::backend;
    auto cpu = be::NewCPU();
    CHECK(cpu->Name() == "cpu" && be::Current()->Name() == "cpu", "default backend is cpu");
    for (const GemmCase& c : kGemmCases) {
        const auto a = r.normals((size_t)c.batch * c.m * c.k);
        const auto b = r.normals((size_t)c.batch * c.k * c.n);
        const auto got = cpu->Gemm(a, b, c.batch, c.m, c.k, c.n, c.ta, c.tb);
        CHECK(close(got, naive_gemm(a, b, c.batch, c.m, c.k, c.n, c.ta, c.tb), 1e-12, 0.0,
                    "cpu Gemm vs naive"),
              "cpu Gemm %d %d %d %d %d %d", c.batch, c.m, c.k, c.n, c.ta, c.tb);
    }
    CHECK(cpu->Gemm({}, {}, 0, 3, 4, 5, false, false).empty(), "Gemm batch=0 is empty");
    CHECK(throws_invalid([&] { cpu->Gemm(std::vector<double>(5), std::vector<double>(20), 1, 2, 3, 4, false, false); }),
          "Gemm short A");

    // backend_test.go:90-111: Use/Current from several threads, then restored.
    auto start = be::Current();
    std::vector<std::thread> ts;
    bool nil_seen = false;
    for (int g = 0; g < 8; g++)
        ts.emplace_back([&] {
            for (int i = 0; i < 1000; i++) {
                auto prev = be::Use(be::NewCPU());
                if (!be::Current()) nil_seen = true;
                be::Use(prev);
            }
        });
    for (auto& t : ts) t.join();
    be::Use(start);
    CHECK(!nil_seen && be::Current() == start, "Use/Current concurrent");

    // backend_test.go:117-126: the CPU backend is not an Elementwiser.
    CHECK(dynamic_cast<const be::Elementwiser*>(cpu.get()) == nullptr, "cpu is not an Elementwiser");

    if (!gonn::hip::Available()) {
        int code = 0;
        try {
            be::NewHIP();
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_NODEVICE, "NewHIP without device: code %d", code);
        code = 0;
        std::vector<double> w(64 * 64, 0.0);
        try {
            gonn::hip::DeviceMHA dm(64, 4, 64, 64, w, {}, w, {}, w, {}, w, {});
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_NODEVICE, "DeviceMHA without device: code %d", code);
    }
    {
        std::vector<double> w(64 * 64, 0.0), shortw(10, 0.0);
        CHECK(throws_invalid([&] { gonn::hip::DeviceMHA(64, 4, 64, 64, w, {}, shortw, {}, w, {}, w, {}); }),
              "DeviceMHA short Wk");
    }
}

static void test_cpu() {
    // Supports: the head dims the kernels cover (replaces D == 64 at
    // nn/attention.go:129).
    CHECK(gonn::hip::Supports(64, 128, 128) && gonn::hip::Supports(128, 7, 300), "Supports 64/128");
    CHECK(!gonn::hip::Supports(32, 128, 128) && !gonn::hip::Supports(256, 128, 128),
          "Supports rejects other D");
    CHECK(!gonn::hip::Supports(64, 0, 128), "Supports rejects empty");

    // Mode switching and its error.
    const int m0 = gonn::hip::Mode();
    gonn::hip::SetMode(1);
    CHECK(gonn::hip::Mode() == 1, "SetMode(1)");
    gonn::hip::SetMode(m0);
    bool threw = false;
    try {
        gonn::hip::SetMode(7);
    } catch (const gonn::hip::Error& e) {
        threw = e.code == GONN_E_INVALID;
    }
    CHECK(threw, "SetMode(7) throws GONN_E_INVALID");

    // Short slices panic in Go; they throw invalid_argument here, before any
    // device work.
    std::vector<double> a(8 * 16 * 64, 0.0), shortv(10, 0.0), o(a.size());
    CHECK(throws_invalid([&] { gonn::hip::FlashAttnF64(a, shortv, a, o, 8, 16, 64, 0.125, true); }),
          "FlashAttnF64 short K");
    CHECK(throws_invalid([&] { gonn::hip::FlashAttnF64Fwd(a, a, a, 0, 16, 64, 0.125, true); }),
          "FlashAttnF64Fwd BH = 0");
    CHECK(throws_invalid([&] {
              gonn::hip::FlashAttnF64Bwd(a, a, a, a, shortv, a, 8, 16, 64, 0.125, true);
          }),
          "FlashAttnF64Bwd short L");

    // Tensor shape ops and the head split match the oracle's Permute copy.
    Rng r(11);
    Tensor x = Tensor::New(r.normals(2 * 5 * 3 * 4), {2, 5, 3, 4});
    Tensor p = x.Permute0213();
    CHECK(p.Shape == std::vector<int>({2, 3, 5, 4}), "Permute shape");
    std::vector<double> ref(x.Numel());
    oracle_heads(x.Data.data(), ref.data(), 2, 5, 3, 4, 0);
    CHECK(p.Data == ref, "Permute0213 == oracle split heads");
    CHECK(p.Permute0213().Data == x.Data, "Permute0213 is an involution");
    CHECK(throws_invalid([&] { x.Reshape({7, 7}); }), "Reshape size check");
    CHECK(throws_invalid([&] { Tensor::New(std::vector<double>(5), {2, 3}); }), "New size check");

    // Linear vs the oracle's Linear.Forward.
    Linear l = make_linear(r, 24, 40);
    Tensor in = Tensor::New(r.normals(3 * 7 * 40), {3, 7, 40});
    Tensor y = l.Forward(in);
    std::vector<double> yref(3 * 7 * 24);
    oracle_linear(in.Data.data(), l.W.Data.data(), l.B.data(), yref.data(), 21, 40, 24);
    CHECK(y.Shape == std::vector<int>({3, 7, 24}), "Linear shape");
    CHECK(close(y.Data, yref, 1e-12, 0.0, "Linear vs oracle"), "Linear vs oracle");
    test_backend_cpu(r);
    {
        using gonn::nn::maskStrides;
        CHECK((maskStrides({5, 7}, 2, 3, 5, 7) == std::array<long, 2>{0, 0}), "mask (Tq,Tk)");
        CHECK((maskStrides({2, 5, 7}, 2, 3, 5, 7) == std::array<long, 2>{35, 0}), "mask (B,Tq,Tk)");
        CHECK((maskStrides({6, 5, 7}, 2, 3, 5, 7) == std::array<long, 2>{105, 35}), "mask (B*H,Tq,Tk)");
        CHECK((maskStrides({2, 3, 5, 7}, 2, 3, 5, 7) == std::array<long, 2>{105, 35}), "mask 4-D");
        CHECK(throws_invalid([&] { maskStrides({5, 8}, 2, 3, 5, 7); }), "mask bad shape");
    }

    // MultiHeadAttention construction and checkQKVDims (nn/attention.go:45-103).
    CHECK(throws_invalid([&] {
              MultiHeadAttention(30, 4, make_linear(r, 30, 30), make_linear(r, 30, 30),
                                 make_linear(r, 30, 30), make_linear(r, 30, 30));
          }),
          "embedDim %% numHeads");
    MultiHeadAttention m(32, 4, make_linear(r, 32, 32), make_linear(r, 32, 32),
                         make_linear(r, 32, 32), make_linear(r, 32, 32));
    Tensor q = Tensor::New(r.normals(2 * 6 * 32), {2, 6, 32});
    Tensor qbad = Tensor::New(r.normals(2 * 6 * 31), {2, 6, 31});
    Tensor k5 = Tensor::New(r.normals(2 * 5 * 32), {2, 5, 32});
    CHECK(throws_invalid([&] { m.Forward(qbad, q, q, false); }), "q feature dim");
    CHECK(throws_invalid([&] { m.Forward(q, q, k5, false); }), "k/v length mismatch");

    // Without a device the fused core reports GONN_E_NODEVICE rather than
    // running anywhere else.
    if (!gonn::hip::Available()) {
        int code = 0;
        try {
            m.Forward(q, q, q, true);
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_NODEVICE, "Forward without device: code %d", code);
        code = 0;
        try {
            std::vector<double> z(4 * 8 * 64, 0.0), oz(z.size());
            gonn::hip::FlashAttnF64(z, z, z, oz, 4, 8, 64, 0.125, false);
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_NODEVICE, "FlashAttnF64 without device: code %d", code);
        code = 0;
        try {
            gonn::hip::KVCache c(2, 2, 16, 64);
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_NODEVICE, "KVCache without device: code %d", code);
    }
    // The cache checks its arguments before the device.
    {
        int code = 0;
        try {
            gonn::hip::KVCache c(2, 2, 16, 96);
        } catch (const gonn::hip::Error& e) {
            code = e.code;
        }
        CHECK(code == GONN_E_UNSUPPORTED, "KVCache D=96: code %d", code);
    }
}

// The HIP backend's GEMM (gonn_hip_gemm_f64) against the host loop at the
// reference's GPU-vs-CPU bar of 1e-10 (tensor/cuda_dispatch_test.go:127-131),
// and the MHA with its projections on it against the oracle.
static void test_backend_gpu() {
    namespace be = gonn::backend;
    auto dev = be::NewHIP();
    auto cpu = be::NewCPU();
    CHECK(dev->Name() == "hip", "NewHIP name");
    Rng r(77);
    std::vector<GemmCase> cases(std::begin(kGemmCases), std::end(kGemmCases));
    cases.push_back({1, 31, 17, 23, false, false});  // cuda_dispatch_test.go:119
    cases.push_back({6, 8, 5, 7, false, false});     // the (2,3,8,5)@(2,3,5,7) batch
    cases.push_back({2, 130, 257, 66, true, true});
    for (const GemmCase& c : cases) {
        const auto a = r.normals((size_t)c.batch * c.m * c.k);
        const auto b = r.normals((size_t)c.batch * c.k * c.n);
        const auto got = dev->Gemm(a, b, c.batch, c.m, c.k, c.n, c.ta, c.tb);
        CHECK(close(got, cpu->Gemm(a, b, c.batch, c.m, c.k, c.n, c.ta, c.tb), 1e-10, 0.0,
                    "hip Gemm vs cpu"),
              "hip Gemm %d %d %d %d %d %d", c.batch, c.m, c.k, c.n, c.ta, c.tb);
    }
    // Elementwiser: f64 kernels against host libm at 1e-12
    // (tensor/cuda_dispatch_test.go:48-106); + - * / bit-identical.
    {
        auto* ew = dynamic_cast<const be::Elementwiser*>(dev.get());
        CHECK(ew != nullptr, "hip backend is an Elementwiser");
        const size_t n = 4099;
        std::vector<double> x = r.normals(n), y = r.normals(n), out(n);
        for (double& v : y) v += 3.0;
        auto host = [](int kind, double v) {
            switch (kind) {
                case be::UnaryReLU: return v > 0.0 ? v : 0.0;
                case be::UnarySigmoid: return 1.0 / (1.0 + std::exp(-v));
                case be::UnaryTanh: return std::tanh(v);
                case be::UnaryExp: return std::exp(v);
                case be::UnaryLog: return std::log(std::fabs(v) + 0.05);
                case be::UnaryGELU:
                    return 0.5 * v * (1.0 + std::tanh(std::sqrt(2.0 / M_PI) * (v + 0.044715 * v * v * v)));
                case be::UnarySiLU: return v / (1.0 + std::exp(-v));
                default: return 0.5 * v * (1.0 + std::erf(v / std::sqrt(2.0)));
            }
        };
        for (int kind = be::UnaryReLU; kind <= be::UnaryGELUExact; kind++) {
            std::vector<double> in = x;
            if (kind == be::UnaryLog)
                for (double& v : in) v = std::fabs(v) + 0.05;
            CHECK(ew && ew->Unary((be::UnaryKind)kind, in, out), "Unary %d accepted", kind);
            std::vector<double> ref(n);
            for (size_t i = 0; i < n; i++) ref[i] = host(kind, x[i]);
            CHECK(close(out, ref, 1e-12, 0.0, "hip Unary vs libm"), "Unary %d", kind);
        }
        CHECK(ew && !ew->Unary(be::UnaryNone, x, out), "UnaryNone declined");
        for (int kind = be::BinaryAdd; kind <= be::BinaryDiv; kind++) {
            CHECK(ew && ew->Binary((be::BinaryKind)kind, x, y, out), "Binary %d accepted", kind);
            bool same = true;
            for (size_t i = 0; i < n; i++) {
                const double ref = kind == be::BinaryAdd ? x[i] + y[i]
                                   : kind == be::BinarySub ? x[i] - y[i]
                                   : kind == be::BinaryMul ? x[i] * y[i]
                                                           : x[i] / y[i];
                same = same && out[i] == ref;
            }
            CHECK(same, "Binary %d bit-identical", kind);
        }
    }
    const auto z = dev->Gemm(std::vector<double>(0), std::vector<double>(0), 2, 3, 0, 4, false, false);
    CHECK(z.size() == 24 && z == std::vector<double>(24, 0.0), "hip Gemm k=0 gives zeros");

    const int B = 2, T = 128, E = 256, H = 4;
    const double ws = 1.0 / std::sqrt((double)E);
    auto lin = [&] {
        Linear l;
        l.W = Tensor::New(r.normals((size_t)E * E, ws), {E, E});
        l.B = r.normals(E, ws);
        return l;
    };
    MultiHeadAttention m(E, H, lin(), lin(), lin(), lin());
    Tensor x = Tensor::New(r.normals((size_t)B * T * E, ws), {B, T, E});
    const std::vector<double> ref = oracle_mha(m, x, x, x, true);
    gonn::hip::SetMode(0);
    const Tensor on_cpu = m.ForwardFused(x, x, x, true);
    auto prev = be::Use(dev);
    const Tensor on_dev = m.ForwardFused(x, x, x, true);
    be::Use(prev);
    CHECK(close(on_dev.Data, ref, 1e-4, 0.0, "MHA, projections on the HIP backend"),
          "MHA on HIP backend vs oracle");
    CHECK(close(on_dev.Data, on_cpu.Data, 1e-9, 0.0, "MHA HIP backend vs CPU backend"),
          "MHA HIP backend vs CPU backend");
}

// The resident layer (weights in HBM) against the oracle and against the
// host-projection path with its projections on the HIP backend.
static void test_resident_gpu() {
    namespace be = gonn::backend;
    Rng r(91);
    const int B = 2, T = 128, E = 256, H = 4;
    const double ws = 1.0 / std::sqrt((double)E);
    auto lin = [&](int in) {
        Linear l;
        l.W = Tensor::New(r.normals((size_t)E * in, 1.0 / std::sqrt((double)in)), {E, in});
        l.B = r.normals(E, ws);
        return l;
    };
    gonn::hip::SetMode(0);
    {
        MultiHeadAttention m(E, H, lin(E), lin(E), lin(E), lin(E));
        Tensor x = Tensor::New(r.normals((size_t)B * T * E, ws), {B, T, E});
        auto res = m.ToDevice();
        const Tensor y = res.Forward(x, x, x, true);
        CHECK(y.Shape == std::vector<int>({B, T, E}), "resident shape");
        CHECK(close(y.Data, oracle_mha(m, x, x, x, true), 1e-4, 0.0, "resident C1 vs oracle"),
              "resident C1 vs oracle");
        auto prev = be::Use(be::NewHIP());
        const Tensor hostp = m.ForwardFused(x, x, x, true);
        be::Use(prev);
        CHECK(close(y.Data, hostp.Data, 1e-12, 0.0, "resident == HIP-backend projections"),
              "resident == host-projection path");
    }
    {
        const int Tq = 40, Tk = 90, kdim = 96, vdim = 160;
        MultiHeadAttention m(E, H, lin(E), lin(kdim), lin(vdim), lin(E));
        Tensor q = Tensor::New(r.normals((size_t)B * Tq * E, ws), {B, Tq, E});
        Tensor k = Tensor::New(r.normals((size_t)B * Tk * kdim, ws), {B, Tk, kdim});
        Tensor v = Tensor::New(r.normals((size_t)B * Tk * vdim, ws), {B, Tk, vdim});
        Tensor pad = Tensor::Zeros({B, Tk});
        for (int t = 33; t < Tk; t++) pad.Data[Tk + t] = 1.0;  // sequence 1 keeps 33 keys
        auto res = m.ToDevice();
        const Tensor ym = res.ForwardMasked(q, k, v, true, pad);
        CHECK(close(ym.Data, oracle_mha(m, q, k, v, true, {Tk, 33}), 1e-4, 0.0,
                    "resident cross + key padding vs oracle"),
              "resident cross + key padding");
        CHECK(close(ym.Data, m.ForwardMasked(q, k, v, true, pad).Data, 1e-9, 0.0,
                    "resident == ForwardMasked"),
              "resident == ForwardMasked");
        CHECK(throws_invalid([&] { res.Forward(q, q, v, false); }), "resident checkQKVDims");
    }
}

// fusedAttnDiff with key padding: the node's backward through
// gonn_hip_flash_attn_f64_bwd_ex against the oracle's autograd chain.
static void test_diff_key_padding_gpu() {
    const int B = 2, H = 2, S = 70, D = 64, BH = B * H;
    const size_t n = (size_t)BH * S * D;
    Rng r(313);
    Tensor q = Tensor::New(r.normals(n), {BH, S, D}), k = Tensor::New(r.normals(n), {BH, S, D}),
           v = Tensor::New(r.normals(n), {BH, S, D}), g = Tensor::New(r.normals(n), {BH, S, D});
    const std::vector<int> lens = {70, 23};
    const double scale = 1.0 / std::sqrt((double)D);
    gonn::hip::SetMode(0);
    gonn::nn::DiffOut f = gonn::nn::fusedAttnDiff(q, k, v, BH, S, D, scale, true, lens, H);
    std::vector<double> ro(n), rq(n), rk(n), rv(n);
    oracle_attn_fwd(q.Data.data(), k.Data.data(), v.Data.data(), ro.data(), nullptr, BH, H, S, S,
                    D, scale, 1, lens.data(), nullptr, 0);
    oracle_attn_bwd_autograd_ex(q.Data.data(), k.Data.data(), v.Data.data(), g.Data.data(),
                                rq.data(), rk.data(), rv.data(), BH, H, S, D, scale, 1,
                                lens.data(), nullptr, 0, 0);
    CHECK(close(f.Out.Data, ro, 1e-4, 0.0, "fusedAttnDiff key padding O"), "diff kv O");
    const auto grads = f.Node.Backward(g);
    CHECK(close(grads[0].Data, rq, 1e-4, 0.0, "fusedAttnDiff key padding dQ"), "diff kv dQ");
    CHECK(close(grads[1].Data, rk, 1e-4, 0.0, "fusedAttnDiff key padding dK"), "diff kv dK");
    CHECK(close(grads[2].Data, rv, 1e-4, 0.0, "fusedAttnDiff key padding dV"), "diff kv dV");
}

// Additive masks (WithAttnMask): fusedAttnDiff with a (B, S, S) mask and key
// padding against the oracle's chain; maskStrides' shape rules.
static void test_attn_mask_gpu() {
    const int B = 2, H = 2, S = 60, D = 64, BH = B * H;
    const size_t n = (size_t)BH * S * D;
    Rng r(414);
    Tensor q = Tensor::New(r.normals(n), {BH, S, D}), k = Tensor::New(r.normals(n), {BH, S, D}),
           v = Tensor::New(r.normals(n), {BH, S, D}), g = Tensor::New(r.normals(n), {BH, S, D});
    Tensor m = Tensor::New(r.normals((size_t)B * S * S, 1.5), {B, S, S});
    for (int b = 0; b < B; b++)
        for (int i = 0; i < S; i++) m.Data[((size_t)b * S + i) * S + 7] = -1e30;  // blocked key
    const std::vector<int> lens = {60, 41};
    const double scale = 1.0 / std::sqrt((double)D);
    std::vector<double> ro(n), rq(n), rk(n), rv(n);
    oracle_attn_fwd_ex(q.Data.data(), k.Data.data(), v.Data.data(), ro.data(), nullptr, BH, H, S,
                       S, D, scale, 1, lens.data(), m.Data.data(), (long)S * S, 0, nullptr, 0);
    oracle_attn_bwd_autograd_ex(q.Data.data(), k.Data.data(), v.Data.data(), g.Data.data(),
                                rq.data(), rk.data(), rv.data(), BH, H, S, D, scale, 1,
                                lens.data(), m.Data.data(), (long)S * S, 0);
    // Both modes: forward and backward run the mode's kernels (the bf16 ones
    // have masked variants), at the mode's bar.
    for (int mode = 0; mode < 2; mode++) {
        gonn::hip::SetMode(mode);
        const double atol = mode ? 2e-2 : 1e-4, rtol = mode ? 1e-2 : 0.0;
        gonn::nn::DiffOut f = gonn::nn::fusedAttnDiff(q, k, v, BH, S, D, scale, true, lens, H, m);
        CHECK(close(f.Out.Data, ro, atol, rtol, "fusedAttnDiff attn mask O"), "mask O");
        const auto grads = f.Node.Backward(g);
        CHECK(close(grads[0].Data, rq, atol, rtol, "fusedAttnDiff attn mask dQ"), "mask dQ");
        CHECK(close(grads[1].Data, rk, atol, rtol, "fusedAttnDiff attn mask dK"), "mask dK");
        CHECK(close(grads[2].Data, rv, atol, rtol, "fusedAttnDiff attn mask dV"), "mask dV");
    }
    gonn::hip::SetMode(0);
}

static void test_gpu() {
    CHECK(gonn::hip::Available(), "no gfx950 device");
    if (!gonn::hip::Available()) return;
    struct Cfg {
        const char* name;
        int B, T, E, H;
        bool causal;
    };
    // C1: B=2, S=128, d_model=256, 4 heads, causal; and a
    // D = 128 variant with a ragged length.
    const Cfg cfgs[] = {{"C1 D=64", 2, 128, 256, 4, true},
                        {"D=128 T=77", 2, 77, 512, 4, true},
                        {"D=64 non-causal", 1, 200, 128, 2, false}};
    for (const Cfg& c : cfgs) {
        Rng r(1000 + c.T);
        const double ws = 1.0 / std::sqrt((double)c.E);
        auto lin = [&] {
            Linear l;
            l.W = Tensor::New(r.normals((size_t)c.E * c.E, ws), {c.E, c.E});
            l.B = r.normals(c.E, ws);
            return l;
        };
        MultiHeadAttention m(c.E, c.H, lin(), lin(), lin(), lin());
        const size_t n = (size_t)c.B * c.T * c.E;
        Tensor q = Tensor::New(r.normals(n, ws), {c.B, c.T, c.E});
        Tensor k = Tensor::New(r.normals(n, ws), {c.B, c.T, c.E});
        Tensor v = Tensor::New(r.normals(n, ws), {c.B, c.T, c.E});
        const std::vector<double> ref = oracle_mha(m, q, k, v, c.causal);
        for (int mode = 0; mode < 2; mode++) {
            gonn::hip::SetMode(mode);
            const double atol = mode ? 2e-2 : 1e-4, rtol = mode ? 1e-2 : 0.0;
            const std::string tag = std::string(c.name) + (mode ? " bf16" : " fp32");
            Tensor out = m.Forward(q, k, v, c.causal);
            CHECK(out.Shape == std::vector<int>({c.B, c.T, c.E}), "%s shape", tag.c_str());
            CHECK(close(out.Data, ref, atol, rtol, (tag + " Forward").c_str()), "%s Forward",
                  tag.c_str());
            // benchmark/mha/main.go:55-73: ForwardFused agrees with Forward.
            Tensor ff = m.ForwardFused(q, k, v, c.causal);
            CHECK(close(ff.Data, out.Data, 0.0, 0.0, (tag + " ForwardFused == Forward").c_str()),
                  "%s ForwardFused", tag.c_str());
        }
    }
    // fusedAttnDiff: the node's backward vs the oracle's autograd.
    for (int D : {64, 128}) {
        Rng r(77 + D);
        const int BH = 3, S = 97;
        const size_t n = (size_t)BH * S * D;
        Tensor qp = Tensor::New(r.normals(n), {1, BH, S, D});
        Tensor kp = Tensor::New(r.normals(n), {1, BH, S, D});
        Tensor vp = Tensor::New(r.normals(n), {1, BH, S, D});
        Tensor g = Tensor::New(r.normals(n), {1, BH, S, D});
        const double scale = 1.0 / std::sqrt((double)D);
        std::vector<double> ro(n), rq(n), rk(n), rv(n);
        oracle_attn_fwd(qp.Data.data(), kp.Data.data(), vp.Data.data(), ro.data(), nullptr, BH, 1,
                        S, S, D, scale, 1, nullptr, nullptr, 0);
        oracle_attn_bwd_autograd(qp.Data.data(), kp.Data.data(), vp.Data.data(), g.Data.data(),
                                 rq.data(), rk.data(), rv.data(), BH, S, D, scale, 1);
        for (int mode = 0; mode < 2; mode++) {
            gonn::hip::SetMode(mode);
            const double atol = mode ? 2e-2 : 1e-4, rtol = mode ? 1e-2 : 0.0;
            const std::string tag = "fusedAttnDiff D=" + std::to_string(D) + (mode ? " bf16" : " fp32");
            auto f = gonn::nn::fusedAttnDiff(qp, kp, vp, BH, S, D, scale, true);
            CHECK(f.Node.Op == "FlashAttn", "node op");
            CHECK(close(f.Out.Data, ro, atol, rtol, (tag + " O").c_str()), "%s O", tag.c_str());
            auto grads = f.Node.Backward(g);
            CHECK(close(grads[0].Data, rq, atol, rtol, (tag + " dQ").c_str()), "%s dQ", tag.c_str());
            CHECK(close(grads[1].Data, rk, atol, rtol, (tag + " dK").c_str()), "%s dK", tag.c_str());
            CHECK(close(grads[2].Data, rv, atol, rtol, (tag + " dV").c_str()), "%s dV", tag.c_str());
        }
    }
    gonn::hip::SetMode(0);
    // TransformerDecoderLayer's cross-attention Forward(x, memory, memory,
    // false) (nn/transformer.go:234), Tq != Tk, through Forward and its
    // LastNode: output vs the oracle's MHA, the node's gradients vs the
    // oracle's rectangular autograd chain on the projected heads.
    for (int D : {64, 128}) {
        const int B = 2, Tq = 45, Tk = 70, H = 2, E = H * D;
        Rng r(4000 + D);
        const double ws = 1.0 / std::sqrt((double)E);
        auto lin = [&] {
            Linear l;
            l.W = Tensor::New(r.normals((size_t)E * E, ws), {E, E});
            l.B = r.normals(E, 0.1);
            return l;
        };
        MultiHeadAttention m(E, H, lin(), lin(), lin(), lin());
        Tensor x = Tensor::New(r.normals((size_t)B * Tq * E, ws), {B, Tq, E});
        Tensor mem = Tensor::New(r.normals((size_t)B * Tk * E, ws), {B, Tk, E});
        const std::vector<double> ref = oracle_mha(m, x, mem, mem, false);
        // projected heads for the gradient reference
        auto heads = [&](const Linear& l, const Tensor& t, int T) {
            Tensor y = l.Forward(t).Reshape({B, T, H, D}).Permute0213();
            return y;
        };
        const Tensor qh = heads(m.QProj, x, Tq), kh = heads(m.KProj, mem, Tk),
                     vh = heads(m.VProj, mem, Tk);
        Tensor g = Tensor::New(r.normals((size_t)B * H * Tq * D), {B, H, Tq, D});
        std::vector<double> rq(qh.Numel()), rk(kh.Numel()), rv(vh.Numel());
        oracle_attn_bwd_autograd_x(qh.Data.data(), kh.Data.data(), vh.Data.data(), g.Data.data(),
                                   rq.data(), rk.data(), rv.data(), B * H, H, Tq, Tk, D,
                                   1.0 / std::sqrt((double)D), 0, nullptr, nullptr, 0, 0);
        for (int mode = 0; mode < 2; mode++) {
            gonn::hip::SetMode(mode);
            const double atol = mode ? 2e-2 : 1e-4, rtol = mode ? 1e-2 : 0.0;
            const std::string tag = "cross Forward D=" + std::to_string(D) + (mode ? " bf16" : " fp32");
            Tensor out = m.Forward(x, mem, mem, false);
            CHECK(close(out.Data, ref, atol, rtol, (tag + " out").c_str()), "%s out", tag.c_str());
            auto grads = m.LastNode.Backward(g);
            CHECK(close(grads[0].Data, rq, atol, rtol, (tag + " dQ").c_str()), "%s dQ", tag.c_str());
            CHECK(close(grads[1].Data, rk, atol, rtol, (tag + " dK").c_str()), "%s dK", tag.c_str());
            CHECK(close(grads[2].Data, rv, atol, rtol, (tag + " dV").c_str()), "%s dV", tag.c_str());
        }
    }
    gonn::hip::SetMode(0);
    // The wider gate: cross-attention (Tq != Tk) through ForwardFused and a
    // suffix key-padding mask through ForwardMasked, against the oracle.
    for (bool causal : {false, true}) {
        const int B = 3, Tq = 40, Tk = 64, E = 256, H = 4;
        Rng r(3000 + causal);
        const double ws = 1.0 / std::sqrt((double)E);
        auto lin = [&] {
            Linear l;
            l.W = Tensor::New(r.normals((size_t)E * E, ws), {E, E});
            l.B = r.normals(E, 0.1);
            return l;
        };
        MultiHeadAttention m(E, H, lin(), lin(), lin(), lin());
        Tensor q = Tensor::New(r.normals((size_t)B * Tq * E), {B, Tq, E});
        Tensor mem = Tensor::New(r.normals((size_t)B * Tk * E), {B, Tk, E});
        const std::string tag = causal ? " causal" : "";
        const Tensor y = m.ForwardFused(q, mem, mem, causal);
        CHECK(close(y.Data, oracle_mha(m, q, mem, mem, causal), 1e-4, 0.0,
                    ("cross ForwardFused" + tag).c_str()), "cross ForwardFused%s", tag.c_str());
        Tensor pad = Tensor::Zeros({B, Tk});
        for (int t = 50; t < Tk; t++) pad.Data[(size_t)1 * Tk + t] = 1.0;
        for (int t = 7; t < Tk; t++) pad.Data[(size_t)2 * Tk + t] = 1.0;
        const Tensor ym = m.ForwardMasked(q, mem, mem, causal, pad);
        CHECK(close(ym.Data, oracle_mha(m, q, mem, mem, causal, {Tk, 50, 7}), 1e-4, 0.0,
                    ("ForwardMasked" + tag).c_str()), "ForwardMasked%s", tag.c_str());
        // a padding mask with holes: added as keyPaddingMaskAdd's -1e30
        Tensor holes = pad;
        holes.Data[3] = 1.0;
        // a blocked leading key (under causal, row 0 sees key 0 alone: keep it)
        holes.Data[(size_t)2 * Tk + (causal ? 1 : 0)] = 1.0;
        std::vector<double> kpAdd((size_t)B * Tq * Tk, 0.0);
        for (int b = 0; b < B; b++)
            for (int i = 0; i < Tq; i++)
                for (int t = 0; t < Tk; t++)
                    if (holes.Data[(size_t)b * Tk + t] != 0) kpAdd[((size_t)b * Tq + i) * Tk + t] = -1e30;
        CHECK(close(m.ForwardMasked(q, mem, mem, causal, holes).Data,
                    oracle_mha(m, q, mem, mem, causal, {}, kpAdd), 1e-4, 0.0,
                    ("ForwardMasked holes" + tag).c_str()), "ForwardMasked holes%s", tag.c_str());
        // rows with no unblocked key: GoNN's -1e30 terms absorb their
        // scores (a uniform average over the keys of the row's maximum
        // summed mask, future keys included); the whole-row form
        Tensor full = pad;
        for (int t = 0; t < Tk; t++) full.Data[(size_t)1 * Tk + t] = 1.0;
        CHECK(close(m.ForwardMasked(q, mem, mem, causal, full).Data,
                    oracle_mha(m, q, mem, mem, causal, {Tk, 0, 7}), 1e-4, 0.0,
                    ("ForwardMasked fully padded" + tag).c_str()),
              "ForwardMasked fully padded%s", tag.c_str());
        {  // row 0 attends key 0 only under causal: blocking it leaves no key
            Tensor am = Tensor::Zeros({Tq, Tk});
            am.Data[0] = -1e30;
            for (int t = 0; t < Tk; t++) am.Data[(size_t)9 * Tk + t] = -1e30;  // row 9 blocked
            std::vector<double> amB((size_t)B * Tq * Tk);
            for (int b = 0; b < B; b++)
                std::copy(am.Data.begin(), am.Data.end(), amB.begin() + (size_t)b * Tq * Tk);
            CHECK(close(m.ForwardMasked(q, mem, mem, causal, Tensor{}, am).Data,
                        oracle_mha(m, q, mem, mem, causal, {}, amB), 1e-4, 0.0,
                        ("ForwardMasked blocked rows" + tag).c_str()),
                  "ForwardMasked blocked rows%s", tag.c_str());
            // refused: a blocked row whose best value keeps part of the score in fp64
            Tensor mid = Tensor::Zeros({Tq, Tk});
            for (int t = 0; t < Tk; t++) mid.Data[(size_t)4 * Tk + t] = -1e20;
            CHECK(throws_invalid([&] { m.ForwardMasked(q, mem, mem, causal, Tensor{}, mid); }),
                  "blocked row between the levels rejected");
        }
    }
    // Incremental decoding: ForwardIncremental over a KV cache in two chunks
    // equals the causal rows of the oracle's MHA over the whole sequence (the
    // cache holds bf16 K/V: bf16 bar).
    for (int H : {4, 2}) {
        const int B = 2, T = 24, E = 256;
        Rng r(2000 + H);
        const double ws = 1.0 / std::sqrt((double)E);
        auto lin = [&] {
            Linear l;
            l.W = Tensor::New(r.normals((size_t)E * E, ws), {E, E});
            l.B = r.normals(E, 0.1);
            return l;
        };
        MultiHeadAttention m(E, H, lin(), lin(), lin(), lin());
        Tensor x = Tensor::New(r.normals((size_t)B * T * E), {B, T, E});
        const std::vector<double> ref = oracle_mha(m, x, x, x, true);
        gonn::hip::KVCache cache = m.NewCache(B, 32);
        auto part = [&](int t0, int t1) {
            std::vector<double> d((size_t)B * (t1 - t0) * E);
            for (int b = 0; b < B; b++)
                for (int t = t0; t < t1; t++)
                    for (int e = 0; e < E; e++)
                        d[((size_t)b * (t1 - t0) + (t - t0)) * E + e] = x.Data[((size_t)b * T + t) * E + e];
            return Tensor::New(std::move(d), {B, t1 - t0, E});
        };
        const Tensor y1 = m.ForwardIncremental(part(0, 10), cache);
        const Tensor y2 = m.ForwardIncremental(part(10, T), cache);
        CHECK(cache.Lengths() == std::vector<int>({T, T}), "cache lengths");
        std::vector<double> got((size_t)B * T * E);
        for (int b = 0; b < B; b++)
            for (int t = 0; t < T; t++)
                for (int e = 0; e < E; e++)
                    got[((size_t)b * T + t) * E + e] =
                        t < 10 ? y1.Data[((size_t)b * 10 + t) * E + e]
                               : y2.Data[((size_t)b * (T - 10) + (t - 10)) * E + e];
        const std::string tag = "ForwardIncremental H=" + std::to_string(H);
        CHECK(close(got, ref, 2e-2, 1e-2, tag.c_str()), "%s", tag.c_str());
        // The resident layer decodes the same chunks on the device.
        {
            auto res = m.ToDevice();
            gonn::hip::KVCache dc = res.NewCache(B, 32);
            const Tensor r1 = res.ForwardIncremental(part(0, 10), dc);
            const Tensor r2 = res.ForwardIncremental(part(10, T), dc);
            CHECK(dc.Lengths() == std::vector<int>({T, T}), "resident cache lengths");
            std::vector<double> rg(got.size());
            for (int b = 0; b < B; b++)
                for (int t = 0; t < T; t++)
                    for (int e = 0; e < E; e++)
                        rg[((size_t)b * T + t) * E + e] =
                            t < 10 ? r1.Data[((size_t)b * 10 + t) * E + e]
                                   : r2.Data[((size_t)b * (T - 10) + (t - 10)) * E + e];
            const std::string rtag = "resident ForwardIncremental H=" + std::to_string(H);
            CHECK(close(rg, ref, 2e-2, 1e-2, rtag.c_str()), "%s", rtag.c_str());
        }
        // past Lmax: rejected, nothing written
        bool threw = false;
        try {
            std::vector<double> z((size_t)B * H * 20 * (E / H), 0.0);
            cache.Append(z, z, 20);
        } catch (const gonn::hip::Error& e) {
            threw = e.code == GONN_E_INVALID;
        }
        CHECK(threw && cache.Lengths() == std::vector<int>({T, T}), "append past Lmax rejected");
        cache.Reset();
        CHECK(cache.Lengths() == std::vector<int>({0, 0}), "Reset");
    }
    test_backend_gpu();
    test_resident_gpu();
    test_diff_key_padding_gpu();
    test_attn_mask_gpu();
}

int main(int argc, char** argv) {
    const std::string what = argc > 1 ? argv[1] : "cpu";
    try {
        if (what == "cpu") test_cpu();
        else if (what == "gpu") test_gpu();
        else {
            std::printf("usage: host_test cpu|gpu\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("FAIL: uncaught exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %s (%d failures)\n", what.c_str(), g_fail ? "FAILED" : "ok", g_fail);
    return g_fail ? 1 : 0;
}
