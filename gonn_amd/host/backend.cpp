// backend.cpp -- gonn::backend, the C++ counterpart of the compute-target
// contract of backend/backend.go:61-118 (Backend, NewCPU, Use, Current) and of
// the CUDA backend's Gemm and Elementwiser methods (backend/cuda/cuda.go:30-106),
// over the C ABI's gonn_hip_gemm_f64 / gonn_hip_unary_f64 / gonn_hip_binary_f64.
#include "gonn_host.hpp"

#include <mutex>
#include <stdexcept>
#include <string>

#include "gonn_hip.h"

namespace gonn {
namespace backend {

namespace {

void check_lengths(const std::vector<double>& a, const std::vector<double>& b, int batch, int m,
                   int k, int n, const char* who) {
    if (batch < 0 || m < 0 || k < 0 || n < 0)
        throw std::invalid_argument(std::string(who) + ": negative GEMM dimension");
    const size_t an = (size_t)batch * m * k, bn = (size_t)batch * k * n;
    if (a.size() < an || b.size() < bn)
        throw std::invalid_argument(std::string(who) + ": A has " + std::to_string(a.size()) +
                                    " elements (need " + std::to_string(an) + "), B " +
                                    std::to_string(b.size()) + " (need " + std::to_string(bn) +
                                    ")");
}

// The host loop (backend/cpu.go): each C[i][j] summed over p in ascending
// order, the order of the reference's naive check (backend_test.go:23-45).
class CpuBackend final : public Backend {
public:
    std::string Name() const override { return "cpu"; }

    std::vector<double> Gemm(const std::vector<double>& a, const std::vector<double>& b, int batch,
                             int m, int k, int n, bool transA, bool transB) const override {
        check_lengths(a, b, batch, m, k, n, "cpu Gemm");
        std::vector<double> c((size_t)batch * m * n, 0.0);
        // Element (i, p) of op(A) is A[i*sa_i + p*sa_p]; likewise op(B).
        const size_t sa_i = transA ? 1 : (size_t)k, sa_p = transA ? (size_t)m : 1;
        const size_t sb_p = transB ? 1 : (size_t)n, sb_j = transB ? (size_t)k : 1;
        for (int z = 0; z < batch; z++) {
            const double* A = a.data() + (size_t)z * m * k;
            const double* B = b.data() + (size_t)z * k * n;
            double* C = c.data() + (size_t)z * m * n;
            for (int i = 0; i < m; i++)
                for (int j = 0; j < n; j++) {
                    double acc = 0.0;
                    for (int p = 0; p < k; p++) acc += A[i * sa_i + p * sa_p] * B[p * sb_p + j * sb_j];
                    C[(size_t)i * n + j] = acc;
                }
        }
        return c;
    }

    void Synchronize() const override {}
};

class HipBackend final : public Backend, public Elementwiser {
public:
    std::string Name() const override { return "hip"; }

    std::vector<double> Gemm(const std::vector<double>& a, const std::vector<double>& b, int batch,
                             int m, int k, int n, bool transA, bool transB) const override {
        check_lengths(a, b, batch, m, k, n, "hip Gemm");
        std::vector<double> c((size_t)batch * m * n, 0.0);
        if (c.empty()) return c;
        const int rc = gonn_hip_gemm_f64(a.empty() ? nullptr : a.data(),
                                         b.empty() ? nullptr : b.data(), c.data(), batch, m, k, n,
                                         transA ? 1 : 0, transB ? 1 : 0);
        if (rc != 0) throw hip::Error(rc, "Gemm");
        return c;
    }

    // Every gonn_hip_gemm_f64 call returns with its result on the host.
    void Synchronize() const override {}

    bool Unary(UnaryKind kind, const std::vector<double>& a,
               std::vector<double>& out) const override {
        if (kind < UnaryReLU || kind > UnaryGELUExact) return false;
        if (out.size() != a.size()) throw std::invalid_argument("hip Unary: len(out) != len(a)");
        if (a.empty()) return true;
        const int rc = gonn_hip_unary_f64(kind, a.data(), out.data(), (long)a.size());
        if (rc != 0) throw hip::Error(rc, "Unary");
        return true;
    }

    bool Binary(BinaryKind kind, const std::vector<double>& a, const std::vector<double>& b,
                std::vector<double>& out) const override {
        if (kind < BinaryAdd || kind > BinaryDiv) return false;
        if (b.size() != a.size() || out.size() != a.size())
            throw std::invalid_argument("hip Binary: operand lengths differ");
        if (a.empty()) return true;
        const int rc = gonn_hip_binary_f64(kind, a.data(), b.data(), out.data(), (long)a.size());
        if (rc != 0) throw hip::Error(rc, "Binary");
        return true;
    }
};

std::mutex g_mu;
std::shared_ptr<Backend>& current() {
    static std::shared_ptr<Backend> b = std::make_shared<CpuBackend>();
    return b;
}

}  // namespace

std::shared_ptr<Backend> NewCPU() { return std::make_shared<CpuBackend>(); }

std::shared_ptr<Backend> NewHIP() {
    if (!hip::Available()) throw hip::Error(GONN_E_NODEVICE, "NewHIP");
    return std::make_shared<HipBackend>();
}

std::shared_ptr<Backend> Use(std::shared_ptr<Backend> b) {
    if (!b) throw std::invalid_argument("backend: Use(nullptr)");
    std::lock_guard<std::mutex> lock(g_mu);
    std::shared_ptr<Backend> prev = std::move(current());
    current() = std::move(b);
    return prev;
}

std::shared_ptr<Backend> Current() {
    std::lock_guard<std::mutex> lock(g_mu);
    return current();
}

}  // namespace backend
}  // namespace gonn
