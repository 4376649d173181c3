// hip_backend.cpp -- gonn::hip, the C++ counterpart of the flash wrappers in
// backend/cuda/cuda.go:125-194, over the C ABI of include/gonn_hip.h.
//
// The reference wrappers allocate the host outputs, pass &slice[0] to C and
// take no lock (cuda.go:128-184); so do these. The reference's C entry points
// return void; the new ABI returns a status, turned into gonn::hip::Error the
// way the Go wrapper panics on it (the GEMM convention of cuda.go:62-64).
#include "gonn_host.hpp"

#include <cstddef>
#include <string>

#include "gonn_hip.h"

namespace gonn {
namespace hip {

Error::Error(int c, const std::string& where)
    : std::runtime_error("hip: " + where + ": " + gonn_hip_strerror(c)), code(c) {}

namespace {

void check(int rc, const char* where) {
    if (rc != 0) throw Error(rc, where);
}

// Go indexes &x[0] of a slice of the required length; a short slice panics.
void need(const std::vector<double>& x, size_t n, const char* what) {
    if (x.size() < n || n == 0)
        throw std::invalid_argument(std::string("hip: ") + what + ": length " +
                                    std::to_string(x.size()) + ", need " + std::to_string(n));
}

void shape_ok(int BH, int S, int d, const char* where) {
    if (BH <= 0 || S <= 0 || d <= 0)
        throw std::invalid_argument(std::string("hip: ") + where + ": BH, S, d must be >= 1");
}

}  // namespace

bool Available() { return gonn_hip_available() == 1; }

bool Supports(int D, int Tq, int Tk) { return gonn_hip_attn_supports(D, Tq, Tk) == 1; }

void SetMode(int mode) { check(gonn_hip_set_attn_mode(mode), "SetMode"); }

int Mode() { return gonn_hip_get_attn_mode(); }

void FlashAttnF64(const std::vector<double>& Q, const std::vector<double>& K,
                  const std::vector<double>& V, std::vector<double>& O, int BH, int S, int d,
                  double scale, bool causal) {
    shape_ok(BH, S, d, "FlashAttnF64");
    const size_t n = (size_t)BH * S * d;
    need(Q, n, "FlashAttnF64 Q");
    need(K, n, "FlashAttnF64 K");
    need(V, n, "FlashAttnF64 V");
    need(O, n, "FlashAttnF64 O");
    check(gonn_hip_flash_attn_f64(Q.data(), K.data(), V.data(), O.data(), BH, S, d, scale,
                                  causal ? 1 : 0),
          "FlashAttnF64");
}

FwdOut FlashAttnF64Fwd(const std::vector<double>& Q, const std::vector<double>& K,
                       const std::vector<double>& V, int BH, int S, int d, double scale,
                       bool causal) {
    shape_ok(BH, S, d, "FlashAttnF64Fwd");
    const size_t n = (size_t)BH * S * d;
    need(Q, n, "FlashAttnF64Fwd Q");
    need(K, n, "FlashAttnF64Fwd K");
    need(V, n, "FlashAttnF64Fwd V");
    FwdOut r;
    r.O.assign(n, 0.0);
    r.L.assign((size_t)BH * S, 0.0);
    check(gonn_hip_flash_attn_f64_fwd(Q.data(), K.data(), V.data(), r.O.data(), r.L.data(), BH, S,
                                      d, scale, causal ? 1 : 0),
          "FlashAttnF64Fwd");
    return r;
}

BwdOut FlashAttnF64Bwd(const std::vector<double>& Q, const std::vector<double>& K,
                       const std::vector<double>& V, const std::vector<double>& O,
                       const std::vector<double>& L, const std::vector<double>& dO, int BH,
                       int S, int d, double scale, bool causal) {
    shape_ok(BH, S, d, "FlashAttnF64Bwd");
    const size_t n = (size_t)BH * S * d;
    need(Q, n, "FlashAttnF64Bwd Q");
    need(K, n, "FlashAttnF64Bwd K");
    need(V, n, "FlashAttnF64Bwd V");
    need(O, n, "FlashAttnF64Bwd O");
    need(L, (size_t)BH * S, "FlashAttnF64Bwd L");
    need(dO, n, "FlashAttnF64Bwd dO");
    BwdOut r;
    r.dQ.assign(n, 0.0);
    r.dK.assign(n, 0.0);
    r.dV.assign(n, 0.0);
    check(gonn_hip_flash_attn_f64_bwd(Q.data(), K.data(), V.data(), O.data(), L.data(), dO.data(),
                                      r.dQ.data(), r.dK.data(), r.dV.data(), BH, S, d, scale,
                                      causal ? 1 : 0),
          "FlashAttnF64Bwd");
    return r;
}

double BenchFlashAttnF64(int BH, int S, int d, int iters, bool causal) {
    const double ms = gonn_hip_bench_flash_attn_f64(BH, S, d, iters, causal ? 1 : 0);
    if (ms < 0) throw Error((int)ms, "BenchFlashAttnF64");
    return ms;
}

}  // namespace hip
}  // namespace gonn
