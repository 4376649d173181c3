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

FwdOut FlashAttnF64ExFwd(const std::vector<double>& Q, const std::vector<double>& K,
                         const std::vector<double>& V, int B, int H, int Sq, int Sk, int d,
                         double scale, bool causal, const std::vector<int>& kvLen) {
    if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || d <= 0)
        throw std::invalid_argument("hip: FlashAttnF64Ex: B, H, Sq, Sk, d must be >= 1");
    const size_t nq = (size_t)B * H * Sq * d, nk = (size_t)B * H * Sk * d;
    need(Q, nq, "FlashAttnF64Ex Q");
    need(K, nk, "FlashAttnF64Ex K");
    need(V, nk, "FlashAttnF64Ex V");
    if (!kvLen.empty() && (int)kvLen.size() != B)
        throw std::invalid_argument("hip: FlashAttnF64Ex: kvLen needs B entries");
    FwdOut r;
    r.O.assign(nq, 0.0);
    r.L.assign((size_t)B * H * Sq, 0.0);
    check(gonn_hip_flash_attn_f64_ex(Q.data(), K.data(), V.data(), r.O.data(), r.L.data(), B, H,
                                     Sq, Sk, d, scale, causal ? 1 : 0,
                                     kvLen.empty() ? nullptr : kvLen.data()),
          "FlashAttnF64Ex");
    return r;
}

std::vector<double> FlashAttnF64Ex(const std::vector<double>& Q, const std::vector<double>& K,
                                   const std::vector<double>& V, int B, int H, int Sq, int Sk,
                                   int d, double scale, bool causal,
                                   const std::vector<int>& kvLen) {
    return FlashAttnF64ExFwd(Q, K, V, B, H, Sq, Sk, d, scale, causal, kvLen).O;
}

// Elements a mask with these strides spans.
static size_t mask_span(int B, int H, int Sq, int Sk, long sb, long sh) {
    if (sb < 0 || sh < 0) throw std::invalid_argument("hip: mask strides must be >= 0");
    return (size_t)(B - 1) * sb + (size_t)(H - 1) * sh + (size_t)Sq * Sk;
}

FwdOut FlashAttnF64Masked(const std::vector<double>& Q, const std::vector<double>& K,
                          const std::vector<double>& V, int B, int H, int Sq, int Sk, int d,
                          double scale, bool causal, const std::vector<int>& kvLen,
                          const std::vector<double>& mask, long maskSB, long maskSH) {
    if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || d <= 0)
        throw std::invalid_argument("hip: FlashAttnF64Masked: B, H, Sq, Sk, d must be >= 1");
    const size_t nq = (size_t)B * H * Sq * d, nk = (size_t)B * H * Sk * d;
    need(Q, nq, "FlashAttnF64Masked Q");
    need(K, nk, "FlashAttnF64Masked K");
    need(V, nk, "FlashAttnF64Masked V");
    if (!mask.empty()) need(mask, mask_span(B, H, Sq, Sk, maskSB, maskSH), "FlashAttnF64Masked mask");
    if (!kvLen.empty() && (int)kvLen.size() != B)
        throw std::invalid_argument("hip: FlashAttnF64Masked: kvLen needs B entries");
    FwdOut r;
    r.O.assign(nq, 0.0);
    r.L.assign((size_t)B * H * Sq, 0.0);
    check(gonn_hip_flash_attn_f64_masked(Q.data(), K.data(), V.data(), r.O.data(), r.L.data(), B,
                                         H, Sq, Sk, d, scale, causal ? 1 : 0,
                                         kvLen.empty() ? nullptr : kvLen.data(),
                                         mask.empty() ? nullptr : mask.data(), maskSB, maskSH),
          "FlashAttnF64Masked");
    return r;
}

BwdOut FlashAttnF64BwdMasked(const std::vector<double>& Q, const std::vector<double>& K,
                             const std::vector<double>& V, const std::vector<double>& O,
                             const std::vector<double>& L, const std::vector<double>& dO, int B,
                             int H, int Sq, int Sk, int d, double scale, bool causal,
                             const std::vector<int>& kvLen, const std::vector<double>& mask,
                             long maskSB, long maskSH) {
    if (B <= 0 || H <= 0) throw std::invalid_argument("hip: FlashAttnF64BwdMasked: B, H must be >= 1");
    shape_ok(B * H, Sq, d, "FlashAttnF64BwdMasked");
    shape_ok(B * H, Sk, d, "FlashAttnF64BwdMasked");
    const size_t nq = (size_t)B * H * Sq * d, nk = (size_t)B * H * Sk * d;
    need(Q, nq, "FlashAttnF64BwdMasked Q");
    need(K, nk, "FlashAttnF64BwdMasked K");
    need(V, nk, "FlashAttnF64BwdMasked V");
    need(O, nq, "FlashAttnF64BwdMasked O");
    need(L, (size_t)B * H * Sq, "FlashAttnF64BwdMasked L");
    need(dO, nq, "FlashAttnF64BwdMasked dO");
    if (!mask.empty()) need(mask, mask_span(B, H, Sq, Sk, maskSB, maskSH), "FlashAttnF64BwdMasked mask");
    if (!kvLen.empty() && (int)kvLen.size() != B)
        throw std::invalid_argument("hip: FlashAttnF64BwdMasked: kvLen needs B entries");
    BwdOut r;
    r.dQ.assign(nq, 0.0);
    r.dK.assign(nk, 0.0);
    r.dV.assign(nk, 0.0);
    check(gonn_hip_flash_attn_f64_bwd_masked(Q.data(), K.data(), V.data(), O.data(), L.data(),
                                             dO.data(), r.dQ.data(), r.dK.data(), r.dV.data(), B,
                                             H, Sq, Sk, d, scale, causal ? 1 : 0,
                                             kvLen.empty() ? nullptr : kvLen.data(),
                                             mask.empty() ? nullptr : mask.data(), maskSB, maskSH),
          "FlashAttnF64BwdMasked");
    return r;
}

BwdOut FlashAttnF64BwdEx(const std::vector<double>& Q, const std::vector<double>& K,
                         const std::vector<double>& V, const std::vector<double>& O,
                         const std::vector<double>& L, const std::vector<double>& dO, int B,
                         int H, int S, int d, double scale, bool causal,
                         const std::vector<int>& kvLen) {
    if (B <= 0 || H <= 0) throw std::invalid_argument("hip: FlashAttnF64BwdEx: B, H must be >= 1");
    shape_ok(B * H, S, d, "FlashAttnF64BwdEx");
    const size_t n = (size_t)B * H * S * d;
    need(Q, n, "FlashAttnF64BwdEx Q");
    need(K, n, "FlashAttnF64BwdEx K");
    need(V, n, "FlashAttnF64BwdEx V");
    need(O, n, "FlashAttnF64BwdEx O");
    need(L, (size_t)B * H * S, "FlashAttnF64BwdEx L");
    need(dO, n, "FlashAttnF64BwdEx dO");
    if (!kvLen.empty() && (int)kvLen.size() != B)
        throw std::invalid_argument("hip: FlashAttnF64BwdEx: kvLen needs B entries");
    BwdOut r;
    r.dQ.assign(n, 0.0);
    r.dK.assign(n, 0.0);
    r.dV.assign(n, 0.0);
    check(gonn_hip_flash_attn_f64_bwd_ex(Q.data(), K.data(), V.data(), O.data(), L.data(),
                                         dO.data(), r.dQ.data(), r.dK.data(), r.dV.data(), B, H, S,
                                         d, scale, causal ? 1 : 0,
                                         kvLen.empty() ? nullptr : kvLen.data()),
          "FlashAttnF64BwdEx");
    return r;
}

KVCache::KVCache(int B, int H, int Lmax, int D) : B_(B), H_(H), Lmax_(Lmax), D_(D) {
    gonn_kvcache* c = nullptr;
    check(gonn_hip_kvcache_create(&c, B, H, Lmax, D), "KVCache");
    h_ = c;
}

KVCache::~KVCache() {
    if (h_) (void)gonn_hip_kvcache_free((gonn_kvcache*)h_);
}

KVCache::KVCache(KVCache&& o) noexcept
    : h_(o.h_), B_(o.B_), H_(o.H_), Lmax_(o.Lmax_), D_(o.D_) {
    o.h_ = nullptr;
}

KVCache& KVCache::operator=(KVCache&& o) noexcept {
    if (this != &o) {
        if (h_) (void)gonn_hip_kvcache_free((gonn_kvcache*)h_);
        h_ = o.h_;
        B_ = o.B_;
        H_ = o.H_;
        Lmax_ = o.Lmax_;
        D_ = o.D_;
        o.h_ = nullptr;
    }
    return *this;
}

void KVCache::Append(const std::vector<double>& k, const std::vector<double>& v, int T,
                     const std::vector<int>& counts) {
    if (!h_) throw std::invalid_argument("hip: KVCache: moved-from cache");
    if (T <= 0) throw std::invalid_argument("hip: KVCache.Append: T must be >= 1");
    const size_t n = (size_t)B_ * H_ * T * D_;
    need(k, n, "KVCache.Append k");
    need(v, n, "KVCache.Append v");
    if (!counts.empty() && (int)counts.size() != B_)
        throw std::invalid_argument("hip: KVCache.Append: counts needs B entries");
    check(gonn_hip_kvcache_append_f64((gonn_kvcache*)h_, k.data(), v.data(), T,
                                      counts.empty() ? nullptr : counts.data()),
          "KVCache.Append");
}

std::vector<double> KVCache::Attend(const std::vector<double>& q, double scale) const {
    if (!h_) throw std::invalid_argument("hip: KVCache: moved-from cache");
    const size_t n = (size_t)B_ * H_ * D_;
    need(q, n, "KVCache.Attend q");
    std::vector<double> o(n, 0.0);
    check(gonn_hip_kvcache_attend_f64((gonn_kvcache*)h_, q.data(), o.data(), scale),
          "KVCache.Attend");
    return o;
}

std::vector<int> KVCache::Lengths() const {
    std::vector<int> len(B_, 0);
    if (h_) check(gonn_hip_kvcache_lengths((const gonn_kvcache*)h_, len.data()), "KVCache.Lengths");
    return len;
}

void KVCache::Reset() {
    if (!h_) throw std::invalid_argument("hip: KVCache: moved-from cache");
    check(gonn_hip_kvcache_reset((gonn_kvcache*)h_), "KVCache.Reset");
}

DeviceMHA::DeviceMHA(int E, int H, int kdim, int vdim, const std::vector<double>& Wq,
                     const std::vector<double>& bq, const std::vector<double>& Wk,
                     const std::vector<double>& bk, const std::vector<double>& Wv,
                     const std::vector<double>& bv, const std::vector<double>& Wo,
                     const std::vector<double>& bo)
    : E_(E), H_(H), kdim_(kdim), vdim_(vdim) {
    if (E <= 0 || H <= 0 || kdim <= 0 || vdim <= 0)
        throw std::invalid_argument("hip: DeviceMHA: dimensions must be >= 1");
    need(Wq, (size_t)E * E, "DeviceMHA Wq");
    need(Wk, (size_t)E * kdim, "DeviceMHA Wk");
    need(Wv, (size_t)E * vdim, "DeviceMHA Wv");
    need(Wo, (size_t)E * E, "DeviceMHA Wo");
    const std::vector<double>* bs[4] = {&bq, &bk, &bv, &bo};
    for (const auto* b : bs)
        if (!b->empty()) need(*b, (size_t)E, "DeviceMHA bias");
    auto bp = [](const std::vector<double>& b) { return b.empty() ? nullptr : b.data(); };
    gonn_mha* m = nullptr;
    check(gonn_hip_mha_create(&m, E, H, kdim, vdim, Wq.data(), bp(bq), Wk.data(), bp(bk),
                              Wv.data(), bp(bv), Wo.data(), bp(bo)),
          "DeviceMHA");
    h_ = m;
}

DeviceMHA::~DeviceMHA() {
    if (h_) (void)gonn_hip_mha_free((gonn_mha*)h_);
}

DeviceMHA::DeviceMHA(DeviceMHA&& o) noexcept
    : h_(o.h_), E_(o.E_), H_(o.H_), kdim_(o.kdim_), vdim_(o.vdim_) {
    o.h_ = nullptr;
}

DeviceMHA& DeviceMHA::operator=(DeviceMHA&& o) noexcept {
    if (this != &o) {
        if (h_) (void)gonn_hip_mha_free((gonn_mha*)h_);
        h_ = o.h_;
        E_ = o.E_;
        H_ = o.H_;
        kdim_ = o.kdim_;
        vdim_ = o.vdim_;
        o.h_ = nullptr;
    }
    return *this;
}

std::vector<double> DeviceMHA::Forward(const std::vector<double>& q, const std::vector<double>& k,
                                       const std::vector<double>& v, int B, int Tq, int Tk,
                                       bool causal, const std::vector<int>& kvLen) const {
    if (!h_) throw std::invalid_argument("hip: DeviceMHA: moved-from handle");
    if (B <= 0 || Tq <= 0 || Tk <= 0)
        throw std::invalid_argument("hip: DeviceMHA.Forward: B, Tq, Tk must be >= 1");
    need(q, (size_t)B * Tq * E_, "DeviceMHA.Forward q");
    need(k, (size_t)B * Tk * kdim_, "DeviceMHA.Forward k");
    need(v, (size_t)B * Tk * vdim_, "DeviceMHA.Forward v");
    if (!kvLen.empty() && (int)kvLen.size() != B)
        throw std::invalid_argument("hip: DeviceMHA.Forward: kvLen needs B entries");
    std::vector<double> out((size_t)B * Tq * E_);
    // Pass the same pointer for k (v) when it is the same vector as q (k), so
    // the library uploads it once.
    const double* kp = &k == &q ? q.data() : k.data();
    const double* vp = &v == &k ? kp : v.data();
    check(gonn_hip_mha_forward_f64((gonn_mha*)h_, q.data(), kp, vp, out.data(), B, Tq, Tk,
                                   causal ? 1 : 0, kvLen.empty() ? nullptr : kvLen.data()),
          "DeviceMHA.Forward");
    return out;
}

std::vector<double> DeviceMHA::ForwardIncremental(const std::vector<double>& x, int B, int T,
                                                  KVCache& cache) const {
    if (!h_) throw std::invalid_argument("hip: DeviceMHA: moved-from handle");
    if (!cache.Handle()) throw std::invalid_argument("hip: KVCache: moved-from cache");
    if (B != cache.B() || T <= 0)
        throw std::invalid_argument("hip: DeviceMHA.ForwardIncremental: B must match the cache, T >= 1");
    const size_t n = (size_t)B * T * E_;
    need(x, n, "DeviceMHA.ForwardIncremental x");
    const size_t wsb = gonn_hip_mha_incremental_workspace_bytes(
        (const gonn_mha*)h_, (const gonn_kvcache*)cache.Handle(), T);
    if (wsb == 0)
        throw std::invalid_argument("hip: DeviceMHA.ForwardIncremental: the cache does not fit "
                                    "the layer (B, H, *, 64|128) of a self-attention");
    // Device buffers for x, out and the workspace, freed on every path.
    struct Bufs {
        gonn_buf x{}, out{}, ws{};
        ~Bufs() {
            (void)gonn_hip_free(&x);
            (void)gonn_hip_free(&out);
            (void)gonn_hip_free(&ws);
        }
    } b;
    check(gonn_hip_alloc(&b.x, n, GONN_F64), "DeviceMHA.ForwardIncremental alloc");
    check(gonn_hip_alloc(&b.out, n, GONN_F64), "DeviceMHA.ForwardIncremental alloc");
    check(gonn_hip_alloc(&b.ws, (wsb + 3) / 4, GONN_I32), "DeviceMHA.ForwardIncremental alloc");
    check(gonn_hip_memcpy_h2d(b.x.ptr, x.data(), n * sizeof(double), nullptr),
          "DeviceMHA.ForwardIncremental upload");
    check(gonn_hip_mha_forward_incremental_dev((gonn_mha*)h_, (gonn_kvcache*)cache.Handle(),
                                               &b.x, &b.out, T, b.ws.ptr, b.ws.bytes, nullptr),
          "DeviceMHA.ForwardIncremental");
    std::vector<double> out(n);
    check(gonn_hip_memcpy_d2h(out.data(), b.out.ptr, n * sizeof(double), nullptr),
          "DeviceMHA.ForwardIncremental download");
    check(gonn_hip_stream_sync(nullptr), "DeviceMHA.ForwardIncremental");
    return out;
}

}  // namespace hip
}  // namespace gonn
