// api.hip -- the C ABI declared in include/gonn_hip.h.
//
// Argument checks run on the host before anything is queued, so every
// GONN_E_* path is testable without a GPU. Device work goes to the caller's
// stream; the f64 compatibility shims are synchronous like the reference's
// (backend/cuda/gonn_cuda.cu:466-560) but check every runtime call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/gonn_hip.h"
#include "common.h"
#include "kernels.h"
#include "kvcache_internal.h"

#define GONN_HIP_VERSION "gonn-hip 0.1.0 (gfx950)"

namespace {

std::atomic<int> g_mode{-1};

// ---- per-kernel event profiler (diagnostics) -----------------------------
// When enabled, every kernel stage launched through this ABI is bracketed by
// two HIP events recorded on the stream it runs on.
struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};
std::mutex g_prof_mu;
std::atomic<bool> g_prof_on{false};
std::vector<ProfRec> g_prof;

struct ProfScope {
    hipEvent_t a = nullptr, b = nullptr;
    const char* name;
    hipStream_t s;
    ProfScope(const char* n, hipStream_t st) : name(n), s(st) {
        if (!n || !g_prof_on.load()) return;
        if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
            a = b = nullptr;
            return;
        }
        (void)hipEventRecord(a, s);
    }
    ~ProfScope() {
        if (!a) return;
        (void)hipEventRecord(b, s);
        std::lock_guard<std::mutex> lock(g_prof_mu);
        g_prof.push_back({name, a, b});
    }
};

int env_mode() {
    const char* e = std::getenv("GONN_HIP_ATTN_MODE");
    if (e && (std::strcmp(e, "bf16") == 0 || std::strcmp(e, "1") == 0)) return GONN_ATTN_BF16_MFMA;
    if (e && (std::strcmp(e, "f64") == 0 || std::strcmp(e, "2") == 0)) return GONN_ATTN_FP64;
    return GONN_ATTN_FP32_MFMA;
}

int current_mode() {
    int m = g_mode.load();
    if (m < 0) {
        int expected = -1;
        g_mode.compare_exchange_strong(expected, env_mode());
        m = g_mode.load();
    }
    return m;
}

bool fail_alloc_injected() {
    const char* e = std::getenv("GONN_HIP_FAIL_ALLOC");
    return e && e[0] == '1';
}

size_t dtype_size(int dt) {
    switch (dt) {
        case GONN_F32: return 4;
        case GONN_BF16: return 2;
        case GONN_F64: return 8;
        case GONN_I32: return 4;
        default: return 0;
    }
}

bool buf_ok(const gonn_buf& b, size_t elems, int dt0, int dt1 = -1) {
    if (!b.ptr) return false;
    if (b.dtype != dt0 && b.dtype != dt1) return false;
    return b.bytes >= elems * dtype_size(b.dtype);
}

int herr(hipError_t e) { return e == hipSuccess ? GONN_OK : (int)e; }

bool head_dim_ok(int D) { return D == 64 || D == 128; }

size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// An additive mask buffer covers every element slices read: the last
// sequence and head at their strides plus Sq x Sk rows.
bool mask_ok(const gonn_buf& m, int64_t sb, int64_t sh, int B, int H, int Sq, int Sk) {
    if (!m.ptr) return true;
    if (sb < 0 || sh < 0) return false;
    const double need = (double)(B - 1) * sb + (double)(H - 1) * sh + (double)Sq * Sk;
    if (need >= 9.0e15) return false;
    return buf_ok(m, (size_t)need, GONN_F32);
}

// The kernels a call runs: every call runs in the requested mode (the bf16
// kernels have masked and cross-attention variants).
int fwd_mode(const gonn_attn_fwd_args* a) { return a->mode; }
int bwd_keys_of(const gonn_attn_bwd_args* a) { return a->Sk > 0 ? a->Sk : a->S; }
int bwd_mode(const gonn_attn_bwd_args* a) { return a->mode; }

// The bf16-MFMA kernels take Q as bf16(q * (sign(scale) * c2)) with
// c2 = |scale| log2(e) (log2(e) and sign 0 for a zero scale), so Q K^T is
// the exp2 argument of the softmax. The forward (which packs Q itself) and the
// backward's pack round the same fp32 products, so the backward recomputes
// exactly the scores whose row sums the forward's LSE normalises.
struct QFold {
    float sign, sabs, c2;
};
QFold q_fold(double scale) {
    QFold f;
    f.sign = scale > 0 ? 1.f : (scale < 0 ? -1.f : 0.f);
    f.sabs = scale == 0.0 ? 1.f : (float)std::fabs(scale);
    f.c2 = f.sabs * gonn::kLog2e;
    return f;
}

// ---- forward -----------------------------------------------------------

int check_fwd(const gonn_attn_fwd_args* a) {
    if (!a) return GONN_E_INVALID;
    if (a->B <= 0 || a->H <= 0 || a->Sq <= 0 || a->Sk <= 0 || a->D <= 0) return GONN_E_INVALID;
    if (a->mode != GONN_ATTN_FP32_MFMA && a->mode != GONN_ATTN_BF16_MFMA) return GONN_E_INVALID;
    if (!std::isfinite(a->scale)) return GONN_E_INVALID;
    if (!head_dim_ok(a->D)) return GONN_E_UNSUPPORTED;
    const size_t BH = (size_t)a->B * a->H;
    if ((double)BH * a->Sq * a->D >= 2147483647.0 * 8 || (double)BH * a->Sk * a->D >= 2147483647.0 * 8)
        return GONN_E_UNSUPPORTED;
    const size_t nq = BH * a->Sq * a->D, nk = BH * a->Sk * a->D;
    if (!mask_ok(a->attn_mask, a->mask_stride_b, a->mask_stride_h, a->B, a->H, a->Sq, a->Sk))
        return GONN_E_INVALID;
    // The bf16 kernels address one slice's mask rows with 32-bit byte offsets.
    if (a->attn_mask.ptr && fwd_mode(a) == GONN_ATTN_BF16_MFMA &&
        (double)a->Sq * a->Sk * 4 >= 4294967295.0)
        return GONN_E_UNSUPPORTED;
    if (fwd_mode(a) == GONN_ATTN_FP32_MFMA) {
        if (!buf_ok(a->q, nq, GONN_F32) || !buf_ok(a->k, nk, GONN_F32) || !buf_ok(a->v, nk, GONN_F32))
            return GONN_E_INVALID;
    } else {
        if (!buf_ok(a->q, nq, GONN_F32, GONN_BF16) || !buf_ok(a->k, nk, GONN_F32, GONN_BF16) ||
            !buf_ok(a->v, nk, GONN_F32, GONN_BF16) || a->k.dtype != a->v.dtype)
            return GONN_E_INVALID;
    }
    if (!buf_ok(a->o, nq, GONN_F32)) return GONN_E_INVALID;
    if (a->lse.ptr && !buf_ok(a->lse, BH * a->Sq, GONN_F32)) return GONN_E_INVALID;
    if (a->kv_len.ptr && !buf_ok(a->kv_len, (size_t)a->B, GONN_I32)) return GONN_E_INVALID;
    return GONN_OK;
}

size_t fwd_ws(const gonn_attn_fwd_args* a) {
    if (fwd_mode(a) != GONN_ATTN_BF16_MFMA) return 0;
    const size_t BH = (size_t)a->B * a->H;
    const size_t Skp = round_up((size_t)a->Sk, 64);
    return 2 * BH * Skp * a->D * sizeof(uint16_t) + 256;
}

// ---- decode ------------------------------------------------------------

// Keys per split workgroup: 2048 (fewer partials, longer streams: 6.8 TB/s
// on C4 against 6.6 at 512) unless that leaves fewer than 2048 workgroups
// for a full cache, then halved down to 64.
int decode_split(const gonn_attn_decode_args* a) {
    if (a->split_keys > 0) return a->split_keys;
    const long long BH = (long long)a->B * a->H;
    int sk = 2048;
    while (sk > 64 && BH * ((a->Lmax + sk - 1) / sk) < 2048) sk /= 2;
    return sk;
}

int check_decode(const gonn_attn_decode_args* a) {
    if (!a) return GONN_E_INVALID;
    if (a->B <= 0 || a->H <= 0 || a->Lmax <= 0 || a->D <= 0) return GONN_E_INVALID;
    if (!std::isfinite(a->scale)) return GONN_E_INVALID;
    if (a->split_keys < 0 || (a->split_keys % 64) != 0) return GONN_E_INVALID;
    if (!head_dim_ok(a->D)) return GONN_E_UNSUPPORTED;
    const size_t BH = (size_t)a->B * a->H;
    if (!buf_ok(a->q, BH * a->D, GONN_F32, GONN_BF16)) return GONN_E_INVALID;
    const size_t nc = BH * (size_t)a->Lmax * a->D;
    if (!buf_ok(a->kcache, nc, GONN_BF16) || !buf_ok(a->vcache, nc, GONN_BF16)) return GONN_E_INVALID;
    if (!buf_ok(a->kv_len, (size_t)a->B, GONN_I32)) return GONN_E_INVALID;
    if (!buf_ok(a->o, BH * a->D, GONN_F32)) return GONN_E_INVALID;
    return GONN_OK;
}

size_t decode_ws(const gonn_attn_decode_args* a) {
    const size_t BH = (size_t)a->B * a->H;
    const int sk = decode_split(a);
    const size_t ns = ((size_t)a->Lmax + sk - 1) / sk;
    return BH * ns * ((size_t)a->D + 2) * sizeof(float) + 1024;
}

// ---- backward ----------------------------------------------------------

int check_bwd(const gonn_attn_bwd_args* a) {
    if (!a) return GONN_E_INVALID;
    if (a->B <= 0 || a->H <= 0 || a->S <= 0 || a->D <= 0 || a->Sk < 0) return GONN_E_INVALID;
    if (a->mode != GONN_ATTN_FP32_MFMA && a->mode != GONN_ATTN_BF16_MFMA) return GONN_E_INVALID;
    if (!std::isfinite(a->scale)) return GONN_E_INVALID;
    if (!head_dim_ok(a->D)) return GONN_E_UNSUPPORTED;
    const int Sk = bwd_keys_of(a);
    const size_t BH = (size_t)a->B * a->H, n = BH * a->S * a->D, nk = BH * Sk * a->D;
    if ((double)n >= 2147483647.0 * 8 || (double)nk >= 2147483647.0 * 8) return GONN_E_UNSUPPORTED;
    const gonn_buf* qs[] = {&a->q, &a->o, &a->dO, &a->dq};
    for (const gonn_buf* b : qs)
        if (!buf_ok(*b, n, GONN_F32)) return GONN_E_INVALID;
    const gonn_buf* ks[] = {&a->k, &a->v, &a->dk, &a->dv};
    for (const gonn_buf* b : ks)
        if (!buf_ok(*b, nk, GONN_F32)) return GONN_E_INVALID;
    if (!buf_ok(a->lse, BH * a->S, GONN_F32)) return GONN_E_INVALID;
    if (a->kv_len.ptr && !buf_ok(a->kv_len, (size_t)a->B, GONN_I32)) return GONN_E_INVALID;
    if (!mask_ok(a->attn_mask, a->mask_stride_b, a->mask_stride_h, a->B, a->H, a->S, Sk))
        return GONN_E_INVALID;
    // The bf16 kernels address one slice's mask rows with 32-bit byte offsets.
    if (a->attn_mask.ptr && bwd_mode(a) == GONN_ATTN_BF16_MFMA &&
        (double)a->S * Sk * 4 >= 4294967295.0)
        return GONN_E_UNSUPPORTED;
    return GONN_OK;
}

// Backward workspace: lse2 and delta (BH,Sp) f32, then in bf16 mode the
// packed operands Qb, dOb (BH,Sp,D), Kb, Vb (BH,Skp,D) and Kt (BH,D,Skp)
// bf16, and the stored dS when the dS path is taken, each region 256-byte
// aligned (Sp, Skp: the query and key counts rounded up to kBwdPad).
struct BwdLayout {
    size_t lse2, delta, packed[5], ds, total;
};

// The bf16 backward stores dS (bf16 blocks of 128 keys x 64 queries; for a
// causal call only the blocks a key block reaches, ds_block_base) and
// computes dQ from it in one GEMM. The stored dS of a call is capped by a
// byte budget: a call whose whole dS exceeds it runs its key blocks in
// chunks of consecutive blocks whose dS fits, each chunk's dK/dV storing its
// dS and the dQ kernel adding that chunk's keys to dQ (BwdParams::kb0, nkb,
// dq_mode), so the workspace stays within the budget. Each further chunk
// costs a dQ round trip and a shorter dK/dV grid (one workgroup per CU, so
// its tail idles CUs): measured at B=1 H=16 S=32768 causal, two chunks ran
// 13.2 ms, five 15.0 ms, and forming S and dP again in the dQ kernel 15.1
// ms; at B=2 H=16 S=8192, three chunks 2.23 ms, the recompute path 2.21 ms.
// Past two chunks the dS path is no faster than the recompute path, which
// needs no dS memory, so by default (budget kDsMaxBytes) a call takes at
// most kMaxAutoChunks chunks and otherwise the recompute path. A budget
// given in GONN_HIP_BWD_DS_MB (MB) always takes the chunks: the caller
// asked for that bound. GONN_HIP_BWD_DQ=recompute takes the recompute path,
// as does the rare shape where one key block of one slice exceeds the
// kernels' 32-bit buffer offsets. A call reads the variables once and sizes,
// checks and lays out its workspace for that one plan, so a workspace sized
// by gonn_hip_attn_workspace_bytes under the same settings fits, and one
// sized under others is either big enough or refused with GONN_E_WORKSPACE
// before any work is queued.
constexpr double kDsMaxBytes = 16.0 * 1024 * 1024 * 1024;
constexpr int kMaxAutoChunks = 2;
struct DqPlan {
    bool use_ds;
    double budget;  // bytes of stored dS per call
};
// The key-block chunks of a dS-path call: consecutive 128-key blocks, as
// many per chunk as keep BH x the chunk's blocks within the budget and one
// slice's part within 32-bit offsets, at least one. f(kb0, nkb, first,
// last) for each chunk in order; returns the most blocks one slice's part
// of a chunk holds.
template <typename F>
long long ds_chunks(size_t BH, int S, int Sk, int causal, double budget, F f) {
    const int nkb = (int)(round_up((size_t)Sk, gonn::kBwdPad) / 128);
    const int nqt = (int)(round_up((size_t)S, gonn::kBwdPad) / 64);
    const double per = (double)gonn::kDsTileElems * 2;  // bytes per block
    auto fits = [&](int kb0, int n) {
        const double b = (double)gonn::ds_chunk_blocks(kb0, n, nqt, causal) * per;
        return b * (double)BH <= budget && b < 2147483648.0;
    };
    long long most = 0;
    for (int kb0 = 0; kb0 < nkb;) {
        int n = 1;
        while (kb0 + n < nkb && fits(kb0, n + 1)) n++;
        most = std::max(most, gonn::ds_chunk_blocks(kb0, n, nqt, causal));
        f(kb0, n, kb0 == 0, kb0 + n == nkb);
        kb0 += n;
    }
    return most;
}
DqPlan bwd_dq_plan(int mode, size_t BH, int S, int Sk, int causal) {
    DqPlan q{false, kDsMaxBytes};
    if (mode != GONN_ATTN_BF16_MFMA) return q;
    const char* e = std::getenv("GONN_HIP_BWD_DQ");
    if (e && std::strcmp(e, "recompute") == 0) return q;
    const char* m = std::getenv("GONN_HIP_BWD_DS_MB");
    const bool given = m && std::atof(m) > 0;
    if (given) q.budget = std::atof(m) * 1024.0 * 1024.0;
    // one key block of one slice: every query tile's block
    const int nqt = (int)(round_up((size_t)S, gonn::kBwdPad) / 64);
    if ((double)nqt * gonn::kDsTileElems * 2 >= 2147483648.0) return q;
    int chunks = 0;
    ds_chunks(BH, S, Sk, causal, q.budget, [&](int, int, bool, bool) { chunks++; });
    q.use_ds = given || chunks <= kMaxAutoChunks;
    return q;
}

BwdLayout bwd_layout(int mode, size_t BH, int S, int Sk, int D, int causal, const DqPlan& plan) {
    BwdLayout L{};
    const size_t Sp = round_up((size_t)S, gonn::kBwdPad), Skp = round_up((size_t)Sk, gonn::kBwdPad);
    size_t off = 0;
    L.lse2 = off;
    off = round_up(off + BH * Sp * 4, 256);
    L.delta = off;
    off = round_up(off + BH * Sp * 4, 256);
    if (mode == GONN_ATTN_BF16_MFMA) {
        // Qb, dOb, Kb, Vb, Kt
        const bool keyside[5] = {false, false, true, true, true};
        for (int i = 0; i < 5; i++) {
            L.packed[i] = off;
            off = round_up(off + BH * (keyside[i] ? Skp : Sp) * D * 2, 256);
        }
        if (plan.use_ds) {
            const long long most =
                ds_chunks(BH, S, Sk, causal, plan.budget, [](int, int, bool, bool) {});
            L.ds = off;
            off = round_up(off + BH * (size_t)most * gonn::kDsTileElems * 2, 256);
        }
    }
    L.total = off;
    return L;
}

size_t bwd_ws(const gonn_attn_bwd_args* a, const DqPlan& plan) {
    return bwd_layout(bwd_mode(a), (size_t)a->B * a->H, a->S, bwd_keys_of(a), a->D, a->causal,
                      plan)
               .total +
           256;
}
DqPlan bwd_dq_plan(const gonn_attn_bwd_args* a) {
    return bwd_dq_plan(bwd_mode(a), (size_t)a->B * a->H, a->S, bwd_keys_of(a), a->causal);
}

// ---- helpers for the host shims ----------------------------------------

#define TRYH_EARLY(x)                                        \
    do {                                                     \
        const hipError_t _e = (x);                           \
        if (_e != hipSuccess) return (int)_e;                \
    } while (0)

// The host (fp64) entry points run on a stream of the calling thread, not on
// the legacy null stream, and wait for that stream only: GoNN runs Backward
// calls concurrently (tensor/autograd.go:10-32), and such callers must not
// serialise on each other's device work. Each device has a fixed pool of
// kHostStreams non-blocking streams (default priority), created on first use
// and kept for the process; a thread draws one slot of the pool the first
// time it calls in and keeps it. cgo spreads calls over many OS threads, so
// the pool bounds the streams: threads beyond kHostStreams share slots,
// which only orders their device work (each call still waits for its own
// stream before returning).
constexpr int kMaxDevices = 64;
constexpr int kHostStreams = 16;
int host_stream(hipStream_t* out) {
    static std::mutex mu;
    static hipStream_t pool[kMaxDevices][kHostStreams] = {};
    static std::atomic<unsigned> next_slot{0};
    thread_local int slot = -1;
    if (slot < 0) slot = (int)(next_slot.fetch_add(1, std::memory_order_relaxed) % kHostStreams);
    int dev = 0;
    TRYH_EARLY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return GONN_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(mu);
    hipStream_t& st = pool[dev][slot];
    if (!st) TRYH_EARLY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *out = st;
    return GONN_OK;
}

// Waits for a host call's stream on every exit path, so no copy from or to
// the caller's host arrays is still queued when the call returns.
struct StreamSync {
    hipStream_t s;
    ~StreamSync() { (void)hipStreamSynchronize(s); }
};

// Scratch device memory of one host call, stream-ordered on that call's
// stream (hipMallocAsync / hipFreeAsync): no device-wide synchronisation.
struct DevMem {
    hipStream_t s;
    std::vector<void*> ptrs;
    explicit DevMem(hipStream_t st) : s(st) {}
    ~DevMem() {
        for (void* p : ptrs) (void)hipFreeAsync(p, s);
    }
    int alloc(void** p, size_t bytes) {
        if (fail_alloc_injected()) return GONN_E_INJECTED;
        if (bytes == 0) bytes = 16;
        if (hipMallocAsync(p, bytes, s) != hipSuccess) {
            (void)hipGetLastError();
            *p = nullptr;
            return GONN_E_NOMEM;
        }
        ptrs.push_back(*p);
        return GONN_OK;
    }
};

int pad_dim(int d) { return d <= 64 ? 64 : 128; }

#define TRY(x)                      \
    do {                            \
        const int _rc = (x);        \
        if (_rc != GONN_OK) return _rc; \
    } while (0)
#define TRYH(x) TRY(herr(x))

// Upload n rows of d doubles and convert to f32 rows of dp (zero-padded).
int upload_padded(DevMem& mem, const double* host, size_t rows, int d, int dp, float** out) {
    void* stage = nullptr;
    void* dst = nullptr;
    TRY(mem.alloc(&stage, rows * d * sizeof(double)));
    TRY(mem.alloc(&dst, rows * dp * sizeof(float)));
    TRYH(hipMemcpyAsync(stage, host, rows * d * sizeof(double), hipMemcpyHostToDevice, mem.s));
    TRYH(gonn::launch_convert_from_f64((const double*)stage, dst, 0, rows, d, dp, mem.s));
    *out = (float*)dst;
    return GONN_OK;
}

int download_padded(DevMem& mem, const float* dev, size_t rows, int d, int dp, double* host) {
    void* stage = nullptr;
    TRY(mem.alloc(&stage, rows * d * sizeof(double)));
    TRYH(gonn::launch_convert_to_f64(dev, 0, (double*)stage, rows, d, dp, mem.s));
    TRYH(hipMemcpyAsync(host, stage, rows * d * sizeof(double), hipMemcpyDeviceToHost, mem.s));
    return GONN_OK;
}

int run_fwd_f32(DevMem& mem, const float* q, const float* k, const float* v, float* o, float* lse,
                int BH, int S, int dp, double scale, int causal) {
    gonn_attn_fwd_args a{};
    const size_t n = (size_t)BH * S * dp;
    a.q = {(void*)q, n * 4, GONN_F32};
    a.k = {(void*)k, n * 4, GONN_F32};
    a.v = {(void*)v, n * 4, GONN_F32};
    a.o = {(void*)o, n * 4, GONN_F32};
    a.lse = {(void*)lse, lse ? (size_t)BH * S * 4 : 0, GONN_F32};
    a.B = BH;
    a.H = 1;
    a.Sq = a.Sk = S;
    a.D = dp;
    a.scale = scale;
    a.causal = causal;
    a.mode = current_mode();
    const size_t wsb = gonn_hip_attn_workspace_bytes(GONN_OP_FWD, &a);
    void* ws = nullptr;
    if (wsb) TRY(mem.alloc(&ws, wsb));
    return gonn_hip_attn_fwd(&a, ws, wsb, mem.s);
}

bool shim_args_ok(int BH, int S, int d) { return BH > 0 && S > 0 && d > 0 && d <= 128; }

// General forward on device f32 buffers: B sequences x H heads, Sq x Sk,
// optional device kv_len[B].
int run_fwd_f32_ex(DevMem& mem, const float* q, const float* k, const float* v, float* o,
                   float* lse, int B, int H, int Sq, int Sk, int dp, double scale, int causal,
                   const int* kv_len, const float* mask = nullptr, size_t mask_n = 0,
                   int64_t mask_sb = 0, int64_t mask_sh = 0) {
    gonn_attn_fwd_args a{};
    a.attn_mask = {(void*)mask, mask ? mask_n * 4 : 0, GONN_F32};
    a.mask_stride_b = mask_sb;
    a.mask_stride_h = mask_sh;
    const size_t BH = (size_t)B * H, nq = BH * Sq * dp, nk = BH * Sk * dp;
    a.q = {(void*)q, nq * 4, GONN_F32};
    a.k = {(void*)k, nk * 4, GONN_F32};
    a.v = {(void*)v, nk * 4, GONN_F32};
    a.o = {(void*)o, nq * 4, GONN_F32};
    a.lse = {(void*)lse, lse ? BH * Sq * 4 : 0, GONN_F32};
    a.kv_len = {(void*)kv_len, kv_len ? (size_t)B * 4 : 0, GONN_I32};
    a.B = B;
    a.H = H;
    a.Sq = Sq;
    a.Sk = Sk;
    a.D = dp;
    a.scale = scale;
    a.causal = causal;
    a.mode = current_mode();
    const size_t wsb = gonn_hip_attn_workspace_bytes(GONN_OP_FWD, &a);
    void* ws = nullptr;
    if (wsb) TRY(mem.alloc(&ws, wsb));
    return gonn_hip_attn_fwd(&a, ws, wsb, mem.s);
}

// Split-KV decode on a checked call with a workspace of at least
// decode_ws(a) bytes. `profile`: bracket the stages with profiler events
// (event creation allocates, so the no-allocation entry passes false).
int run_decode(const gonn_attn_decode_args* a, void* ws, hipStream_t s, bool profile) {
    gonn::DecodeParams p{};
    const int sk = decode_split(a);
    p.q = a->q.ptr;
    p.kc = a->kcache.ptr;
    p.vc = a->vcache.ptr;
    p.kv_len = (const int*)a->kv_len.ptr;
    p.o = (float*)a->o.ptr;
    p.B = a->B;
    p.H = a->H;
    p.Lmax = a->Lmax;
    p.split_keys = sk;
    p.nsplit = (a->Lmax + sk - 1) / sk;
    float* w = (float*)round_up((size_t)ws, 256);
    p.part_ml = w;
    p.part_o = w + round_up((size_t)a->B * a->H * p.nsplit * 2, 64);
    p.scale_log2 = (float)a->scale * gonn::kLog2e;
    {
        ProfScope ps(profile ? "decode_split" : nullptr, s);
        TRYH(gonn::launch_decode_split(p, a->D, a->q.dtype == GONN_BF16, s));
    }
    ProfScope ps(profile ? "decode_combine" : nullptr, s);
    return herr(gonn::launch_decode_combine(p, a->D, s));
}

// ---- no-allocation scratch ----------------------------------------------
// One library-owned device array per GPU for callers that cannot allocate
// (gonn_hip_attn_decode_noalloc). In host code `scratch` names a host-side
// stand-in, not the device array: its device address is looked up once per
// device with hipGetSymbolAddress (on the first call on that device, with
// the device current) and only that address is ever handed to kernels. The
// array keeps the last call's contents; the decode kernels write every
// partial they later read, so nothing needs clearing between calls.
constexpr size_t kNoAllocScratchBytes = GONN_NOALLOC_SCRATCH_BYTES;  // 32 MiB per device
struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
    int rc = GONN_OK;
};
ScratchSlot g_scratch[kMaxDevices];

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

int noalloc_scratch(void** out) {
    int dev = 0;
    TRYH(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return GONN_E_UNSUPPORTED;
    ScratchSlot& slot = g_scratch[dev];
    std::call_once(slot.once, [&slot] {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        slot.rc = herr(e);
        slot.ptr = e == hipSuccess ? p : nullptr;
    });
    if (slot.rc != GONN_OK) return slot.rc;
    if (!slot.ptr) return GONN_E_NODEVICE;
    *out = slot.ptr;
    return GONN_OK;
}
}  // namespace

// The KV-cache handle of the C ABI (opaque to callers).
struct gonn_kvcache {
    int B = 0, H = 0, Lmax = 0, D = 0;
    void* k = nullptr;    // bf16 (B,H,Lmax,D)
    void* v = nullptr;
    int* d_len = nullptr;  // device int32[B]: cached positions per sequence
    int* d_pc = nullptr;   // device int32[2B]: positions and counts of an append
    void* ws = nullptr;    // decode workspace
    size_t ws_bytes = 0;
    std::vector<int> h_len;  // host copy of the lengths (authoritative)
    std::vector<int> h_pc;
    // Set when a failed call left the device lengths advanced past h_len and
    // putting them back failed too: every call that reads them then returns
    // GONN_E_INVALID until gonn_hip_kvcache_reset succeeds.
    bool stale = false;
};

namespace {

void kv_release(gonn_kvcache* c) {
    void* ptrs[] = {c->k, c->v, c->d_len, c->d_pc, c->ws};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    c->k = c->v = c->ws = nullptr;
    c->d_len = c->d_pc = nullptr;
}

gonn_attn_decode_args kv_decode_args(const gonn_kvcache* c) {
    gonn_attn_decode_args a{};
    const size_t n = (size_t)c->B * c->H * c->Lmax * c->D;
    a.kcache = {c->k, n * 2, GONN_BF16};
    a.vcache = {c->v, n * 2, GONN_BF16};
    a.kv_len = {c->d_len, (size_t)c->B * 4, GONN_I32};
    a.B = c->B;
    a.H = c->H;
    a.Lmax = c->Lmax;
    a.D = c->D;
    a.split_keys = 0;
    return a;
}

// Checks an append of T rows per sequence (counts: host int[B] or null = T);
// fills c->h_pc with (positions, counts).
int kv_check_append(gonn_kvcache* c, int T, const int* counts) {
    if (T <= 0 || c->stale) return GONN_E_INVALID;
    c->h_pc.assign(2 * (size_t)c->B, 0);
    for (int b = 0; b < c->B; b++) {
        const int n = counts ? counts[b] : T;
        if (n < 0 || n > T) return GONN_E_INVALID;
        if ((long long)c->h_len[b] + n > c->Lmax) return GONN_E_INVALID;
        c->h_pc[b] = c->h_len[b];
        c->h_pc[c->B + b] = n;
    }
    return GONN_OK;
}

// Launches the append (k, v device, f32 or bf16 (B,H,T,D)) and advances the
// lengths; synchronous.
int kv_append_dev(gonn_kvcache* c, const void* k, const void* v, int src_bf16, int T,
                  hipStream_t s) {
    TRYH(hipMemcpyAsync(c->d_pc, c->h_pc.data(), 2 * (size_t)c->B * sizeof(int),
                        hipMemcpyHostToDevice, s));
    TRYH(gonn::launch_kv_append(k, v, src_bf16, c->k, c->v, c->d_pc, c->d_pc + c->B, c->B, c->H,
                                T, c->Lmax, c->D, s));
    // The new lengths become the handle's only once the append and their
    // upload have completed, so a failed call leaves host and device
    // lengths as they were.
    std::vector<int> len(c->h_len);
    for (int b = 0; b < c->B; b++) len[b] += c->h_pc[c->B + b];
    TRYH(hipMemcpyAsync(c->d_len, len.data(), (size_t)c->B * sizeof(int), hipMemcpyHostToDevice,
                        s));
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        // The upload of the new lengths may have run: put the committed ones
        // back (a failure there marks the handle stale).
        (void)gonn::kvcache_restore(c);
        return herr(e);
    }
    c->h_len.swap(len);
    return GONN_OK;
}

// Split size of the causal multi-token attend: the decode rule of
// decode_split with one (b,h) counted once per query group.
int causal_split(const gonn_kvcache* c, int T) {
    const long long units = (long long)c->B * c->H * ((T + gonn::kDecodeGroup - 1) / gonn::kDecodeGroup);
    int sk = 2048;
    while (sk > 64 && units * ((c->Lmax + sk - 1) / sk) < 2048) sk /= 2;
    return sk;
}

}  // namespace

namespace gonn {

void kvcache_dims(const gonn_kvcache* c, int* B, int* H, int* Lmax, int* D) {
    *B = c->B;
    *H = c->H;
    *Lmax = c->Lmax;
    *D = c->D;
}

int kvcache_append_pending(gonn_kvcache* c, const float* k, const float* v, int T, hipStream_t s,
                           std::vector<int>* new_len) {
    TRY(kv_check_append(c, T, nullptr));
    TRYH(hipMemcpyAsync(c->d_pc, c->h_pc.data(), 2 * (size_t)c->B * sizeof(int),
                        hipMemcpyHostToDevice, s));
    TRYH(launch_kv_append(k, v, 0, c->k, c->v, c->d_pc, c->d_pc + c->B, c->B, c->H, T, c->Lmax,
                          c->D, s));
    *new_len = c->h_len;
    for (int b = 0; b < c->B; b++) (*new_len)[b] += T;
    return herr(hipMemcpyAsync(c->d_len, new_len->data(), (size_t)c->B * sizeof(int),
                               hipMemcpyHostToDevice, s));
}

void kvcache_commit(gonn_kvcache* c, std::vector<int>* new_len) { c->h_len.swap(*new_len); }

int kvcache_restore(gonn_kvcache* c) {
    const hipError_t e =
        hipMemcpy(c->d_len, c->h_len.data(), (size_t)c->B * sizeof(int), hipMemcpyHostToDevice);
    c->stale = e != hipSuccess;
    return herr(e);
}

bool kvcache_usable(const gonn_kvcache* c) { return c && !c->stale; }

size_t kvcache_attend_causal_ws(const gonn_kvcache* c, int T) {
    if (!c || T <= 0) return 0;
    const int sk = causal_split(c, T);
    const size_t ns = ((size_t)c->Lmax + sk - 1) / sk;
    const size_t parts = (size_t)c->B * c->H * T * ns;
    return round_up(parts * 2, 64) * sizeof(float) + parts * c->D * sizeof(float) + 1024;
}

int kvcache_attend_causal_run(gonn_kvcache* c, const float* q, float* o, int T, double scale,
                              void* ws, hipStream_t s, bool profile) {
    DecodeParams p{};
    const int sk = causal_split(c, T);
    p.q = q;
    p.kc = c->k;
    p.vc = c->v;
    p.kv_len = c->d_len;
    p.o = o;
    p.B = c->B;
    p.H = c->H;
    p.Lmax = c->Lmax;
    p.T = T;
    p.split_keys = sk;
    p.nsplit = (c->Lmax + sk - 1) / sk;
    float* w = (float*)round_up((size_t)ws, 256);
    p.part_ml = w;
    p.part_o = w + round_up((size_t)c->B * c->H * T * p.nsplit * 2, 64);
    p.scale_log2 = (float)scale * kLog2e;
    {
        ProfScope ps(profile ? "decode_causal_split" : nullptr, s);
        TRYH(launch_decode_causal_split(p, c->D, s));
    }
    ProfScope ps(profile ? "decode_causal_combine" : nullptr, s);
    return herr(launch_decode_causal_combine(p, c->D, s));
}

}  // namespace gonn

extern "C" {

const char* gonn_hip_version(void) { return GONN_HIP_VERSION; }

const char* gonn_hip_strerror(int code) {
    switch (code) {
        case GONN_OK: return "success";
        case GONN_E_INVALID: return "invalid argument (shape, null pointer, dtype or short buffer)";
        case GONN_E_UNSUPPORTED: return "unsupported configuration (head dim must be 64 or 128)";
        case GONN_E_WORKSPACE: return "workspace missing or too small";
        case GONN_E_NOMEM: return "device allocation failed";
        case GONN_E_NODEVICE: return "no usable gfx950 device";
        case GONN_E_INJECTED: return "failure injected by GONN_HIP_FAIL_ALLOC";
        case GONN_E_BLAS: return "rocBLAS call failed";
        default: break;
    }
    if (code > 0) return hipGetErrorString((hipError_t)code);
    return "unknown error";
}

int gonn_hip_available(void) {
    static int cached = -1;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (cached >= 0) return cached;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        cached = 0;
        return 0;
    }
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        cached = 0;
        return 0;
    }
    cached = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
    return cached;
}

int gonn_hip_attn_supports(int D, int Sq, int Sk) {
    return head_dim_ok(D) && Sq > 0 && Sk > 0 ? 1 : 0;
}

int gonn_hip_set_attn_mode(int mode) {
    if (mode != GONN_ATTN_FP32_MFMA && mode != GONN_ATTN_BF16_MFMA && mode != GONN_ATTN_FP64)
        return GONN_E_INVALID;
    g_mode.store(mode);
    return GONN_OK;
}

int gonn_hip_get_attn_mode(void) { return current_mode(); }

size_t gonn_hip_attn_workspace_bytes(int op, const void* args) {
    if (!args) return 0;
    switch (op) {
        case GONN_OP_FWD: {
            const auto* a = (const gonn_attn_fwd_args*)args;
            if (a->B <= 0 || a->H <= 0 || a->Sk <= 0 || a->D <= 0) return 0;
            return fwd_ws(a);
        }
        case GONN_OP_BWD: {
            const auto* a = (const gonn_attn_bwd_args*)args;
            if (a->B <= 0 || a->H <= 0 || a->S <= 0 || !head_dim_ok(a->D)) return 0;
            return bwd_ws(a, bwd_dq_plan(a));
        }
        case GONN_OP_DECODE: {
            const auto* a = (const gonn_attn_decode_args*)args;
            if (a->B <= 0 || a->H <= 0 || a->Lmax <= 0 || a->D <= 0) return 0;
            return decode_ws(a);
        }
        default: return 0;
    }
}

int gonn_hip_attn_fwd(const gonn_attn_fwd_args* a, void* ws, size_t ws_bytes, void* stream) {
    TRY(check_fwd(a));
    const size_t need = fwd_ws(a);
    if (need && (!ws || ws_bytes < need)) return GONN_E_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    const int BH = a->B * a->H;
    gonn::FwdParams p{};
    p.o = (float*)a->o.ptr;
    p.lse = a->lse.ptr ? (float*)a->lse.ptr : nullptr;
    p.BH = BH;
    p.Sq = a->Sq;
    p.Sk = a->Sk;
    p.H = a->H;
    p.kv_len = a->kv_len.ptr ? (const int*)a->kv_len.ptr : nullptr;
    const QFold qf = q_fold(a->scale);
    p.qsign = qf.sign;
    p.scale_abs = qf.sabs;
    p.scale_log2 = qf.c2;
    p.q = a->q.ptr;
    const int mode = fwd_mode(a);
    if (a->attn_mask.ptr) {
        p.mask = (const float*)a->attn_mask.ptr;
        p.mask_sb = a->mask_stride_b;
        p.mask_sh = a->mask_stride_h;
        p.mask_mul = 1.f / p.scale_abs;
    }
    if (mode == GONN_ATTN_BF16_MFMA) {
        const int Skp = (int)round_up((size_t)a->Sk, 64);
        uint8_t* w = (uint8_t*)round_up((size_t)ws, 256);
        const size_t half = (size_t)BH * Skp * a->D * sizeof(uint16_t);
        void* Kb = w;
        void* Vt = w + half;
        {
            ProfScope ps("pack_kv", s);
            gonn::PackParams pp{};
            pp.src[0] = a->k.ptr;
            pp.row[0] = Kb;
            pp.src[1] = a->v.ptr;
            pp.tr[1] = Vt;
            pp.mul[0] = pp.mul[1] = 1.f;
            pp.S = a->Sk;
            pp.Sp = Skp;
            TRYH(gonn::launch_pack(pp, 2, a->k.dtype == GONN_BF16, BH, a->D, s));
        }
        p.k = Kb;
        p.v = Vt;
        p.Skp = Skp;
    } else {
        p.k = a->k.ptr;
        p.v = a->v.ptr;
        p.Skp = a->Sk;
    }
    ProfScope ps(mode == GONN_ATTN_BF16_MFMA ? "fwd_bf16" : "fwd_f32", s);
    return herr(gonn::launch_fwd(p, mode, a->D, a->causal, a->q.dtype == GONN_BF16, s));
}

int gonn_hip_attn_bwd(const gonn_attn_bwd_args* a, void* ws, size_t ws_bytes, void* stream) {
    TRY(check_bwd(a));
    const DqPlan plan = bwd_dq_plan(a);  // the dQ path of this call, read once
    const bool use_ds = plan.use_ds;
    const size_t need = bwd_ws(a, plan);
    if (!ws || ws_bytes < need) return GONN_E_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    const int BH = a->B * a->H, S = a->S, D = a->D;
    const int Sp = (int)round_up((size_t)S, gonn::kBwdPad);
    const int mode = bwd_mode(a);
    const BwdLayout L = bwd_layout(mode, (size_t)BH, S, bwd_keys_of(a), D, a->causal, plan);
    uint8_t* w = (uint8_t*)round_up((size_t)ws, 256);
    gonn::BwdParams p{};
    if (a->attn_mask.ptr) {
        p.mask = (const float*)a->attn_mask.ptr;
        p.mask_sb = a->mask_stride_b;
        p.mask_sh = a->mask_stride_h;
    }
    p.lse2 = (const float*)(w + L.lse2);
    p.delta = (const float*)(w + L.delta);
    p.dq = (float*)a->dq.ptr;
    p.dk = (float*)a->dk.ptr;
    p.dv = (float*)a->dv.ptr;
    p.BH = BH;
    p.S = S;
    p.Sp = Sp;
    p.Sk = bwd_keys_of(a);
    p.Skp = (int)round_up((size_t)p.Sk, gonn::kBwdPad);
    p.scale = (float)a->scale;
    p.scale_log2 = (float)(a->scale * (double)gonn::kLog2e);
    // bf16 kernels: Q packed exactly as the bf16 forward packs it (see
    // q_fold), so S = Q K^T is already the exp2 argument's scale and
    // dK = |scale| / c2 * (dS^T Q).
    const QFold qf = q_fold(a->scale);
    p.c2b = 1.f;
    p.dqs = (float)a->scale;
    p.dks = (float)(std::fabs(a->scale) / (double)qf.c2);
    p.kv_len = a->kv_len.ptr ? (const int*)a->kv_len.ptr : nullptr;
    p.H = a->H;
    {
        ProfScope ps("bwd_prep", s);
        TRYH(gonn::launch_bwd_prep((const float*)a->o.ptr, (const float*)a->dO.ptr,
                                   (const float*)a->lse.ptr, (float*)(w + L.lse2),
                                   (float*)(w + L.delta), BH, S, Sp, D,
                                   mode == GONN_ATTN_BF16_MFMA, s));
    }
    if (mode == GONN_ATTN_BF16_MFMA) {
        void* Qb = w + L.packed[0];
        void* dOb = w + L.packed[1];
        void* Kb = w + L.packed[2];
        void* Vb = w + L.packed[3];
        void* Kt = w + L.packed[4];
        ProfScope ps("bwd_pack", s);
        gonn::PackParams p1{};
        p1.src[0] = a->q.ptr;
        p1.row[0] = Qb;
        p1.src[1] = a->dO.ptr;
        p1.row[1] = dOb;
        p1.mul[0] = qf.sign * qf.c2;
        p1.mul[1] = 1.f;
        p1.S = S;
        p1.Sp = Sp;
        TRYH(gonn::launch_pack(p1, 2, 0, BH, D, s));
        gonn::PackParams p2{};
        p2.src[0] = a->k.ptr;
        p2.row[0] = Kb;
        p2.tr[0] = Kt;
        p2.src[1] = a->v.ptr;
        p2.row[1] = Vb;
        p2.mul[0] = p2.mul[1] = 1.f;
        p2.S = p.Sk;
        p2.Sp = p.Skp;
        TRYH(gonn::launch_pack(p2, 2, 0, BH, D, s));
        p.q = Qb;
        p.dO = dOb;
        p.k = Kb;
        p.v = Vb;
        p.kt = Kt;
    } else {
        p.q = a->q.ptr;
        p.dO = a->dO.ptr;
        p.k = a->k.ptr;
        p.v = a->v.ptr;
    }
    p.ds = use_ds ? (bf16*)(w + L.ds) : nullptr;
    if (!use_ds) {
        {
            ProfScope ps("bwd_dkdv", s);
            TRYH(gonn::launch_bwd_dkdv(p, mode, D, a->causal, s));
        }
        ProfScope ps("bwd_dq", s);
        return herr(gonn::launch_bwd_dq(p, mode, D, a->causal, s));
    }
    // dS path: one chunk of every key block, or chunks within the budget.
    int nchunks = 0;
    ds_chunks((size_t)BH, S, p.Sk, a->causal, plan.budget,
              [&](int, int, bool, bool) { nchunks++; });
    hipError_t err = hipSuccess;
    ds_chunks((size_t)BH, S, p.Sk, a->causal, plan.budget,
              [&](int kb0, int nkb, bool first, bool last) {
                  if (err != hipSuccess) return;
                  if (nchunks > 1) {
                      p.kb0 = kb0;
                      p.nkb = nkb;
                      p.dq_mode = first ? 1 : (last ? 3 : 2);
                  }
                  {
                      ProfScope ps("bwd_dkdv", s);
                      err = gonn::launch_bwd_dkdv(p, mode, D, a->causal, s);
                  }
                  if (err != hipSuccess) return;
                  ProfScope ps("bwd_dq", s);
                  err = gonn::launch_bwd_dq_ds(p, D, a->causal, s);
              });
    return herr(err);
}

int gonn_hip_attn_decode(const gonn_attn_decode_args* a, void* ws, size_t ws_bytes, void* stream) {
    TRY(check_decode(a));
    const size_t need = decode_ws(a);
    if (!ws || ws_bytes < need) return GONN_E_WORKSPACE;
    return run_decode(a, ws, (hipStream_t)stream, true);
}

int gonn_hip_attn_decode_noalloc(const gonn_attn_decode_args* a, void* stream) {
    TRY(check_decode(a));
    if (decode_ws(a) > kNoAllocScratchBytes) return GONN_E_WORKSPACE;
    void* ws = nullptr;
    TRY(noalloc_scratch(&ws));
    return run_decode(a, ws, (hipStream_t)stream, false);
}


int gonn_hip_alloc(gonn_buf* b, size_t n_elems, int dtype) {
    if (!b || dtype_size(dtype) == 0) return GONN_E_INVALID;
    b->ptr = nullptr;
    b->bytes = 0;
    b->dtype = dtype;
    if (fail_alloc_injected()) return GONN_E_INJECTED;
    const size_t bytes = n_elems * dtype_size(dtype);
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) {
        (void)hipGetLastError();
        return GONN_E_NOMEM;
    }
    b->ptr = p;
    b->bytes = bytes;
    return GONN_OK;
}

int gonn_hip_free(gonn_buf* b) {
    if (!b) return GONN_E_INVALID;
    if (b->ptr) {
        const hipError_t e = hipFree(b->ptr);
        b->ptr = nullptr;
        b->bytes = 0;
        return herr(e);
    }
    return GONN_OK;
}

int gonn_hip_upload_from_f64(gonn_buf* dst, const double* src, size_t n, void* stream) {
    if (!dst || !dst->ptr || (!src && n)) return GONN_E_INVALID;
    if (dst->dtype != GONN_F32 && dst->dtype != GONN_BF16 && dst->dtype != GONN_F64)
        return GONN_E_INVALID;
    if (dst->bytes < n * dtype_size(dst->dtype)) return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    hipStream_t s = (hipStream_t)stream;
    if (dst->dtype == GONN_F64) {
        TRYH(hipMemcpyAsync(dst->ptr, src, n * 8, hipMemcpyHostToDevice, s));
        return herr(hipStreamSynchronize(s));
    }
    DevMem mem(s);
    void* stage = nullptr;
    TRY(mem.alloc(&stage, n * 8));
    TRYH(hipMemcpyAsync(stage, src, n * 8, hipMemcpyHostToDevice, s));
    TRYH(gonn::launch_convert_from_f64((const double*)stage, dst->ptr, dst->dtype == GONN_BF16, n,
                                       1, 1, s));
    return herr(hipStreamSynchronize(s));
}

int gonn_hip_download_to_f64(double* dst, const gonn_buf* src, size_t n, void* stream) {
    if (!src || !src->ptr || (!dst && n)) return GONN_E_INVALID;
    if (src->dtype != GONN_F32 && src->dtype != GONN_BF16 && src->dtype != GONN_F64)
        return GONN_E_INVALID;
    if (src->bytes < n * dtype_size(src->dtype)) return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    hipStream_t s = (hipStream_t)stream;
    if (src->dtype == GONN_F64) {
        TRYH(hipMemcpyAsync(dst, src->ptr, n * 8, hipMemcpyDeviceToHost, s));
        return herr(hipStreamSynchronize(s));
    }
    DevMem mem(s);
    void* stage = nullptr;
    TRY(mem.alloc(&stage, n * 8));
    TRYH(gonn::launch_convert_to_f64(src->ptr, src->dtype == GONN_BF16, (double*)stage, n, 1, 1, s));
    TRYH(hipMemcpyAsync(dst, stage, n * 8, hipMemcpyDeviceToHost, s));
    return herr(hipStreamSynchronize(s));
}

int gonn_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if ((!dst || !src) && bytes) return GONN_E_INVALID;
    hipStream_t s = (hipStream_t)stream;
    TRYH(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    return herr(hipStreamSynchronize(s));
}

int gonn_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if ((!dst || !src) && bytes) return GONN_E_INVALID;
    hipStream_t s = (hipStream_t)stream;
    TRYH(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    return herr(hipStreamSynchronize(s));
}

int gonn_hip_stream_sync(void* stream) { return herr(hipStreamSynchronize((hipStream_t)stream)); }

// ---- exact fp64 path of the f64 entry points (GONN_ATTN_FP64) ----
namespace {

int upload_f64(DevMem& mem, const double* host, size_t n, double** out) {
    void* dst = nullptr;
    TRY(mem.alloc(&dst, n * sizeof(double)));
    TRYH(hipMemcpyAsync(dst, host, n * sizeof(double), hipMemcpyHostToDevice, mem.s));
    *out = (double*)dst;
    return GONN_OK;
}

int upload_kv_len(DevMem& mem, const int* kv_len, int B, const int** out) {
    *out = nullptr;
    if (!kv_len) return GONN_OK;
    void* dst = nullptr;
    TRY(mem.alloc(&dst, (size_t)B * sizeof(int)));
    TRYH(hipMemcpyAsync(dst, kv_len, (size_t)B * sizeof(int), hipMemcpyHostToDevice, mem.s));
    *out = (const int*)dst;
    return GONN_OK;
}

// The causal split of the fp64 forward (gonn::f64_fwd_split_plan): device
// item table and partials from `mem`, set in p. `items` holds the host
// table until the stream has copied it.
int f64_fwd_split_setup(DevMem& mem, gonn::F64Params& p, std::vector<int>& items) {
    gonn::F64FwdSplit sp = gonn::f64_fwd_split_plan(p);
    if (sp.items.empty()) return GONN_OK;
    items = std::move(sp.items);
    void *it = nullptr, *part = nullptr;
    TRY(mem.alloc(&it, items.size() * sizeof(int)));
    TRY(mem.alloc(&part, sp.part_bytes));
    TRYH(hipMemcpyAsync(it, items.data(), items.size() * sizeof(int), hipMemcpyHostToDevice,
                        mem.s));
    p.items = (const int*)it;
    p.nitems = (int)items.size();
    p.split_q0 = sp.split_q0;
    p.part = (double*)part;
    return GONN_OK;
}

// The causal split of the fp64 backward (gonn::f64_bwd_split_plan): device
// item tables and partials from `mem`, set in p; `items` and `items_k` hold
// the host tables until the stream has copied them.
int f64_bwd_split_setup(DevMem& mem, gonn::F64Params& p, std::vector<int>& items,
                        std::vector<int>& items_k) {
    gonn::F64BwdSplit sp = gonn::f64_bwd_split_plan(p);
    items = std::move(sp.items);
    items_k = std::move(sp.items_k);
    if (!items.empty()) {
        void *it = nullptr, *part = nullptr;
        TRY(mem.alloc(&it, items.size() * sizeof(int)));
        TRY(mem.alloc(&part, sp.part_bytes));
        TRYH(hipMemcpyAsync(it, items.data(), items.size() * sizeof(int), hipMemcpyHostToDevice,
                            mem.s));
        p.items = (const int*)it;
        p.nitems = (int)items.size();
        p.split_q0 = sp.split_q0;
        p.part = (double*)part;
    }
    if (!items_k.empty()) {
        void *it = nullptr, *part = nullptr;
        TRY(mem.alloc(&it, items_k.size() * sizeof(int)));
        TRY(mem.alloc(&part, sp.part_k_bytes));
        TRYH(hipMemcpyAsync(it, items_k.data(), items_k.size() * sizeof(int),
                            hipMemcpyHostToDevice, mem.s));
        p.items_k = (const int*)it;
        p.nitems_k = (int)items_k.size();
        p.split_k1 = sp.split_k1;
        p.part_k = (double*)part;
    }
    return GONN_OK;
}

// Forward on host fp64 data: O (and L when non-null) back in host memory.
int f64_exact_fwd(const double* Q, const double* K, const double* V, double* O, double* L, int B,
                  int H, int Sq, int Sk, int d, double scale, int causal, const int* kv_len,
                  const double* mask, size_t mask_n, long mask_sb, long mask_sh) {
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const size_t nq = (size_t)B * H * Sq * d, nk = (size_t)B * H * Sk * d;
    gonn::F64Params p{};
    double *q, *k, *v, *o, *l = nullptr, *m = nullptr;
    TRY(upload_f64(mem, Q, nq, &q));
    TRY(upload_f64(mem, K, nk, &k));
    TRY(upload_f64(mem, V, nk, &v));
    if (mask) TRY(upload_f64(mem, mask, mask_n, &m));
    TRY(upload_kv_len(mem, kv_len, B, &p.kv_len));
    TRY(mem.alloc((void**)&o, nq * sizeof(double)));
    if (L) TRY(mem.alloc((void**)&l, (size_t)B * H * Sq * sizeof(double)));
    p.q = q;
    p.k = k;
    p.v = v;
    p.out_o = o;
    p.out_lse = l;
    p.mask = m;
    p.mask_sb = mask_sb;
    p.mask_sh = mask_sh;
    p.B = B;
    p.H = H;
    p.Sq = Sq;
    p.Sk = Sk;
    p.d = d;
    p.scale = scale;
    p.causal = causal;
    std::vector<int> items;
    TRY(f64_fwd_split_setup(mem, p, items));
    {
        ProfScope ps("fwd_f64", hs);
        TRYH(gonn::launch_f64_fwd(p, hs));
    }
    TRYH(hipMemcpyAsync(O, o, nq * sizeof(double), hipMemcpyDeviceToHost, hs));
    if (L)
        TRYH(hipMemcpyAsync(L, l, (size_t)B * H * Sq * sizeof(double), hipMemcpyDeviceToHost,
                            hs));
    return herr(hipStreamSynchronize(hs));
}

// Backward on host fp64 data from the saved O and L (natural-log LSE).
int f64_exact_bwd(const double* Q, const double* K, const double* V, const double* O,
                  const double* L, const double* dO, double* dQ, double* dK, double* dV, int B,
                  int H, int Sq, int Sk, int d, double scale, int causal, const int* kv_len,
                  const double* mask, size_t mask_n, long mask_sb, long mask_sh) {
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const size_t rq = (size_t)B * H * Sq, nq = rq * d, nk = (size_t)B * H * Sk * d;
    gonn::F64Params p{};
    double *q, *k, *v, *o, *l, *g, *m = nullptr;
    TRY(upload_f64(mem, Q, nq, &q));
    TRY(upload_f64(mem, K, nk, &k));
    TRY(upload_f64(mem, V, nk, &v));
    TRY(upload_f64(mem, O, nq, &o));
    TRY(upload_f64(mem, L, rq, &l));
    TRY(upload_f64(mem, dO, nq, &g));
    if (mask) TRY(upload_f64(mem, mask, mask_n, &m));
    TRY(upload_kv_len(mem, kv_len, B, &p.kv_len));
    TRY(mem.alloc((void**)&p.delta, rq * sizeof(double)));
    TRY(mem.alloc((void**)&p.dq, nq * sizeof(double)));
    TRY(mem.alloc((void**)&p.dk, nk * sizeof(double)));
    TRY(mem.alloc((void**)&p.dv, nk * sizeof(double)));
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = l;
    p.dO = g;
    p.mask = m;
    p.mask_sb = mask_sb;
    p.mask_sh = mask_sh;
    p.B = B;
    p.H = H;
    p.Sq = Sq;
    p.Sk = Sk;
    p.d = d;
    p.scale = scale;
    p.causal = causal;
    std::vector<int> items, items_k;
    TRY(f64_bwd_split_setup(mem, p, items, items_k));
    {
        ProfScope ps("bwd_f64", hs);
        TRYH(gonn::launch_f64_bwd(p, hs));
    }
    TRYH(hipMemcpyAsync(dQ, p.dq, nq * sizeof(double), hipMemcpyDeviceToHost, hs));
    TRYH(hipMemcpyAsync(dK, p.dk, nk * sizeof(double), hipMemcpyDeviceToHost, hs));
    TRYH(hipMemcpyAsync(dV, p.dv, nk * sizeof(double), hipMemcpyDeviceToHost, hs));
    return herr(hipStreamSynchronize(hs));
}

}  // namespace

int gonn_hip_flash_attn_f64(const double* Q, const double* K, const double* V, double* O, int BH,
                            int S, int d, double scale, int causal) {
    if (current_mode() == GONN_ATTN_FP64) {
        if (!shim_args_ok(BH, S, d) || !Q || !K || !V || !O) return GONN_E_INVALID;
        if (!gonn_hip_available()) return GONN_E_NODEVICE;
        return f64_exact_fwd(Q, K, V, O, nullptr, BH, 1, S, S, d, scale, causal, nullptr,
                             nullptr, 0, 0, 0);
    }
    if (!shim_args_ok(BH, S, d) || !Q || !K || !V || !O) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const int dp = pad_dim(d);
    const size_t rows = (size_t)BH * S;
    float *q, *k, *v, *o;
    TRY(upload_padded(mem, Q, rows, d, dp, &q));
    TRY(upload_padded(mem, K, rows, d, dp, &k));
    TRY(upload_padded(mem, V, rows, d, dp, &v));
    TRY(mem.alloc((void**)&o, rows * dp * 4));
    TRY(run_fwd_f32(mem, q, k, v, o, nullptr, BH, S, dp, scale, causal));
    TRY(download_padded(mem, o, rows, d, dp, O));
    return herr(hipStreamSynchronize(hs));
}

int gonn_hip_flash_attn_f64_fwd(const double* Q, const double* K, const double* V, double* O,
                                double* L, int BH, int S, int d, double scale, int causal) {
    if (!shim_args_ok(BH, S, d) || !Q || !K || !V || !O || !L) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    if (current_mode() == GONN_ATTN_FP64)
        return f64_exact_fwd(Q, K, V, O, L, BH, 1, S, S, d, scale, causal, nullptr, nullptr, 0, 0,
                             0);
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const int dp = pad_dim(d);
    const size_t rows = (size_t)BH * S;
    float *q, *k, *v, *o, *l;
    TRY(upload_padded(mem, Q, rows, d, dp, &q));
    TRY(upload_padded(mem, K, rows, d, dp, &k));
    TRY(upload_padded(mem, V, rows, d, dp, &v));
    TRY(mem.alloc((void**)&o, rows * dp * 4));
    TRY(mem.alloc((void**)&l, rows * 4));
    TRY(run_fwd_f32(mem, q, k, v, o, l, BH, S, dp, scale, causal));
    TRY(download_padded(mem, o, rows, d, dp, O));
    TRY(download_padded(mem, l, rows, 1, 1, L));
    return herr(hipStreamSynchronize(hs));
}

int gonn_hip_flash_attn_f64_ex(const double* Q, const double* K, const double* V, double* O,
                               double* L, int B, int H, int Sq, int Sk, int d, double scale,
                               int causal, const int* kv_len) {
    return gonn_hip_flash_attn_f64_masked(Q, K, V, O, L, B, H, Sq, Sk, d, scale, causal, kv_len,
                                          nullptr, 0, 0);
}

// Elements an additive mask with these strides spans (0: bad strides).
static size_t mask_elems(int B, int H, int Sq, int Sk, long sb, long sh) {
    if (sb < 0 || sh < 0) return 0;
    const double n = (double)(B - 1) * sb + (double)(H - 1) * sh + (double)Sq * Sk;
    return n < 9.0e15 ? (size_t)n : 0;
}

int gonn_hip_flash_attn_f64_masked(const double* Q, const double* K, const double* V, double* O,
                                   double* L, int B, int H, int Sq, int Sk, int d, double scale,
                                   int causal, const int* kv_len, const double* mask,
                                   long mask_sb, long mask_sh) {
    if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || d <= 0 || d > 128) return GONN_E_INVALID;
    if (!Q || !K || !V || !O || !std::isfinite(scale)) return GONN_E_INVALID;
    const size_t mn = mask ? mask_elems(B, H, Sq, Sk, mask_sb, mask_sh) : 0;
    if (mask && !mn) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    if (current_mode() == GONN_ATTN_FP64)
        return f64_exact_fwd(Q, K, V, O, L, B, H, Sq, Sk, d, scale, causal, kv_len, mask, mn,
                             mask_sb, mask_sh);
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const int dp = pad_dim(d);
    const size_t rq = (size_t)B * H * Sq, rk = (size_t)B * H * Sk;
    float *q, *k, *v, *o, *l = nullptr, *m = nullptr;
    int* kl = nullptr;
    TRY(upload_padded(mem, Q, rq, d, dp, &q));
    TRY(upload_padded(mem, K, rk, d, dp, &k));
    TRY(upload_padded(mem, V, rk, d, dp, &v));
    if (mask) TRY(upload_padded(mem, mask, mn, 1, 1, &m));
    TRY(mem.alloc((void**)&o, rq * dp * 4));
    if (L) TRY(mem.alloc((void**)&l, rq * 4));
    if (kv_len) {
        TRY(mem.alloc((void**)&kl, (size_t)B * 4));
        TRYH(hipMemcpyAsync(kl, kv_len, (size_t)B * 4, hipMemcpyHostToDevice, mem.s));
    }
    TRY(run_fwd_f32_ex(mem, q, k, v, o, l, B, H, Sq, Sk, dp, scale, causal, kl, m, mn, mask_sb,
                       mask_sh));
    TRY(download_padded(mem, o, rq, d, dp, O));
    if (L) TRY(download_padded(mem, l, rq, 1, 1, L));
    return herr(hipStreamSynchronize(hs));
}

int gonn_hip_flash_attn_f64_bwd(const double* Q, const double* K, const double* V, const double* O,
                                const double* L, const double* dO, double* dQ, double* dK,
                                double* dV, int BH, int S, int d, double scale, int causal) {
    return gonn_hip_flash_attn_f64_bwd_ex(Q, K, V, O, L, dO, dQ, dK, dV, BH, 1, S, d, scale, causal,
                                          nullptr);
}

int gonn_hip_flash_attn_f64_bwd_ex(const double* Q, const double* K, const double* V,
                                   const double* O, const double* L, const double* dO, double* dQ,
                                   double* dK, double* dV, int B, int H, int S, int d,
                                   double scale, int causal, const int* kv_len) {
    return gonn_hip_flash_attn_f64_bwd_masked(Q, K, V, O, L, dO, dQ, dK, dV, B, H, S, S, d, scale,
                                              causal, kv_len, nullptr, 0, 0);
}

int gonn_hip_flash_attn_f64_bwd_masked(const double* Q, const double* K, const double* V,
                                       const double* O, const double* L, const double* dO,
                                       double* dQ, double* dK, double* dV, int B, int H, int Sq,
                                       int Sk, int d, double scale, int causal,
                                       const int* kv_len, const double* mask, long mask_sb,
                                       long mask_sh) {
    if (B <= 0 || H <= 0 || !shim_args_ok(B * H, Sq, d) || !shim_args_ok(B * H, Sk, d) || !Q ||
        !K || !V || !O || !L || !dO || !dQ || !dK || !dV)
        return GONN_E_INVALID;
    const size_t mn = mask ? mask_elems(B, H, Sq, Sk, mask_sb, mask_sh) : 0;
    if (mask && !mn) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    if (current_mode() == GONN_ATTN_FP64)
        return f64_exact_bwd(Q, K, V, O, L, dO, dQ, dK, dV, B, H, Sq, Sk, d, scale, causal, kv_len,
                             mask, mn, mask_sb, mask_sh);
    const int BH = B * H;
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    const int dp = pad_dim(d);
    const size_t rq = (size_t)BH * Sq, rk = (size_t)BH * Sk, nq = rq * dp, nk = rk * dp;
    float *q, *k, *v, *o, *l, *g, *dq, *dk, *dv;
    TRY(upload_padded(mem, Q, rq, d, dp, &q));
    TRY(upload_padded(mem, K, rk, d, dp, &k));
    TRY(upload_padded(mem, V, rk, d, dp, &v));
    TRY(upload_padded(mem, O, rq, d, dp, &o));
    TRY(upload_padded(mem, L, rq, 1, 1, &l));
    TRY(upload_padded(mem, dO, rq, d, dp, &g));
    TRY(mem.alloc((void**)&dq, nq * 4));
    TRY(mem.alloc((void**)&dk, nk * 4));
    TRY(mem.alloc((void**)&dv, nk * 4));
    int* kl = nullptr;
    float* m = nullptr;
    if (mask) TRY(upload_padded(mem, mask, mn, 1, 1, &m));
    if (kv_len) {
        TRY(mem.alloc((void**)&kl, (size_t)B * 4));
        TRYH(hipMemcpyAsync(kl, kv_len, (size_t)B * 4, hipMemcpyHostToDevice, mem.s));
    }
    gonn_attn_bwd_args a{};
    a.q = {q, nq * 4, GONN_F32};
    a.k = {k, nk * 4, GONN_F32};
    a.v = {v, nk * 4, GONN_F32};
    a.o = {o, nq * 4, GONN_F32};
    a.lse = {l, rq * 4, GONN_F32};
    a.dO = {g, nq * 4, GONN_F32};
    a.dq = {dq, nq * 4, GONN_F32};
    a.dk = {dk, nk * 4, GONN_F32};
    a.dv = {dv, nk * 4, GONN_F32};
    a.kv_len = {kl, kl ? (size_t)B * 4 : 0, GONN_I32};
    a.attn_mask = {m, m ? mn * 4 : 0, GONN_F32};
    a.mask_stride_b = mask_sb;
    a.mask_stride_h = mask_sh;
    a.B = B;
    a.H = H;
    a.S = Sq;
    a.Sk = Sk;
    a.D = dp;
    a.scale = scale;
    a.causal = causal;
    a.mode = current_mode();
    a.deterministic = 1;
    const size_t wsb = gonn_hip_attn_workspace_bytes(GONN_OP_BWD, &a);
    void* ws = nullptr;
    if (wsb) TRY(mem.alloc(&ws, wsb));
    TRY(gonn_hip_attn_bwd(&a, ws, wsb, mem.s));
    TRY(download_padded(mem, dq, rq, d, dp, dQ));
    TRY(download_padded(mem, dk, rk, d, dp, dK));
    TRY(download_padded(mem, dv, rk, d, dp, dV));
    return herr(hipStreamSynchronize(hs));
}

// Mean ms per call of `call` over `iters` calls on the null stream (after
// five untimed ones), from one event pair; -1 if a call or an event fails.
extern "C++" template <typename F>
static double time_calls(F call, int iters) {
    for (int i = 0; i < 5; i++)
        if (!call()) return -1.0;
    if (hipDeviceSynchronize() != hipSuccess) return -1.0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
              hipEventRecord(e0, nullptr) == hipSuccess;
    for (int i = 0; ok && i < iters; i++) ok = call();
    ok = ok && hipEventRecord(e1, nullptr) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
    float ms = 0.f;
    ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return ok ? (double)ms / iters : -1.0;
}

// Mean ms per call of the f64 mode's forward over `iters` calls (after 5
// untimed), on zeroed device fp64 buffers, null stream.
static double bench_f64_exact(int BH, int S, int d, int iters, int causal) {
    DevMem mem(nullptr);
    const size_t n = (size_t)BH * S * d;
    double *q, *k, *v, *o;
    if (mem.alloc((void**)&q, n * 8) || mem.alloc((void**)&k, n * 8) ||
        mem.alloc((void**)&v, n * 8) || mem.alloc((void**)&o, n * 8))
        return (double)GONN_E_NOMEM;
    if (gonn::launch_fill_zero(q, n * 8, nullptr) || gonn::launch_fill_zero(k, n * 8, nullptr) ||
        gonn::launch_fill_zero(v, n * 8, nullptr))
        return -1.0;
    gonn::F64Params p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.out_o = o;
    p.B = BH;
    p.H = 1;
    p.Sq = p.Sk = S;
    p.d = d;
    p.scale = 1.0 / std::sqrt((double)d);
    p.causal = causal;
    std::vector<int> items;
    if (f64_fwd_split_setup(mem, p, items) != GONN_OK) return -1.0;
    return time_calls([&] { return gonn::launch_f64_fwd(p, nullptr) == hipSuccess; }, iters);
}

// Mean ms per call of the f64 mode's backward (D = rowsum(dO * O), dQ,
// dK/dV) over `iters` calls (after 5 untimed), on zeroed device fp64
// buffers (LSE 0: every key live), null stream.
static double bench_f64_exact_bwd(int BH, int S, int d, int iters, int causal) {
    DevMem mem(nullptr);
    const size_t n = (size_t)BH * S * d, nr = (size_t)BH * S;
    double *q, *k, *v, *o, *g, *l, *dl, *dq, *dk, *dv;
    if (mem.alloc((void**)&q, n * 8) || mem.alloc((void**)&k, n * 8) ||
        mem.alloc((void**)&v, n * 8) || mem.alloc((void**)&o, n * 8) ||
        mem.alloc((void**)&g, n * 8) || mem.alloc((void**)&l, nr * 8) ||
        mem.alloc((void**)&dl, nr * 8) || mem.alloc((void**)&dq, n * 8) ||
        mem.alloc((void**)&dk, n * 8) || mem.alloc((void**)&dv, n * 8))
        return (double)GONN_E_NOMEM;
    for (double* x : {q, k, v, o, g})
        if (gonn::launch_fill_zero(x, n * 8, nullptr)) return -1.0;
    if (gonn::launch_fill_zero(l, nr * 8, nullptr)) return -1.0;
    gonn::F64Params p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.dO = g;
    p.lse = l;
    p.delta = dl;
    p.dq = dq;
    p.dk = dk;
    p.dv = dv;
    p.B = BH;
    p.H = 1;
    p.Sq = p.Sk = S;
    p.d = d;
    p.scale = 1.0 / std::sqrt((double)d);
    p.causal = causal;
    std::vector<int> items, items_k;
    if (f64_bwd_split_setup(mem, p, items, items_k) != GONN_OK) return -1.0;
    return time_calls([&] { return gonn::launch_f64_bwd(p, nullptr) == hipSuccess; }, iters);
}

double gonn_hip_bench_flash_attn_f64_bwd(int BH, int S, int d, int iters, int causal) {
    if (!shim_args_ok(BH, S, d) || iters <= 0) return (double)GONN_E_INVALID;
    if (!gonn_hip_available()) return (double)GONN_E_NODEVICE;
    if (current_mode() != GONN_ATTN_FP64) return (double)GONN_E_INVALID;
    return bench_f64_exact_bwd(BH, S, d, iters, causal);
}

double gonn_hip_bench_flash_attn_f64(int BH, int S, int d, int iters, int causal) {
    if (!shim_args_ok(BH, S, d) || iters <= 0) return (double)GONN_E_INVALID;
    if (!gonn_hip_available()) return (double)GONN_E_NODEVICE;
    if (current_mode() == GONN_ATTN_FP64) return bench_f64_exact(BH, S, d, iters, causal);
    DevMem mem(nullptr);
    const int dp = pad_dim(d);
    const size_t n = (size_t)BH * S * dp;
    float *q, *k, *v, *o;
    if (mem.alloc((void**)&q, n * 4) || mem.alloc((void**)&k, n * 4) ||
        mem.alloc((void**)&v, n * 4) || mem.alloc((void**)&o, n * 4))
        return (double)GONN_E_NOMEM;
    if (gonn::launch_fill_zero(q, n * 4, nullptr) || gonn::launch_fill_zero(k, n * 4, nullptr) ||
        gonn::launch_fill_zero(v, n * 4, nullptr))
        return -1.0;
    const double scale = 1.0 / std::sqrt((double)d);
    gonn_attn_fwd_args a{};
    a.q = {q, n * 4, GONN_F32};
    a.k = {k, n * 4, GONN_F32};
    a.v = {v, n * 4, GONN_F32};
    a.o = {o, n * 4, GONN_F32};
    a.B = BH;
    a.H = 1;
    a.Sq = a.Sk = S;
    a.D = dp;
    a.scale = scale;
    a.causal = causal;
    a.mode = current_mode();
    const size_t wsb = gonn_hip_attn_workspace_bytes(GONN_OP_FWD, &a);
    void* ws = nullptr;
    if (wsb && mem.alloc(&ws, wsb)) return (double)GONN_E_NOMEM;
    return time_calls([&] { return gonn_hip_attn_fwd(&a, ws, wsb, nullptr) == GONN_OK; }, iters);
}

int gonn_hip_profile_enable(int on) {
    g_prof_on.store(on != 0);
    return GONN_OK;
}

int gonn_hip_profile_reset(void) {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    for (auto& r : g_prof) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    g_prof.clear();
    return GONN_OK;
}

int gonn_hip_profile_read(const char* kernel, double* total_ms, int* count) {
    if (!kernel || !total_ms || !count) return GONN_E_INVALID;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    double tot = 0.0;
    int n = 0;
    for (auto& r : g_prof) {
        if (std::strcmp(r.name, kernel) != 0) continue;
        TRYH(hipEventSynchronize(r.b));
        float ms = 0.f;
        TRYH(hipEventElapsedTime(&ms, r.a, r.b));
        tot += ms;
        n++;
    }
    *total_ms = tot;
    *count = n;
    return GONN_OK;
}

int gonn_hip_selftest_mfma(void) {
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    return gonn::selftest_mfma();
}

// ---- KV cache ---------------------------------------------------------------

int gonn_hip_kvcache_create(gonn_kvcache** out, int B, int H, int Lmax, int D) {
    if (!out) return GONN_E_INVALID;
    *out = nullptr;
    if (B <= 0 || H <= 0 || Lmax <= 0 || D <= 0) return GONN_E_INVALID;
    if (!head_dim_ok(D)) return GONN_E_UNSUPPORTED;
    const size_t n = (size_t)B * H * Lmax * D;
    if ((double)n * 2 >= 9.0e18 || (double)B * H * Lmax >= 2147483647.0) return GONN_E_UNSUPPORTED;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    if (fail_alloc_injected()) return GONN_E_INJECTED;
    gonn_kvcache* c = new (std::nothrow) gonn_kvcache;
    if (!c) return GONN_E_NOMEM;
    c->B = B;
    c->H = H;
    c->Lmax = Lmax;
    c->D = D;
    c->h_len.assign(B, 0);
    gonn_attn_decode_args a = kv_decode_args(c);
    c->ws_bytes = decode_ws(&a);
    const size_t bytes[] = {n * 2, n * 2, (size_t)B * 4, (size_t)B * 8, c->ws_bytes};
    void** slots[] = {&c->k, &c->v, (void**)&c->d_len, (void**)&c->d_pc, &c->ws};
    for (int i = 0; i < 5; i++) {
        if (hipMalloc(slots[i], bytes[i] ? bytes[i] : 16) != hipSuccess) {
            (void)hipGetLastError();
            *slots[i] = nullptr;
            kv_release(c);
            delete c;
            return GONN_E_NOMEM;
        }
    }
    const hipError_t e = hipMemset(c->d_len, 0, (size_t)B * 4);
    if (e != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        kv_release(c);
        delete c;
        return herr(e != hipSuccess ? e : hipErrorUnknown);
    }
    *out = c;
    return GONN_OK;
}

int gonn_hip_kvcache_free(gonn_kvcache* c) {
    if (!c) return GONN_OK;
    kv_release(c);
    delete c;
    return GONN_OK;
}

int gonn_hip_kvcache_reset(gonn_kvcache* c) {
    if (!c) return GONN_E_INVALID;
    std::fill(c->h_len.begin(), c->h_len.end(), 0);
    TRYH(hipMemcpy(c->d_len, c->h_len.data(), (size_t)c->B * 4, hipMemcpyHostToDevice));
    c->stale = false;  // host and device lengths agree again
    return GONN_OK;
}

int gonn_hip_kvcache_lengths(const gonn_kvcache* c, int* len) {
    if (!c || !len) return GONN_E_INVALID;
    for (int b = 0; b < c->B; b++) len[b] = c->h_len[b];
    return GONN_OK;
}

int gonn_hip_kvcache_append(gonn_kvcache* c, const gonn_buf* k, const gonn_buf* v, int T,
                            const int* counts, void* stream) {
    if (!c || !k || !v) return GONN_E_INVALID;
    if (k->dtype != v->dtype || (k->dtype != GONN_F32 && k->dtype != GONN_BF16))
        return GONN_E_INVALID;
    if (T <= 0) return GONN_E_INVALID;
    const size_t n = (size_t)c->B * c->H * T * c->D;
    if (!buf_ok(*k, n, k->dtype) || !buf_ok(*v, n, v->dtype)) return GONN_E_INVALID;
    if (((uintptr_t)k->ptr | (uintptr_t)v->ptr) & 15) return GONN_E_INVALID;
    TRY(kv_check_append(c, T, counts));
    return kv_append_dev(c, k->ptr, v->ptr, k->dtype == GONN_BF16, T, (hipStream_t)stream);
}

int gonn_hip_kvcache_append_f64(gonn_kvcache* c, const double* k, const double* v, int T,
                                const int* counts) {
    if (!c || !k || !v) return GONN_E_INVALID;
    TRY(kv_check_append(c, T, counts));
    const size_t rows = (size_t)c->B * c->H * T;
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    float *kd = nullptr, *vd = nullptr;
    TRY(upload_padded(mem, k, rows, c->D, c->D, &kd));
    TRY(upload_padded(mem, v, rows, c->D, c->D, &vd));
    return kv_append_dev(c, kd, vd, 0, T, hs);
}

int gonn_hip_kvcache_attend(gonn_kvcache* c, const gonn_buf* q, gonn_buf* o, double scale,
                            void* stream) {
    if (!c || !q || !o || c->stale) return GONN_E_INVALID;
    gonn_attn_decode_args a = kv_decode_args(c);
    a.q = *q;
    a.o = *o;
    a.scale = scale;
    return gonn_hip_attn_decode(&a, c->ws, c->ws_bytes, stream);
}

int gonn_hip_kvcache_attend_f64(gonn_kvcache* c, const double* q, double* o, double scale) {
    if (!c || !q || !o || c->stale) return GONN_E_INVALID;
    const size_t rows = (size_t)c->B * c->H;
    hipStream_t hs = nullptr;
    TRY(host_stream(&hs));
    DevMem mem(hs);
    StreamSync wait_on_exit{hs};
    float* qd = nullptr;
    void* od = nullptr;
    TRY(upload_padded(mem, q, rows, c->D, c->D, &qd));
    TRY(mem.alloc(&od, rows * c->D * sizeof(float)));
    gonn_buf qb{qd, rows * c->D * 4, GONN_F32}, ob{od, rows * c->D * 4, GONN_F32};
    TRY(gonn_hip_kvcache_attend(c, &qb, &ob, scale, hs));
    TRY(download_padded(mem, (const float*)od, rows, c->D, c->D, o));
    return herr(hipStreamSynchronize(hs));
}

size_t gonn_hip_kvcache_attend_causal_workspace_bytes(const gonn_kvcache* c, int T) {
    return gonn::kvcache_attend_causal_ws(c, T);
}

int gonn_hip_kvcache_attend_causal(gonn_kvcache* c, const gonn_buf* q, gonn_buf* o, int T,
                                   double scale, void* ws, size_t ws_bytes, void* stream) {
    if (!c || !q || !o || T <= 0 || !std::isfinite(scale) || c->stale) return GONN_E_INVALID;
    const size_t n = (size_t)c->B * c->H * T * c->D;
    if (!buf_ok(*q, n, GONN_F32) || !buf_ok(*o, n, GONN_F32)) return GONN_E_INVALID;
    // The T queries' own positions are the last T cached ones.
    for (int b = 0; b < c->B; b++)
        if (c->h_len[b] < T) return GONN_E_INVALID;
    if (!ws || ws_bytes < gonn::kvcache_attend_causal_ws(c, T)) return GONN_E_WORKSPACE;
    return gonn::kvcache_attend_causal_run(c, (const float*)q->ptr, (float*)o->ptr, T, scale, ws,
                                           (hipStream_t)stream, true);
}

}  // extern "C"
