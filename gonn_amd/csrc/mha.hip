// mha.hip -- device-resident multi-head attention forward: the MHA of
// nn/attention.go:107-148 (projections nn/linear.go:40-59, head split, fused
// core, head merge, output projection) with its weights held in HBM and every
// intermediate kept there.
//
// The reference moves data across PCIe around each GEMM (gonn_cuda.cu:147-177,
// through tensor/dispatch.go:111-113) and again around the fused core
// (gonn_cuda.cu:466-529). Here one call uploads x once and downloads the
// output once (gonn_hip_mha_forward_f64); gonn_hip_mha_forward_dev takes
// device buffers, a caller workspace and a stream, and allocates nothing.
//
// Per forward, on one stream:
//   Y_p = x_p W_p^T            rocBLAS fp64 (gonn_hip_gemm_f64_dev), p = q, k, v;
//                              one GEMM against the stacked (3E, E) weights for
//                              self-attention with kdim = vdim = E
//   heads_p = split(Y_p + b_p)  fp32 (B, H, T, dp), zero-padded to dp = 64 | 128
//   O = attention core          gonn_hip_attn_fwd (current MFMA mode)
//   ctx = merge(O)              fp64 (B, Tq, E)
//   out = ctx Wo^T + bo         rocBLAS fp64, then the bias
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/gonn_hip.h"
#include "kvcache_internal.h"

namespace {

int herr(hipError_t e) { return e == hipSuccess ? GONN_OK : (int)e; }

#define TRY(x)                          \
    do {                                \
        const int _rc = (x);            \
        if (_rc != GONN_OK) return _rc; \
    } while (0)

size_t al(size_t x) { return (x + 255) / 256 * 256; }

unsigned grid_for(size_t n) {
    const size_t want = (n + 255) / 256;
    return (unsigned)(want < 4096 ? (want ? want : 1) : 4096);
}

// heads[b][h][t][d] = Y[b][t][h D + d] + bias[h D + d] for d < D, 0 for D <= d < dp;
// rows of Y are ldy apart (E, or 3E for the fused q/k/v projection).
__global__ __launch_bounds__(256) void split_heads_kernel(const double* __restrict__ Y,
                                                          const double* __restrict__ bias,
                                                          float* __restrict__ heads, int T, int H,
                                                          int D, int dp, size_t ldy, size_t total) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % dp);
        const size_t r = i / dp;
        const int t = (int)(r % T);
        const size_t bh = r / T;
        const int h = (int)(bh % H);
        const size_t b = bh / H;
        float v = 0.f;
        if (d < D) {
            const size_t e = (size_t)h * D + d;
            v = (float)(Y[(b * T + t) * ldy + e] + bias[e]);
        }
        heads[i] = v;
    }
}

// The three splits of a fused projection in one launch: Y rows hold
// [Q | K | V] (3E apart); tensor p of heads3[p] (each `per` values) takes
// columns p E .. p E + E - 1 and bias3 + p E.
__global__ __launch_bounds__(256) void split_heads3_kernel(const double* __restrict__ Y,
                                                           const double* __restrict__ bias3,
                                                           float* __restrict__ h0,
                                                           float* __restrict__ h1,
                                                           float* __restrict__ h2, int T, int H,
                                                           int D, int dp, size_t per) {
    const size_t E = (size_t)H * D;
    for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < 3 * per;
         j += (size_t)gridDim.x * blockDim.x) {
        const int p = (int)(j / per);
        const size_t i = j - (size_t)p * per;
        const int d = (int)(i % dp);
        const size_t r = i / dp;
        const int t = (int)(r % T);
        const size_t bh = r / T;
        const int h = (int)(bh % H);
        const size_t b = bh / H;
        float v = 0.f;
        if (d < D) {
            const size_t e = (size_t)h * D + d;
            v = (float)(Y[(b * T + t) * 3 * E + p * E + e] + bias3[p * E + e]);
        }
        (p == 0 ? h0 : p == 1 ? h1 : h2)[i] = v;
    }
}

// ctx[b][t][h D + d] = O[b][h][t][d].
__global__ __launch_bounds__(256) void merge_heads_kernel(const float* __restrict__ O,
                                                          double* __restrict__ ctx, int T, int H,
                                                          int D, int dp, size_t total) {
    const size_t E = (size_t)H * D;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t e = i % E, bt = i / E;
        const int h = (int)(e / D), d = (int)(e % D);
        const int t = (int)(bt % T);
        const size_t b = bt / T;
        ctx[i] = (double)O[((b * H + h) * T + t) * dp + d];
    }
}

// Y[n][o] += bias[o].
__global__ __launch_bounds__(256) void add_bias_kernel(double* __restrict__ Y,
                                                       const double* __restrict__ bias, int E,
                                                       size_t total) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        Y[i] += bias[i % E];
}

gonn_buf f64buf(const void* p, size_t n) { return gonn_buf{(void*)p, n * sizeof(double), GONN_F64}; }

}  // namespace

// The handle of the C ABI (opaque to callers).
struct gonn_mha {
    int E = 0, H = 0, D = 0, dp = 0, kdim = 0, vdim = 0;
    // q, k, v, out weights (E, in), one allocation in that order, so that for
    // kdim = vdim = E the first three form one (3E, E) matrix: a
    // self-attention forward projects q, k and v with a single GEMM.
    double* W[4] = {nullptr, nullptr, nullptr, nullptr};
    double* b[4] = {nullptr, nullptr, nullptr, nullptr};  // (E) each, one allocation
    std::mutex mu;       // guards the host entry's workspace
    void* ws = nullptr;  // grow-only workspace of gonn_hip_mha_forward_f64
    size_t ws_bytes = 0;
};

namespace {

void mha_release(gonn_mha* m) {
    if (m->W[0]) (void)hipFree(m->W[0]);
    if (m->b[0]) (void)hipFree(m->b[0]);
    if (m->ws) (void)hipFree(m->ws);
}

// Workspace layout of one forward (256-byte aligned pieces, in order):
//   Yq (B Tq E) f64 | Yk (B Tk E) | Yv (B Tk E) | hq (B H Tq dp) f32 | hk | hv |
//   ho (B H Tq dp) | kv_len (B) i32 | attention workspace (either MFMA mode)
struct Layout {
    size_t yq, yk, yv, hq, hk, hv, ho, kl, aw, aw_bytes, total;
};

Layout layout(const gonn_mha* m, int B, int Tq, int Tk) {
    Layout L{};
    const size_t nq = (size_t)B * Tq, nk = (size_t)B * Tk;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += al(bytes);
        return at;
    };
    L.yq = take(nq * m->E * 8);
    L.yk = take(nk * m->E * 8);
    L.yv = take(nk * m->E * 8);
    L.hq = take(nq * m->H * m->dp * 4);
    L.hk = take(nk * m->H * m->dp * 4);
    L.hv = take(nk * m->H * m->dp * 4);
    L.ho = take(nq * m->H * m->dp * 4);
    L.kl = take((size_t)B * 4);
    gonn_attn_fwd_args a{};
    a.B = B;
    a.H = m->H;
    a.Sq = Tq;
    a.Sk = Tk;
    a.D = m->dp;
    a.mode = GONN_ATTN_FP32_MFMA;
    size_t aw = gonn_hip_attn_workspace_bytes(GONN_OP_FWD, &a);
    a.mode = GONN_ATTN_BF16_MFMA;
    const size_t aw1 = gonn_hip_attn_workspace_bytes(GONN_OP_FWD, &a);
    if (aw1 > aw) aw = aw1;
    L.aw_bytes = aw;
    L.aw = take(aw);
    L.total = off + 256;  // room to align the base
    return L;
}

bool shape_ok(const gonn_mha* m, int B, int Tq, int Tk) {
    if (!m || B <= 0 || Tq <= 0 || Tk <= 0) return false;
    const double big = 9.0e15;
    return (double)B * Tq * m->E < big && (double)B * Tk * m->E < big &&
           (double)B * Tk * (m->kdim > m->vdim ? m->kdim : m->vdim) < big &&
           (double)B * m->H * (Tq > Tk ? Tq : Tk) * m->dp < 2147483647.0 * 8;
}

// The forward on device data; x* are fp64 (B, T, in) device pointers.
int run_forward(gonn_mha* m, const double* xq, const double* xk, const double* xv, double* out,
                int B, int Tq, int Tk, int causal, const int* kv_len_dev, uint8_t* w,
                const Layout& L, hipStream_t s) {
    const int E = m->E, H = m->H, D = m->D, dp = m->dp;
    const size_t nq = (size_t)B * Tq, nk = (size_t)B * Tk;
    double* Y[3] = {(double*)(w + L.yq), (double*)(w + L.yk), (double*)(w + L.yv)};
    float* hd[3] = {(float*)(w + L.hq), (float*)(w + L.hk), (float*)(w + L.hv)};
    const double* x[3] = {xq, xk, xv};
    const int in[3] = {E, m->kdim, m->vdim};
    const size_t rows[3] = {nq, nk, nk};
    const int T[3] = {Tq, Tk, Tk};
    // Self-attention with square projections: one GEMM against the stacked
    // (3E, E) weights writes [Q | K | V] rows of 3E into Yq's slot, which the
    // layout follows with Yk's and Yv's (room for 3 nq E values).
    const bool fused = xq == xk && xk == xv && Tq == Tk && m->kdim == E && m->vdim == E;
    if (fused) {
        const gonn_buf A = f64buf(xq, nq * E), Wb = f64buf(m->W[0], (size_t)3 * E * E);
        gonn_buf C = f64buf(Y[0], nq * 3 * E);
        TRY(gonn_hip_gemm_f64_dev(&A, &Wb, &C, 1, (int)nq, E, 3 * E, 0, 1, s));
        const size_t per = nq * H * dp;
        hipLaunchKernelGGL(split_heads3_kernel, dim3(grid_for(3 * per)), dim3(256), 0, s, Y[0],
                           m->b[0], hd[0], hd[1], hd[2], Tq, H, D, dp, per);
        TRY(herr(hipGetLastError()));
    } else {
        for (int p = 0; p < 3; p++) {
            const gonn_buf A = f64buf(x[p], rows[p] * in[p]),
                           Wb = f64buf(m->W[p], (size_t)E * in[p]);
            gonn_buf C = f64buf(Y[p], rows[p] * E);
            TRY(gonn_hip_gemm_f64_dev(&A, &Wb, &C, 1, (int)rows[p], in[p], E, 0, 1, s));
            const size_t tot = rows[p] * H * dp;
            hipLaunchKernelGGL(split_heads_kernel, dim3(grid_for(tot)), dim3(256), 0, s, Y[p],
                               m->b[p], hd[p], T[p], H, D, dp, (size_t)E, tot);
            TRY(herr(hipGetLastError()));
        }
    }
    gonn_attn_fwd_args a{};
    const size_t hq = nq * H * dp, hk = nk * H * dp;
    float* ho = (float*)(w + L.ho);
    a.q = {hd[0], hq * 4, GONN_F32};
    a.k = {hd[1], hk * 4, GONN_F32};
    a.v = {hd[2], hk * 4, GONN_F32};
    a.o = {ho, hq * 4, GONN_F32};
    a.kv_len = {(void*)kv_len_dev, kv_len_dev ? (size_t)B * 4 : 0, GONN_I32};
    a.B = B;
    a.H = H;
    a.Sq = Tq;
    a.Sk = Tk;
    a.D = dp;
    a.scale = 1.0 / std::sqrt((double)D);  // nn/attention.go:136
    a.causal = causal;
    // The core runs on the layer's fp32 device intermediates: in the f64
    // entries' fp64 mode it takes the fp32-MFMA kernels.
    const int mode = gonn_hip_get_attn_mode();
    a.mode = mode == GONN_ATTN_FP64 ? GONN_ATTN_FP32_MFMA : mode;
    TRY(gonn_hip_attn_fwd(&a, w + L.aw, L.aw_bytes, s));
    // Merge into Yq's slot (the projections are done with it), then project.
    double* ctx = Y[0];
    const size_t tot = nq * E;
    hipLaunchKernelGGL(merge_heads_kernel, dim3(grid_for(tot)), dim3(256), 0, s, ho, ctx, Tq, H, D,
                       dp, tot);
    TRY(herr(hipGetLastError()));
    const gonn_buf A = f64buf(ctx, tot), Wb = f64buf(m->W[3], (size_t)E * E);
    gonn_buf C = f64buf(out, tot);
    TRY(gonn_hip_gemm_f64_dev(&A, &Wb, &C, 1, (int)nq, E, E, 0, 1, s));
    hipLaunchKernelGGL(add_bias_kernel, dim3(grid_for(tot)), dim3(256), 0, s, out, m->b[3], E, tot);
    return herr(hipGetLastError());
}

// Workspace of the incremental forward (256-byte aligned pieces): Y (B T 3E)
// f64 | hq, hk, hv, ho (B H T dp) f32 | causal-attend workspace.
struct IncLayout {
    size_t y, hq, hk, hv, ho, aw, total;
};

IncLayout inc_layout(const gonn_mha* m, const gonn_kvcache* c, int B, int T) {
    IncLayout L{};
    const size_t n = (size_t)B * T;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += al(bytes);
        return at;
    };
    L.y = take(n * 3 * m->E * 8);
    L.hq = take(n * m->H * m->dp * 4);
    L.hk = take(n * m->H * m->dp * 4);
    L.hv = take(n * m->H * m->dp * 4);
    L.ho = take(n * m->H * m->dp * 4);
    L.aw = take(gonn::kvcache_attend_causal_ws(c, T));
    L.total = off + 256;
    return L;
}

// The cache must hold this layer's heads at the padded head dim, and the
// layer must be a square self-attention (one stacked q/k/v projection).
bool inc_ok(const gonn_mha* m, const gonn_kvcache* c, int T, int* B) {
    if (!m || !c || T <= 0) return false;
    int H = 0, Lmax = 0, D = 0;
    gonn::kvcache_dims(c, B, &H, &Lmax, &D);
    return H == m->H && D == m->dp && m->kdim == m->E && m->vdim == m->E && T <= Lmax &&
           (double)*B * T * 3 * m->E < 9.0e15;
}

// Incremental self-attention on device data: x, out fp64 (B, T, E).
int run_incremental(gonn_mha* m, gonn_kvcache* c, const double* x, double* out, int B, int T,
                    uint8_t* w, const IncLayout& L, hipStream_t s) {
    if (!gonn::kvcache_usable(c)) return GONN_E_INVALID;
    const int E = m->E, H = m->H, D = m->D, dp = m->dp;
    const size_t n = (size_t)B * T;
    double* Y = (double*)(w + L.y);
    float* hq = (float*)(w + L.hq);
    float* hk = (float*)(w + L.hk);
    float* hv = (float*)(w + L.hv);
    float* ho = (float*)(w + L.ho);
    {
        const gonn_buf A = f64buf(x, n * E), Wb = f64buf(m->W[0], (size_t)3 * E * E);
        gonn_buf C = f64buf(Y, n * 3 * E);
        TRY(gonn_hip_gemm_f64_dev(&A, &Wb, &C, 1, (int)n, E, 3 * E, 0, 1, s));
        const size_t per = n * H * dp;
        hipLaunchKernelGGL(split_heads3_kernel, dim3(grid_for(3 * per)), dim3(256), 0, s, Y,
                           m->b[0], hq, hk, hv, T, H, D, dp, per);
        TRY(herr(hipGetLastError()));
    }
    std::vector<int> new_len;
    TRY(gonn::kvcache_append_pending(c, hk, hv, T, s, &new_len));
    int rc = gonn::kvcache_attend_causal_run(c, hq, ho, T, 1.0 / std::sqrt((double)D), w + L.aw, s,
                                             true);  // nn/attention.go:136
    if (rc == GONN_OK) {
        const size_t tot = n * E;
        hipLaunchKernelGGL(merge_heads_kernel, dim3(grid_for(tot)), dim3(256), 0, s, ho, Y, T, H,
                           D, dp, tot);
        rc = herr(hipGetLastError());
        if (rc == GONN_OK) {
            const gonn_buf A = f64buf(Y, tot), Wb = f64buf(m->W[3], (size_t)E * E);
            gonn_buf C = f64buf(out, tot);
            rc = gonn_hip_gemm_f64_dev(&A, &Wb, &C, 1, (int)n, E, E, 0, 1, s);
        }
        if (rc == GONN_OK) {
            hipLaunchKernelGGL(add_bias_kernel, dim3(grid_for(tot)), dim3(256), 0, s, out,
                               m->b[3], E, tot);
            rc = herr(hipGetLastError());
        }
    }
    // The new lengths become the cache's once everything has run.
    if (rc == GONN_OK) rc = herr(hipStreamSynchronize(s));
    if (rc == GONN_OK) {
        gonn::kvcache_commit(c, &new_len);
    } else {
        // The enqueued upload may have advanced the device lengths: put the
        // committed ones back. The call's own error is returned; if the
        // restore fails as well, the handle is marked stale, so later calls
        // fail instead of attending positions that were never committed.
        (void)hipStreamSynchronize(s);
        const int rr = gonn::kvcache_restore(c);
        (void)rr;
    }
    return rc;
}

}  // namespace

extern "C" {

size_t gonn_hip_mha_incremental_workspace_bytes(const gonn_mha* m, const gonn_kvcache* c, int T) {
    int B = 0;
    if (!inc_ok(m, c, T, &B)) return 0;
    return inc_layout(m, c, B, T).total;
}

int gonn_hip_mha_forward_incremental_dev(gonn_mha* m, gonn_kvcache* c, const gonn_buf* x,
                                         gonn_buf* out, int T, void* ws, size_t ws_bytes,
                                         void* stream) {
    int B = 0;
    if (!inc_ok(m, c, T, &B) || !x || !out) return GONN_E_INVALID;
    const size_t n = (size_t)B * T * m->E;
    if (x->dtype != GONN_F64 || !x->ptr || x->bytes < n * 8 || out->dtype != GONN_F64 ||
        !out->ptr || out->bytes < n * 8)
        return GONN_E_INVALID;
    const IncLayout L = inc_layout(m, c, B, T);
    if (!ws || ws_bytes < L.total) return GONN_E_WORKSPACE;
    uint8_t* base = (uint8_t*)al((size_t)ws);
    return run_incremental(m, c, (const double*)x->ptr, (double*)out->ptr, B, T, base, L,
                           (hipStream_t)stream);
}

int gonn_hip_mha_create(gonn_mha** out, int E, int H, int kdim, int vdim, const double* Wq,
                        const double* bq, const double* Wk, const double* bk, const double* Wv,
                        const double* bv, const double* Wo, const double* bo) {
    if (!out) return GONN_E_INVALID;
    *out = nullptr;
    if (E <= 0 || H <= 0 || E % H != 0 || kdim <= 0 || vdim <= 0) return GONN_E_INVALID;
    if (!Wq || !Wk || !Wv || !Wo) return GONN_E_INVALID;
    const int D = E / H;
    if (D > 128) return GONN_E_UNSUPPORTED;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    gonn_mha* m = new (std::nothrow) gonn_mha;
    if (!m) return GONN_E_NOMEM;
    m->E = E;
    m->H = H;
    m->D = D;
    m->dp = D <= 64 ? 64 : 128;
    m->kdim = kdim;
    m->vdim = vdim;
    const double* W[4] = {Wq, Wk, Wv, Wo};
    const double* b[4] = {bq, bk, bv, bo};
    const int in[4] = {E, kdim, vdim, E};
    const size_t wall = (size_t)E * (2 * (size_t)E + kdim + vdim);
    if (hipMalloc(&m->W[0], wall * 8) != hipSuccess || hipMalloc(&m->b[0], (size_t)4 * E * 8) != hipSuccess) {
        (void)hipGetLastError();
        mha_release(m);
        delete m;
        return GONN_E_NOMEM;
    }
    for (int i = 1; i < 4; i++) {
        m->W[i] = m->W[i - 1] + (size_t)E * in[i - 1];
        m->b[i] = m->b[i - 1] + E;
    }
    for (int i = 0; i < 4; i++) {
        const size_t wn = (size_t)E * in[i];
        int rc = herr(hipMemcpy(m->W[i], W[i], wn * 8, hipMemcpyHostToDevice));
        // A missing bias is zero (nn.Linear without bias).
        if (!rc) rc = b[i] ? herr(hipMemcpy(m->b[i], b[i], (size_t)E * 8, hipMemcpyHostToDevice))
                           : herr(hipMemset(m->b[i], 0, (size_t)E * 8));
        if (rc) {
            mha_release(m);
            delete m;
            return rc;
        }
    }
    *out = m;
    return GONN_OK;
}

int gonn_hip_mha_free(gonn_mha* m) {
    if (!m) return GONN_OK;
    mha_release(m);
    delete m;
    return GONN_OK;
}

size_t gonn_hip_mha_workspace_bytes(const gonn_mha* m, int B, int Tq, int Tk) {
    if (!shape_ok(m, B, Tq, Tk)) return 0;
    return layout(m, B, Tq, Tk).total;
}

int gonn_hip_mha_forward_f64(gonn_mha* m, const double* q, const double* k, const double* v,
                             double* out, int B, int Tq, int Tk, int causal, const int* kv_len) {
    if (!shape_ok(m, B, Tq, Tk) || !q || !k || !v || !out) return GONN_E_INVALID;
    if (kv_len)
        for (int b = 0; b < B; b++)
            if (kv_len[b] < 0) return GONN_E_INVALID;
    std::lock_guard<std::mutex> lock(m->mu);
    const Layout L = layout(m, B, Tq, Tk);
    // Staging for x (self-attention uploads x once) and the output.
    const size_t nq = (size_t)B * Tq * m->E, nk = (size_t)B * Tk * m->kdim, nv = (size_t)B * Tk * m->vdim;
    const bool kq = k == q && nk == nq, vk = v == k && nv == nk;
    const size_t sq = al(nq * 8), sk = kq ? 0 : al(nk * 8), sv = vk ? 0 : al(nv * 8);
    const size_t need = L.total + sq + sk + sv + al(nq * 8);
    if (m->ws_bytes < need) {
        if (m->ws) (void)hipFree(m->ws);
        m->ws = nullptr;
        m->ws_bytes = 0;
        if (hipMalloc(&m->ws, need) != hipSuccess) {
            (void)hipGetLastError();
            return GONN_E_NOMEM;
        }
        m->ws_bytes = need;
    }
    uint8_t* base = (uint8_t*)m->ws;  // hipMalloc is 256-byte aligned
    double* dq = (double*)(base + L.total);
    double* dk = kq ? dq : (double*)((uint8_t*)dq + sq);
    double* dv = vk ? dk : (double*)((uint8_t*)dq + sq + sk);
    double* dout = (double*)((uint8_t*)dq + sq + sk + sv);
    TRY(herr(hipMemcpy(dq, q, nq * 8, hipMemcpyHostToDevice)));
    if (!kq) TRY(herr(hipMemcpy(dk, k, nk * 8, hipMemcpyHostToDevice)));
    if (!vk) TRY(herr(hipMemcpy(dv, v, nv * 8, hipMemcpyHostToDevice)));
    int* kl = nullptr;
    if (kv_len) {
        kl = (int*)(base + L.kl);
        TRY(herr(hipMemcpy(kl, kv_len, (size_t)B * 4, hipMemcpyHostToDevice)));
    }
    TRY(run_forward(m, dq, dk, dv, dout, B, Tq, Tk, causal, kl, base, L, nullptr));
    return herr(hipMemcpy(out, dout, nq * 8, hipMemcpyDeviceToHost));
}

int gonn_hip_mha_forward_dev(gonn_mha* m, const gonn_buf* q, const gonn_buf* k, const gonn_buf* v,
                             gonn_buf* out, int B, int Tq, int Tk, int causal, const gonn_buf* kv_len,
                             void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(m, B, Tq, Tk) || !q || !k || !v || !out) return GONN_E_INVALID;
    auto ok = [](const gonn_buf* b, size_t n) {
        return b->dtype == GONN_F64 && b->ptr && b->bytes >= n * 8;
    };
    const size_t nq = (size_t)B * Tq * m->E;
    if (!ok(q, nq) || !ok(k, (size_t)B * Tk * m->kdim) || !ok(v, (size_t)B * Tk * m->vdim) ||
        !ok(out, nq))
        return GONN_E_INVALID;
    if (kv_len && kv_len->ptr && (kv_len->dtype != GONN_I32 || kv_len->bytes < (size_t)B * 4))
        return GONN_E_INVALID;
    const Layout L = layout(m, B, Tq, Tk);
    if (!ws || ws_bytes < L.total) return GONN_E_WORKSPACE;
    uint8_t* base = (uint8_t*)al((size_t)ws);
    return run_forward(m, (const double*)q->ptr, (const double*)k->ptr, (const double*)v->ptr,
                       (double*)out->ptr, B, Tq, Tk, causal,
                       kv_len && kv_len->ptr ? (const int*)kv_len->ptr : nullptr, base, L,
                       (hipStream_t)stream);
}

}  // extern "C"
