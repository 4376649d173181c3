// gemm.hip -- fp64 GEMM of the HIP backend: the counterpart of the CUDA
// backend's gonn_gemm (backend/cuda/gonn_cuda.cu:147-177) behind
// backend.Backend.Gemm (backend/backend.go:61-78), used by the MHA
// projections (nn/linear.go:40-59) around the attention core.
//
// Row-major batched C = op(A) op(B) with op(A) (m,k), op(B) (k,n), C (m,n).
// rocBLAS is column-major; a row-major matrix is its own transpose viewed
// column-major, so the call computes C^T = op(B)^T op(A)^T with the stored
// row-major column counts as leading dimensions. fp64 runs on the fp64
// MFMA path of gfx950 inside rocBLAS (a plain library GEMM).
//
// Skinny case (batch 1, C = A W^T with W row-major (n, k), m <= 256 as
// skinny_ok bounds it, k a multiple of 128: the projections of a decoding
// step, m = B x T rows against E x E weights): a kernel of its own. rocBLAS takes about 445 us
// for m = 64, k = 4096 whatever n (4096 or 12288; 4.8 and 14 TFLOP/s),
// the time of a few output tiles walking the whole k range serially; the
// whole of that GEMM is 2.1 GFLOP (27 us at the 78.6 TFLOP/s fp64 peak).
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/gonn_hip.h"

namespace {

std::mutex g_mu;                  // guards the handle and the host workspace
rocblas_handle g_handle = nullptr;
void* g_ws[3] = {nullptr, nullptr, nullptr};
size_t g_ws_bytes[3] = {0, 0, 0};

int herr(hipError_t e) { return e == hipSuccess ? GONN_OK : (int)e; }

bool fail_alloc_injected() {
    const char* e = std::getenv("GONN_HIP_FAIL_ALLOC");
    return e && e[0] == '1';
}

int ensure_handle() {
    if (g_handle) return GONN_OK;
    if (rocblas_create_handle(&g_handle) != rocblas_status_success) {
        g_handle = nullptr;
        return GONN_E_BLAS;
    }
    return GONN_OK;
}

int ws_reserve(int i, size_t bytes) {
    if (g_ws_bytes[i] >= bytes) return GONN_OK;
    if (fail_alloc_injected()) return GONN_E_INJECTED;
    if (g_ws[i]) (void)hipFree(g_ws[i]);
    g_ws[i] = nullptr;
    g_ws_bytes[i] = 0;
    if (hipMalloc(&g_ws[i], bytes) != hipSuccess) {
        (void)hipGetLastError();
        g_ws[i] = nullptr;
        return GONN_E_NOMEM;
    }
    g_ws_bytes[i] = bytes;
    return GONN_OK;
}

bool args_ok(int batch, int m, int k, int n) {
    return batch >= 0 && m >= 0 && k >= 0 && n >= 0 &&
           (double)batch * m * k < 9.0e15 && (double)batch * k * n < 9.0e15 &&
           (double)batch * m * n < 9.0e15;
}

// C = 0 for an empty inner dimension. A kernel rather than a memset node, so
// that a caller capturing the stream into a graph replays it correctly.
__global__ void zero_kernel(double* __restrict__ c, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) c[i] = 0.0;
}

// ---- skinny C = A W^T (m <= 256) on v_mfma_f64_16x16x4_f64 ----
// One workgroup of 4 waves per 16 NW output columns and 64 rows (a row chunk);
// wave w takes the k range
// [w k/4, (w+1) k/4) and all (up to 4) 16-row tiles of A, and the 4 waves'
// partial tiles are summed through LDS in wave order (deterministic, no
// global workspace). MFMA k-slots are free to map to any k as long as A and
// B agree: lane group q = lane / 16 takes 8 consecutive k of each 32-k chunk,
// so every lane loads 64 contiguous bytes of its A row and its W row (four
// 16-byte loads each), and the next chunk's loads are issued before the
// current chunk's 32 MFMAs. A variant takes 32 output columns per
// workgroup (NW = 2) with 16 k per lane group and chunk. A row chunk
// (64 x k, 2 MB at k = 4096) is re-read from L2 by every workgroup of the
// chunk. The row chunks of one
// column tile get block indices 8 apart, so they run on one XCD and read
// that tile of W from its L2: W streams from HBM once.
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
constexpr int kSkinnyMaxRows = 256;

template <int NW, int SKS>
__global__ __launch_bounds__(256, 2) void gemm_f64_skinny_nt(const double* __restrict__ A,
                                                             const double* __restrict__ W,
                                                             double* __restrict__ C, int m, int k,
                                                             int n) {
    constexpr int CHUNK = 4 * SKS;  // k per chunk
    constexpr int H = SKS / 2;      // 16-byte loads per row per chunk
    __shared__ double red[4][NW * 4 * 4 * 64];  // [wave][(j, mt, r, lane)]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = lane & 15, q = lane >> 4;
    // Block -> (column tile, row chunk): with 8 | column tiles, block L runs
    // on XCD L % 8 and the nm chunks of tile 8 (L / 8 / nm) + L % 8 share it.
    const int nm = (m + 63) / 64, ntile = (n + 16 * NW - 1) / (16 * NW), L = blockIdx.x;
    int tile, chunk;
    if (ntile % 8 == 0) {
        tile = (L >> 3) / nm * 8 + (L & 7);
        chunk = (L >> 3) % nm;
    } else {
        tile = L / nm;
        chunk = L % nm;
    }
    A += (size_t)chunk * 64 * k;
    C += (size_t)chunk * 64 * n;
    m = m - chunk * 64 < 64 ? m - chunk * 64 : 64;
    const int n0 = tile * 16 * NW;
    const double* wrow[NW];
    bool wlive[NW];
    for (int j = 0; j < NW; j++) {
        const int col = n0 + 16 * j + i;
        wlive[j] = col < n;
        wrow[j] = W + (size_t)(wlive[j] ? col : 0) * k;
    }
    const double* arow[4];
    bool live[4];
    for (int mt = 0; mt < 4; mt++) {
        const int r = 16 * mt + i;
        live[mt] = r < m;
        arow[mt] = A + (size_t)(live[mt] ? r : 0) * k;
    }
    const int kw = k / 4, kb = wave * kw;
    f64x4 acc[NW][4];
    for (int j = 0; j < NW; j++)
        for (int mt = 0; mt < 4; mt++) acc[j][mt] = f64x4{0.0, 0.0, 0.0, 0.0};
    // Two register buffers (X, Y) of one chunk each; the chunk loop is
    // unrolled by two so that no buffer is indexed at run time.
    f64x2 wX[NW][H], aX[4][H], wY[NW][H], aY[4][H];
    auto load = [&](f64x2 (*wv)[H], f64x2 (*av)[H], int c0) {
        const int kk = c0 + q * SKS;
        for (int j = 0; j < NW; j++)
            for (int h = 0; h < H; h++)
                wv[j][h] = wlive[j] ? *(const f64x2*)(wrow[j] + kk + 2 * h) : f64x2{0.0, 0.0};
        for (int mt = 0; mt < 4; mt++)
            for (int h = 0; h < H; h++)
                av[mt][h] = live[mt] ? *(const f64x2*)(arow[mt] + kk + 2 * h) : f64x2{0.0, 0.0};
    };
    auto compute = [&](const f64x2 (*wv)[H], const f64x2 (*av)[H]) {
        for (int st = 0; st < SKS; st++)
            for (int j = 0; j < NW; j++)
                for (int mt = 0; mt < 4; mt++)
                    if (16 * mt < m)  // uniform: row tiles past m are skipped
                        acc[j][mt] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                            av[mt][st >> 1][st & 1], wv[j][st >> 1][st & 1], acc[j][mt], 0, 0, 0);
    };
    const int nch = kw / CHUNK;  // >= 1 (k % 128 == 0)
    load(wX, aX, kb);
    for (int c = 0; c < nch; c += 2) {
        if (c + 1 < nch) load(wY, aY, kb + (c + 1) * CHUNK);
        compute(wX, aX);
        if (c + 1 >= nch) break;
        if (c + 2 < nch) load(wX, aX, kb + (c + 2) * CHUNK);
        compute(wY, aY);
    }
    for (int j = 0; j < NW; j++)
        for (int mt = 0; mt < 4; mt++)
            for (int r = 0; r < 4; r++)
                red[wave][((j * 4 + mt) * 4 + r) * 64 + lane] = acc[j][mt][r];
    __syncthreads();
    // Output element e = (j, mt, r, lane): row 16 mt + 4 r + lane / 16,
    // column n0 + 16 j + lane % 16 (the f64 16x16 accumulator layout, probed
    // on gfx950: register r of lane l holds row 4 r + l / 16, column l % 16).
    for (int e = threadIdx.x; e < NW * 4 * 4 * 64; e += 256) {
        const int j = e >> 10, mt = (e >> 8) & 3, r = (e >> 6) & 3, ln = e & 63;
        const int row = 16 * mt + 4 * r + (ln >> 4), cc = n0 + 16 * j + (ln & 15);
        if (row < m && cc < n)
            C[(size_t)row * n + cc] = ((red[0][e] + red[1][e]) + red[2][e]) + red[3][e];
    }
}

// Shapes the skinny kernel takes: every m <= 64 (rocBLAS spends ~445 us on
// any such call at k = 4096, the skinny kernel 27-32 TFLOP/s), and m <= 256
// while the product is at most 16 GFLOP (the skinny kernel's 35-47 TFLOP/s
// against rocBLAS's ~445 us floor and 57 TFLOP/s beyond it, measured at
// k = 4096 on one MI355X: 128 x 12288 382 against 448 us, 256 x 4096 184
// against 443 us, 256 x 12288 566 against 452 us).
bool skinny_ok(int batch, int m, int k, int n, int transA, int transB) {
    if (batch != 1 || transA || !transB || m < 1 || k < 128 || k % 128 != 0 || n < 1) return false;
    return m <= 64 || (m <= kSkinnyMaxRows && 2.0 * m * n * k <= 1.6e10);
}

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev] &&
        hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    return cus[dev];
}

int run_skinny(const double* dA, const double* dB, double* dC, int m, int k, int n,
               hipStream_t s) {
    // 32 columns per workgroup halve the re-reads of A where that still
    // leaves a workgroup per CU (128 x 4096: 111 against 154 us; 64 x 4096,
    // 128 workgroups: 106 against 78 us).
    const long long wide = (long long)((n + 31) / 32) * ((m + 63) / 64);
    const int nw = wide >= device_cus() ? 2 : 1;
    const unsigned blocks = (unsigned)((n + 16 * nw - 1) / (16 * nw)) * (unsigned)((m + 63) / 64);
    if (nw == 2)
        hipLaunchKernelGGL((gemm_f64_skinny_nt<2, 4>), dim3(blocks), dim3(256), 0, s, dA, dB, dC, m,
                           k, n);
    else
        hipLaunchKernelGGL((gemm_f64_skinny_nt<1, 8>), dim3(blocks), dim3(256), 0, s, dA, dB, dC, m,
                           k, n);
    return herr(hipGetLastError());
}

// Caller holds g_mu and the handle exists. GONN_HIP_GEMM=rocblas keeps the
// skinny shapes on rocBLAS too.
int run_gemm(const double* dA, const double* dB, double* dC, int batch, int m, int k, int n,
             int transA, int transB, hipStream_t s) {
    const char* e = std::getenv("GONN_HIP_GEMM");
    if (skinny_ok(batch, m, k, n, transA, transB) && !(e && std::strcmp(e, "rocblas") == 0))
        return run_skinny(dA, dB, dC, m, k, n, s);
    if (rocblas_set_stream(g_handle, s) != rocblas_status_success) return GONN_E_BLAS;
    const double alpha = 1.0, beta = 0.0;
    const rocblas_operation opA = transA ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation opB = transB ? rocblas_operation_transpose : rocblas_operation_none;
    const int lda = transA ? m : k;  // stored row-major column counts
    const int ldb = transB ? k : n;
    const rocblas_status st = rocblas_dgemm_strided_batched(
        g_handle, opB, opA, n, m, k, &alpha, dB, ldb, (rocblas_stride)k * n, dA, lda,
        (rocblas_stride)m * k, &beta, dC, n, (rocblas_stride)m * n, batch);
    return st == rocblas_status_success ? GONN_OK : GONN_E_BLAS;
}

}  // namespace

extern "C" {

int gonn_hip_gemm_f64(const double* A, const double* B, double* C, int batch, int m, int k, int n,
                      int transA, int transB) {
    if (!args_ok(batch, m, k, n)) return GONN_E_INVALID;
    const size_t an = (size_t)batch * m * k, bn = (size_t)batch * k * n, cn = (size_t)batch * m * n;
    if (cn == 0) return GONN_OK;
    if (!C || (an && !A) || (bn && !B)) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    if (k == 0) {  // empty inner dimension: C = 0
        for (size_t i = 0; i < cn; i++) C[i] = 0.0;
        return GONN_OK;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    int rc = ensure_handle();
    if (rc) return rc;
    if ((rc = ws_reserve(0, an * 8)) || (rc = ws_reserve(1, bn * 8)) || (rc = ws_reserve(2, cn * 8)))
        return rc;
    double* dA = (double*)g_ws[0];
    double* dB = (double*)g_ws[1];
    double* dC = (double*)g_ws[2];
    if ((rc = herr(hipMemcpy(dA, A, an * 8, hipMemcpyHostToDevice)))) return rc;
    if ((rc = herr(hipMemcpy(dB, B, bn * 8, hipMemcpyHostToDevice)))) return rc;
    if ((rc = run_gemm(dA, dB, dC, batch, m, k, n, transA, transB, nullptr))) return rc;
    return herr(hipMemcpy(C, dC, cn * 8, hipMemcpyDeviceToHost));
}

int gonn_hip_gemm_f64_dev(const gonn_buf* A, const gonn_buf* B, gonn_buf* C, int batch, int m,
                          int k, int n, int transA, int transB, void* stream) {
    if (!A || !B || !C || !args_ok(batch, m, k, n)) return GONN_E_INVALID;
    const size_t an = (size_t)batch * m * k, bn = (size_t)batch * k * n, cn = (size_t)batch * m * n;
    if (A->dtype != GONN_F64 || B->dtype != GONN_F64 || C->dtype != GONN_F64) return GONN_E_INVALID;
    if ((an && (!A->ptr || A->bytes < an * 8)) || (bn && (!B->ptr || B->bytes < bn * 8)) ||
        (cn && (!C->ptr || C->bytes < cn * 8)))
        return GONN_E_INVALID;
    if (cn == 0) return GONN_OK;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    hipStream_t s = (hipStream_t)stream;
    if (k == 0) {
        const size_t blocks = std::min<size_t>((cn + 255) / 256, 4096);
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (double*)C->ptr, cn);
        return herr(hipGetLastError());
    }
    std::lock_guard<std::mutex> lock(g_mu);
    const int rc = ensure_handle();
    if (rc) return rc;
    return run_gemm((const double*)A->ptr, (const double*)B->ptr, (double*)C->ptr, batch, m, k, n,
                    transA, transB, s);
}

}  // extern "C"
