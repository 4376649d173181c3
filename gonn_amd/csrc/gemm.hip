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
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstdlib>
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

// Caller holds g_mu and the handle exists.
int run_gemm(const double* dA, const double* dB, double* dC, int batch, int m, int k, int n,
             int transA, int transB, hipStream_t s) {
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
