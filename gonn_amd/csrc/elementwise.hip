// elementwise.hip -- fp64 elementwise ops of the HIP backend: the counterpart
// of backend.Elementwiser (backend/backend.go:80-92) and of the CUDA
// backend's gonn_unary / gonn_binary (backend/cuda/gonn_cuda.h:39-43,
// gonn_cuda.cu:82-107). The op kinds and their numeric values are the
// reference's append-only ABI (backend.go:26-58).
//
// HBM-bound streaming: each thread moves 16 bytes per operand per iteration
// (two doubles, one global_load_dwordx4), in a grid-stride loop over a grid
// sized to fill every CU a few times; a ragged tail is handled by the
// thread that owns it. Math is fp64 device libm (ocml).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "../../include/gonn_hip.h"

namespace {

template <int K>
__device__ __forceinline__ double unary_op(double x) {
    if constexpr (K == GONN_UN_RELU) return x > 0.0 ? x : 0.0;
    else if constexpr (K == GONN_UN_SIGMOID) return 1.0 / (1.0 + exp(-x));
    else if constexpr (K == GONN_UN_TANH) return tanh(x);
    else if constexpr (K == GONN_UN_EXP) return exp(x);
    else if constexpr (K == GONN_UN_LOG) return log(x);
    // tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
    else if constexpr (K == GONN_UN_GELU)
        return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
    else if constexpr (K == GONN_UN_SILU) return x / (1.0 + exp(-x));
    // erf form: 0.5 x (1 + erf(x / sqrt(2)))
    else return 0.5 * x * (1.0 + erf(x * 0.7071067811865476));
}

template <int K>
__device__ __forceinline__ double binary_op(double a, double b) {
    if constexpr (K == GONN_BIN_ADD) return a + b;
    else if constexpr (K == GONN_BIN_SUB) return a - b;
    else if constexpr (K == GONN_BIN_MUL) return a * b;
    else return a / b;
}

typedef double f64x2 __attribute__((ext_vector_type(2)));

template <int K>
__global__ __launch_bounds__(256) void unary_kernel(const double* __restrict__ a,
                                                    double* __restrict__ c, size_t n) {
    const size_t n2 = n / 2, stride = (size_t)gridDim.x * blockDim.x;
    const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (size_t i = t0; i < n2; i += stride) {
        const f64x2 x = *(const f64x2*)(a + 2 * i);
        f64x2 y;
        y[0] = unary_op<K>(x[0]);
        y[1] = unary_op<K>(x[1]);
        *(f64x2*)(c + 2 * i) = y;
    }
    if ((n & 1) && t0 == 0) c[n - 1] = unary_op<K>(a[n - 1]);
}

template <int K>
__global__ __launch_bounds__(256) void binary_kernel(const double* __restrict__ a,
                                                     const double* __restrict__ b,
                                                     double* __restrict__ c, size_t n) {
    const size_t n2 = n / 2, stride = (size_t)gridDim.x * blockDim.x;
    const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (size_t i = t0; i < n2; i += stride) {
        const f64x2 x = *(const f64x2*)(a + 2 * i), y = *(const f64x2*)(b + 2 * i);
        f64x2 z;
        z[0] = binary_op<K>(x[0], y[0]);
        z[1] = binary_op<K>(x[1], y[1]);
        *(f64x2*)(c + 2 * i) = z;
    }
    if ((n & 1) && t0 == 0) c[n - 1] = binary_op<K>(a[n - 1], b[n - 1]);
}

int herr(hipError_t e) { return e == hipSuccess ? GONN_OK : (int)e; }

// Workgroups for n elements: one pair per thread up to 8 workgroups per CU
// (2048 on 256 CUs), then grid-stride.
unsigned grid_for(size_t n) {
    const size_t want = (n / 2 + 255) / 256;
    return (unsigned)std::max<size_t>(1, std::min<size_t>(want, 2048));
}

int launch_unary(int kind, const double* a, double* c, size_t n, hipStream_t s) {
    const dim3 grid(grid_for(n)), block(256);
    switch (kind) {
        case GONN_UN_RELU: unary_kernel<GONN_UN_RELU><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_SIGMOID: unary_kernel<GONN_UN_SIGMOID><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_TANH: unary_kernel<GONN_UN_TANH><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_EXP: unary_kernel<GONN_UN_EXP><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_LOG: unary_kernel<GONN_UN_LOG><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_GELU: unary_kernel<GONN_UN_GELU><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_SILU: unary_kernel<GONN_UN_SILU><<<grid, block, 0, s>>>(a, c, n); break;
        case GONN_UN_GELU_EXACT:
            unary_kernel<GONN_UN_GELU_EXACT><<<grid, block, 0, s>>>(a, c, n);
            break;
        default: return GONN_E_INVALID;
    }
    return herr(hipGetLastError());
}

int launch_binary(int kind, const double* a, const double* b, double* c, size_t n, hipStream_t s) {
    const dim3 grid(grid_for(n)), block(256);
    switch (kind) {
        case GONN_BIN_ADD: binary_kernel<GONN_BIN_ADD><<<grid, block, 0, s>>>(a, b, c, n); break;
        case GONN_BIN_SUB: binary_kernel<GONN_BIN_SUB><<<grid, block, 0, s>>>(a, b, c, n); break;
        case GONN_BIN_MUL: binary_kernel<GONN_BIN_MUL><<<grid, block, 0, s>>>(a, b, c, n); break;
        case GONN_BIN_DIV: binary_kernel<GONN_BIN_DIV><<<grid, block, 0, s>>>(a, b, c, n); break;
        default: return GONN_E_INVALID;
    }
    return herr(hipGetLastError());
}

bool unary_kind_ok(int k) { return k >= GONN_UN_RELU && k <= GONN_UN_GELU_EXACT; }
bool binary_kind_ok(int k) { return k >= GONN_BIN_ADD && k <= GONN_BIN_DIV; }

// Staging for the host entry points: a grow-only device workspace behind one
// mutex (the reference's Go wrapper holds its backend mutex around the same
// calls, cuda.go:72-106).
std::mutex g_mu;
void* g_ws[3] = {nullptr, nullptr, nullptr};
size_t g_ws_bytes[3] = {0, 0, 0};

int ws_reserve(int i, size_t bytes) {
    if (g_ws_bytes[i] >= bytes) return GONN_OK;
    if (g_ws[i]) (void)hipFree(g_ws[i]);
    g_ws[i] = nullptr;
    g_ws_bytes[i] = 0;
    if (hipMalloc(&g_ws[i], bytes) != hipSuccess) {
        (void)hipGetLastError();
        return GONN_E_NOMEM;
    }
    g_ws_bytes[i] = bytes;
    return GONN_OK;
}

bool buf_ok(const gonn_buf* b, size_t n) {
    return b && b->dtype == GONN_F64 && (n == 0 || (b->ptr && b->bytes >= n * sizeof(double)));
}

}  // namespace

extern "C" {

int gonn_hip_unary_f64(int kind, const double* A, double* C, long n) {
    if (!unary_kind_ok(kind) || n < 0) return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    if (!A || !C) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    const size_t bytes = (size_t)n * sizeof(double);
    std::lock_guard<std::mutex> lock(g_mu);
    int rc;
    if ((rc = ws_reserve(0, bytes)) || (rc = ws_reserve(2, bytes))) return rc;
    double* dA = (double*)g_ws[0];
    double* dC = (double*)g_ws[2];
    if ((rc = herr(hipMemcpy(dA, A, bytes, hipMemcpyHostToDevice)))) return rc;
    if ((rc = launch_unary(kind, dA, dC, (size_t)n, nullptr))) return rc;
    return herr(hipMemcpy(C, dC, bytes, hipMemcpyDeviceToHost));
}

int gonn_hip_binary_f64(int kind, const double* A, const double* B, double* C, long n) {
    if (!binary_kind_ok(kind) || n < 0) return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    if (!A || !B || !C) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    const size_t bytes = (size_t)n * sizeof(double);
    std::lock_guard<std::mutex> lock(g_mu);
    int rc;
    if ((rc = ws_reserve(0, bytes)) || (rc = ws_reserve(1, bytes)) || (rc = ws_reserve(2, bytes)))
        return rc;
    double* dA = (double*)g_ws[0];
    double* dB = (double*)g_ws[1];
    double* dC = (double*)g_ws[2];
    if ((rc = herr(hipMemcpy(dA, A, bytes, hipMemcpyHostToDevice)))) return rc;
    if ((rc = herr(hipMemcpy(dB, B, bytes, hipMemcpyHostToDevice)))) return rc;
    if ((rc = launch_binary(kind, dA, dB, dC, (size_t)n, nullptr))) return rc;
    return herr(hipMemcpy(C, dC, bytes, hipMemcpyDeviceToHost));
}

int gonn_hip_unary_f64_dev(int kind, const gonn_buf* A, gonn_buf* C, long n, void* stream) {
    if (!unary_kind_ok(kind) || n < 0 || !buf_ok(A, (size_t)n) || !buf_ok(C, (size_t)n))
        return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    if (((uintptr_t)A->ptr | (uintptr_t)C->ptr) & 15) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    return launch_unary(kind, (const double*)A->ptr, (double*)C->ptr, (size_t)n,
                        (hipStream_t)stream);
}

int gonn_hip_binary_f64_dev(int kind, const gonn_buf* A, const gonn_buf* B, gonn_buf* C, long n,
                            void* stream) {
    if (!binary_kind_ok(kind) || n < 0 || !buf_ok(A, (size_t)n) || !buf_ok(B, (size_t)n) ||
        !buf_ok(C, (size_t)n))
        return GONN_E_INVALID;
    if (n == 0) return GONN_OK;
    if (((uintptr_t)A->ptr | (uintptr_t)B->ptr | (uintptr_t)C->ptr) & 15) return GONN_E_INVALID;
    if (!gonn_hip_available()) return GONN_E_NODEVICE;
    return launch_binary(kind, (const double*)A->ptr, (const double*)B->ptr, (double*)C->ptr,
                         (size_t)n, (hipStream_t)stream);
}

}  // extern "C"
