// util.hip -- conversion and fill kernels used at the ABI boundary, and the
// MFMA layout self-test.
#include <vector>

#include "common.h"
#include "kernels.h"

namespace gonn {

__global__ void convert_from_f64_kernel(const double* __restrict__ src, void* __restrict__ dst,
                                        int dst_bf16, size_t rows, int d, int dpad) {
    const size_t n = rows * (size_t)dpad;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / dpad;
        const int c = (int)(i - r * dpad);
        const double x = c < d ? src[r * d + c] : 0.0;
        if (dst_bf16)
            ((bf16*)dst)[i] = to_bf16((float)x);
        else
            ((float*)dst)[i] = (float)x;
    }
}

__global__ void convert_to_f64_kernel(const void* __restrict__ src, int src_bf16,
                                      double* __restrict__ dst, size_t rows, int d, int dpad) {
    const size_t n = rows * (size_t)d;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / d;
        const int c = (int)(i - r * d);
        const size_t j = r * dpad + c;
        dst[i] = src_bf16 ? (double)bf16_to_f32(((const uint16_t*)src)[j])
                          : (double)((const float*)src)[j];
    }
}

__global__ void fill_zero_kernel(uint32_t* __restrict__ dst, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = 0u;
}

static unsigned grid_for(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    if (g == 0) g = 1;
    return (unsigned)g;
}

hipError_t launch_convert_from_f64(const double* src, void* dst, int dst_bf16, size_t rows, int d,
                                   int dpad, hipStream_t s) {
    convert_from_f64_kernel<<<grid_for(rows * dpad), 256, 0, s>>>(src, dst, dst_bf16, rows, d, dpad);
    return hipGetLastError();
}

hipError_t launch_convert_to_f64(const void* src, int src_bf16, double* dst, size_t rows, int d,
                                 int dpad, hipStream_t s) {
    convert_to_f64_kernel<<<grid_for(rows * d), 256, 0, s>>>(src, src_bf16, dst, rows, d, dpad);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t s) {
    // bytes is a multiple of 4 for every buffer this library clears
    const size_t n = bytes / 4;
    fill_zero_kernel<<<grid_for(n), 256, 0, s>>>((uint32_t*)dst, n);
    return hipGetLastError();
}

// ---- MFMA layout self-test -------------------------------------------------
// A(32x16), B(16x32) hold small integers (exact in bf16 and fp32). Lane l loads
// A[l%32][8(l/32)+j] and B[8(l/32)+j][l%32], j = 0..7, runs one bf16 MFMA and
// stores its 16 accumulators; likewise one fp32 MFMA with K = 2.
__global__ void selftest_kernel(const float* A, const float* B, float* out_bf16, float* out_f32) {
    const int l = threadIdx.x, g = l >> 5, n = l & 31;
    bf16x8 a, b;
    for (int j = 0; j < 8; j++) {
        a[j] = to_bf16(A[n * 16 + 8 * g + j]);
        b[j] = to_bf16(B[(8 * g + j) * 32 + n]);
    }
    f32x16 c = mfma_bf16(a, b, f32x16{});
    for (int r = 0; r < 16; r++) out_bf16[l * 16 + r] = c[r];
    // fp32: A2(32x2) = A[:, 0:2], B2(2x32) = B[0:2, :]
    f32x16 c2 = mfma_f32(A[n * 16 + g], B[g * 32 + n], f32x16{});
    for (int r = 0; r < 16; r++) out_f32[l * 16 + r] = c2[r];
}

int selftest_mfma() {
    std::vector<float> A(32 * 16), B(16 * 32);
    for (int i = 0; i < 32; i++)
        for (int k = 0; k < 16; k++) A[i * 16 + k] = (float)((i * 3 + k * 5) % 7 - 3);
    for (int k = 0; k < 16; k++)
        for (int j = 0; j < 32; j++) B[k * 32 + j] = (float)((k * 2 + j * 3) % 5 - 2);
    float *dA, *dB, *d1, *d2;
    if (hipMalloc(&dA, A.size() * 4) || hipMalloc(&dB, B.size() * 4) || hipMalloc(&d1, 1024 * 4) ||
        hipMalloc(&d2, 1024 * 4))
        return -4;
    (void)hipMemcpy(dA, A.data(), A.size() * 4, hipMemcpyHostToDevice);
    (void)hipMemcpy(dB, B.data(), B.size() * 4, hipMemcpyHostToDevice);
    selftest_kernel<<<1, 64>>>(dA, dB, d1, d2);
    std::vector<float> o1(1024), o2(1024);
    hipError_t e = hipMemcpy(o1.data(), d1, 1024 * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(o2.data(), d2, 1024 * 4, hipMemcpyDeviceToHost);
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(d1);
    (void)hipFree(d2);
    if (e != hipSuccess) return (int)e;
    int bad = 0;
    for (int l = 0; l < 64; l++)
        for (int r = 0; r < 16; r++) {
            const int row = 8 * (r / 4) + 4 * (l / 32) + (r % 4), col = l % 32;
            float ref = 0.f, ref2 = 0.f;
            for (int k = 0; k < 16; k++) ref += A[row * 16 + k] * B[k * 32 + col];
            for (int k = 0; k < 2; k++) ref2 += A[row * 16 + k] * B[k * 32 + col];
            if (o1[l * 16 + r] != ref) bad++;
            if (o2[l * 16 + r] != ref2) bad++;
        }
    return bad;
}

}  // namespace gonn
