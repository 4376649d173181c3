// calib.hip -- box calibration for the benchmark (no counterpart in the
// reference): a fixed MFMA loop on constant or random operands, whose rate
// and clock tell a slow box from a slow kernel (and, on random operands,
// give the rate the power limit leaves any bf16 MFMA kernel), and a one-wave
// clock probe that reads the shader clock against the fixed 100 MHz counter
// while other work runs.
#include <hip/hip_runtime.h>

#include <vector>

#include "common.h"
#include "../../include/gonn_hip.h"

namespace gonn {
namespace {

constexpr int kCalibChains = 8;  // independent accumulator chains per wave

// A value in [-1, 1) from a 32-bit integer hash (operand data for the random
// mode; any well-mixed bits do).
__device__ __forceinline__ float hash_unit(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return (float)(x >> 8) * (2.f / 16777216.f) - 1.f;
}

// Each wave issues `iters` rounds of kCalibChains independent
// v_mfma_f32_32x32x16_bf16 (no memory traffic in the loop); the grid holds
// two waves per SIMD. Operands: constant (few toggling bits) or, with
// `random`, distinct uniform [-1, 1) bf16 values per lane and chain, chain
// c multiplying A(c) by B(c + j) in round j of eight -- the switching of
// real data, which sets the clock the power limit allows. Wave 0 of each
// workgroup stores its s_memtime / s_memrealtime spans over the loop.
__global__ __launch_bounds__(256, 2) void mfma_calib_kernel(int iters, int random, float* sink,
                                                            unsigned long long* span) {
    bf16x8 a[kCalibChains], b[kCalibChains];
    const uint32_t id = blockIdx.x * 256u + threadIdx.x;
    for (int c = 0; c < kCalibChains; c++)
        for (int i = 0; i < 8; i++) {
            const uint32_t h = (id * kCalibChains + c) * 16u + i;
            a[c][i] = random ? (bf16)hash_unit(h) : (bf16)(1.0f + 0.0078125f * (threadIdx.x & 7));
            b[c][i] = random ? (bf16)hash_unit(h + 8u) : (bf16)(0.5f);
        }
    f32x16 acc[kCalibChains];
    for (int c = 0; c < kCalibChains; c++) acc[c] = f32x16{};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it += kCalibChains) {
#pragma unroll
        for (int j = 0; j < kCalibChains; j++)
#pragma unroll
            for (int c = 0; c < kCalibChains; c++)
                acc[c] = mfma_bf16(a[c], b[(c + j) % kCalibChains], acc[c]);
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
    for (int c = 0; c < kCalibChains; c++)
        for (int r = 0; r < 16; r++) s += acc[c][r];
    if (s == -1.f) sink[threadIdx.x] = s;  // never true: keeps the loop live
    if (threadIdx.x == 0) {
        span[2 * blockIdx.x] = t1 - t0;
        span[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// One lane reads s_memtime (shader clock) and s_memrealtime (100 MHz) at its
// start and again once `ref_ticks` reference ticks have passed (it sleeps in
// between, so it takes almost no issue slots), and stores both spans.
__global__ void clock_probe_kernel(unsigned long long ref_ticks, unsigned long long* out) {
    if (threadIdx.x != 0) return;
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    unsigned long long r = r0;
    while (r - r0 < ref_ticks) {
        __builtin_amdgcn_s_sleep(32);
        r = __builtin_amdgcn_s_memrealtime();
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    out[0] = t1 - t0;
    out[1] = r - r0;
}

__device__ unsigned long long g_clock_span[2];

int cus_of_current_device(int* cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return GONN_E_NODEVICE;
    if (hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return GONN_E_NODEVICE;
    return GONN_OK;
}

}  // namespace
}  // namespace gonn

extern "C" {

int gonn_hip_calib_mfma(int random, double* tflops, double* ghz) {
    if (!tflops || !ghz) return GONN_E_INVALID;
    *tflops = 0.0;
    *ghz = 0.0;
    int cus = 0;
    const int rc = gonn::cus_of_current_device(&cus);
    if (rc != GONN_OK) return rc;
    const int grid = 2 * cus;  // 4 waves each: two waves per SIMD
    const int iters = 40000;   // a multiple of kCalibChains
    float* sink = nullptr;
    unsigned long long* span = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&sink, 256 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&span, (size_t)grid * 2 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    float ms = 0.f;
    std::vector<unsigned long long> h((size_t)grid * 2, 0);
    if (e == hipSuccess) {
        const int r = random ? 1 : 0;
        hipLaunchKernelGGL(gonn::mfma_calib_kernel, dim3(grid), dim3(256), 0, s, iters / 4, r,
                           sink, span);
        (void)hipEventRecord(e0, s);
        hipLaunchKernelGGL(gonn::mfma_calib_kernel, dim3(grid), dim3(256), 0, s, iters, r, sink,
                           span);
        (void)hipEventRecord(e1, s);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e == hipSuccess)
            e = hipMemcpy(h.data(), span, h.size() * sizeof(unsigned long long),
                          hipMemcpyDeviceToHost);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (sink) (void)hipFree(sink);
    if (span) (void)hipFree(span);
    if (e != hipSuccess) return (int)e;
    const double flop = (double)grid * 4 * iters * gonn::kCalibChains * 32.0 * 32.0 * 16.0 * 2.0;
    *tflops = ms > 0.f ? flop / (ms * 1e-3) / 1e12 : 0.0;
    double sum = 0.0;
    int n = 0;
    for (int i = 0; i < grid; i++)
        if (h[2 * i + 1]) {
            sum += (double)h[2 * i] / ((double)h[2 * i + 1] * 10.0);  // ticks of 10 ns
            n++;
        }
    *ghz = n ? sum / n : 0.0;
    return GONN_OK;
}

int gonn_hip_calib_clock_start(double ms, void* stream) {
    if (!(ms > 0.0) || ms > 60000.0) return GONN_E_INVALID;
    unsigned long long* out = nullptr;
    hipError_t e = hipGetSymbolAddress((void**)&out, HIP_SYMBOL(gonn::g_clock_span));
    if (e != hipSuccess) return (int)e;
    const unsigned long long ticks = (unsigned long long)(ms * 1e5);  // 100 MHz
    hipLaunchKernelGGL(gonn::clock_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, ticks,
                       out);
    return (int)hipGetLastError();
}

int gonn_hip_calib_clock_read(double* ghz) {
    if (!ghz) return GONN_E_INVALID;
    unsigned long long span[2] = {0, 0};
    const hipError_t e = hipMemcpyFromSymbol(span, HIP_SYMBOL(gonn::g_clock_span), sizeof(span));
    if (e != hipSuccess) return (int)e;
    *ghz = span[1] ? (double)span[0] / ((double)span[1] * 10.0) : 0.0;  // ticks of 10 ns
    return GONN_OK;
}

}  // extern "C"
