// kernels.h -- launch interface between the C ABI (api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace gonn {

struct FwdParams {
    const void* q;  // (BH,Sq,D) f32 or bf16
    const void* k;  // bf16 mode: Kb (BH,Skp,D) bf16; fp32 mode: K (BH,Sk,D) f32
    const void* v;  // bf16 mode: Vt (BH,D,Skp) bf16; fp32 mode: V (BH,Sk,D) f32
    float* o;       // (BH,Sq,D)
    float* lse;     // (BH,Sq) or null
    int BH, Sq, Sk, Skp, nqb;
    float scale_log2;  // |scale| * log2(e)
    float scale_abs;   // |scale|
    float qsign;       // sign(scale) (Q is negated for a negative scale)
};

struct DecodeParams {
    const void* q;     // (B,H,D) f32 or bf16
    const void* kc;    // (B,H,Lmax,D) bf16
    const void* vc;    // (B,H,Lmax,D) bf16
    const int* kv_len; // [B]
    float* o;          // (B,H,D)
    float* part_o;     // (B*H, nsplit, D) unnormalised partial outputs
    float* part_ml;    // (B*H, nsplit, 2) partial (max, sum) in log2 units
    int B, H, Lmax, nsplit, split_keys;
    float scale_log2;  // scale * log2(e) (any sign)
};

struct BwdParams {
    // bf16 mode operands live in the workspace (see api.hip); fp32 mode uses
    // the caller's buffers directly.
    const void* q;    // Q   (BH,S,D)
    const void* k;    // K   (BH,S,D)
    const void* v;    // V   (BH,S,D)
    const void* qt;   // Q^T (BH,D,Sp) key-permuted, bf16 mode only
    const void* kt;   // K^T (BH,D,Sp) key-permuted, bf16 mode only
    const void* dot;  // dO^T (BH,D,Sp) key-permuted, bf16 mode only
    const void* dO;   // dO  (BH,S,D)
    const float* lse; // (BH,S) natural log
    const float* delta; // (BH,S) rowsum(dO * O)
    float* dq;        // (BH,S,D)
    float* dk;
    float* dv;
    int BH, S, Sp;
    float scale;       // signed scale
    float scale_log2;  // scale * log2(e)
};

hipError_t launch_pack_kv(const void* K, const void* V, int in_bf16, void* Kb, void* Vt, int BH,
                          int Sk, int Skp, int D, hipStream_t s);
hipError_t launch_fwd(const FwdParams& p, int mode, int D, int causal, int q_bf16,
                      hipStream_t s);
hipError_t launch_decode_split(const DecodeParams& p, int D, int q_bf16, hipStream_t s);
hipError_t launch_decode_combine(const DecodeParams& p, int D, hipStream_t s);
hipError_t launch_bwd(const BwdParams& p, int mode, int D, int causal, const float* O,
                      void* ws, hipStream_t s);
size_t bwd_workspace_bytes(int mode, int BH, int S, int D);

// f64 <-> f32/bf16 conversion with optional head-dim padding:
// dst (rows, dpad) <- src (rows, d); pad columns are zero.
hipError_t launch_convert_from_f64(const double* src, void* dst, int dst_bf16, size_t rows,
                                   int d, int dpad, hipStream_t s);
hipError_t launch_convert_to_f64(const void* src, int src_bf16, double* dst, size_t rows, int d,
                                 int dpad, hipStream_t s);
hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t s);

int selftest_mfma();

}  // namespace gonn
