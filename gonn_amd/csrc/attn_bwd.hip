// attn_bwd.hip -- flash-attention backward (dQ, dK, dV) for gfx950 (MI355X).
//
// Replaces the reference's fp64 one-thread-per-query-row backward
// flash_attn_bwd_f64_kernel (backend/cuda/gonn_cuda.cu:341-383) and follows
// its identities (gonn_cuda.cu:333-340), with s = scale * q.k and
// P_ij = exp(s_ij - L_i):
//   D_i  = dO_i . O_i
//   dP_ij = dO_i . v_j
//   dS_ij = P_ij (dP_ij - D_i)
//   dQ_i = scale * sum_j dS_ij k_j      dK_j = scale * sum_i dS_ij q_i
//   dV_j = sum_i P_ij dO_i
// The reference accumulates dK and dV with fp64 atomics; here every output
// element is owned by exactly one workgroup, so results are deterministic:
//   prep  lse2 = L * log2(e) (+inf on pad rows, so padded queries get P = 0)
//         and D (0 on pad rows), one 16-lane row per query;
//   dkdv  one workgroup per 128-key block of one (b,h) slice, 32 keys per
//         wave. K and V of the block stay in VGPRs; Q / dO tiles (and their
//         transposes in bf16 mode) stream through double-buffered LDS. Per
//         query tile: S = Q K^T and dP = dO V^T on MFMA with one KEY per lane
//         (the 16 accumulators of a lane are 16 queries), P and dS in
//         registers, then dV^T += dO^T P and dK^T += Q^T dS on MFMA straight
//         from those registers;
//   dq    one workgroup per 128-query block, 32 queries per wave (the forward
//         kernel's shape): S^T = K Q^T and dP^T = V dO^T with one QUERY per
//         lane, so L_i and D_i are lane scalars; dQ^T += K^T dS^T.
// Causal work skips fully masked tiles and masks only diagonal ones.
//
// bf16 mode reads the packed bf16 operands of attn_pack.hip (row-major Qb,
// dOb, Kb, Vb and the vt_pos-permuted transposes Qt, dOt, Kt, all padded to
// Sp rows); fp32 mode reads the caller's fp32 (BH,S,D) buffers directly with
// v_mfma_f32_32x32x2_f32, clamping rows past S (masked or never written).
#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// prep: grid ceil(BH*Sp/16), 256 threads (16 lanes per query row).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const float* __restrict__ O,
                                                       const float* __restrict__ dO,
                                                       const float* __restrict__ lse,
                                                       float* __restrict__ lse2,
                                                       float* __restrict__ delta, int BH, int S,
                                                       int Sp) {
    constexpr int EPL = D / 16;
    const int tid = threadIdx.x, c = tid & 15;
    const size_t row = (size_t)blockIdx.x * 16 + (tid >> 4);
    if (row >= (size_t)BH * Sp) return;  // whole 16-lane rows leave together
    const int bh = (int)(row / Sp), i = (int)(row - (size_t)bh * Sp);
    float acc = 0.f;
    if (i < S) {
        const size_t off = ((size_t)bh * S + i) * D + c * EPL;
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const f32x4 o = *(const f32x4*)(O + off + e);
            const f32x4 g = *(const f32x4*)(dO + off + e);
            for (int j = 0; j < 4; j++) acc = __builtin_fmaf(o[j], g[j], acc);
        }
    }
    acc = row_sum16(acc);
    if (c == 0) {
        delta[row] = i < S ? acc : 0.f;
        lse2[row] = i < S ? lse[(size_t)bh * S + i] * kLog2e : INFINITY;
    }
}

// ---------------------------------------------------------------------------
// bf16 dK/dV.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_bf16_kernel(BwdParams p) {
    constexpr int BN = 128;       // keys per workgroup
    constexpr int BM = 64;        // queries per tile
    constexpr int RST = D + 8;    // Q / dO tile row stride (bf16)
    constexpr int TST = BM + 8;   // Q^T / dO^T tile row stride (bf16)
    constexpr int RTILE = BM * RST, TTILE = D * TST, BUF = 2 * (RTILE + TTILE);
    constexpr int RCH = BM * D / 8 / 256;  // 16-byte chunks per thread per tile
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;
    __shared__ __attribute__((aligned(16))) bf16 smem[2 * BUF];
    __shared__ float s_lse[2][BM], s_del[2][BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;
    int bh, kb;
    map_block(blockIdx.x, Sp / BN, p.BH, false, bh, kb);
    const int kw = kb * BN + wave * 32;  // first key of this wave
    const int kj = kw + ln;              // this lane's key

    // K and V rows of this lane's key as MFMA B operands (k = d, column = key).
    bf16x8 kf[NKS], vf[NKS];
    {
        const bf16* kr = (const bf16*)p.k + ((size_t)bh * Sp + kj) * D + g * 8;
        const bf16* vr = (const bf16*)p.v + ((size_t)bh * Sp + kj) * D + g * 8;
        for (int ks = 0; ks < NKS; ks++) {
            kf[ks] = *(const bf16x8*)(kr + ks * 16);
            vf[ks] = *(const bf16x8*)(vr + ks * 16);
        }
    }

    const bf16* Qg = (const bf16*)p.q + (size_t)bh * Sp * D;
    const bf16* dOg = (const bf16*)p.dO + (size_t)bh * Sp * D;
    const bf16* Qtg = (const bf16*)p.qt + (size_t)bh * D * Sp;
    const bf16* dOtg = (const bf16*)p.dot + (size_t)bh * D * Sp;
    const float* lg = p.lse2 + (size_t)bh * Sp;
    const float* dg = p.delta + (size_t)bh * Sp;

    u32x4 rq[RCH], rdo[RCH], rqt[RCH], rdot[RCH];
    float rl = 0.f, rd = 0.f;
    auto gload = [&](int qb) {
        const int q0 = qb * BM;
        for (int i = 0; i < RCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            rq[i] = *(const u32x4*)(Qg + (size_t)(q0 + row) * D + col);
            rdo[i] = *(const u32x4*)(dOg + (size_t)(q0 + row) * D + col);
        }
        for (int i = 0; i < RCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BM / 8), col = (c % (BM / 8)) * 8;
            rqt[i] = *(const u32x4*)(Qtg + (size_t)row * Sp + q0 + col);
            rdot[i] = *(const u32x4*)(dOtg + (size_t)row * Sp + q0 + col);
        }
        if (tid < BM) {
            rl = lg[q0 + tid];
            rd = dg[q0 + tid];
        }
    };
    auto sstore = [&](int buf) {
        bf16* sQ = smem + buf * BUF;
        bf16* sdO = sQ + RTILE;
        bf16* sQt = sdO + RTILE;
        bf16* sdOt = sQt + TTILE;
        for (int i = 0; i < RCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            *(u32x4*)(sQ + row * RST + col) = rq[i];
            *(u32x4*)(sdO + row * RST + col) = rdo[i];
        }
        for (int i = 0; i < RCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BM / 8), col = (c % (BM / 8)) * 8;
            *(u32x4*)(sQt + row * TST + col) = rqt[i];
            *(u32x4*)(sdOt + row * TST + col) = rdot[i];
        }
        if (tid < BM) {
            s_lse[buf][tid] = rl;
            s_del[buf][tid] = rd;
        }
    };

    f32x16 dvacc[NDT], dkacc[NDT];
    for (int t = 0; t < NDT; t++) dvacc[t] = dkacc[t] = f32x16{};
    const float c2 = p.scale_log2;
    // Queries below the block's first key see none of its keys.
    const int qb0 = CAUSAL ? (kb * BN) / BM : 0;
    const int qb1 = (S + BM - 1) / BM;

    if (qb0 < qb1) {
        gload(qb0);
        sstore(0);
    }
    __syncthreads();
    for (int qb = qb0; qb < qb1; qb++) {
        const int buf = (qb - qb0) & 1;
        if (qb + 1 < qb1) gload(qb + 1);
        const int q0 = qb * BM;
        // A wave whose first key lies past the tile's last query is fully
        // masked on this tile (wave-uniform).
        if (!CAUSAL || kw <= q0 + BM - 1) {
            const bf16* sQ = smem + buf * BUF;
            const bf16* sdO = sQ + RTILE;
            const bf16* sQt = sdO + RTILE;
            const bf16* sdOt = sQt + TTILE;
            // S, dP: 64 queries x 32 keys as two 32x32 tiles (mt = query half).
            f32x16 sacc[2] = {f32x16{}, f32x16{}}, dpacc[2] = {f32x16{}, f32x16{}};
            for (int ks = 0; ks < NKS; ks++)
                for (int mt = 0; mt < 2; mt++) {
                    const int off = (mt * 32 + ln) * RST + ks * 16 + g * 8;
                    sacc[mt] = mfma_bf16(*(const bf16x8*)(sQ + off), kf[ks], sacc[mt]);
                    dpacc[mt] = mfma_bf16(*(const bf16x8*)(sdO + off), vf[ks], dpacc[mt]);
                }
            const bool need_mask = CAUSAL && (q0 < kw + 31);
            for (int mt = 0; mt < 2; mt++)
                for (int r = 0; r < 16; r++) {
                    const int qr = mt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    float pv = fast_exp2(__builtin_fmaf(sacc[mt][r], c2, -s_lse[buf][qr]));
                    if (need_mask && kj > q0 + qr) pv = 0.f;
                    sacc[mt][r] = pv;
                    dpacc[mt][r] = pv * (dpacc[mt][r] - s_del[buf][qr]);
                }
            // dV^T += dO^T P and dK^T += Q^T dS over 4 k-steps of 16 queries.
            for (int ks = 0; ks < BM / 16; ks++) {
                const int mt = ks >> 1, b0 = (ks & 1) * 8;
                const bf16x8 pb = pack8(sacc[mt][b0 + 0], sacc[mt][b0 + 1], sacc[mt][b0 + 2],
                                        sacc[mt][b0 + 3], sacc[mt][b0 + 4], sacc[mt][b0 + 5],
                                        sacc[mt][b0 + 6], sacc[mt][b0 + 7]);
                const bf16x8 db = pack8(dpacc[mt][b0 + 0], dpacc[mt][b0 + 1], dpacc[mt][b0 + 2],
                                        dpacc[mt][b0 + 3], dpacc[mt][b0 + 4], dpacc[mt][b0 + 5],
                                        dpacc[mt][b0 + 6], dpacc[mt][b0 + 7]);
                for (int t = 0; t < NDT; t++) {
                    const int off = (t * 32 + ln) * TST + ks * 16 + g * 8;
                    dvacc[t] = mfma_bf16(*(const bf16x8*)(sdOt + off), pb, dvacc[t]);
                    dkacc[t] = mfma_bf16(*(const bf16x8*)(sQt + off), db, dkacc[t]);
                }
            }
        }
        if (qb + 1 < qb1) sstore(buf ^ 1);
        __syncthreads();
    }

    if (kj < S) {
        const float sc = p.scale;
        float* dkr = p.dk + ((size_t)bh * S + kj) * D;
        float* dvr = p.dv + ((size_t)bh * S + kj) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a, b;
                for (int i = 0; i < 4; i++) {
                    a[i] = dkacc[t][rq4 * 4 + i] * sc;
                    b[i] = dvacc[t][rq4 * 4 + i];
                }
                *(f32x4*)(dkr + t * 32 + rq4 * 8 + g * 4) = a;
                *(f32x4*)(dvr + t * 32 + rq4 * 8 + g * 4) = b;
            }
    }
}

// ---------------------------------------------------------------------------
// bf16 dQ.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_dq_bf16_kernel(BwdParams p) {
    constexpr int BM = 128, BN = 64;
    constexpr int KST = D + 8;   // K / V tile row stride (bf16)
    constexpr int TST = BN + 8;  // K^T tile row stride (bf16)
    constexpr int KTILE = BN * KST, TTILE = D * TST, BUF = 2 * KTILE + TTILE;
    constexpr int KCH = BN * D / 8 / 256;
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;
    __shared__ __attribute__((aligned(16))) bf16 smem[2 * BUF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;
    int bh, qb;
    map_block(blockIdx.x, Sp / BM, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qi = q0 + wave * 32 + ln;  // this lane's query (< Sp)

    bf16x8 qf[NKS], df[NKS];
    {
        const bf16* qr = (const bf16*)p.q + ((size_t)bh * Sp + qi) * D + g * 8;
        const bf16* dr = (const bf16*)p.dO + ((size_t)bh * Sp + qi) * D + g * 8;
        for (int ks = 0; ks < NKS; ks++) {
            qf[ks] = *(const bf16x8*)(qr + ks * 16);
            df[ks] = *(const bf16x8*)(dr + ks * 16);
        }
    }
    const float lq = p.lse2[(size_t)bh * Sp + qi];
    const float dl = p.delta[(size_t)bh * Sp + qi];

    int kend = S;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int ntiles = (kend + BN - 1) / BN;
    const bf16* Kg = (const bf16*)p.k + (size_t)bh * Sp * D;
    const bf16* Vg = (const bf16*)p.v + (size_t)bh * Sp * D;
    const bf16* Ktg = (const bf16*)p.kt + (size_t)bh * D * Sp;

    u32x4 rk[KCH], rv[KCH], rkt[KCH];
    auto gload = [&](int kt) {
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            rk[i] = *(const u32x4*)(Kg + (size_t)(kt * BN + row) * D + col);
            rv[i] = *(const u32x4*)(Vg + (size_t)(kt * BN + row) * D + col);
        }
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BN / 8), col = (c % (BN / 8)) * 8;
            rkt[i] = *(const u32x4*)(Ktg + (size_t)row * Sp + kt * BN + col);
        }
    };
    auto sstore = [&](int buf) {
        bf16* sK = smem + buf * BUF;
        bf16* sV = sK + KTILE;
        bf16* sKt = sV + KTILE;
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            *(u32x4*)(sK + row * KST + col) = rk[i];
            *(u32x4*)(sV + row * KST + col) = rv[i];
        }
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BN / 8), col = (c % (BN / 8)) * 8;
            *(u32x4*)(sKt + row * TST + col) = rkt[i];
        }
    };

    f32x16 dqacc[NDT];
    for (int t = 0; t < NDT; t++) dqacc[t] = f32x16{};
    const float c2 = p.scale_log2;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ntiles) gload(kt + 1);
        const bf16* sK = smem + buf * BUF;
        const bf16* sV = sK + KTILE;
        const bf16* sKt = sV + KTILE;

        f32x16 sacc[2] = {f32x16{}, f32x16{}}, dpacc[2] = {f32x16{}, f32x16{}};
        for (int ks = 0; ks < NKS; ks++)
            for (int mt = 0; mt < 2; mt++) {
                const int off = (mt * 32 + ln) * KST + ks * 16 + g * 8;
                sacc[mt] = mfma_bf16(*(const bf16x8*)(sK + off), qf[ks], sacc[mt]);
                dpacc[mt] = mfma_bf16(*(const bf16x8*)(sV + off), df[ks], dpacc[mt]);
            }
        const int kbase = kt * BN;
        const bool need_mask = (kbase + BN > S) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) {
                float pv = fast_exp2(__builtin_fmaf(sacc[mt][r], c2, -lq));
                if (need_mask) {
                    const int key = kbase + mt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (key >= S || (CAUSAL && key > qi)) pv = 0.f;
                }
                dpacc[mt][r] = pv * (dpacc[mt][r] - dl);
            }
        // dQ^T += K^T dS^T over 4 k-steps of 16 keys.
        for (int ks = 0; ks < BN / 16; ks++) {
            const int mt = ks >> 1, b0 = (ks & 1) * 8;
            const bf16x8 db = pack8(dpacc[mt][b0 + 0], dpacc[mt][b0 + 1], dpacc[mt][b0 + 2],
                                    dpacc[mt][b0 + 3], dpacc[mt][b0 + 4], dpacc[mt][b0 + 5],
                                    dpacc[mt][b0 + 6], dpacc[mt][b0 + 7]);
            for (int t = 0; t < NDT; t++) {
                const int off = (t * 32 + ln) * TST + ks * 16 + g * 8;
                dqacc[t] = mfma_bf16(*(const bf16x8*)(sKt + off), db, dqacc[t]);
            }
        }
        if (kt + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    if (qi < S) {
        const float sc = p.scale;
        float* dqr = p.dq + ((size_t)bh * S + qi) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a;
                for (int i = 0; i < 4; i++) a[i] = dqacc[t][rq4 * 4 + i] * sc;
                *(f32x4*)(dqr + t * 32 + rq4 * 8 + g * 4) = a;
            }
    }
}

// ---------------------------------------------------------------------------
// fp32 dK/dV (v_mfma_f32_32x32x2_f32). k-slot map of the D-contractions:
// step i, group g <-> d = g*(D/2) + i; of the query contractions: step r,
// group g <-> query 8(r/4) + 4g + r%4, the row an accumulator register holds.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_f32_kernel(BwdParams p) {
    constexpr int BN = 128, BM = 32;
    constexpr int RST = D + 4;  // Q / dO tile row stride (floats)
    constexpr int RTILE = BM * RST, BUF = 2 * RTILE;
    constexpr int CH = BM * D / 4 / 256;
    constexpr int HD = D / 2;
    constexpr int NDT = D / 32;
    __shared__ __attribute__((aligned(16))) float smem[2 * BUF];
    __shared__ float s_lse[2][BM], s_del[2][BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;
    int bh, kb;
    map_block(blockIdx.x, Sp / BN, p.BH, false, bh, kb);
    const int kw = kb * BN + wave * 32;
    const int kj = kw + ln;

    float kf[HD], vf[HD];
    {
        const int kr = kj < S ? kj : S - 1;  // pad keys are computed, never written
        const float* kp = (const float*)p.k + ((size_t)bh * S + kr) * D + g * HD;
        const float* vp = (const float*)p.v + ((size_t)bh * S + kr) * D + g * HD;
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = *(const f32x4*)(kp + i), b = *(const f32x4*)(vp + i);
            for (int j = 0; j < 4; j++) {
                kf[i + j] = a[j];
                vf[i + j] = b[j];
            }
        }
    }
    const float* Qg = (const float*)p.q + (size_t)bh * S * D;
    const float* dOg = (const float*)p.dO + (size_t)bh * S * D;
    const float* lg = p.lse2 + (size_t)bh * Sp;
    const float* dg = p.delta + (size_t)bh * Sp;

    f32x4 rq[CH], rdo[CH];
    float rl = 0.f, rd = 0.f;
    auto gload = [&](int qb) {
        const int q0 = qb * BM;
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            int q = q0 + row;
            q = q < S ? q : S - 1;  // clamped rows have lse2 = +inf: P = 0
            rq[i] = *(const f32x4*)(Qg + (size_t)q * D + col);
            rdo[i] = *(const f32x4*)(dOg + (size_t)q * D + col);
        }
        if (tid < BM) {
            rl = lg[q0 + tid];
            rd = dg[q0 + tid];
        }
    };
    auto sstore = [&](int buf) {
        float* sQ = smem + buf * BUF;
        float* sdO = sQ + RTILE;
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            *(f32x4*)(sQ + row * RST + col) = rq[i];
            *(f32x4*)(sdO + row * RST + col) = rdo[i];
        }
        if (tid < BM) {
            s_lse[buf][tid] = rl;
            s_del[buf][tid] = rd;
        }
    };

    f32x16 dvacc[NDT], dkacc[NDT];
    for (int t = 0; t < NDT; t++) dvacc[t] = dkacc[t] = f32x16{};
    const float c2 = p.scale_log2;
    const int qb0 = CAUSAL ? (kb * BN) / BM : 0;
    const int qb1 = (S + BM - 1) / BM;

    if (qb0 < qb1) {
        gload(qb0);
        sstore(0);
    }
    __syncthreads();
    for (int qb = qb0; qb < qb1; qb++) {
        const int buf = (qb - qb0) & 1;
        if (qb + 1 < qb1) gload(qb + 1);
        const int q0 = qb * BM;
        if (!CAUSAL || kw <= q0 + BM - 1) {
            const float* sQ = smem + buf * BUF;
            const float* sdO = sQ + RTILE;
            f32x16 sacc = f32x16{}, dpacc = f32x16{};
            const float* qrow = sQ + ln * RST + g * HD;
            const float* drow = sdO + ln * RST + g * HD;
            for (int i = 0; i < HD; i += 4) {
                const f32x4 a = *(const f32x4*)(qrow + i), b = *(const f32x4*)(drow + i);
                for (int j = 0; j < 4; j++) {
                    sacc = mfma_f32(a[j], kf[i + j], sacc);
                    dpacc = mfma_f32(b[j], vf[i + j], dpacc);
                }
            }
            const bool need_mask = CAUSAL && (q0 < kw + 31);
            for (int r = 0; r < 16; r++) {
                const int qr = 8 * (r >> 2) + 4 * g + (r & 3);
                float pv = fast_exp2(__builtin_fmaf(sacc[r], c2, -s_lse[buf][qr]));
                if (need_mask && kj > q0 + qr) pv = 0.f;
                sacc[r] = pv;
                dpacc[r] = pv * (dpacc[r] - s_del[buf][qr]);
            }
            for (int r = 0; r < 16; r++) {
                const int qr = 8 * (r >> 2) + 4 * g + (r & 3);
                const float* dor = sdO + qr * RST + ln;
                const float* qr_ = sQ + qr * RST + ln;
                for (int t = 0; t < NDT; t++) {
                    dvacc[t] = mfma_f32(dor[t * 32], sacc[r], dvacc[t]);
                    dkacc[t] = mfma_f32(qr_[t * 32], dpacc[r], dkacc[t]);
                }
            }
        }
        if (qb + 1 < qb1) sstore(buf ^ 1);
        __syncthreads();
    }

    if (kj < S) {
        const float sc = p.scale;
        float* dkr = p.dk + ((size_t)bh * S + kj) * D;
        float* dvr = p.dv + ((size_t)bh * S + kj) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a, b;
                for (int i = 0; i < 4; i++) {
                    a[i] = dkacc[t][rq4 * 4 + i] * sc;
                    b[i] = dvacc[t][rq4 * 4 + i];
                }
                *(f32x4*)(dkr + t * 32 + rq4 * 8 + g * 4) = a;
                *(f32x4*)(dvr + t * 32 + rq4 * 8 + g * 4) = b;
            }
    }
}

// ---------------------------------------------------------------------------
// fp32 dQ.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void bwd_dq_f32_kernel(BwdParams p) {
    constexpr int BM = 128, BN = 32;
    constexpr int KST = D + 4;  // K / V tile row stride (floats)
    constexpr int KTILE = BN * KST, BUF = 2 * KTILE;
    constexpr int CH = BN * D / 4 / 256;
    constexpr int HD = D / 2;
    constexpr int NDT = D / 32;
    __shared__ __attribute__((aligned(16))) float smem[2 * BUF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;
    int bh, qb;
    map_block(blockIdx.x, Sp / BM, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qi = q0 + wave * 32 + ln;

    float qf[HD], df[HD];
    {
        const int qr = qi < S ? qi : S - 1;  // pad queries have lse2 = +inf: P = 0
        const float* qp = (const float*)p.q + ((size_t)bh * S + qr) * D + g * HD;
        const float* dp = (const float*)p.dO + ((size_t)bh * S + qr) * D + g * HD;
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = *(const f32x4*)(qp + i), b = *(const f32x4*)(dp + i);
            for (int j = 0; j < 4; j++) {
                qf[i + j] = a[j];
                df[i + j] = b[j];
            }
        }
    }
    const float lq = p.lse2[(size_t)bh * Sp + qi];
    const float dl = p.delta[(size_t)bh * Sp + qi];

    int kend = S;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int ntiles = (kend + BN - 1) / BN;
    const float* Kg = (const float*)p.k + (size_t)bh * S * D;
    const float* Vg = (const float*)p.v + (size_t)bh * S * D;

    f32x4 rk[CH], rv[CH];
    auto gload = [&](int kt) {
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            int key = kt * BN + row;
            key = key < S ? key : S - 1;  // clamped rows are masked
            rk[i] = *(const f32x4*)(Kg + (size_t)key * D + col);
            rv[i] = *(const f32x4*)(Vg + (size_t)key * D + col);
        }
    };
    auto sstore = [&](int buf) {
        float* sK = smem + buf * BUF;
        float* sV = sK + KTILE;
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            *(f32x4*)(sK + row * KST + col) = rk[i];
            *(f32x4*)(sV + row * KST + col) = rv[i];
        }
    };

    f32x16 dqacc[NDT];
    for (int t = 0; t < NDT; t++) dqacc[t] = f32x16{};
    const float c2 = p.scale_log2;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ntiles) gload(kt + 1);
        const float* sK = smem + buf * BUF;
        const float* sV = sK + KTILE;

        f32x16 sacc = f32x16{}, dpacc = f32x16{};
        const float* krow = sK + ln * KST + g * HD;
        const float* vrow = sV + ln * KST + g * HD;
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = *(const f32x4*)(krow + i), b = *(const f32x4*)(vrow + i);
            for (int j = 0; j < 4; j++) {
                sacc = mfma_f32(a[j], qf[i + j], sacc);
                dpacc = mfma_f32(b[j], df[i + j], dpacc);
            }
        }
        const int kbase = kt * BN;
        const bool need_mask = (kbase + BN > S) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
        for (int r = 0; r < 16; r++) {
            float pv = fast_exp2(__builtin_fmaf(sacc[r], c2, -lq));
            if (need_mask) {
                const int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key >= S || (CAUSAL && key > qi)) pv = 0.f;
            }
            dpacc[r] = pv * (dpacc[r] - dl);
        }
        for (int r = 0; r < 16; r++) {
            const int key = 8 * (r >> 2) + 4 * g + (r & 3);
            const float* kr = sK + key * KST + ln;
            for (int t = 0; t < NDT; t++) dqacc[t] = mfma_f32(kr[t * 32], dpacc[r], dqacc[t]);
        }
        if (kt + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    if (qi < S) {
        const float sc = p.scale;
        float* dqr = p.dq + ((size_t)bh * S + qi) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a;
                for (int i = 0; i < 4; i++) a[i] = dqacc[t][rq4 * 4 + i] * sc;
                *(f32x4*)(dqr + t * 32 + rq4 * 8 + g * 4) = a;
            }
    }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
hipError_t launch_bwd_prep(const float* O, const float* dO, const float* lse, float* lse2,
                           float* delta, int BH, int S, int Sp, int D, hipStream_t s) {
    const size_t rows = (size_t)BH * Sp;
    const unsigned grid = (unsigned)((rows + 15) / 16);
    if (D == 64)
        bwd_prep_kernel<64><<<grid, 256, 0, s>>>(O, dO, lse, lse2, delta, BH, S, Sp);
    else if (D == 128)
        bwd_prep_kernel<128><<<grid, 256, 0, s>>>(O, dO, lse, lse2, delta, BH, S, Sp);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

#define GONN_BWD_LAUNCH(KERNEL)                                                      \
    do {                                                                             \
        if (D == 64) {                                                               \
            if (causal) KERNEL<64, true><<<grid, 256, 0, s>>>(p);                    \
            else KERNEL<64, false><<<grid, 256, 0, s>>>(p);                          \
        } else if (D == 128) {                                                       \
            if (causal) KERNEL<128, true><<<grid, 256, 0, s>>>(p);                   \
            else KERNEL<128, false><<<grid, 256, 0, s>>>(p);                         \
        } else {                                                                     \
            return hipErrorInvalidValue;                                             \
        }                                                                            \
    } while (0)

hipError_t launch_bwd_dkdv(const BwdParams& p, int mode, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0) return hipErrorInvalidValue;
    const dim3 grid((p.Sp / 128) * p.BH);
    if (mode == 1) GONN_BWD_LAUNCH(bwd_dkdv_bf16_kernel);
    else GONN_BWD_LAUNCH(bwd_dkdv_f32_kernel);
    return hipGetLastError();
}

hipError_t launch_bwd_dq(const BwdParams& p, int mode, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0) return hipErrorInvalidValue;
    const dim3 grid((p.Sp / 128) * p.BH);
    if (mode == 1) GONN_BWD_LAUNCH(bwd_dq_bf16_kernel);
    else GONN_BWD_LAUNCH(bwd_dq_f32_kernel);
    return hipGetLastError();
}

#undef GONN_BWD_LAUNCH

}  // namespace gonn
