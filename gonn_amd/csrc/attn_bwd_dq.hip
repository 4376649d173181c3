// attn_bwd_dq.hip -- bf16 dQ kernel of the flash-attention backward for
// gfx950 (MI355X); the other backward stages are in attn_bwd.hip, whose header
// states the identities (reference: backend/cuda/gonn_cuda.cu:333-383).
//
// Compiled on its own with -mllvm -amdgpu-mfma-vgpr-form=1: at one wave per
// SIMD the compiler otherwise gives every MFMA an AGPR accumulator, and the
// score tiles the VALU reads would have to be copied out of AGPRs each step
// (v_accvgpr_read, about 80 per step, which do not overlap the MFMAs). In
// VGPR form the score and dQ accumulators live in VGPRs and only the Q / dO
// fragments (pure MFMA operands) are held in AGPRs.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// bf16 dQ.
//
// One workgroup per 128-query block, 32 queries per wave (the forward's
// shape): S^T = K Q^T and dP^T = V dO^T with one QUERY per lane, so L and D
// are lane scalars, and dQ^T += K^T dS^T. One wave per SIMD. Three-stage
// software pipeline, as in the dK/dV kernel: step t issues
//   MFMA  S^T(t+1), dP^T(t+1)            (K, V row tiles of key tile t+1)
//   VALU  dS(t) = exp2(S c - L) (dP - D), packed to bf16
//   MFMA  dQ^T += K^T(t-1) dS^T(t-1)     (transposed K tile of t-1)
// hand-scheduled in slots; dS(t) overwrites dS(t-1) 16 keys at a time after
// the dQ MFMAs that read them were issued. Step t loads K, V of tile t+2 and
// K^T of tile t into the 2-slot rings (one barrier per step). Masks (causal
// diagonal, key end) exist only on the last key tiles of a query block.
//
// The step is issue-bound inside its one wave (about 7.5 instructions per
// MFMA slot: VALU, LDS operand reads and their waits, tile-load blocks). The
// tile loads go into the first kDqDmaSpan slots, so that they have most of
// a step to arrive (an L2 miss takes about a microsecond); the dP^T
// accumulator starts at -D, which saves the subtraction per score.
// ---------------------------------------------------------------------------
// Softmax micro-ops of one 16-key k-step (4 score pairs): j -> pair, kind
// (0 / 1: FMA + exp2 of score 0 / 1 of the pair, 2: products + bf16 pack).
constexpr int kDqPairOf[12] = {0, 0, 1, 1, 0, 2, 2, 1, 3, 3, 2, 3};
constexpr int kDqKindOf[12] = {0, 1, 0, 1, 2, 0, 1, 2, 0, 1, 2, 2};
// Slot of micro-op j of k-step q in a step of GW MFMAs per k-step whose
// first HCn MFMAs of each group are the dQ products reading pd[q].
template <int GW, int HCn>
constexpr int dq_uop_slot(int q, int j) {
    int s = q * GW + (j * GW) / 12;
    if (kDqKindOf[j] == 2 && HCn > 0 && s < q * GW + HCn - 1) s = q * GW + HCn - 1;
    return s;
}

constexpr int kDqDmaSpan = 24;     // slots over which the step's tile loads are spread
constexpr int kDqLookahead = 3;    // LDS operand lead (deeper measured no faster)
constexpr bool kDqFragsInAgpr = true;

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(256, 1) void bwd_dq_bf16_kernel(BwdParams p) {
    constexpr int BM = 128, BN = 64;
    constexpr int KST = D + 8;   // K / V tile row stride (bf16)
    constexpr int TST = BN + 8;  // K^T tile row stride (bf16)
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;
    constexpr int RCP = KST / 8, RCD = D / 8, NRP = BN * RCP;
    constexpr int TCP = TST / 8, TCD = BN / 8, NTP = D * TCP;
    constexpr int NRI = (NRP + 255) / 256, NTI = (NTP + 255) / 256;
    constexpr int RLAST = NRP - (NRI - 1) * 256, TLAST = NTP - (NTI - 1) * 256;
    static_assert(RLAST % 64 == 0 && TLAST % 64 == 0, "partial loads must be whole waves");
    constexpr int RTILE = BN * KST, TTILE = D * TST;
    constexpr uint32_t RTB = RTILE * 2, TTB = TTILE * 2;
    __shared__ __attribute__((aligned(16))) bf16 sK[2 * RTILE];
    __shared__ __attribute__((aligned(16))) bf16 sV[2 * RTILE];
    __shared__ __attribute__((aligned(16))) bf16 sKt[2 * TTILE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;
    int bh, qb;
    map_block(blockIdx.x, Sp / BM, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qw = q0 + wave * 32;       // first query of this wave
    const int qi = qw + ln;              // this lane's query (< Sp)
    const int Skv = bwd_keys(p, bh);     // keys taking part (key padding)
    if (Skv == 0) {  // no key: the forward gave O = 0; dQ = 0
        bwd_zero_rows<D>(p.dq, S, bh, q0, BM);
        return;
    }

    bf16x8 qf[NKS], df[NKS];
    {
        const bf16* qr = (const bf16*)p.q + ((size_t)bh * Sp + qi) * D + g * 8;
        const bf16* dr = (const bf16*)p.dO + ((size_t)bh * Sp + qi) * D + g * 8;
        for (int ks = 0; ks < NKS; ks++) {
            qf[ks] = *(const bf16x8*)(qr + ks * 16);
            df[ks] = *(const bf16x8*)(dr + ks * 16);
            // The fragments are only MFMA operands: keeping them in AGPRs
            // leaves the VGPRs to the score tiles the VALU works on.
            if constexpr (kDqFragsInAgpr) asm volatile("" : "+a"(qf[ks]), "+a"(df[ks]));
        }
    }
    const float lq = p.lse2[(size_t)bh * Sp + qi];
    const float dl = p.delta[(size_t)bh * Sp + qi];
    // dP^T accumulates onto -D (D is per query, i.e. per lane), so the
    // accumulator holds dP - D.
    f32x16 dinit;
    for (int r = 0; r < 16; r++) dinit[r] = -dl;

    int kend = Skv;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int nt = (kend + BN - 1) / BN;
    // K, V and K^T hold Sk key rows padded to Skp (Sk != S for
    // cross-attention).
    const int Skp = p.Skp;
    const bf16* Kg = (const bf16*)p.k + (size_t)bh * Skp * D;
    const bf16* Vg = (const bf16*)p.v + (size_t)bh * Skp * D;
    const bf16* Ktg = (const bf16*)p.kt + (size_t)bh * D * Skp;

    uint32_t roff[NRI], toff[NTI];
    for (int i = 0; i < NRI; i++) {
        const int pos = i * 256 + tid, r = pos / RCP, ch = pos % RCP;
        roff[i] = (uint32_t)(((pos < NRP ? r : 0) * D + (ch < RCD ? ch : 0) * 8) * 2);
    }
    for (int i = 0; i < NTI; i++) {
        const int pos = i * 256 + tid, r = pos / TCP, ch = pos % TCP;
        toff[i] = (uint32_t)(((pos < NTP ? r : 0) * Skp + (ch < TCD ? ch : 0) * 8) * 2);
    }
    const uint32_t rlast = wave * 64 < RLAST, tlast = wave * 64 < TLAST;  // wave-uniform
    const uint32_t slice = (uint32_t)Skp * D * 2;  // bytes of one (b,h) slice of K, V, K^T
    const brsrc rk = make_rsrc(Kg, slice), rv = make_rsrc(Vg, slice), rkt = make_rsrc(Ktg, slice);
    const uint32_t lk = lds_addr(sK) + wave * 1024, lv = lds_addr(sV) + wave * 1024;
    const uint32_t lkt = lds_addr(sKt) + wave * 1024;
    // Load j of the row tiles (K: j < NRI, V: j >= NRI) of key tile kt.
    // (Issued when the wave-uniform `on` is set: a scalar branch inside the
    // load statement keeps the step one basic block.)
    auto dma_row = [&](int kt, int slot, int j, uint32_t on) {
        const uint32_t so = (uint32_t)kt * BN * D * 2;
        const int i = j % NRI;
        const brsrc r = j < NRI ? rk : rv;
        const uint32_t dst = (j < NRI ? lk : lv) + slot * RTB + i * 4096;
        dma16_if(r, dst, roff[i], so, i < NRI - 1 ? on : on & rlast);
    };
    // Load j of the K^T tile of key tile kt.
    auto dma_tr = [&](int kt, int slot, int j, uint32_t on) {
        const uint32_t so = (uint32_t)kt * BN * 2;
        const uint32_t dst = lkt + slot * TTB + j * 4096;
        dma16_if(rkt, dst, toff[j], so, j < NTI - 1 ? on : on & tlast);
    };

    const uint32_t rq0 = (uint32_t)(ln * KST + g * 8) * 2, tq0 = (uint32_t)(ln * TST + g * 8) * 2;
    const char* cK = (const char*)sK;
    const char* cV = (const char*)sV;
    const char* cKt = (const char*)sKt;

    // Masks of key tile kt on S^T: key >= Skv (end of the slice or key
    // padding), or causal key > query. The exponent scale c2b is positive,
    // so -inf gives P = 0 and dS = 0.
    auto needs_mask = [&](int kt) {
        const int kbase = kt * BN;
        return (kbase + BN > Skv) || (CAUSAL && kbase + BN - 1 > qw);
    };
    auto mask = [&](int kt, f32x16* s) {
        const int kbase = kt * BN + 4 * g;
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) {
                const int key = kbase + mt * 32 + 8 * (r >> 2) + (r & 3);
                const bool off = key >= Skv || (CAUSAL && key > qi);
                s[mt][r] = off ? -INFINITY : s[mt][r];
            }
    };

    f32x16 dqacc[NDT];
    for (int t = 0; t < NDT; t++) dqacc[t] = f32x16{};
    const float c2 = p.c2b;
    // Additive mask (MASK variant): this lane's query row; the values of
    // S^T(t+1) are loaded at the start of step t and added at its end, when
    // that tile is complete.
    MaskRow mrow{};
    f32x4 mreg[8];
    if constexpr (MASK) mrow.init(p.mask, p.mask_sb, p.mask_sh, p.H, S, p.Sk, bh, qi);
    u32x4 pd[4];  // dS of the tile dQ consumes next, bf16 pairs per word
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

    // One pipeline step. sA <- S^T(t+1), dA <- dP^T(t+1); sB, dB = tile t.
    auto step = [&](auto ha_tag, auto hb_tag, auto hc_tag, int t, f32x16* sA, f32x16* dA,
                    f32x16* sB, f32x16* dB) __attribute__((always_inline)) {
        constexpr bool HA = decltype(ha_tag)::value;  // S^T/dP^T of tile t+1
        constexpr bool HB = decltype(hb_tag)::value;  // dS of tile t
        constexpr bool HC = decltype(hc_tag)::value;  // dQ of tile t-1
        const uint32_t dr = HA && t + 2 < nt, dt = HB;
        if constexpr (HB)
            if (needs_mask(t)) mask(t, sB);
        if constexpr (MASK && HA) mrow.load(t + 1, g, mreg);
        const uint32_t rsl = (uint32_t)((t + 1) & 1) * RTB;  // K, V of tile t+1
        const uint32_t tsl = (uint32_t)((t + 1) & 1) * TTB;  // K^T of tile t-1

        constexpr int HCn = HC ? NDT : 0, HAn = HA ? NKS : 0;
        constexpr int GW = HCn + HAn;
        constexpr int NM = 4 * GW;
        constexpr int LA = kDqLookahead;  // LDS operand lead (MFMA slots)
        constexpr int NO = LA < 4 ? 4 : 8;
        constexpr int NDMA = 2 * NRI + NTI;
        // Tile loads, one per MFMA slot from slot 1 on, spread over the first
        // kDqDmaSpan slots of the step (all of them when 0).
        constexpr int SPAN = kDqDmaSpan > 0 && kDqDmaSpan < NM ? kDqDmaSpan : NM;
        constexpr int DS = SPAN / NDMA > 0 ? SPAN / NDMA : 1;
        bf16x8 opr[NO];
        auto fetch = [&](auto E) {
            constexpr int e = decltype(E)::value, ks = e / GW, w = e % GW;
            if constexpr (w < HCn) {
                opr[e % NO] = *(const bf16x8*)(cKt + tsl + tq0 + (w * 32 * TST + ks * 16) * 2);
            } else {
                constexpr int u = w - HCn, kk = ks * (NKS / 4) + u / 4, mt = u & 1;
                const char* base = ((u & 2) ? cV : cK) + rsl + rq0;
                opr[e % NO] = *(const bf16x8*)(base + (mt * 32 * KST + kk * 16) * 2);
            }
        };
        auto issue = [&](auto E) {
            constexpr int e = decltype(E)::value, ks = e / GW, w = e % GW;
            if constexpr (w < HCn) {
                dqacc[w] = mfma_bf16(opr[e % NO], __builtin_bit_cast(bf16x8, pd[ks]), dqacc[w]);
            } else {
                constexpr int u = w - HCn, kk = ks * (NKS / 4) + u / 4, mt = u & 1;
                if constexpr (u & 2)
                    dA[mt] = mfma_bf16(opr[e % NO], df[kk], kk == 0 ? dinit : dA[mt]);
                else
                    sA[mt] = mfma_bf16(opr[e % NO], qf[kk], kk == 0 ? f32x16{} : sA[mt]);
            }
        };
        // dS of tile t as 16 score pairs k (registers (k%8)*2, +1 of
        // sB/dB[k/8]; 16-key k-step k/4 of the dQ product), each in three
        // micro-ops: E0 / E1 (FMA + exp2 of one score, ~20 VALU cycles) and
        // P (two products and the bf16 pair into pd, ~12 cycles). The 12
        // micro-ops of k-step q are spread one per MFMA slot over its group
        // of GW slots, so no slot carries more VALU than its MFMA hides; a
        // P micro-op of k-step q comes after the dQ MFMAs that read pd[q].
        float ue[16][2];
        auto uop = [&](auto Q, auto J) {
            constexpr int q = decltype(Q)::value, j = decltype(J)::value;
            constexpr int k = 4 * q + kDqPairOf[j], mt = k >> 3, r = (k & 7) * 2;
            if constexpr (kDqKindOf[j] < 2) {
                constexpr int h = kDqKindOf[j];
                ue[k][h] = fast_exp2(__builtin_fmaf(sB[mt][r + h], c2, -lq));
                pin(ue[k][h]);
            } else {
                const float d0 = ue[k][0] * dB[mt][r];
                const float d1 = ue[k][1] * dB[mt][r + 1];
                const bf16x2 pr = {to_bf16(d0), to_bf16(d1)};
                pd[k >> 2][k & 3] = __builtin_bit_cast(uint32_t, pr);
                pin(pd[k >> 2][k & 3]);
            }
        };
        auto uops_at = [&](auto E) {
            constexpr int e = decltype(E)::value;
            if constexpr (HB) {
                static_for<4>([&](auto Q) {
                    static_for<12>([&](auto J) {
                        constexpr int at = dq_uop_slot<GW, HCn>(decltype(Q)::value, decltype(J)::value);
                        if constexpr (e < NM ? at == e : at >= NM) uop(Q, J);
                    });
                });
            }
        };
        static_for<LA>([&](auto E) {
            if constexpr (decltype(E)::value < NM) fetch(E);
        });
        static_for<NM>([&](auto E) {
            constexpr int e = decltype(E)::value;
            if constexpr (e + LA < NM) fetch(std::integral_constant<int, e + LA>{});
            issue(E);
            if constexpr (e >= 1 && (e - 1) % DS == 0 && (e - 1) / DS < NDMA) {
                constexpr int d = (e - 1) / DS;
                if constexpr (d < 2 * NRI) dma_row(t + 2, t & 1, d, dr);
                else dma_tr(t, t & 1, d - 2 * NRI, dt);
            }
            uops_at(E);
            __builtin_amdgcn_sched_barrier(0);
        });
        static_for<NDMA>([&](auto Dd) {
            constexpr int d = decltype(Dd)::value;
            if constexpr (NM == 0 || 1 + d * DS >= NM) {
                if constexpr (d < 2 * NRI) dma_row(t + 2, t & 1, d, dr);
                else dma_tr(t, t & 1, d - 2 * NRI, dt);
            }
        });
        uops_at(std::integral_constant<int, NM>{});
        GONN_VMCNT(0);
        __syncthreads();
        if constexpr (MASK && HA) MaskRow::add(mreg, sA);
    };
    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;

    // Prologue: K, V of tiles 0 and 1; S^T/dP^T of tile 0.
    for (int j = 0; j < 2 * NRI; j++) dma_row(0, 0, j, 1);
    for (int j = 0; j < 2 * NRI; j++) dma_row(1, 1, j, nt > 1);
    GONN_VMCNT(0);
    __syncthreads();
    f32x16 sX[2], dX[2], sY[2], dY[2];
    for (int mt = 0; mt < 2; mt++) {
        sX[mt] = f32x16{};
        dX[mt] = dinit;
    }
    for (int kk = 0; kk < NKS; kk++)
        for (int mt = 0; mt < 2; mt++) {
            sX[mt] = mfma_bf16(*(const bf16x8*)(cK + rq0 + (mt * 32 * KST + kk * 16) * 2), qf[kk], sX[mt]);
            dX[mt] = mfma_bf16(*(const bf16x8*)(cV + rq0 + (mt * 32 * KST + kk * 16) * 2), df[kk], dX[mt]);
        }
    if constexpr (MASK) {
        mrow.load(0, g, mreg);
        MaskRow::add(mreg, sX);
    }
    __syncthreads();  // row slot 0 is reloaded by step 0

    if (nt == 1) {
        step(No{}, Yes{}, No{}, 0, sY, dY, sX, dX);
        step(No{}, No{}, Yes{}, 1, sX, dX, sY, dY);
    } else {
        step(Yes{}, Yes{}, No{}, 0, sY, dY, sX, dX);
        int t = 1;
        for (; t + 2 < nt; t += 2) {
            step(Yes{}, Yes{}, Yes{}, t, sX, dX, sY, dY);
            step(Yes{}, Yes{}, Yes{}, t + 1, sY, dY, sX, dX);
        }
        if (t + 1 < nt) {
            step(Yes{}, Yes{}, Yes{}, t, sX, dX, sY, dY);
            step(No{}, Yes{}, Yes{}, t + 1, sY, dY, sX, dX);
            step(No{}, No{}, Yes{}, t + 2, sX, dX, sY, dY);
        } else {
            step(No{}, Yes{}, Yes{}, t, sX, dX, sY, dY);
            step(No{}, No{}, Yes{}, t + 1, sY, dY, sX, dX);
        }
    }

    if (qi < S) {
        const float sc = p.dqs;
        float* dqr = p.dq + ((size_t)bh * S + qi) * D;
        for (int d = 0; d < NDT; d++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a;
                for (int k = 0; k < 4; k++) a[k] = dqacc[d][rq4 * 4 + k] * sc;
                *(f32x4*)(dqr + d * 32 + rq4 * 8 + g * 4) = a;
            }
    }
}

hipError_t launch_bwd_dq_bf16(const BwdParams& p, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0 || p.Skp % kBwdPad != 0) return hipErrorInvalidValue;
    const dim3 grid((p.Sp / 128) * p.BH);
    const bool m = p.mask != nullptr;
    if (D == 64) {
        if (causal) m ? bwd_dq_bf16_kernel<64, true, true><<<grid, 256, 0, s>>>(p)
                      : bwd_dq_bf16_kernel<64, true, false><<<grid, 256, 0, s>>>(p);
        else m ? bwd_dq_bf16_kernel<64, false, true><<<grid, 256, 0, s>>>(p)
               : bwd_dq_bf16_kernel<64, false, false><<<grid, 256, 0, s>>>(p);
    } else if (D == 128) {
        if (causal) m ? bwd_dq_bf16_kernel<128, true, true><<<grid, 256, 0, s>>>(p)
                      : bwd_dq_bf16_kernel<128, true, false><<<grid, 256, 0, s>>>(p);
        else m ? bwd_dq_bf16_kernel<128, false, true><<<grid, 256, 0, s>>>(p)
               : bwd_dq_bf16_kernel<128, false, false><<<grid, 256, 0, s>>>(p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gonn
