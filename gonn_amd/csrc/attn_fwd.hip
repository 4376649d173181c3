// attn_fwd.hip -- flash-attention forward for gfx950 (MI355X).
//
// Replaces the reference's fp64 one-thread-per-row kernels
// flash_attn_f64_tiled / flash_attn_f64_kernel (backend/cuda/gonn_cuda.cu:302-331,
// :389-450). Same result definition: O = softmax(scale*QK^T + mask) V and
// L = m + ln(l) per query row (gonn_cuda.cu:330, :448), causal mask j > i.
//
// Design (one workgroup = 4 wave64s = 128 query rows of one (b,h) slice):
//  * each wave owns 32 query rows; its Q fragment stays in VGPRs;
//  * K/V tiles are staged in LDS (double buffered, one barrier per tile),
//    loaded with 128-bit coalesced global loads one tile ahead;
//  * S^T = K Q^T on MFMA, so every lane holds scores of ONE query: the row
//    max/sum of the online softmax is in-lane plus one v_permlane32_swap;
//  * O^T += V^T P^T on MFMA straight from the S^T registers (no LDS trip for
//    P); the output accumulator then also holds one query per lane, so the
//    rescale by exp2(m_old - m_new) is in-lane;
//  * scale*log2(e) is folded into one FMA before v_exp_f32;
//  * masking only on tiles that cross the diagonal or the key end;
//  * blockIdx -> (head, q-block) is head-major within each XCD (workgroups are
//    dealt round-robin to the 8 XCDs), longest causal q-blocks first, so the
//    q-blocks sharing one head's K/V run on the same XCD's L2.
//
// Two arithmetic modes:
//  bf16: v_mfma_f32_32x32x16_bf16. The pack kernel (attn_pack.hip) converts K
//        to bf16 (BH,Skp,D) and V to a transposed bf16 layout Vt (BH,D,Skp)
//        whose 16-key groups are permuted (vt_pos) so each lane's PV operand
//        is one 16-byte read. Skp = Sk rounded up to 64; the pad is zero and
//        masked.
//  fp32: v_mfma_f32_32x32x2_f32 straight from the fp32 K/V (no pack).
#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// bf16-MFMA forward.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, typename QT>
__global__ __launch_bounds__(256, 2) void fwd_bf16_kernel(FwdParams p) {
    constexpr int BM = 128, BN = 64;
    constexpr int KST = D + 8;   // K tile row stride (bf16)
    constexpr int VST = BN + 8;  // Vt tile row stride (bf16)
    constexpr int KTILE = BN * KST, VTILE = D * VST;
    constexpr int KCH = BN * D / 8 / 256;  // 16-byte chunks per thread (K)
    constexpr int VCH = D * BN / 8 / 256;  // (Vt)
    constexpr int NKS = D / 16;            // k-steps of the QK^T product
    constexpr int NDT = D / 32;            // 32-row d-tiles of O^T
    __shared__ __attribute__((aligned(16))) bf16 smem[2 * (KTILE + VTILE)];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    int bh, qb;
    map_block(blockIdx.x, p.nqb, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qi = q0 + wave * 32 + ln;  // this lane's query row
    const int Sq = p.Sq, Sk = p.Sk, Skp = p.Skp;

    // Q fragment: qf[ks] = Q[qi][16ks + 8g .. +7] in bf16.
    bf16x8 qf[NKS];
    {
        const QT* qrow = (const QT*)p.q + ((size_t)bh * Sq + (qi < Sq ? qi : 0)) * D;
        const float sg = qi < Sq ? p.qsign : 0.f;
        for (int ks = 0; ks < NKS; ks++) {
            const int d0 = ks * 16 + g * 8;
            float v[8];
            if constexpr (sizeof(QT) == 4) {
                const f32x4 a = *(const f32x4*)(qrow + d0), b = *(const f32x4*)(qrow + d0 + 4);
                for (int i = 0; i < 4; i++) { v[i] = a[i]; v[4 + i] = b[i]; }
            } else {
                const u16x8 a = *(const u16x8*)(qrow + d0);
                for (int i = 0; i < 8; i++) v[i] = bf16_to_f32(a[i]);
            }
            qf[ks] = pack8(v[0] * sg, v[1] * sg, v[2] * sg, v[3] * sg, v[4] * sg, v[5] * sg,
                           v[6] * sg, v[7] * sg);
        }
    }

    int kend = Sk;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int ntiles = (kend + BN - 1) / BN;

    const bf16* Kg = (const bf16*)p.k + (size_t)bh * Skp * D;
    const bf16* Vg = (const bf16*)p.v + (size_t)bh * D * Skp;

    u32x4 kreg[KCH], vreg[VCH];
    auto gload = [&](int kt) {
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            kreg[i] = *(const u32x4*)(Kg + (size_t)(kt * BN + row) * D + col);
        }
        for (int i = 0; i < VCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BN / 8), col = (c % (BN / 8)) * 8;
            vreg[i] = *(const u32x4*)(Vg + (size_t)row * Skp + kt * BN + col);
        }
    };
    auto sstore = [&](int buf) {
        bf16* sK = smem + buf * (KTILE + VTILE);
        bf16* sV = sK + KTILE;
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 8), col = (c % (D / 8)) * 8;
            *(u32x4*)(sK + row * KST + col) = kreg[i];
        }
        for (int i = 0; i < VCH; i++) {
            const int c = tid + i * 256;
            const int row = c / (BN / 8), col = (c % (BN / 8)) * 8;
            *(u32x4*)(sV + row * VST + col) = vreg[i];
        }
    };

    f32x16 oacc[NDT];
    for (int t = 0; t < NDT; t++) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;
    const float c2 = p.scale_log2;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ntiles) gload(kt + 1);
        const bf16* sK = smem + buf * (KTILE + VTILE);
        const bf16* sV = sK + KTILE;

        // S^T (64 keys x 32 queries) as two 32x32 tiles.
        f32x16 sacc[2] = {f32x16{}, f32x16{}};
        for (int ks = 0; ks < NKS; ks++) {
            for (int mt = 0; mt < 2; mt++) {
                const bf16x8 a = *(const bf16x8*)(sK + (mt * 32 + ln) * KST + ks * 16 + g * 8);
                sacc[mt] = mfma_bf16(a, qf[ks], sacc[mt]);
            }
        }
        // Masks: causal (key > query) and the key end (key >= Sk).
        const int kbase = kt * BN;
        const bool need_mask = (kbase + BN > Sk) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
        if (need_mask) {
            for (int mt = 0; mt < 2; mt++)
                for (int r = 0; r < 16; r++) {
                    const int key = kbase + mt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (key >= Sk || (CAUSAL && key > qi)) sacc[mt][r] = -INFINITY;
                }
        }
        // Online softmax (all registers of a lane belong to query qi).
        float mx = -INFINITY;
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[mt][r]);
        mx = pair_max32(mx);
        const float mnew = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.f : fast_exp2((m - mnew) * c2);
        const float mc = mnew * c2;
        float rs = 0.f;
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) {
                const float e = fast_exp2(__builtin_fmaf(sacc[mt][r], c2, -mc));
                sacc[mt][r] = e;
                rs += e;
            }
        l = l * alpha + rs;
        m = mnew;
        for (int t = 0; t < NDT; t++) oacc[t] *= alpha;

        // O^T += V^T P^T over 4 k-steps of 16 keys.
        for (int ks = 0; ks < BN / 16; ks++) {
            const int mt = ks >> 1, b0 = (ks & 1) * 8;
            const bf16x8 pb = pack8(sacc[mt][b0 + 0], sacc[mt][b0 + 1], sacc[mt][b0 + 2],
                                    sacc[mt][b0 + 3], sacc[mt][b0 + 4], sacc[mt][b0 + 5],
                                    sacc[mt][b0 + 6], sacc[mt][b0 + 7]);
            for (int t = 0; t < NDT; t++) {
                const bf16x8 a = *(const bf16x8*)(sV + (t * 32 + ln) * VST + ks * 16 + g * 8);
                oacc[t] = mfma_bf16(a, pb, oacc[t]);
            }
        }
        if (kt + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    const float lt = pair_sum32(l);
    if (qi < Sq) {
        const float inv = 1.f / lt;
        float* orow = p.o + ((size_t)bh * Sq + qi) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq = 0; rq < 4; rq++) {
                f32x4 v;
                for (int i = 0; i < 4; i++) v[i] = oacc[t][rq * 4 + i] * inv;
                *(f32x4*)(orow + t * 32 + rq * 8 + g * 4) = v;
            }
        if (p.lse && g == 0) p.lse[(size_t)bh * Sq + qi] = m * p.scale_abs + fast_log2(lt) * kLn2;
    }
}

// ---------------------------------------------------------------------------
// fp32-MFMA forward (32 keys per tile).
// k-slot map of the QK^T product: step ks, group g <-> d = g*(D/2) + ks, so a
// lane reads its K row and holds its Q row as contiguous runs of floats.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fwd_f32_kernel(FwdParams p) {
    constexpr int BM = 128, BN = 32;
    constexpr int KST = D + 4, VST = D + 8;  // LDS row strides (floats)
    constexpr int KTILE = BN * KST, VTILE = BN * VST;
    constexpr int CH = BN * D / 4 / 256;  // 16-byte chunks per thread (each of K, V)
    constexpr int HD = D / 2;
    constexpr int NDT = D / 32;
    __shared__ __attribute__((aligned(16))) float smem[2 * (KTILE + VTILE)];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    int bh, qb;
    map_block(blockIdx.x, p.nqb, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qi = q0 + wave * 32 + ln;
    const int Sq = p.Sq, Sk = p.Sk;

    float qf[HD];
    {
        const float* qrow = (const float*)p.q + ((size_t)bh * Sq + (qi < Sq ? qi : 0)) * D + g * HD;
        const float sg = qi < Sq ? p.qsign : 0.f;
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = *(const f32x4*)(qrow + i);
            for (int j = 0; j < 4; j++) qf[i + j] = a[j] * sg;
        }
    }

    int kend = Sk;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int ntiles = (kend + BN - 1) / BN;
    const float* Kg = (const float*)p.k + (size_t)bh * Sk * D;
    const float* Vg = (const float*)p.v + (size_t)bh * Sk * D;

    f32x4 kreg[CH], vreg[CH];
    auto gload = [&](int kt) {
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            int key = kt * BN + row;
            key = key < Sk ? key : Sk - 1;  // clamped rows are masked
            kreg[i] = *(const f32x4*)(Kg + (size_t)key * D + col);
            vreg[i] = *(const f32x4*)(Vg + (size_t)key * D + col);
        }
    };
    auto sstore = [&](int buf) {
        float* sK = smem + buf * (KTILE + VTILE);
        float* sV = sK + KTILE;
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            *(f32x4*)(sK + row * KST + col) = kreg[i];
            *(f32x4*)(sV + row * VST + col) = vreg[i];
        }
    };

    f32x16 oacc[NDT];
    for (int t = 0; t < NDT; t++) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;
    const float c2 = p.scale_log2;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ntiles) gload(kt + 1);
        const float* sK = smem + buf * (KTILE + VTILE);
        const float* sV = sK + KTILE;

        f32x16 sacc = f32x16{};
        const float* krow = sK + ln * KST + g * HD;
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = *(const f32x4*)(krow + i);
            sacc = mfma_f32(a[0], qf[i + 0], sacc);
            sacc = mfma_f32(a[1], qf[i + 1], sacc);
            sacc = mfma_f32(a[2], qf[i + 2], sacc);
            sacc = mfma_f32(a[3], qf[i + 3], sacc);
        }
        const int kbase = kt * BN;
        const bool need_mask = (kbase + BN > Sk) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
        if (need_mask) {
            for (int r = 0; r < 16; r++) {
                const int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key >= Sk || (CAUSAL && key > qi)) sacc[r] = -INFINITY;
            }
        }
        float mx = -INFINITY;
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[r]);
        mx = pair_max32(mx);
        const float mnew = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.f : fast_exp2((m - mnew) * c2);
        const float mc = mnew * c2;
        float rs = 0.f;
        for (int r = 0; r < 16; r++) {
            const float e = fast_exp2(__builtin_fmaf(sacc[r], c2, -mc));
            sacc[r] = e;
            rs += e;
        }
        l = l * alpha + rs;
        m = mnew;
        for (int t = 0; t < NDT; t++) oacc[t] *= alpha;

        // O^T[d][q] += sum_key V[key][d] P[key][q]; step r <-> key 8(r/4)+4g+r%4.
        for (int r = 0; r < 16; r++) {
            const int key = 8 * (r >> 2) + 4 * g + (r & 3);
            const float* vrow = sV + key * VST + ln;
            for (int t = 0; t < NDT; t++) oacc[t] = mfma_f32(vrow[t * 32], sacc[r], oacc[t]);
        }
        if (kt + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    const float lt = pair_sum32(l);
    if (qi < Sq) {
        const float inv = 1.f / lt;
        float* orow = p.o + ((size_t)bh * Sq + qi) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq = 0; rq < 4; rq++) {
                f32x4 v;
                for (int i = 0; i < 4; i++) v[i] = oacc[t][rq * 4 + i] * inv;
                *(f32x4*)(orow + t * 32 + rq * 8 + g * 4) = v;
            }
        if (p.lse && g == 0) p.lse[(size_t)bh * Sq + qi] = m * p.scale_abs + fast_log2(lt) * kLn2;
    }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <int D, bool C>
static void launch_bf16_d(const FwdParams& p, int q_bf16, dim3 grid, hipStream_t s) {
    if (q_bf16)
        fwd_bf16_kernel<D, C, bf16><<<grid, 256, 0, s>>>(p);
    else
        fwd_bf16_kernel<D, C, float><<<grid, 256, 0, s>>>(p);
}

hipError_t launch_fwd(const FwdParams& p, int mode, int D, int causal, int q_bf16,
                      hipStream_t s) {
    dim3 grid(p.nqb * p.BH);
    if (mode == 1) {
        if (D == 64) {
            if (causal) launch_bf16_d<64, true>(p, q_bf16, grid, s);
            else launch_bf16_d<64, false>(p, q_bf16, grid, s);
        } else if (D == 128) {
            if (causal) launch_bf16_d<128, true>(p, q_bf16, grid, s);
            else launch_bf16_d<128, false>(p, q_bf16, grid, s);
        } else {
            return hipErrorInvalidValue;
        }
    } else {
        if (D == 64) {
            if (causal) fwd_f32_kernel<64, true><<<grid, 256, 0, s>>>(p);
            else fwd_f32_kernel<64, false><<<grid, 256, 0, s>>>(p);
        } else if (D == 128) {
            if (causal) fwd_f32_kernel<128, true><<<grid, 256, 0, s>>>(p);
            else fwd_f32_kernel<128, false><<<grid, 256, 0, s>>>(p);
        } else {
            return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace gonn
