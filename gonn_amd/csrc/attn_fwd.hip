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
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// bf16-MFMA forward.
//
// Pipeline (one barrier per 64-key tile): K and V have separate double
// buffers in LDS and V lags K by one tile. K(t+2) and V(t+1) stream from HBM
// straight into the LDS buffers step t no longer reads
// (buffer_load_dwordx4 ... lds: lane L of a wave writes 16 bytes at dst + 16 L),
// so no VGPRs stage them. The tiles keep a padded row stride (one spare
// 16-byte slot per row: conflict-free MFMA operand reads); the lanes that
// land on a pad slot load a dummy chunk.
//
// Step t (after the rare lazy rescale, one basic block): for each 16-key
// k-step of P(t), the exp2 / bf16 pack / row sum of the next k-step, the PV
// MFMAs of this one (NDT accumulator chains) and a quarter of the
// S^T(t+1) = K(t+1) Q^T MFMAs (2 chains), so 2 + NDT independent chains are
// in flight; LDS operand reads run a few MFMAs ahead. Then the mask (last
// two tiles only) and the row max of S^T(t+1). The loop is unrolled by two
// so S^T(t) and S^T(t+1) alternate between two register sets without copies.
// The wave raises its issue priority over the MFMA stream so the co-resident
// workgroup's VALU work fills its gaps. Counters and timing: VALU work per
// MFMA is well under the MFMA time; the loss is per-step latency (tile
// loads, the row-max chain, the barrier).
//
// Lazy rescaling: the running reference max m only moves when a lane's tile
// max exceeds it by more than kLazyLog2 (in log2 units), so P <= 2^kLazyLog2
// and the O / l rescale (64 multiplies per lane) runs only on those tiles. The
// result is exact in real arithmetic: O = sum_j 2^((s_j - m) c) v_j /
// sum_j 2^((s_j - m) c) for any fixed m, and LSE = m |scale| + ln(l).
// ---------------------------------------------------------------------------
constexpr float kLazyLog2 = 8.0f;

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSgVALU = 0x002, kSgMFMA = 0x008, kSgDSR = 0x100;

template <int D, bool CAUSAL, typename QT>
__global__ __launch_bounds__(256, 2) void fwd_bf16_kernel(FwdParams p) {
    constexpr int BM = 128, BN = 64;
    constexpr int KST = D + 8;   // K tile row stride (bf16)
    constexpr int VST = BN + 8;  // Vt tile row stride (bf16)
    constexpr int KTILE = BN * KST, VTILE = D * VST;
    constexpr int NKS = D / 16;            // k-steps of the QK^T product
    constexpr int NDT = D / 32;            // 32-row d-tiles of O^T
    __shared__ __attribute__((aligned(16))) bf16 sKb[2 * KTILE];
    __shared__ __attribute__((aligned(16))) bf16 sVb[2 * VTILE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
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
    // Direct-to-LDS tile loads. Position p = 16-byte slot of a padded tile;
    // instruction i of thread tid fills slot i*256 + tid.
    constexpr int KCP = KST / 8, KCD = D / 8, NKP = BN * KCP;  // K: slots per row, data slots
    constexpr int VCP = VST / 8, VCD = BN / 8, NVP = D * VCP;
    constexpr int NKI = (NKP + 255) / 256, NVI = (NVP + 255) / 256;
    constexpr int KLAST = NKP - (NKI - 1) * 256, VLAST = NVP - (NVI - 1) * 256;
    static_assert(KLAST % 64 == 0 && VLAST % 64 == 0, "partial instructions must be whole waves");
    // Byte offsets inside one global tile (32-bit: the loads use a scalar
    // 64-bit base plus a per-lane 32-bit offset).
    uint32_t koff[NKI], voff[NVI];
    for (int i = 0; i < NKI; i++) {
        const int pos = i * 256 + tid, row = pos / KCP, ch = pos % KCP;
        koff[i] = (uint32_t)(((pos < NKP ? row : 0) * D + (ch < KCD ? ch : 0) * 8) * 2);
    }
    for (int i = 0; i < NVI; i++) {
        const int pos = i * 256 + tid, row = pos / VCP, ch = pos % VCP;
        voff[i] = (uint32_t)(((pos < NVP ? row : 0) * Skp + (ch < VCD ? ch : 0) * 8) * 2);
    }
    const brsrc krs = make_rsrc(Kg, (uint32_t)Skp * D * 2);
    const brsrc vrs = make_rsrc(Vg, (uint32_t)Skp * D * 2);
    // LDS byte address of this wave's first slot in K / Vt buffer 0.
    const uint32_t kl = lds_addr(sKb) + wave * 64 * 16, vl = lds_addr(sVb) + wave * 64 * 16;
    auto dma_k = [&](int kt, int buf) {
        const uint32_t dst = kl + buf * KTILE * 2;
        for (int i = 0; i < NKI; i++)
            if (i < NKI - 1 || tid < KLAST) dma16(krs, dst + i * 4096, koff[i], kt * BN * D * 2);
    };
    auto dma_v = [&](int kt, int buf) {
        const uint32_t dst = vl + buf * VTILE * 2;
        for (int i = 0; i < NVI; i++)
            if (i < NVI - 1 || tid < VLAST) dma16(vrs, dst + i * 4096, voff[i], kt * BN * 2);
    };
    // Wait for this thread's tile loads.
    auto dma_wait = [] { GONN_VMCNT(0); };
    // S^T (64 keys x 32 queries) of one K tile as two 32x32 tiles.
    auto qk = [&](int buf, f32x16* s) {
        const bf16* sK = sKb + buf * KTILE + ln * KST + g * 8;
        s[0] = f32x16{};
        s[1] = f32x16{};
        for (int ks = 0; ks < NKS; ks++)
            for (int mt = 0; mt < 2; mt++) {
                const bf16x8 a = *(const bf16x8*)(sK + mt * 32 * KST + ks * 16);
                s[mt] = mfma_bf16(a, qf[ks], s[mt]);
            }
    };

    f32x16 oacc[NDT];
    for (int t = 0; t < NDT; t++) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;
    const float c2 = p.scale_log2;

    // Causal (key > query) and key-end (key >= Sk) masks of tile kt.
    auto mask = [&](int kt, f32x16* s) {
        const int kbase = kt * BN + 4 * g;
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) {
                const int key = kbase + mt * 32 + 8 * (r >> 2) + (r & 3);
                const bool off = key >= Sk || (CAUSAL && key > qi);
                s[mt][r] = off ? -INFINITY : s[mt][r];
            }
    };
    auto needs_mask = [&](int kt) {
        const int kbase = kt * BN;
        return (kbase + BN > Sk) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
    };
    // Row max of this lane's query over a tile (both lane halves).
    auto tile_max = [&](const f32x16* s) {
        float t8[8];
        for (int i = 0; i < 8; i++)
            t8[i] = fmaxf(fmaxf(s[i >> 2][(i & 3) * 4 + 0], s[i >> 2][(i & 3) * 4 + 1]),
                          fmaxf(s[i >> 2][(i & 3) * 4 + 2], s[i >> 2][(i & 3) * 4 + 3]));
        const float mx = fmaxf(fmaxf(fmaxf(t8[0], t8[1]), fmaxf(t8[2], t8[3])),
                               fmaxf(fmaxf(t8[4], t8[5]), fmaxf(t8[6], t8[7])));
        return pair_max32(mx);
    };
    float mxc;  // row max of the tile the next step consumes
    bool grow;  // that tile moves the reference max

    // One tile step: softmax + PV of `cur` (tile kt, already masked, its row
    // max in mxc); with NEXT, also S^T(kt+1) into `nxt`, its mask and row max,
    // and the prefetch of K(kt+2) / V(kt+1).
    auto step = [&](auto next_tag, int kt, f32x16* cur, f32x16* nxt) {
        constexpr bool NEXT = decltype(next_tag)::value;
        const int buf = kt & 1;
        if constexpr (NEXT) {
            // K(kt+2) -> the K buffer read by the previous step, V(kt+1) -> the
            // V buffer read by the previous step. A K index past the end is
            // clamped: the load is redundant and its buffer is not read again.
            dma_k(kt + 2 < ntiles ? kt + 2 : ntiles - 1, buf);
            dma_v(kt + 1, buf ^ 1);
        }
        // Lazy rescale (wave-uniform branch, rare after the first tile).
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float mnew = grow ? mxc : m;
            const float alpha = (m == -INFINITY) ? 0.f : fast_exp2((m - mnew) * c2);
            l *= alpha;
            for (int t = 0; t < NDT; t++) oacc[t] *= alpha;
            m = mnew;
        }
        const float mc = (m == -INFINITY) ? 0.f : m * c2;

        // ---- one basic block: PV(kt) and S^T(kt+1) MFMAs interleaved (up to
        // 6 independent accumulator chains), P for the next PV k-step computed
        // between them ----
        // Raised issue priority while this wave runs its MFMA stream, so the
        // co-resident wave's VALU work fills the gaps rather than the reverse.
        __builtin_amdgcn_s_setprio(1);
        float part[4] = {0.f, 0.f, 0.f, 0.f};
        bf16x8 pb[4];
        auto make_p = [&](int ks) {
            const int mt = ks >> 1, b0 = (ks & 1) * 8;
            float e[8];
            for (int i = 0; i < 8; i++) {
                e[i] = fast_exp2(__builtin_fmaf(cur[mt][b0 + i], c2, -mc));
                part[i & 3] += e[i];
            }
            pb[ks] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
        };
        const bf16* sV = sVb + buf * VTILE + ln * VST + g * 8;
        const bf16* sK = sKb + (buf ^ 1) * KTILE + ln * KST + g * 8;
        if constexpr (NEXT) {
            nxt[0] = f32x16{};
            nxt[1] = f32x16{};
        }
        constexpr int SKS = NKS / 4;  // S^T k-steps per PV k-step
        make_p(0);
        for (int ks = 0; ks < 4; ks++) {
            if (ks + 1 < 4) make_p(ks + 1);
            for (int t = 0; t < NDT; t++) {
                const bf16x8 a = *(const bf16x8*)(sV + t * 32 * VST + ks * 16);
                oacc[t] = mfma_bf16(a, pb[ks], oacc[t]);
            }
            if constexpr (NEXT) {
                for (int kk = ks * SKS; kk < (ks + 1) * SKS; kk++)
                    for (int mt = 0; mt < 2; mt++) {
                        const bf16x8 a = *(const bf16x8*)(sK + mt * 32 * KST + kk * 16);
                        nxt[mt] = mfma_bf16(a, qf[kk], nxt[mt]);
                    }
            }
        }
        l += (part[0] + part[1]) + (part[2] + part[3]);
        {
            // 24 VALU make one P k-step; each chunk of MFMAs carries one.
            constexpr int kMf = NDT + (NEXT ? 2 * SKS : 0);  // MFMAs per chunk
            constexpr int kVa = (24 + kMf - 1) / kMf;
            __builtin_amdgcn_sched_group_barrier(kSgVALU, 24, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDSR, 4, 0);
            for (int ks = 0; ks < 4; ks++)
                for (int i = 0; i < kMf; i++) {
                    __builtin_amdgcn_sched_group_barrier(kSgMFMA, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(kSgDSR, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(kSgVALU, kVa, 0);
                }
        }
        __builtin_amdgcn_s_setprio(0);
        if constexpr (NEXT) {
            if (needs_mask(kt + 1)) mask(kt + 1, nxt);
            mxc = tile_max(nxt);
            grow = (mxc - m) * c2 > kLazyLog2;
        }
        dma_wait();
        __syncthreads();
    };
    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;

    // Prologue: K(0), V(0), K(1) in LDS; S^T(0) in registers.
    dma_k(0, 0);
    dma_v(0, 0);
    if (ntiles > 1) dma_k(1, 1);
    dma_wait();
    __syncthreads();
    f32x16 s0[2], s1[2];
    qk(0, s0);
    if (needs_mask(0)) mask(0, s0);
    mxc = tile_max(s0);
    grow = (mxc - m) * c2 > kLazyLog2;
    // Step 0 streams K(2) into the buffer qk(0) just read: every wave must be
    // done reading it first.
    __syncthreads();

    int kt = 0;
    for (; kt + 2 < ntiles; kt += 2) {
        step(Yes{}, kt, s0, s1);
        step(Yes{}, kt + 1, s1, s0);
    }
    if (kt + 1 < ntiles) {
        step(Yes{}, kt, s0, s1);
        step(No{}, kt + 1, s1, s0);
    } else {
        step(No{}, kt, s0, s1);
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
