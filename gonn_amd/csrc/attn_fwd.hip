// attn_fwd.hip -- flash-attention forward for gfx950 (MI355X).
//
// Replaces the reference's fp64 one-thread-per-row kernels
// flash_attn_f64_tiled / flash_attn_f64_kernel (backend/cuda/gonn_cuda.cu:302-331,
// :389-450). Same result definition: O = softmax(scale*QK^T + mask) V and
// L = m + ln(l) per query row (gonn_cuda.cu:330, :448), causal mask j > i.
//
// Design (one workgroup = 4 wave64s = 128 query rows of one (b,h) slice):
//  * each wave owns 32 query rows; its Q fragment stays in VGPRs;
//  * K/V tiles are staged in LDS (two-slot rings, one barrier per tile); the
//    bf16 kernel fills them with direct-to-LDS 128-bit loads (buffer_load
//    ... lds) one to three tiles ahead, the fp32 kernel through registers;
//  * S^T = K Q^T on MFMA, so every lane holds scores of ONE query: the row
//    max/sum of the online softmax is in-lane plus one v_permlane32_swap;
//  * O^T += V^T P^T on MFMA straight from the S^T registers (no LDS trip for
//    P); the output accumulator then also holds one query per lane, so the
//    rescale by exp2(m_old - m_new) is in-lane;
//  * scale*log2(e) is folded into the packed Q (bf16 mode) or into one
//    multiply before v_exp_f32 (fp32 mode);
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
#include <atomic>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// Lazy rescaling (both MFMA forwards): the running reference max only moves
// when a tile's scores exceed it by more than kLazyLog2 (log2 units), so P
// stays bounded and the O / l rescale runs only on those tiles. The result
// is exact in real arithmetic: O = sum_j 2^((s_j - m) c) v_j /
// sum_j 2^((s_j - m) c) for any fixed m, and LSE = m |scale| + ln(l).
// ---------------------------------------------------------------------------
constexpr float kLazyLog2 = 8.0f;

// Keys of slice bh that take part: Sk, or the sequence's kv_len clamped to
// [0, Sk] (a prefix key-padding mask).
GONN_DEV int fwd_keys(const FwdParams& p, int bh) {
    if (!p.kv_len) return p.Sk;
    int l = p.kv_len[bh / p.H];
    l = l < 0 ? 0 : (l > p.Sk ? p.Sk : l);
    return __builtin_amdgcn_readfirstlane(l);
}

// Rows q0 .. q0 + rows - 1 of slice bh when the slice has no key at all:
// O = 0, LSE = -inf.
template <int D>
GONN_DEV void fwd_empty_rows(const FwdParams& p, int bh, int q0, int rows) {
    const int r1 = q0 + rows < p.Sq ? q0 + rows : p.Sq;
    if (r1 <= q0) return;
    float* o = p.o + ((size_t)bh * p.Sq + q0) * D;
    for (int i = threadIdx.x; i < (r1 - q0) * D; i += blockDim.x) o[i] = 0.f;
    if (p.lse)
        for (int r = q0 + threadIdx.x; r < r1; r += blockDim.x) p.lse[(size_t)bh * p.Sq + r] = -INFINITY;
}

// ---------------------------------------------------------------------------
// bf16-MFMA forward for D = 128: 4 wave64s (32 query rows each) per
// workgroup, two workgroups per CU (two waves per SIMD).
//
// Three-stage software pipeline. Step t issues, with no dependency between
// them inside the step:
//   MFMA  O^T += V(t)^T P(t)            (P(t) packed by step t-1)
//   MFMA  S^T(t+2) = K(t+2) Q^T - mc     (K(t+2) landed by the end of step t-1)
//   VALU  P(t+1) = exp2(S^T(t+1)) packed to bf16, row sums
// so the MFMA stream never waits on the softmax of the tile it is computing.
//
// The step is issue-bound (each wave issues its own MFMAs, their LDS operand
// reads and waits, the softmax VALU and the tile loads), so the per-score work
// is cut to one exp2, half a bf16 pack and half a v_dot2:
//  * |scale| log2(e) is folded into the packed Q and the first MFMA of each
//    S^T tile accumulates onto a register block holding -mc, so the MFMA
//    result already is the exp2 argument s c - mc (no per-score FMA);
//  * no per-tile row max: P = exp2(s c - mc) is exact for any offset mc,
//    which only has to keep P bounded. A tile whose row sum exceeds 2^14 (or
//    is not finite) takes a rare, wave-uniform branch that computes the tile
//    max, moves mc to it, recomputes the tile's P, shifts the S^T tile already
//    accumulated against the old offset and rescales l and O by
//    alpha = 2^(old - new). Otherwise every score is below mc + 14, so P, l
//    and O stay far inside fp32 range, and their relative precision does not
//    depend on mc. The first tile (prologue) uses its exact max.
//
// LDS: two-slot rings of K tiles (64 keys x D) and Vt tiles (D x 64 keys)
// filled straight from HBM/L2 by buffer_load ... lds, one barrier per step;
// step t loads K(t+3) and V(t+1), one step ahead, in every other slot of the
// first 16 of its 32 MFMA slots (the last load then still has half the step
// to arrive before the step's closing wait). The prologue stages K(0) in Vt
// slot 1 (free until step 0 loads V(1)), so K(0), K(1), K(2), V(0) and the Q
// fragment arrive in one memory round trip. Tiles are stored without padding
// in the swizzled layout of slab_swz (conflict-free MFMA operand reads,
// 64 contiguous bytes per row per load, no dummy or partial loads: four load
// instructions per 16 KB tile). Each load's M0 (its LDS base) is written one
// slot ahead, so the M0 -> LDS-DMA wait state is filled by an MFMA, not a nop.
//
// Every step has the same form: the last two steps compute S^T of tiles past
// the end and the last one their softmax; those keys lie past the key end
// (or the causal diagonal), so the mask sets the whole tile to -inf and
// P = 0 adds nothing to l or O. One step form keeps the register allocation
// the same in every step (tail variants spilled), for two masked S^T tiles
// per q-block.
// ---------------------------------------------------------------------------
constexpr float kSumBound = 16384.f;  // 2^14: row-sum bound of one 64-key tile
// Wave issue priority (s_setprio) during a step's MFMA stream.
constexpr int kFwdStreamPrio = 1;
// Waves per workgroup of the pipelined bf16 forward.
constexpr int kFwdWaves = 4;
// Resident workgroups per CU the pipelined forward is compiled for (its
// register budget): two, or one for D = 128 with the additive mask's
// registers. The kernel is written for any D that is a multiple of 32 and
// runs every bf16 call (D = 64 and 128). At D = 64 it takes 185-209 VGPRs:
// two workgroups per CU run C2's 768 q-blocks in 1.5 rounds, where an older
// two-stage kernel fitted three per CU in one round, and it is still 3%
// faster there (leaner softmax: no per-tile row max, no per-tile
// accumulator seeding); built for three per CU it spills (112 B/lane) and is
// 40% slower. With the additive mask at D = 64 it replaced that kernel too:
// 77.6 -> 76.9 us non-causal, 70.7 -> 68.3 us causal on the C2 shape with a
// (B, S, S) mask (same box, three interleaved rounds). Non-causal unmasked
// D = 64 (C2) keeps its S^T tiles absolute (P = exp2(s - mc), one subtract
// per score, the MASK variant's form), which frees the 16 registers of the
// -mc block: 168 VGPRs, three workgroups per CU, C2's 768 q-blocks in one
// round: 39.7 -> 37.8 us (same box, three interleaved rounds). Causal
// D = 64 stays at two (three measured +3.7% at S = 4096).
constexpr int fwd_pipe_wgs(int D, bool mask, bool causal) {
    return mask ? (D == 128 ? 1 : 2) : (D == 64 && !causal ? 3 : 2);
}

template <int D, bool CAUSAL, typename QT, bool MASK>
__global__ __launch_bounds__(256, fwd_pipe_wgs(D, MASK, CAUSAL)) void fwd_bf16_pipe_kernel(FwdParams p) {
    constexpr int NW = kFwdWaves, BM = NW * 32, BN = 64, NT = NW * 64;
    constexpr int NKS = D / 16, NDT = D / 32;
    // Absolute S^T tiles (P = exp2(s - mc)) instead of tiles accumulated
    // onto -mc: with the additive mask, and for non-causal D = 64.
    constexpr bool ABS = MASK || (D == 64 && !CAUSAL);
    // Swizzled tiles without padding (layout at slab_swz): 16 KB per tile
    // at D = 128, two-slot K and Vt rings, 64 KB per workgroup. Step t loads
    // K(t+3) and V(t+1), each one step ahead of its use.
    constexpr uint32_t KTB = BN * D * 2, VTB = D * BN * 2;  // slot bytes
    constexpr int KSLOTS = 2, VSLOTS = 2;
    constexpr int KLEAD = 3, VLEAD = 1;
    __shared__ __attribute__((aligned(16))) bf16 sKb[KSLOTS * BN * D];
    __shared__ __attribute__((aligned(16))) bf16 sVb[VSLOTS * D * BN];
    // Additive mask (MASK variant): one 64-key tile of this wave's 32 rows,
    // 8 KB per wave, written and read by that wave only.
    __shared__ __attribute__((aligned(16))) float sMk[MASK ? NW * 32 * BN : 4];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    int bh, qb;
    map_block(blockIdx.x, p.nqb, p.BH, CAUSAL, bh, qb, CAUSAL ? p.hgroup : 1);
    const int Sq = p.Sq, Sk = fwd_keys(p, bh), Skp = p.Skp;
    if (Sk == 0) {  // uniform: the whole slice is padded
        fwd_empty_rows<D>(p, bh, qb * BM, BM);
        return;
    }
    const int q0 = qb * BM, qw = q0 + wave * 32, qi = qw + ln;
    const float c2 = p.scale_log2;
    int ntiles;
    {
        int kend = Sk;
        if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
        ntiles = (kend + BN - 1) / BN;
    }
    // Additive mask (MASK variant): the values of S^T(t+2) are loaded at the
    // start of step t and added when that tile is complete, at the step's
    // end. A lane's own scores are 4-key runs of its query's row, 32 bytes of
    // it per load instruction: loaded straight into registers, one
    // instruction touches 32 rows' cache lines for 32 bytes of each, and the
    // mask stream cost the D = 64 forward 30 of its 74 us. So each wave
    // stages its 32 rows of the tile in its own LDS slot instead, each load
    // instruction filling 4 whole 256-byte rows (16-byte chunk c of row r at
    // chunk slot c ^ (r % 16), which keeps the lanes' reads conflict-free),
    // and reads its values back after the step's closing wait. The prologue's
    // two tiles go straight to registers.
    MaskRow mrow{};
    f32x4 mreg[8];
    uint32_t moff[MASK ? 8 : 1];
    if constexpr (MASK) {
        mrow.init(p.mask, p.mask_sb, p.mask_sh, p.H, p.Sq, p.Sk, bh, qi);
        for (int i = 0; i < 8; i++) {
            const int r = 4 * i + (lane >> 4), q = qw + r < Sq ? qw + r : Sq - 1;
            moff[i] = (uint32_t)(q * p.Sk) * 4u + (uint32_t)(((lane & 15) ^ (r & 15)) * 16);
        }
    }
    const uint32_t mkl = lds_addr(sMk) + wave * 32 * BN * 4;
    auto mask_dma = [&](int kt) {
        for (int i = 0; i < 8; i++) dma16(mrow.rs, mkl + i * 1024, moff[i], (uint32_t)kt * BN * 4);
    };
    auto mask_add_lds = [&](f32x16* s) {
        const char* base = (const char*)sMk + wave * 32 * BN * 4 + ln * BN * 4;
        for (int mt = 0; mt < 2; mt++)
            for (int j = 0; j < 4; j++) {
                const int c = 8 * mt + 2 * j + g;
                const f32x4 m = *(const f32x4*)(base + ((c ^ (ln & 15)) << 4));
                for (int e = 0; e < 4; e++)
                    s[mt][4 * j + e] = __builtin_fmaf(m[e], kLog2e, s[mt][4 * j + e]);
            }
    };

    // Q fragment: qf[ks] = Q[qi][16ks + 8g .. +7] * sign(scale) * c2, in bf16.
    // Loaded in the prologue after the first tile loads are issued, so the
    // Q load and the K/V tile loads share one memory round trip.
    bf16x8 qf[NKS];
    auto load_q = [&]() {
        const QT* qrow = (const QT*)p.q + ((size_t)bh * Sq + (qi < Sq ? qi : 0)) * D;
        const float sg = qi < Sq ? p.qsign * c2 : 0.f;
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
    };

    // ---- tile loads: instruction i of thread tid fills 16-byte position
    // i*NT + tid of a tile (slab_chunk gives the row and chunk it holds) ----
    constexpr int NKP = BN * D / 8, NVP = D * BN / 8;  // 16-byte chunks per tile
    static_assert(NKP % NT == 0 && NVP % NT == 0, "tiles are whole load instructions");
    constexpr int NKI = NKP / NT, NVI = NVP / NT;      // loads per tile
    uint32_t koff[NKI], voff[NVI];
    for (int i = 0; i < NKI; i++) {
        int r, c;
        slab_chunk(i * NT + tid, BN, r, c);
        koff[i] = (uint32_t)((r * D + c * 8) * 2);
        slab_chunk(i * NT + tid, D, r, c);
        voff[i] = (uint32_t)((r * Skp + c * 8) * 2);
    }
    const bf16* Kg = (const bf16*)p.k + (size_t)bh * Skp * D;
    const bf16* Vg = (const bf16*)p.v + (size_t)bh * D * Skp;
    const brsrc krs = make_rsrc(Kg, (uint32_t)Skp * D * 2);
    const brsrc vrs = make_rsrc(Vg, (uint32_t)Skp * D * 2);
    const uint32_t kl = lds_addr(sKb) + wave * 1024, vl = lds_addr(sVb) + wave * 1024;
    // Load i of K tile kt into the K-layout tile at LDS address base (this
    // wave's part of it; M0 written by the call).
    auto dma_ki_at = [&](int kt, uint32_t base, int i) {
        dma16(krs, base + i * NT * 16, koff[i], kt * BN * D * 2);
    };
    auto dma_k = [&](int kt, int slot) {
        for (int i = 0; i < NKI; i++) dma_ki_at(kt, kl + slot * KTB, i);
    };
    // K(0) is staged in Vt slot 1, which no tile occupies before step 0
    // loads V(1), so the prologue issues K(0), K(1), K(2) and V(0) at once.
    static_assert(KTB <= VTB, "a K tile fits in a Vt slot");
    auto dma_k0_staged = [&]() {
        for (int i = 0; i < NKI; i++) dma_ki_at(0, vl + VTB, i);
    };
    auto dma_v = [&](int kt, int slot) {
        for (int i = 0; i < NVI; i++)
            dma16(vrs, vl + slot * VTB + i * NT * 16, voff[i], kt * BN * 2);
    };

    // ---- MFMA operand reads: K row mt*32 + ln, Vt row dt*32 + ln; chunk
    // 2ks + g. In the layout of slab_swz the byte offset of (row, chunk) in a tile is
    // (chunk / 4) * rows * 64 + row * 64 + ((chunk % 4) ^ h(row)) * 16; for
    // row = 32 m + ln and chunk = 2 ks + g the lane part depends on ks only
    // through ks & 1, so two lane offsets serve every K and Vt read. ----
    const int hs = slab_swz(ln);
    const uint32_t qa0 = (uint32_t)(ln * 64 + ((0 + g) ^ hs) * 16);  // k-step even
    const uint32_t qa1 = (uint32_t)(ln * 64 + ((2 + g) ^ hs) * 16);  // k-step odd
    const char* sKc = (const char*)sKb;
    const char* sVc = (const char*)sVb;
    auto kfrag = [&](uint32_t base, int ks, int mt) {
        return *(const bf16x8*)(sKc + (base + ((ks & 1) ? qa1 : qa0)) +
                                ((ks >> 1) * BN + mt * 32) * 64);
    };
    auto vfrag = [&](uint32_t base, int ks, int dt) {
        return *(const bf16x8*)(sVc + (base + ((ks & 1) ? qa1 : qa0)) +
                                ((ks >> 1) * D + dt * 32) * 64);
    };

    f32x16 oacc[NDT];
    for (int dt = 0; dt < NDT; dt++) oacc[dt] = f32x16{};
    // mc: this lane's running offset (log2 units); l: row sum relative to it;
    // nmc: -mc in every element, the first S^T accumulator of each tile.
    // ABS (the MASK variant, and non-causal D = 64): S^T tiles stay
    // absolute (nmc unused) and P = exp2(s - mc).
    // An additive mask can make a whole tile huge and negative (-1e30 blocks
    // keys); an offset taken from such a tile would absorb every later score
    // if it were folded into the accumulator, so the offset stays out of it.
    float mc = 0.f, l = 0.f, alpha = 1.f;
    f32x16 nmc = f32x16{};

    // Key kt * BN + 4g + c of register (mt, r), c = 32 mt + 8 (r / 4) + r % 4,
    // is masked when past the key end or (causal) past this lane's query,
    // i.e. when c exceeds one per-lane threshold: a compare against a
    // constant and a select per score.
    auto mask = [&](int kt, f32x16* s) {
        int lim = Sk - 1;
        if (CAUSAL) lim = qi < lim ? qi : lim;
        const int thr = lim - (kt * BN + 4 * g);
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++) {
                const int c = mt * 32 + 8 * (r >> 2) + (r & 3);
                s[mt][r] = c > thr ? -INFINITY : s[mt][r];
            }
    };
    auto needs_mask = [&](int kt) {
        const int kb = kt * BN;
        return (kb + BN > Sk) || (CAUSAL && kb + BN - 1 > qw);
    };
    auto tile_max = [&](const f32x16* s) {
        float t8[8];
        for (int i = 0; i < 8; i++)
            t8[i] = fmaxf(fmaxf(s[i >> 2][(i & 3) * 4 + 0], s[i >> 2][(i & 3) * 4 + 1]),
                          fmaxf(s[i >> 2][(i & 3) * 4 + 2], s[i >> 2][(i & 3) * 4 + 3]));
        const float mx = fmaxf(fmaxf(fmaxf(t8[0], t8[1]), fmaxf(t8[2], t8[3])),
                               fmaxf(fmaxf(t8[4], t8[5]), fmaxf(t8[6], t8[7])));
        return pair_max32(mx);
    };
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one2 = {(__bf16)1.0f, (__bf16)1.0f};
    // Whole-tile P = exp2(s + off) as packed bf16 pairs, and its row sum
    // (prologue and the rare rescale branch).
    auto p_tile = [&](const f32x16* s, u32x4* pk, float off) {
        float part[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < 16; k++) {
            const int mt = k >> 3, r = (k & 7) * 2;
            const bf16x2 pr = {to_bf16(fast_exp2(s[mt][r] + off)),
                               to_bf16(fast_exp2(s[mt][r + 1] + off))};
            part[k & 3] = __builtin_amdgcn_fdot2_f32_bf16(pr, one2, part[k & 3], false);
            pk[k >> 2][k & 3] = __builtin_bit_cast(uint32_t, pr);
        }
        return (part[0] + part[1]) + (part[2] + part[3]);
    };
    u32x4 pp[4];  // P of the tile PV consumes next, bf16 pairs per 32-bit word

    // One pipeline step (see the header). sA <- S^T(t+2) - mc, sB = S^T(t+1) - mc;
    // pp holds P(t) and is overwritten with P(t+1) 16 keys at a time, each
    // part after the PV MFMAs that read it were issued.
    //
    // The step is scheduled by hand: slot e issues the LDS read of MFMA e+3,
    // MFMA e, possibly one tile load (or the M0 write of the next slot's
    // load) and the softmax micro-op mapped to it, and a sched_barrier keeps
    // the compiler from regrouping slots (left to itself it serialises the
    // S^T chains behind their LDS reads). MFMA order per 16-key PV k-step j:
    // PV(j, dt = 0..3), then S^T k-steps 2j and 2j+1 (mt = 0, 1), so six
    // accumulator chains interleave.
    // TAIL: 0 a full step; 1 the block's next-to-last step (no S^T(t+2) and
    // no K load: that tile is past the block); 2 its last step (no P(t+1)
    // and no tile loads either, and a wave whose rows all precede tile t's
    // first key skips its PV MFMAs: P(t) is zero there).
    auto step = [&](int t, f32x16* sA, f32x16* sB, auto TAILC) __attribute__((always_inline)) {
        constexpr int TAIL = decltype(TAILC)::value;
        const bool pv_dead = CAUSAL && TAIL == 2 && t * BN > qw + 31;
        const int kslot = (t + KLEAD) & (KSLOTS - 1);
        const int vslot = (t + 1) & 1;
        // Tiles past the last one are clamped to it: such a load refills a
        // slot no later step reads as real data (its S^T tile is masked).
        const int kload = t + KLEAD < ntiles ? t + KLEAD : ntiles - 1;
        const int vload = t + VLEAD < ntiles ? t + VLEAD : ntiles - 1;
        // Diagonal / key-end tiles only (a wave-uniform branch ahead of the
        // step's MFMA stream).
        if constexpr (TAIL < 2)
            if (needs_mask(t + 1)) mask(t + 1, sB);
        if constexpr (MASK && TAIL == 0) mask_dma(t + 2 < ntiles ? t + 2 : ntiles - 1);
        const uint32_t vb = (uint32_t)(t & 1) * VTB;
        const uint32_t kb = (uint32_t)((t + 2) & (KSLOTS - 1)) * KTB;

        constexpr int SKS = NKS / 4;       // S^T k-steps per PV k-step
        constexpr int GW = NDT + 2 * SKS;  // MFMAs per PV k-step group
        constexpr int NM = 4 * GW;         // MFMAs in the step
        constexpr int NU = 16;             // softmax micro-ops (one score pair each)
        constexpr int LA = 3;              // LDS read lead (MFMAs)
        constexpr int NDMA = NKI + NVI;    // tile loads of a step (K first)
        // Slots between tile loads: two (an M0 write needs the slot before
        // its load), so every load of the step is issued in its first
        // 2 NDMA slots and has the rest of the step to arrive.
        constexpr int DS = 2;
        static_assert(DS * NDMA <= NM, "the step's tile loads fit in its slots");
        bf16x8 opr[4];
        auto fetch = [&](auto E) {
            constexpr int e = decltype(E)::value, j = e / GW, w = e % GW;
            if constexpr (w < NDT) opr[e & 3] = vfrag(vb, j, w);
            else if constexpr (TAIL == 0)
                opr[e & 3] = kfrag(kb, SKS * j + ((w - NDT) >> 1), (w - NDT) & 1);
        };
        auto issue = [&](auto E) {
            constexpr int e = decltype(E)::value, j = e / GW, w = e % GW;
            if constexpr (w < NDT) {
                if (TAIL < 2 || !pv_dead)
                    oacc[w] = mfma_bf16(opr[e & 3], __builtin_bit_cast(bf16x8, pp[j]), oacc[w]);
            } else if constexpr (TAIL == 0) {
                constexpr int kk = SKS * j + ((w - NDT) >> 1), mt = (w - NDT) & 1;
                sA[mt] = mfma_bf16(opr[e & 3], qf[kk], kk == 0 ? (ABS ? f32x16{} : nmc) : sA[mt]);
            }
        };
        // Tile load d (0 .. NDMA-1) at slot 1 + d*DS: the K(t+3) loads, then
        // the V(t+1) loads. Its M0 is written at the slot before.
        auto dma_slot = [&](auto E) {
            constexpr int e = decltype(E)::value;
            // Tail steps load no K tile (TAIL >= 1) and no V tile (TAIL 2).
            constexpr int d0 = TAIL == 0 ? 0 : (TAIL == 1 ? NKI : NDMA);
            if constexpr (e % DS == 0 && e / DS < NDMA && e / DS >= d0) {
                constexpr int d = e / DS;
                const uint32_t lds = d < NKI ? kl + kslot * KTB + d * NT * 16
                                             : vl + vslot * VTB + (d - NKI) * NT * 16;
                dma_set_m0(lds);
            }
            if constexpr (e >= 1 && (e - 1) % DS == 0 && (e - 1) / DS < NDMA &&
                          (e - 1) / DS >= d0) {
                constexpr int d = (e - 1) / DS;
                if constexpr (d < NKI) dma16_m0(krs, koff[d], kload * BN * D * 2);
                else dma16_m0(vrs, voff[d - NKI], vload * BN * 2);
            }
        };
        float part[4] = {0.f, 0.f, 0.f, 0.f};
        // Score pair k (16 keys j = k / 4 of P(t+1)) in two micro-ops two
        // slots apart so no slot waits on a dependent VALU result: (0) exp2,
        // (1) bf16 pack into pp and row sum. Stage 1 lands in slot uslot(k),
        // after the PV MFMAs of k-step j read pp[j]; micro-ops past the
        // stream's end run after it.
        auto uslot = [](int k) { return (k >> 2) * GW + NDT + (k & 3); };
        float ub[16][2];
        auto uop = [&](auto U, auto S) {
            constexpr int k = decltype(U)::value, stage = decltype(S)::value;
            constexpr int mt = k >> 3, r = (k & 7) * 2;
            if constexpr (stage == 0) {
                if constexpr (ABS) {
                    ub[k][0] = fast_exp2(sB[mt][r] - mc);
                    ub[k][1] = fast_exp2(sB[mt][r + 1] - mc);
                } else {
                    ub[k][0] = fast_exp2(sB[mt][r]);
                    ub[k][1] = fast_exp2(sB[mt][r + 1]);
                }
                pin(ub[k][0]);
                pin(ub[k][1]);
            } else {
                const bf16x2 pr = {to_bf16(ub[k][0]), to_bf16(ub[k][1])};
                part[k & 3] = __builtin_amdgcn_fdot2_f32_bf16(pr, one2, part[k & 3], false);
                pp[k >> 2][k & 3] = __builtin_bit_cast(uint32_t, pr);
                pin(pp[k >> 2][k & 3]);
                pin(part[k & 3]);
            }
        };
        // Run the micro-ops of slot e (stage st of pair k sits at slot
        // uslot(k) - 2 + 2 st); e = NM runs everything past the stream's end.
        auto uops_at = [&](auto E) {
            constexpr int e = decltype(E)::value;
            if constexpr (TAIL == 2) return;  // P(t+1) is past the block
            static_for<2>([&](auto S) {
                static_for<NU>([&](auto U) {
                    constexpr int at = uslot(decltype(U)::value) - 2 + 2 * decltype(S)::value;
                    if constexpr (e < NM ? at == e : at >= NM) uop(U, S);
                });
            });
        };
        // Raised issue priority over the MFMA stream: on a SIMD shared with
        // the other workgroup's wave, that wave's step start and barrier
        // then fill the gaps of this stream rather than delay it.
        __builtin_amdgcn_s_setprio(kFwdStreamPrio);
        static_for<LA>([&](auto E) { fetch(E); });
        static_for<NM>([&](auto E) {
            constexpr int e = decltype(E)::value;
            if constexpr (e + LA < NM) fetch(std::integral_constant<int, e + LA>{});
            issue(E);
            dma_slot(E);
            // Softmax micro-ops; their results are pinned (an empty asm) so
            // IR passes cannot sink the work out of its slot.
            uops_at(E);
            __builtin_amdgcn_sched_barrier(0);
        });
        uops_at(std::integral_constant<int, NM>{});
        __builtin_amdgcn_s_setprio(0);
        float ts = (part[0] + part[1]) + (part[2] + part[3]);
        alpha = 1.f;
        // Rare: the tile's P is not bounded by the current offset (or is not
        // finite). Move the offset to the tile max (log2 units), redo the
        // tile, and shift S^T(t+2), accumulated against the old offset.
        if constexpr (ABS) {
            // Absolute tiles. Also taken while the row holds nothing (l = 0:
            // every earlier key blocked or -inf), so the offset follows the
            // first tile with a finite score instead of staying at a level
            // below which the tile's P would underflow.
            // (Not in the last step: no P(t+1) there, and sB is not a tile.)
            if (TAIL < 2 && __builtin_amdgcn_ballot_w64(!(ts <= kSumBound) || l == 0.f)) {
                const float mx = tile_max(sB);
                const bool empty = pair_sum32(l) == 0.f;
                const float mn =
                    mx > -INFINITY && (empty || mx - mc > kLazyLog2) ? mx : mc;
                alpha = empty ? 0.f : fast_exp2(mc - mn);
                mc = mn;
                ts = p_tile(sB, pp, -mc);
            }
        } else if (TAIL < 2 && __builtin_amdgcn_ballot_w64(!(ts <= kSumBound))) {
            const float mx = tile_max(sB);  // relative to mc
            const float dlt = mx > kLazyLog2 ? -mx : 0.f;
            alpha = fast_exp2(dlt);
            mc -= dlt;
            ts = p_tile(sB, pp, dlt);
            for (int mt = 0; mt < 2; mt++) sA[mt] += dlt;
            nmc = f32x16{} - mc;
        }
        l = l * alpha + ts;

        // K(t+3) and V(t+1), which step t+1 reads, have landed.
        GONN_VMCNT(0);
        __syncthreads();
        if constexpr (MASK && TAIL == 0) mask_add_lds(sA);
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f))
            for (int dt = 0; dt < NDT; dt++) oacc[dt] *= alpha;
    };

    // ---- prologue: S^T(0) -> P(0), S^T(1); the rings hold what step 0 needs ----
    f32x16 s0[2], s1[2];
    // S^T of the K-layout tile starting at LDS byte `tile`.
    auto qk_tile = [&](const char* tile, f32x16* s, f32x16 c) {
        s[0] = c;
        s[1] = c;
        for (int ks = 0; ks < NKS; ks++)
            for (int mt = 0; mt < 2; mt++)
                s[mt] = mfma_bf16(*(const bf16x8*)(tile + ((ks & 1) ? qa1 : qa0) +
                                                   ((ks >> 1) * BN + mt * 32) * 64),
                                  qf[ks], s[mt]);
    };
    auto last = [&](int kt) { return kt < ntiles ? kt : ntiles - 1; };
    // One memory round trip: K(0) (staged in Vt slot 1), K(1), K(2), V(0)
    // and the Q fragment are all in flight together.
    dma_k0_staged();
    dma_k(last(1), 1);
    dma_k(last(2), 0);
    dma_v(0, 0);
    load_q();
    GONN_VMCNT(0);
    __syncthreads();
    qk_tile(sVc + VTB, s0, f32x16{});
    // K(1), or for a one-tile block a masked copy of K(0): issued before the
    // VALU of tile 0 so the two overlap; -mc is added once mc is known.
    qk_tile(sKc + KTB, s1, f32x16{});
    if constexpr (MASK) {
        mrow.load(0, g, mreg);
        MaskRow::add(mreg, s0);
    }
    // First tile: exact offset (its max; key 0 is never masked by the
    // causal or key-end mask, so it is finite unless the additive mask
    // makes it -inf).
    if (needs_mask(0)) mask(0, s0);
    mc = tile_max(s0);
    if constexpr (ABS) {
        if (!(mc > -INFINITY)) mc = 0.f;  // a first tile of -inf: no offset yet
    } else {
        nmc = f32x16{} - mc;
        for (int mt = 0; mt < 2; mt++) s1[mt] += nmc;
    }
    l = p_tile(s0, pp, -mc);
    if constexpr (MASK) {
        mrow.load(last(1), g, mreg);
        MaskRow::add(mreg, s1);
    }
    // K(0) and K(1) read by every wave: step 0 loads V(2) and K(3) over them.
    __syncthreads();

    {
        // S^T(k) lives in s[k & 1]. Full steps up to the block's last two,
        // then the tail steps: 1 reads S^T(ntiles - 1) as sB, 2 reads only
        // P(ntiles - 1) (no S^T tile). One copy of each tail step: when the
        // next-to-last index is odd, s0 and s1 trade contents first.
        const std::integral_constant<int, 0> full;
        const std::integral_constant<int, 1> tail1;
        const std::integral_constant<int, 2> tail2;
        const int nfull = ntiles - 2;
        int t = 0;
        for (; t + 1 < nfull; t += 2) {
            step(t, s0, s1, full);
            step(t + 1, s1, s0, full);
        }
        if (t < nfull) step(t++, s0, s1, full);
        if (ntiles >= 2) {
            if (t & 1)
                for (int mt = 0; mt < 2; mt++) {
                    const f32x16 x = s0[mt];
                    s0[mt] = s1[mt];
                    s1[mt] = x;
                }
            step(t, s0, s1, tail1);
        }
        step(ntiles - 1, s1, s0, tail2);
    }
    // The last steps leave V loads in flight; they write this workgroup's
    // LDS, so they land before the waves exit.
    GONN_VMCNT(0);

    const float lt = pair_sum32(l);
    const float inv = 1.f / lt;
    if constexpr (D == 128) {
        // O through LDS (the rings are free now): each wave writes its 32
        // normalised rows, 16-byte chunk c of row r at chunk slot c ^ r, and
        // reads them back so that each store instruction writes two whole
        // rows (1 KB contiguous) instead of 32 rows x 32 bytes: C3 0.594 ->
        // 0.586 ms (same-box A/B). At D = 64 the direct stores were as fast.
        constexpr int NC = D / 4;            // 16-byte chunks per row
        constexpr int RPI = 64 / NC;         // rows per store instruction
        constexpr uint32_t WB = 32 * D * 4;  // bytes per wave
        static_assert(2 * WB <= sizeof(sKb) && 2 * WB <= sizeof(sVb), "O staging fits");
        char* reg = (char*)(wave < 2 ? (void*)sKb : (void*)sVb) + (wave & 1) * WB;
        __syncthreads();  // every wave is past its last ring read
        for (int dt = 0; dt < NDT; dt++)
            for (int rq = 0; rq < 4; rq++) {
                f32x4 v;
                for (int i = 0; i < 4; i++) v[i] = oacc[dt][rq * 4 + i] * inv;
                const int c = dt * 8 + rq * 2 + g;
                *(f32x4*)(reg + ln * D * 4 + ((c ^ (ln & (NC - 1))) * 16)) = v;
            }
        __syncthreads();
        for (int i = 0; i < 32 / RPI; i++) {
            const int r = i * RPI + lane / NC, c = lane % NC;
            const f32x4 v = *(const f32x4*)(reg + r * D * 4 + ((c ^ (r & (NC - 1))) * 16));
            if (qw + r < Sq) *(f32x4*)(p.o + ((size_t)bh * Sq + qw + r) * D + c * 4) = v;
        }
    } else if (qi < Sq) {
        float* orow = p.o + ((size_t)bh * Sq + qi) * D;
        for (int dt = 0; dt < NDT; dt++)
            for (int rq = 0; rq < 4; rq++) {
                f32x4 v;
                for (int i = 0; i < 4; i++) v[i] = oacc[dt][rq * 4 + i] * inv;
                *(f32x4*)(orow + dt * 32 + rq * 8 + g * 4) = v;
            }
    }
    // LSE = (mc + log2 l) * ln 2, natural-log units of the scaled scores.
    if (qi < Sq && p.lse && g == 0) p.lse[(size_t)bh * Sq + qi] = (mc + fast_log2(lt)) * kLn2;
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
    const int Sq = p.Sq, Sk = fwd_keys(p, bh), Ss = p.Sk;  // keys taking part, slice stride
    if (Sk == 0) {  // uniform: the whole slice is padded
        fwd_empty_rows<D>(p, bh, q0, BM);
        return;
    }

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
    const float* Kg = (const float*)p.k + (size_t)bh * Ss * D;
    const float* Vg = (const float*)p.v + (size_t)bh * Ss * D;
    // The additive mask's row of this lane's query (rows Ss apart).
    const float* mrow = p.mask ? p.mask + (size_t)(bh / p.H) * p.mask_sb +
                                     (size_t)(bh % p.H) * p.mask_sh +
                                     (size_t)(qi < Sq ? qi : 0) * Ss
                               : nullptr;

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
        if (mrow) {  // scale * s + m = scale_abs * (sacc + m / scale_abs)
            for (int r = 0; r < 16; r++) {
                const int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key < Sk) sacc[r] += mrow[key] * p.mask_mul;
            }
        }
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
        // exp2((s - max) c2): the difference is formed before the scaling, so
        // scores equal to the max give exactly 1 at any magnitude (an additive
        // -1e30 mask on every key of a tile gives ties, as in fp64).
        const float mref = (mnew == -INFINITY) ? 0.f : mnew;
        float rs = 0.f;
        for (int r = 0; r < 16; r++) {
            const float e = fast_exp2((sacc[r] - mref) * c2);
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
static void launch_bf16_pipe(const FwdParams& p, int q_bf16, dim3 grid, hipStream_t s) {
    if (p.mask) {
        if (q_bf16) fwd_bf16_pipe_kernel<D, C, bf16, true><<<grid, kFwdWaves * 64, 0, s>>>(p);
        else fwd_bf16_pipe_kernel<D, C, float, true><<<grid, kFwdWaves * 64, 0, s>>>(p);
    } else {
        if (q_bf16) fwd_bf16_pipe_kernel<D, C, bf16, false><<<grid, kFwdWaves * 64, 0, s>>>(p);
        else fwd_bf16_pipe_kernel<D, C, float, false><<<grid, kFwdWaves * 64, 0, s>>>(p);
    }
}

// Compute units of the current device, looked up once per device (the
// lookup is idempotent, so concurrent first calls may both run it).
static int device_cus() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cache[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
    int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        c = 256;
    cache[dev].store(c, std::memory_order_relaxed);
    return c;
}

hipError_t launch_fwd(const FwdParams& p_in, int mode, int D, int causal, int q_bf16,
                      hipStream_t s) {
    FwdParams p = p_in;
    // Query rows per workgroup.
    const int bm = mode == 1 ? kFwdWaves * 32 : 128;  // both bf16 kernels: 128 rows
    p.nqb = (p.Sq + bm - 1) / bm;
    dim3 grid(p.nqb * p.BH);
    // Causal dispatch groups: about two XCDs' worth of workgroup slots
    // (2 x CUs / 8 XCDs x 2 resident workgroups) of q-blocks per group.
    p.hgroup = 1;
    if (causal && mode == 1 && D == 128) {
        // Two XCDs' worth measured 1% faster on C3 than one (interleaved
        // runs), and the same on C5.
        const int slots = device_cus() / 8 * (8 / kFwdWaves);
        p.hgroup = 2 * slots / p.nqb > 1 ? 2 * slots / p.nqb : 1;
    }
    if (mode == 1) {
        if (D == 64) {
            if (causal) launch_bf16_pipe<64, true>(p, q_bf16, grid, s);
            else launch_bf16_pipe<64, false>(p, q_bf16, grid, s);
        } else if (D == 128) {
            if (causal) launch_bf16_pipe<128, true>(p, q_bf16, grid, s);
            else launch_bf16_pipe<128, false>(p, q_bf16, grid, s);
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
