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
//         wave. K and V of the block stay in VGPRs; Q / dO tiles stream
//         through LDS rings (bf16 mode reads their transposes from the same
//         tiles with ds_read_b64_tr_b16). Per query tile: S = Q K^T and
//         dP = dO V^T on MFMA with one KEY per lane (the 16 accumulators of a
//         lane are 16 queries), P and dS in registers, then dV^T += dO^T P
//         and dK^T += Q^T dS on MFMA straight from those registers; bf16 mode
//         also stores dS for the dQ kernel;
//   dq    bf16 mode: dQ^T = K^T dS^T from the stored dS (attn_bwd_dqds.hip),
//         or, past the dS buffer's limits, one workgroup per 128-query block
//         that forms S^T = K Q^T and dP^T = V dO^T again with one QUERY per
//         lane (attn_bwd_dq.hip, built with other MFMA flags); fp32 mode: the
//         latter form, in this file.
// Causal work skips fully masked tiles and masks only diagonal ones.
//
// bf16 mode reads the packed bf16 operands of attn_pack.hip (row-major Qb,
// dOb, Kb, Vb and the vt_pos-permuted transpose Kt, padded to Sp / Skp
// rows); fp32 mode reads the caller's fp32 (BH,S,D) buffers directly with
// v_mfma_f32_32x32x2_f32, clamping rows past S (masked or never written).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace gonn {

// ---------------------------------------------------------------------------
// prep: grid ceil(BH*Sp/16), 256 threads (16 lanes per query row).
// delta = rowsum(dO * O). With round_do (bf16 mode) dO is rounded to bf16
// first, the operand the dP = dO V^T product sees, so that dS = P (dP - delta)
// loses the dO rounding in both terms alike and its rows still sum to ~0.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const float* __restrict__ O,
                                                       const float* __restrict__ dO,
                                                       const float* __restrict__ lse,
                                                       float* __restrict__ lse2,
                                                       float* __restrict__ delta, int BH, int S,
                                                       int Sp, int round_do) {
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
            for (int j = 0; j < 4; j++)
                acc = __builtin_fmaf(o[j], round_do ? (float)to_bf16(g[j]) : g[j], acc);
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
//
// One workgroup per 128-key block (32 keys per wave, held as the MFMA B
// operand in VGPRs), query tiles of 64 streamed through LDS, one wave per
// SIMD with the full register file. Three-stage software pipeline: step i
// issues, with no dependency between them inside the step,
//   MFMA  S(i+1) = Q K^T, dP(i+1) = dO V^T        (row tiles of query tile i+1)
//   VALU  P(i) = exp2(S c - L log2e), dS(i) = P (dP - D), packed to bf16
//   MFMA  dV^T += dO^T P(i-1), dK^T += Q^T dS(i-1) (row tiles of i-1, read
//         transposed)
// so no MFMA waits on the VALU of its own step. P(i) / dS(i) overwrite
// P(i-1) / dS(i-1) 16 queries at a time, after the dV / dK MFMAs that read
// those 16 queries were issued. The step is scheduled by hand: slot e issues
// the LDS read of MFMA e+3, MFMA e, a tile load and the VALU micro-ops mapped
// to it, fenced by sched_barrier (the compiler's own schedule serialises
// MFMA chains behind their LDS reads). MFMA order per 16-query k-step ks:
// dV(ks, d-tiles), dK(ks, d-tiles), then a quarter of S/dP(i+1): 4 NDT + 4
// accumulator chains interleave.
//
// LDS: the Q and dO tiles of 64 queries sit in 4-slot rings in the swizzled
// slab layout of slab_swz, without padding. Step i reads tile i+1 (S, dP)
// and tile i-1 (dV, dK) and keeps tile i for step i+1; it loads tile i+2
// into the slot of tile i-2 and L/D of tile i+1, all landing by the end of
// step i (one barrier per step). The dV / dK MFMAs take dO^T and Q^T as
// their A operand (d rows, query k-slots): ds_read_b64_tr_b16 reads them
// from the row tiles, so no transposed copy of Q or dO is packed, streamed
// or staged. Causal masks exist only on the first two query tiles of a key
// block (its query tiles start at the block's first key).
// ---------------------------------------------------------------------------
constexpr int kDkdvLookahead = 3;
constexpr int kDkdvDmaSpan = 16;  // slots over which a step's tile loads are spread (0: all)

// S / dP products of the bf16 dK/dV kernel with VGPR accumulators and the
// K / V fragment (B operand) in AGPRs, so the softmax VALU reads S and dP
// where the MFMA leaves them. Left to the compiler, at one wave per SIMD
// every MFMA of the kernel gets an AGPR accumulator and S / dP were copied
// out with 64 v_accvgpr_read per step (same results bit for bit without
// them; C5 dK/dV 1.287-1.291 -> 1.251-1.259 ms, cross 0.392-0.393 ->
// 0.379-0.383 ms, same box, three interleaved rounds). The compiler does not
// track MFMA hazards through inline asm, so the kernel provides the wait
// states, each in an asm statement that the registers pass through (so the
// compiler cannot schedule an access of them ahead of it): the fragments go
// into AGPRs through an s_nop 4 each, then an s_nop 7 precedes the first of
// these MFMAs; three s_nop 7 (24 wait states, above the result latency of
// this 32-cycle MFMA) separate each step's last S / dP MFMA from any VALU
// access of its accumulators. Chained MFMAs on one accumulator and A
// operands loaded from LDS (the compiler's waitcnt covers them) need none.
GONN_DEV void mfma_vacc0(f32x16& d, bf16x8 a, bf16x8 b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
}
GONN_DEV void mfma_vacc(f32x16& d, bf16x8 a, bf16x8 b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_bf16_kernel(BwdParams p) {
    constexpr int BN = 128;      // keys per workgroup
    constexpr int BM = 64;       // queries per tile
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;
    // A Q / dO tile: BM rows x D/8 chunks of 16 bytes (slab layout), filled
    // by NRI load instructions of 256 x 16 bytes.
    constexpr int RTILE = BM * D;  // bf16 elements
    constexpr uint32_t RTB = RTILE * 2;
    constexpr int NRI = RTILE / 8 / 256;
    static_assert(NRI * 256 * 8 == RTILE, "whole load instructions per tile");
    constexpr int NSLOT = 4;
    // S / dP accumulators in VGPRs (mfma_vacc), except with the additive
    // mask: its registers leave no room (at D = 64 the compiler then moves
    // values between VGPRs and AGPRs, and D = 128 already spills).
    constexpr bool VACC = !MASK;
    __shared__ __attribute__((aligned(16))) bf16 sQ[NSLOT * RTILE];
    __shared__ __attribute__((aligned(16))) bf16 sdO[NSLOT * RTILE];
    __shared__ __attribute__((aligned(16))) float sLD[2][2 * BM];  // L*log2e, then D

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    const int S = p.S, Sp = p.Sp;  // query rows (Q, dO, L, D padded to Sp)
    const int Sk = p.Sk, Skp = p.Skp;  // key rows (K, V padded to Skp)
    // This launch's key blocks: [kb0, kb0 + nkbc) (a chunk of the dS path, or all).
    const int nkbc = p.nkb ? p.nkb : Skp / BN;
    int bh, kb;
    map_block(blockIdx.x, nkbc, p.BH, false, bh, kb);
    kb += p.kb0;
    const int kw = kb * BN + wave * 32;  // first key of this wave
    const int kj = kw + ln;              // this lane's key
    // Keys >= Skv are padded: zero probability for every query, so their dK
    // and dV rows are 0, and the other keys' gradients do not involve them.
    const int Skv = bwd_keys(p, bh);
    // Top-left causal: key j is seen by queries i >= j only, so a block past
    // the last query has no gradient either (cross-attention, Sq < Sk).
    const int qb0 = CAUSAL ? (kb * BN) / BM : 0;  // earlier queries see none of these keys
    const int nq = (S + BM - 1) / BM - qb0;
    if (kb * BN >= Skv || nq <= 0) {
        bwd_zero_rows<D>(p.dk, Sk, bh, kb * BN, BN);
        bwd_zero_rows<D>(p.dv, Sk, bh, kb * BN, BN);
        return;
    }

    bf16x8 kf[NKS], vf[NKS];
    {
        const bf16* kr = (const bf16*)p.k + ((size_t)bh * Skp + kj) * D + g * 8;
        const bf16* vr = (const bf16*)p.v + ((size_t)bh * Skp + kj) * D + g * 8;
        for (int ks = 0; ks < NKS; ks++) {
            kf[ks] = *(const bf16x8*)(kr + ks * 16);
            vf[ks] = *(const bf16x8*)(vr + ks * 16);
        }
    }
    if constexpr (VACC) {  // fragments into AGPRs, then wait states (mfma_vacc)
        for (int ks = 0; ks < NKS; ks++) {
            asm volatile("s_nop 4" : "+a"(kf[ks]));
            asm volatile("s_nop 4" : "+a"(vf[ks]));
        }
        asm volatile("s_nop 7");
    }
    const bf16* Qg = (const bf16*)p.q + (size_t)bh * Sp * D;
    const bf16* dOg = (const bf16*)p.dO + (size_t)bh * Sp * D;
    const float* lg = p.lse2 + (size_t)bh * Sp;
    const float* dg = p.delta + (size_t)bh * Sp;

    // Byte offset in the (b,h) slice of the chunk this thread loads into
    // tile position i*256 + tid (slab_chunk gives its row and chunk).
    uint32_t roff[NRI];
    for (int i = 0; i < NRI; i++) {
        int r, c;
        slab_chunk(i * 256 + tid, BM, r, c);
        roff[i] = (uint32_t)((r * D + c * 8) * 2);
    }
    const uint32_t slice = (uint32_t)Sp * D * 2;  // bytes of one (b,h) slice
    const brsrc rq = make_rsrc(Qg, slice), rdo = make_rsrc(dOg, slice);
    const brsrc rl = make_rsrc(lg, (uint32_t)Sp * 4), rd = make_rsrc(dg, (uint32_t)Sp * 4);
    const uint32_t lq = lds_addr(sQ) + wave * 1024, ldo = lds_addr(sdO) + wave * 1024;
    // Load j of the row tiles (Q: j < NRI, dO: j >= NRI) of query tile qb,
    // issued when the wave-uniform `on` is set (a scalar branch inside the
    // load statement keeps the step one basic block).
    auto dma_row = [&](int qb, int slot, int j, uint32_t on) {
        const uint32_t so = (uint32_t)qb * BM * D * 2;
        const int i = j % NRI;
        const brsrc r = j < NRI ? rq : rdo;
        const uint32_t dst = (j < NRI ? lq : ldo) + slot * RTB + i * 4096;
        dma16_if(r, dst, roff[i], so, on);
    };
    // L and D of query tile qb: wave 0, lanes 0-15 load the 64 L values
    // (bytes 0-255 of sLD[slot]), lanes 16-31 the 64 D values (256-511).
    auto dma_ld = [&](int qb, int slot) {
        if (wave == 0) {
            const uint32_t dl = lds_addr(sLD) + slot * 2 * BM * 4;
            if (lane < 16) dma16(rl, dl, (lane & 15) * 16, (uint32_t)qb * BM * 4);
            else if (lane < 32) dma16(rd, dl, (lane & 15) * 16, (uint32_t)qb * BM * 4);
        }
    };

    // ---- MFMA operand reads (bytes from a slot's start) ----
    // S / dP A operand (Q / dO rows, d k-slots; ds_read_b128): row 32 mt + ln,
    // chunk 2 kk + g at ((kk / 2) * BM + 32 mt) * 64 + (kk odd ? ra1 : ra0)
    // (slab layout; h(32 mt + ln) = h(ln)).
    const int hs = slab_swz(ln);
    const uint32_t ra0 = (uint32_t)(ln * 64 + ((0 + g) ^ hs) * 16);
    const uint32_t ra1 = (uint32_t)(ln * 64 + ((2 + g) ^ hs) * 16);
    // dV / dK A operand (dO^T / Q^T: row d = 32 t + ln, k-slots 0-3 = queries
    // 16 ks + 4g + 0..3, k-slots 4-7 = 16 ks + 8 + 4g + 0..3, the order of
    // the P / dS words in pp / pd) by two ds_read_b64_tr_b16. That
    // instruction gives lane L of a 16-lane group element L % 4 of the 8-byte
    // reads of group lanes 4i + L / 4 (i = 0..3). Group lane s reads query
    // row base + s / 4 at d = 32 t + 16 ((ln >> 4) & 1) + 4 (s % 4), so lane
    // L receives d = 32 t + 16 ((ln >> 4) & 1) + L for queries base + 0..3.
    // In the slab layout: slab t, row base + s / 4, chunk 2 ((ln >> 4) & 1) +
    // (s / 2) % 2, byte 8 (s % 2); h(row) = g (+2 for the upper quads). A
    // half-wave reads 4 rows x 64 bytes of one slab: 4 distinct 16-bank
    // quarters, no conflict.
    const int s16 = lane & 15;
    const int tcx = 2 * ((ln >> 4) & 1) + ((s16 >> 1) & 1);
    const uint32_t ta0 = (uint32_t)((4 * g + (s16 >> 2)) * 64 + (tcx ^ g) * 16 + 8 * (s16 & 1));
    const uint32_t ta1 =
        (uint32_t)((8 + 4 * g + (s16 >> 2)) * 64 + (tcx ^ (2 + g)) * 16 + 8 * (s16 & 1));
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    typedef __attribute__((address_space(3))) char lds_char;
    lds_char* const tQ = (lds_char*)sQ;
    lds_char* const tdO = (lds_char*)sdO;
    const char* cQ = (const char*)sQ;
    const char* cdO = (const char*)sdO;
    auto rowa = [&](int kk, int mt) {  // S / dP operand offset inside a slot
        return (uint32_t)(((kk >> 1) * BM + mt * 32) * 64) + ((kk & 1) ? ra1 : ra0);
    };

    f32x16 dvacc[NDT], dkacc[NDT];
    for (int t = 0; t < NDT; t++) dvacc[t] = dkacc[t] = f32x16{};
    const float c2 = p.c2b;
    // Additive mask (MASK variant): this lane's key column; the values of
    // S(i+1) are loaded at the start of step i and added at its end, when
    // that tile is complete.
    MaskCol mcol{};
    f32x4 mreg[8];
    if constexpr (MASK) mcol.init(p.mask, p.mask_sb, p.mask_sh, p.H, S, Sk, bh, kj);
    u32x4 pp[4], pd[4];  // P and dS of the tile dV/dK consume next, bf16 pairs per word
    // dS-store path (layout at BwdParams::ds): this key block's dS for every
    // query tile. Lane (ln, g) holds, in pd[ks], the dS of its key for the
    // 8 queries of chunk 2 ks + g of a 64-query tile (queries 16 ks +
    // {4g..4g+3, 8+4g..8+4g+3}, the vt_pos order); a block keeps the 16-byte
    // pieces of each half of the 128 keys chunk by chunk, so one store
    // writes contiguous 512-byte runs and the dQ kernel reads the 64 keys of
    // one of its steps as one contiguous 8 KB. A padded key (kj >= Skv) stores zeros. Without
    // p.ds the resource has no range and every store is dropped.
    const bool store_ds = p.ds != nullptr;
    // This key block's blocks (query tiles qb0 .. Sp/64 - 1) in the chunk's
    // stored dS.
    const size_t ds0 = (size_t)(bh * ds_chunk_blocks(p.kb0, nkbc, Sp / BM, CAUSAL) +
                                ds_block_base(kb, Sp / BM, CAUSAL) -
                                ds_block_base(p.kb0, Sp / BM, CAUSAL));
    const brsrc dsrs = make_rsrc(store_ds ? p.ds + ds0 * kDsTileElems : p.ds,
                                 store_ds ? (uint32_t)(Sp / BM - qb0) * kDsTileElems * 2 : 0u);
    // Piece (key / 64) * 512 + chunk * 64 + key % 64 of a block, chunk 2e + g
    // for store e.
    const uint32_t dsvo = (uint32_t)(((wave >> 1) * 512 + (wave & 1) * 32 + ln + g * 64) * 16);
    const bool ds_live = kj < Skv;

    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    // Causal mask (key > query) of S(i): only the first two query tiles of a
    // key block cross the diagonal. Applied between steps, once S(i) is
    // complete and before the step that exponentiates it reads it. The
    // exponent scale c2b is positive (a negative scale is folded into the
    // packed Q), so a masked score of -inf gives P = 0 and dS = 0.
    auto causal_mask = [&](int i, f32x16* s) {
        const int kq = kj - (qb0 + i) * BM - 4 * g;  // key minus the lane group's base query
        for (int mt = 0; mt < 2; mt++)
            for (int r = 0; r < 16; r++)
                s[mt][r] = kq > mt * 32 + 8 * (r >> 2) + (r & 3) ? -INFINITY : s[mt][r];
    };
    // One pipeline step. sA <- S(i+1), dA <- dP(i+1); sB, dB = S(i), dP(i).
    auto step = [&](auto ha_tag, auto hb_tag, auto hc_tag, int i, f32x16* sA,
                    f32x16* dA, f32x16* sB, f32x16* dB) __attribute__((always_inline)) {
        constexpr bool HA = decltype(ha_tag)::value;  // S/dP of tile i+1
        constexpr bool HB = decltype(hb_tag)::value;  // P/dS of tile i
        constexpr bool HC = decltype(hc_tag)::value;  // dV/dK of tile i-1
        const int qb = qb0 + i;
        if constexpr (MASK && HA) mcol.load(qb + 1, g, mreg);
        // Loads for the next steps: row tiles i+2, L/D i+1.
        const uint32_t dr = HA && i + 2 < nq;
        const bool dl = HA;
        if (dl) dma_ld(qb + 1, (i + 1) & 1);
        const uint32_t rsl = (uint32_t)((i + 1) & 3) * RTB;   // row tile i+1 (S, dP)
        const uint32_t tsl = (uint32_t)((i + 3) & 3) * RTB;   // row tile i-1 (dV, dK)
        const uint32_t nsl = (uint32_t)((i + 2) & 3);     // slot of row tile i+2
        const int lsl = i & 1;                                 // L/D of tile i

        constexpr int HCn = HC ? 2 * NDT : 0, HAn = HA ? NKS : 0;
        constexpr int GW = HCn + HAn;  // MFMAs per 16-query k-step group
        constexpr int NM = 4 * GW;
        constexpr int LA = kDkdvLookahead;  // LDS operand lead (MFMA slots)
        constexpr int NO = LA < 4 ? 4 : 8;
        constexpr int NDMA = 2 * NRI;
        constexpr int SPAN = kDkdvDmaSpan > 0 && kDkdvDmaSpan < NM ? kDkdvDmaSpan : NM;
        constexpr int DS = SPAN / NDMA > 0 ? SPAN / NDMA : 1;
        bf16x8 opr[NO];
        auto fetch = [&](auto E) {
            constexpr int e = decltype(E)::value, ks = e / GW, w = e % GW;
            if constexpr (w < HCn) {
                constexpr int t = w % NDT;
                lds_char* const base = (w < NDT ? tdO : tQ) + tsl + (t * BM + 16 * ks) * 64;
                const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + ta0));
                const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + ta1));
                const s4 b8[2] = {lo, hi};
                opr[e % NO] = __builtin_bit_cast(bf16x8, b8);
            } else {
                constexpr int u = w - HCn, kk = ks * (NKS / 4) + u / 4, mt = u & 1;
                const char* base = ((u & 2) ? cdO : cQ) + rsl;
                opr[e % NO] = *(const bf16x8*)(base + rowa(kk, mt));
            }
        };
        auto issue = [&](auto E) {
            constexpr int e = decltype(E)::value, ks = e / GW, w = e % GW;
            if constexpr (w < HCn) {
                constexpr int t = w % NDT;
                if constexpr (w < NDT)
                    dvacc[t] = mfma_bf16(opr[e % NO], __builtin_bit_cast(bf16x8, pp[ks]), dvacc[t]);
                else
                    dkacc[t] = mfma_bf16(opr[e % NO], __builtin_bit_cast(bf16x8, pd[ks]), dkacc[t]);
            } else {
                constexpr int u = w - HCn, kk = ks * (NKS / 4) + u / 4, mt = u & 1;
                f32x16& acc = (u & 2) ? dA[mt] : sA[mt];
                const bf16x8& b = (u & 2) ? vf[kk] : kf[kk];
                if constexpr (!VACC) acc = mfma_bf16(opr[e % NO], b, kk == 0 ? f32x16{} : acc);
                else if constexpr (kk == 0) mfma_vacc0(acc, opr[e % NO], b);
                else mfma_vacc(acc, opr[e % NO], b);
            }
        };
        // VALU of tile i in 8 groups k = mt*4 + j4 (registers 4 j4 .. +3 of
        // sB/dB[mt], queries mt*32 + 8 j4 + 4g + 0..3), each in five
        // micro-ops: R (read L, D), A0/A1 (exp2 of two scores), B0/B1 (dS of
        // two scores, bf16 pairs of P and dS). Group k fills words of k-step
        // ks = k/2: its B micro-ops sit after the dV/dK MFMAs of ks.
        f32x4 uL[8], uD[8];
        float ue[8][4];
        auto ub = [](int k, int st) {  // slot of micro-op st (0 R, 1 A0, 2 A1, 3 B0, 4 B1)
            int b0 = (k >> 1) * GW + (HCn ? HCn - 1 : 0) + 2 * (k & 1);
            const int off[5] = {-5, -3, -2, 0, 1};
            const int s = b0 + off[st];
            return s < 0 ? 0 : s;
        };
        auto uop = [&](auto K, auto ST) {
            constexpr int k = decltype(K)::value, st = decltype(ST)::value;
            constexpr int mt = k >> 2, j4 = k & 3, ks = k >> 1, w0 = (j4 & 1) * 2;
            if constexpr (st == 0) {
                uL[k] = *(const f32x4*)&sLD[lsl][mt * 32 + 8 * j4 + 4 * g];
                uD[k] = *(const f32x4*)&sLD[lsl][BM + mt * 32 + 8 * j4 + 4 * g];
            } else if constexpr (st <= 2) {
                constexpr int e0 = (st - 1) * 2;
                for (int e = e0; e < e0 + 2; e++) {
                    ue[k][e] = fast_exp2(__builtin_fmaf(sB[mt][4 * j4 + e], c2, -uL[k][e]));
                    pin(ue[k][e]);
                }
            } else {
                constexpr int e0 = (st - 3) * 2;
                const float d0 = ue[k][e0] * (dB[mt][4 * j4 + e0] - uD[k][e0]);
                const float d1 = ue[k][e0 + 1] * (dB[mt][4 * j4 + e0 + 1] - uD[k][e0 + 1]);
                const bf16x2 pr = {to_bf16(ue[k][e0]), to_bf16(ue[k][e0 + 1])};
                const bf16x2 dr2 = {to_bf16(d0), to_bf16(d1)};
                pp[ks][w0 + e0 / 2] = __builtin_bit_cast(uint32_t, pr);
                pd[ks][w0 + e0 / 2] = __builtin_bit_cast(uint32_t, dr2);
                pin(pp[ks][w0 + e0 / 2]);
                pin(pd[ks][w0 + e0 / 2]);
            }
        };
        auto uops_at = [&](auto E) {
            constexpr int e = decltype(E)::value;
            if constexpr (HB) {
                static_for<5>([&](auto ST) {
                    static_for<8>([&](auto K) {
                        constexpr int at = ub(decltype(K)::value, decltype(ST)::value);
                        if constexpr (e < NM ? at == e : at >= NM) uop(K, ST);
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
            // dS-store path: the dS of tile i-1 (pd, read by this step's dK
            // MFMAs) goes out one k-step at a time, at slot 2 of each k-step
            // group (pd[es] is overwritten by the VALU from slot 7 of the
            // group on). Spread over the step and after the tile loads,
            // which sit in its first 16 slots (together 2% faster at C5
            // than four stores in a row at the step's start and loads over
            // 40 slots).
            if constexpr (HC && e % GW == 2 && e / GW < 4) {
                typedef int i32x4 __attribute__((ext_vector_type(4)));
                constexpr int es = e / GW;
                const u32x4 v = ds_live ? pd[es] : u32x4{};
                // Non-temporal (nt): the stream of dS is read once, by the dQ
                // kernel, and would otherwise evict the Q / dO tiles this
                // kernel re-reads from L2.
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(i32x4, v), dsrs, dsvo,
                    (uint32_t)((qb - 1 - qb0) * kDsTileElems * 2 + es * 2048), 2);
            }
            // Tile loads spread over the first SPAN slots: 1, 1 + DS, ...
            if constexpr (e >= 1 && (e - 1) % DS == 0 && (e - 1) / DS < NDMA)
                dma_row(qb + 2, nsl, (e - 1) / DS, dr);
            uops_at(E);
            __builtin_amdgcn_sched_barrier(0);
        });
        // Loads not placed in the stream (a step with too few MFMAs).
        static_for<NDMA>([&](auto Dd) {
            constexpr int d = decltype(Dd)::value;
            if constexpr (NM == 0 || 1 + d * DS >= NM) dma_row(qb + 2, nsl, d, dr);
        });
        uops_at(std::integral_constant<int, NM>{});
        // Wait states between this step's last S / dP MFMA and VALU access.
        // The accumulators pass through the statement, so no access of them
        // is scheduled before it.
        if constexpr (VACC && HA)
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+v"(sA[0]), "+v"(sA[1]), "+v"(dA[0]), "+v"(dA[1]));
        GONN_VMCNT(0);
        __syncthreads();
        if constexpr (MASK && HA) MaskRow::add(mreg, sA);
    };
    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;

    // Prologue: row tiles 0, 1 and L/D of tile 0; S/dP of tile 0.
    for (int j = 0; j < 2 * NRI; j++) dma_row(qb0, 0, j, 1);
    for (int j = 0; j < 2 * NRI; j++) dma_row(qb0 + 1, 1, j, nq > 1);
    dma_ld(qb0, 0);
    GONN_VMCNT(0);
    __syncthreads();
    f32x16 sX[2], dX[2], sY[2], dY[2];
    for (int mt = 0; mt < 2; mt++) sX[mt] = dX[mt] = f32x16{};
    for (int kk = 0; kk < NKS; kk++)
        for (int mt = 0; mt < 2; mt++) {
            const bf16x8 aq = *(const bf16x8*)(cQ + rowa(kk, mt));
            const bf16x8 ad = *(const bf16x8*)(cdO + rowa(kk, mt));
            if constexpr (!VACC) {
                sX[mt] = mfma_bf16(aq, kf[kk], sX[mt]);
                dX[mt] = mfma_bf16(ad, vf[kk], dX[mt]);
            } else if (kk == 0) {
                mfma_vacc0(sX[mt], aq, kf[kk]);
                mfma_vacc0(dX[mt], ad, vf[kk]);
            } else {
                mfma_vacc(sX[mt], aq, kf[kk]);
                mfma_vacc(dX[mt], ad, vf[kk]);
            }
        }
    if constexpr (VACC)
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                     : "+v"(sX[0]), "+v"(sX[1]), "+v"(dX[0]), "+v"(dX[1]));
    if constexpr (MASK) {
        mcol.load(qb0, g, mreg);
        MaskRow::add(mreg, sX);
    }

    // Steps 0 .. nq: step i has S/dP(i+1) while i+1 < nq, P/dS(i) while
    // i < nq, dV/dK(i-1) from i = 1. Step i writes S/dP(i+1) into the
    // register set the next step reads as S/dP(i): the full steps
    // 1 .. nq-2 run in pairs (sX, sY), then (sY, sX); an odd count peels
    // step 1 and copies its S/dP(2) into sY, so one copy of each tail step
    // (the next-to-last reads sY) follows the loop.
    if constexpr (CAUSAL) causal_mask(0, sX);
    if (nq == 1) {
        step(No{}, Yes{}, No{}, 0, sY, dY, sX, dX);
        step(No{}, No{}, Yes{}, 1, sX, dX, sY, dY);
    } else {
        step(Yes{}, Yes{}, No{}, 0, sY, dY, sX, dX);
        if constexpr (CAUSAL) causal_mask(1, sY);
        int i = 1;
        if ((nq - 2) & 1) {
            step(Yes{}, Yes{}, Yes{}, 1, sX, dX, sY, dY);
            for (int mt = 0; mt < 2; mt++) {
                sY[mt] = sX[mt];
                dY[mt] = dX[mt];
            }
            i = 2;
        }
        for (; i < nq - 1; i += 2) {
            step(Yes{}, Yes{}, Yes{}, i, sX, dX, sY, dY);
            step(Yes{}, Yes{}, Yes{}, i + 1, sY, dY, sX, dX);
        }
        step(No{}, Yes{}, Yes{}, nq - 1, sX, dX, sY, dY);
        step(No{}, No{}, Yes{}, nq, sY, dY, sX, dX);
    }

    if (kj < Sk) {
        const float sc = p.dks;
        const bool live = kj < Skv;  // a padded key of a partial block: zeros
        float* dkr = p.dk + ((size_t)bh * Sk + kj) * D;
        float* dvr = p.dv + ((size_t)bh * Sk + kj) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a, b;
                for (int k = 0; k < 4; k++) {
                    a[k] = live ? dkacc[t][rq4 * 4 + k] * sc : 0.f;
                    b[k] = live ? dvacc[t][rq4 * 4 + k] : 0.f;
                }
                *(f32x4*)(dkr + t * 32 + rq4 * 8 + g * 4) = a;
                *(f32x4*)(dvr + t * 32 + rq4 * 8 + g * 4) = b;
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
    const int S = p.S, Sp = p.Sp, Sk = p.Sk;  // S queries, Sk keys
    int bh, kb;
    map_block(blockIdx.x, p.Skp / BN, p.BH, false, bh, kb);
    const int kw = kb * BN + wave * 32;
    const int kj = kw + ln;
    const int Skv = bwd_keys(p, bh);  // keys >= Skv are padded: dK = dV = 0
    if (kb * BN >= Skv) {
        bwd_zero_rows<D>(p.dk, Sk, bh, kb * BN, BN);
        bwd_zero_rows<D>(p.dv, Sk, bh, kb * BN, BN);
        return;
    }

    float kf[HD], vf[HD];
    {
        const int kr = kj < Sk ? kj : Sk - 1;  // pad keys are computed, never written
        const float* kp = (const float*)p.k + ((size_t)bh * Sk + kr) * D + g * HD;
        const float* vp = (const float*)p.v + ((size_t)bh * Sk + kr) * D + g * HD;
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
    // The additive mask's column of this lane's key (rows S apart), if any.
    const float* mcol = p.mask ? p.mask + (size_t)(bh / p.H) * p.mask_sb +
                                     (size_t)(bh % p.H) * p.mask_sh + (kj < Sk ? kj : Sk - 1)
                               : nullptr;

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
                float off = -s_lse[buf][qr];
                if (mcol) {  // mask[q][kj], clamped rows and keys are not used
                    const int qq = q0 + qr < S ? q0 + qr : S - 1;
                    off += mcol[(size_t)qq * Sk] * kLog2e;
                }
                float pv = fast_exp2(__builtin_fmaf(sacc[r], c2, off));
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

    if (kj < Sk) {
        const float sc = p.scale;
        const bool live = kj < Skv;
        float* dkr = p.dk + ((size_t)bh * Sk + kj) * D;
        float* dvr = p.dv + ((size_t)bh * Sk + kj) * D;
        for (int t = 0; t < NDT; t++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a, b;
                for (int i = 0; i < 4; i++) {
                    a[i] = live ? dkacc[t][rq4 * 4 + i] * sc : 0.f;
                    b[i] = live ? dvacc[t][rq4 * 4 + i] : 0.f;
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
    const int S = p.S, Sp = p.Sp, Sk = p.Sk;  // S queries, Sk keys
    int bh, qb;
    map_block(blockIdx.x, Sp / BM, p.BH, CAUSAL, bh, qb);
    const int q0 = qb * BM;
    const int qi = q0 + wave * 32 + ln;
    const int Skv = bwd_keys(p, bh);  // keys taking part (key padding)
    if (Skv == 0) {
        bwd_zero_rows<D>(p.dq, S, bh, q0, BM);
        return;
    }

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

    int kend = Skv;
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    const int ntiles = (kend + BN - 1) / BN;
    const float* Kg = (const float*)p.k + (size_t)bh * Sk * D;
    const float* Vg = (const float*)p.v + (size_t)bh * Sk * D;
    // The additive mask's row of this lane's query, if any.
    const float* mrow = p.mask ? p.mask + (size_t)(bh / p.H) * p.mask_sb +
                                     (size_t)(bh % p.H) * p.mask_sh +
                                     (size_t)(qi < S ? qi : S - 1) * Sk
                               : nullptr;

    f32x4 rk[CH], rv[CH];
    auto gload = [&](int kt) {
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            int key = kt * BN + row;
            key = key < Sk ? key : Sk - 1;  // clamped rows are masked
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
        const bool need_mask = (kbase + BN > Skv) || (CAUSAL && kbase + BN - 1 > q0 + wave * 32);
        for (int r = 0; r < 16; r++) {
            float off = -lq;  // log2 units: s scale log2e + m log2e - L log2e
            if (mrow) {
                const int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key < Skv) off += mrow[key] * kLog2e;
            }
            float pv = fast_exp2(__builtin_fmaf(sacc[r], c2, off));
            if (need_mask) {
                const int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key >= Skv || (CAUSAL && key > qi)) pv = 0.f;
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
                           float* delta, int BH, int S, int Sp, int D, int round_do,
                           hipStream_t s) {
    const size_t rows = (size_t)BH * Sp;
    const unsigned grid = (unsigned)((rows + 15) / 16);
    if (D == 64)
        bwd_prep_kernel<64><<<grid, 256, 0, s>>>(O, dO, lse, lse2, delta, BH, S, Sp, round_do);
    else if (D == 128)
        bwd_prep_kernel<128><<<grid, 256, 0, s>>>(O, dO, lse, lse2, delta, BH, S, Sp, round_do);
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

template <int D, bool C>
static void launch_dkdv_bf16(const BwdParams& p, dim3 grid, hipStream_t s) {
    if (p.mask) bwd_dkdv_bf16_kernel<D, C, true><<<grid, 256, 0, s>>>(p);
    else bwd_dkdv_bf16_kernel<D, C, false><<<grid, 256, 0, s>>>(p);
}

hipError_t launch_bwd_dkdv(const BwdParams& p, int mode, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0 || p.Skp % kBwdPad != 0) return hipErrorInvalidValue;
    // A key-block chunk (bf16 kernels only) lies inside the slice's blocks.
    const int nkb = p.Skp / 128;
    if (p.kb0 < 0 || p.nkb < 0 || p.kb0 + p.nkb > nkb || (p.nkb == 0 && p.kb0 != 0) ||
        (mode != 1 && p.nkb != 0))
        return hipErrorInvalidValue;
    const dim3 grid((p.nkb ? p.nkb : nkb) * p.BH);
    if (mode == 1) {
        if (D == 64) {
            if (causal) launch_dkdv_bf16<64, true>(p, grid, s);
            else launch_dkdv_bf16<64, false>(p, grid, s);
        } else if (D == 128) {
            if (causal) launch_dkdv_bf16<128, true>(p, grid, s);
            else launch_dkdv_bf16<128, false>(p, grid, s);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    GONN_BWD_LAUNCH(bwd_dkdv_f32_kernel);
    return hipGetLastError();
}

hipError_t launch_bwd_dq(const BwdParams& p, int mode, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0) return hipErrorInvalidValue;
    const dim3 grid((p.Sp / 128) * p.BH);
    if (mode == 1) return launch_bwd_dq_bf16(p, D, causal, s);
    GONN_BWD_LAUNCH(bwd_dq_f32_kernel);
    return hipGetLastError();
}

#undef GONN_BWD_LAUNCH

}  // namespace gonn
