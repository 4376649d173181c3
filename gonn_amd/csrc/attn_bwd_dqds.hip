// attn_bwd_dqds.hip -- dQ of the bf16 backward from the dS the dK/dV kernel
// stored (the dS-store path).
//
// Same result as bwd_dq_bf16_kernel (attn_bwd_dq.hip): dQ_i = scale *
// sum_j dS_ij k_j over the keys query i attends (the reference's identity,
// backend/cuda/gonn_cuda.cu:333-340). There the dQ kernel forms S and dP a
// second time to get dS (three GEMM-equivalents per (query, key) pair); here
// bwd_dkdv_bf16_kernel writes the dS it already formed, so dQ is one GEMM:
//
//   dQ^T (D x 256 queries of a block) = K^T (D x keys) . dS^T (keys x queries)
//
// The stored dS (layout at BwdParams::ds) keeps each 16-query group in the
// vt_pos order in which a dK/dV lane holds it. K^T is the packed Kt
// (BH, D, Skp) of attn_pack.hip, whose 16-key groups carry the same
// permutation, so the A and B operands of v_mfma_f32_32x32x16_bf16 agree on
// the key of every k-slot.
//
// One workgroup per 256 queries (8 waves x 32 queries), one per CU, key
// tiles of 64 streamed through three-slot LDS rings (step t loads tile t+2).
// The kernel is bound by its two load streams, dS from HBM and Kt from L2
// (timing builds without the MFMAs run as long); 256 queries per workgroup
// halve the Kt bytes per query against 128. Measured at C5: the dS stream
// alone runs at about 5.4 TB/s, whether one or three tiles are in flight,
// and with the block order or the piece order inside a block changed.
//  * Kt tile: D rows x 64 keys in the swizzled slab layout (slab_swz), read
//    as the A operand with one ds_read_b128 per MFMA;
//  * dS^T tile: 64 keys x 256 queries, stored chunk-major: 32 columns of
//    8 queries, each 64 keys x 16 bytes, 1088 bytes apart (64 bytes of pad).
//    One load instruction fills one column from 1 KB contiguous in HBM. It
//    is read as the B operand with ds_read_b64_tr_b16: per 16-lane group
//    that instruction returns to lane L the element L % 4 of the 8-byte
//    reads of lanes 4i + L / 4 (i = 0..3); with lane s of the group reading
//    key k0 + s / 4 at query column c0 + 4 (s % 4), lane L receives keys
//    k0 .. k0+3 of column c0 + L, i.e. 4 k-slots of the MFMA B operand.
//    Two such reads (keys 16ks + 4g.. and 16ks + 8 + 4g..) fill the 8
//    k-slots of lane group g in Kt's key order. A half-wave reads 4 keys x
//    32 queries, 4 columns x 64 bytes, which the 1088-byte column stride
//    puts on 64 distinct banks.
// Causal: a query block attends keys below its end (top-left mask); the
// masked (key > query) entries of the diagonal tiles were stored as zeros,
// and a wave skips the key tiles past its own 64-query tile.
// Key padding: keys at or past kv_len were stored as zeros, and key tiles
// past the last valid key are not read. Query columns past S hold values
// the dK/dV kernel never wrote; a dQ^T column depends on its own dS^T column
// only, and those rows are not written.
#include "common.h"
#include "kernels.h"

namespace gonn {

constexpr int kDqDsWaves = 8;  // waves (32 queries each) per workgroup

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kDqDsWaves * 64, 1) void bwd_dq_ds_kernel(BwdParams p) {
    constexpr int NW = kDqDsWaves, BM = NW * 32, BN = 64, NT = NW * 64;
    constexpr int NDT = D / 32;
    constexpr int NSLOT = 3, PF = NSLOT - 1;  // ring slots, tiles loaded ahead
    constexpr int SCB = BN * 16 + 64;  // dS^T tile column stride (bytes)
    constexpr int NSC = BM / 8;        // dS^T tile columns
    constexpr uint32_t KTB = D * BN * 2, STB = NSC * SCB;
    __shared__ __attribute__((aligned(16))) bf16 sK[NSLOT * D * BN];
    __shared__ __attribute__((aligned(16))) char sS[NSLOT * STB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    int bh, qb;
    map_block(blockIdx.x, (p.Sp + BM - 1) / BM, p.BH, CAUSAL, bh, qb);
    const int S = p.S, Sp = p.Sp, Skp = p.Skp;
    const int q0 = qb * BM;
    if (q0 >= S) return;  // padding rows only
    int kend = bwd_keys(p, bh);
    if (CAUSAL && q0 + BM < kend) kend = q0 + BM;
    // Key tiles [t0, t1) of this launch: the chunk's key blocks (two 64-key
    // tiles each) that hold keys this block attends.
    const int nkbc = p.nkb ? p.nkb : Skp / 128;
    const int t0 = 2 * p.kb0;
    int t1 = (kend + BN - 1) / BN;
    if (t1 > 2 * (p.kb0 + nkbc)) t1 = 2 * (p.kb0 + nkbc);
    const int ntiles = t1 > t0 ? t1 - t0 : 0;

    // ---- tile loads (direct to LDS): instruction i of thread tid fills the
    // 16-byte position i*NT + tid of a Kt tile (slab_chunk gives its row and
    // chunk); every thread issues NKI + NSC/4 loads per tile ----
    constexpr int NKI = D * BN / 8 / NT;
    static_assert(NKI * NT * 8 == D * BN, "whole Kt load instructions");
    static_assert(NSC % NW == 0, "dS^T columns spread over the waves");
    constexpr int NLD = NKI + NSC / NW;  // loads per tile per thread
    uint32_t koff[NKI];
    for (int i = 0; i < NKI; i++) {
        int r, c;
        slab_chunk(i * NT + tid, D, r, c);
        koff[i] = (uint32_t)((r * Skp + c * 8) * 2);
    }
    const bf16* Ktg = (const bf16*)p.kt + (size_t)bh * D * Skp;
    const brsrc krs = make_rsrc(Ktg, (uint32_t)D * Skp * 2);
    // This slice's stored dS blocks (placement at ds_block_base): key-block
    // major, so concurrent workgroups of a head read adjacent blocks (a
    // query-major order, which makes each workgroup's reads one stream but
    // puts concurrent workgroups 1 MB apart, measured 10% slower).
    const int nqt = Sp / 64, qt0 = q0 / 64;
    const long long nblk = ds_chunk_blocks(p.kb0, nkbc, nqt, CAUSAL);
    const long long cbase = ds_block_base(p.kb0, nqt, CAUSAL);  // the chunk's first block
    const brsrc srs = make_rsrc((const bf16*)p.ds + (size_t)(bh * nblk) * kDsTileElems,
                                (uint32_t)(nblk * kDsTileElems * 2));
    const uint32_t kl = lds_addr(sK) + wave * 1024, sl = lds_addr(sS);
    // A load no step reads (a tile past the last, or a dS column whose
    // waves skip this key tile) still issues, so every wave's vmcnt counts
    // match, but against a zero-size buffer: it moves no bytes.
    const brsrc nul = make_rsrc(p.ds, 0u);
    // Local tile u of this launch: key tile t0 + u.
    auto load_tile = [&](int u, int slot) {
        const bool real = u < ntiles;
        const int t = t0 + (real ? u : ntiles - 1);
        const brsrc kr = real ? krs : nul;
        for (int i = 0; i < NKI; i++)
            dma16(kr, kl + slot * KTB + i * NT * 16, koff[i], (uint32_t)t * BN * 2);
        // Column c = NW i + wave: query tile qt0 + c / 8, chunk c % 8, the 64
        // keys of half t % 2 of key block t / 2: lane L loads key L. A query
        // tile outside the key block's stored range (before its first tile,
        // causal, or past Sp) is clamped into it: only a wave that skips this
        // key tile, or dQ rows past S (not written), read that column.
        const int kb = t / 2, f = ds_first_qt(kb, CAUSAL);
        const long long kbase = ds_block_base(kb, nqt, CAUSAL) - cbase;
        for (int i = 0; i < NSC / NW; i++) {
            const int c = NW * i + wave;
            int qt = qt0 + c / 8;
            qt = qt < f ? f : (qt < nqt ? qt : nqt - 1);
            const uint32_t so = (uint32_t)((kbase + (qt - f)) * kDsTileElems * 2 +
                                           ((t % 2) * 512 + (c % 8) * 64) * 16);
            // Column c is read by the waves of query tile qt0 + c / 8.
            const bool need = real && (!CAUSAL || t <= qt0 + c / 8);
            dma16_nt(need ? srs : nul, sl + slot * STB + c * SCB, (uint32_t)lane * 16, so);
        }
    };

    // ---- operand reads ----
    // A (Kt): row dt*32 + ln, chunk 2ks + g, at (dt*32 + (ks/2)*D) * 64 +
    // (ks odd ? ka1 : ka0) in the slab layout.
    const int hs = slab_swz(ln);
    const uint32_t ka0 = (uint32_t)(ln * 64 + ((0 + g) ^ hs) * 16);
    const uint32_t ka1 = (uint32_t)(ln * 64 + ((2 + g) ^ hs) * 16);
    // B (dS^T): this lane reads key 4g + (lane & 15) / 4 (+16ks, +8 for the
    // second half of the k-slots) at query column qc = 32 wave + 16
    // ((lane >> 4) & 1) + 4 (lane & 3): column qc / 8, byte 2 (qc % 8).
    const int s16 = lane & 15;
    const int qc = 32 * wave + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);
    const uint32_t sb = (uint32_t)((qc / 8) * SCB + (4 * g + (s16 >> 2)) * 16 + (qc % 8) * 2);
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    typedef __attribute__((address_space(3))) char lds_char;
    lds_char* const sS3 = (lds_char*)sS;
    // byte: offset from the start of sS
    auto tr_read = [&](uint32_t byte) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(sS3 + byte));
    };

    // Lane (ln, g) holds query column 32 wave + ln of the block (stored
    // order), i.e. query q0 + 16 (c / 16) + vt_pos(c % 16); dQ^T register r
    // of d-tile dt is d = 32 dt + 8 (r / 4) + 4 g + r % 4.
    const int c = 32 * wave + ln;
    const int qi = q0 + (c & ~15) + vt_pos(c & 15);
    float* dqr = p.dq + ((size_t)bh * S + (qi < S ? qi : S - 1)) * D;
    f32x16 acc[NDT];
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x16{};
    if (p.dq_mode >= 2) {  // continue the partial sum an earlier chunk stored
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int rq4 = 0; rq4 < 4; rq4++) {
                const f32x4 a = *(const f32x4*)(dqr + dt * 32 + rq4 * 8 + g * 4);
                for (int k = 0; k < 4; k++) acc[dt][rq4 * 4 + k] = a[k];
            }
        // Landed here: otherwise the compiler guards the accumulators' first
        // use inside the step loop with waits that also cover the tile loads
        // in flight, and every step waits for its own prefetch (+22% at C5).
        GONN_VMCNT(0);
    }
    // Tiles past the last are loads of no bytes into a slot no step reads,
    // so every step issues NLD loads and the wait for tile t+1 at the end of
    // step t is always "all but the newest PF-1 tiles".
    if (ntiles > 0) {
        for (int j = 0; j < PF; j++) load_tile(j, j);
        GONN_VMCNT((PF - 1) * NLD);
        __syncthreads();
        for (int u = 0; u < ntiles; u++) {
            const int t = t0 + u, cur = u % NSLOT;
            load_tile(u + PF, (u + PF) % NSLOT);
            const char* kbase = (const char*)sK + cur * KTB;
            const uint32_t sbase = cur * STB + sb;
            // Causal: this wave's 32 queries lie in query tile qt0 + wave/2,
            // which sees key tiles up to its own index; later key tiles are
            // fully masked, and the dK/dV kernel (whose key block kb starts
            // at query tile 2 kb) wrote no dS for some of them. Wave-uniform;
            // the loads above stay uniform so every wave's vmcnt counts match.
            const bool live = !CAUSAL || t <= qt0 + (wave >> 1);
            for (int ks = 0; ks < (live ? BN / 16 : 0); ks++) {
                const s4 lo = tr_read(sbase + (uint32_t)(16 * ks) * 16);
                const s4 hi = tr_read(sbase + (uint32_t)(16 * ks + 8) * 16);
                const s4 b8[2] = {lo, hi};
                const bf16x8 bop = __builtin_bit_cast(bf16x8, b8);
                for (int dt = 0; dt < NDT; dt++) {
                    const bf16x8 aop = *(const bf16x8*)(kbase + (ks & 1 ? ka1 : ka0) +
                                                        (dt * 32 + (ks >> 1) * D) * 64);
                    acc[dt] = mfma_bf16(aop, bop, acc[dt]);
                }
            }
            GONN_VMCNT((PF - 1) * NLD);
            __syncthreads();
        }
        GONN_VMCNT(0);
    }

    if (qi < S) {
        // dqs on the whole sum (modes 0 and 3); a partial is stored as it is.
        const float sc = (p.dq_mode == 1 || p.dq_mode == 2) ? 1.f : p.dqs;
        for (int dt = 0; dt < NDT; dt++)
            for (int rq4 = 0; rq4 < 4; rq4++) {
                f32x4 a;
                for (int k = 0; k < 4; k++) a[k] = acc[dt][rq4 * 4 + k] * sc;
                *(f32x4*)(dqr + dt * 32 + rq4 * 8 + g * 4) = a;
            }
    }
}

hipError_t launch_bwd_dq_ds(const BwdParams& p, int D, int causal, hipStream_t s) {
    if (p.Sp % kBwdPad != 0 || p.Skp % kBwdPad != 0 || !p.ds || !p.kt)
        return hipErrorInvalidValue;
    if (p.kb0 < 0 || p.nkb < 0 || p.kb0 + p.nkb > p.Skp / 128 || (p.nkb == 0 && p.kb0 != 0) ||
        p.dq_mode < 0 || p.dq_mode > 3 || (p.nkb == 0 && p.dq_mode != 0))
        return hipErrorInvalidValue;
    constexpr int BM = kDqDsWaves * 32, NT = kDqDsWaves * 64;
    const dim3 grid(((p.Sp + BM - 1) / BM) * p.BH);
    if (D == 64) {
        if (causal) bwd_dq_ds_kernel<64, true><<<grid, NT, 0, s>>>(p);
        else bwd_dq_ds_kernel<64, false><<<grid, NT, 0, s>>>(p);
    } else if (D == 128) {
        if (causal) bwd_dq_ds_kernel<128, true><<<grid, NT, 0, s>>>(p);
        else bwd_dq_ds_kernel<128, false><<<grid, NT, 0, s>>>(p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gonn
