// kernels.h -- launch interface between the C ABI (api.hip) and the kernels.
#pragma once
#include <vector>

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "common.h"

namespace gonn {

struct FwdParams {
    const void* q;  // (BH,Sq,D) f32 or bf16
    const void* k;  // bf16 mode: Kb (BH,Skp,D) bf16; fp32 mode: K (BH,Sk,D) f32
    const void* v;  // bf16 mode: Vt (BH,D,Skp) bf16; fp32 mode: V (BH,Sk,D) f32
    float* o;       // (BH,Sq,D)
    float* lse;     // (BH,Sq) or null
    int BH, Sq, Sk, Skp, nqb;
    float scale_log2;  // c2 = |scale| * log2(e) (log2(e) for a zero scale)
    float scale_abs;   // |scale| (1 for a zero scale)
    float qsign;       // sign(scale) (Q is negated for a negative scale; 0 for 0)
    int hgroup;        // slices whose blocks are dispatched interleaved (map_block)
    const int* kv_len; // [BH / H] valid keys per sequence, or null (all Sk)
    int H;             // heads per sequence (slice bh belongs to sequence bh / H)
    // Optional additive mask (WithAttnMask): slice bh = b*H + h adds
    // mask[b*mask_sb + h*mask_sh + q*Sk + key] to the scaled scores; only the
    // fp32 kernel reads it. mask_mul = 1 / scale_abs (raw score units).
    const float* mask;
    long long mask_sb, mask_sh;
    float mask_mul;
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
    // Causal multi-token attend only: T new queries per (b,h) (q and o are
    // (B,H,T,D) f32), the last T cached positions of each sequence; query t
    // sees keys [0, kv_len[b] - (T - 1 - t)). Partials are (B*H*T, nsplit).
    int T;
};

// Up to two sources packed by one launch (attn_pack.hip): src[i] (BH,S,D)
// f32 or bf16 -> row[i] (BH,Sp,D) bf16 and/or tr[i] (BH,D,Sp) bf16
// (transposed, 16-groups permuted by vt_pos), times mul[i]. Null outputs are
// skipped.
struct PackParams {
    const void* src[2];
    void* row[2];
    void* tr[2];
    float mul[2];  // each source is multiplied by mul before rounding to bf16
    int S, Sp;
};

struct BwdParams {
    // bf16 mode: packed operands in the workspace (row-major (BH,Sp,D), K^T
    // (BH,D,Skp)); fp32 mode: the caller's (BH,S,D) f32 buffers in q, k, v,
    // dO and a null kt.
    const void* q;
    const void* k;
    const void* v;
    const void* dO;
    const void* kt;   // K^T  bf16 mode only
    // dS-store path (bf16 mode): dS in blocks of kDsTileElems bf16 (one
    // 128-key block x one 64-query tile), slice bh at block bh *
    // ds_slice_blocks(..), key block kb's blocks from ds_block_base(kb, ..)
    // on, one per query tile from ds_first_qt(kb, causal) (the tiles a causal
    // key block reaches) to Sp/64; inside a block,
    // 16-byte piece ((key / 64) * 512 + c * 64 + key % 64) (key of the
    // block's 128) holds the key's dS for the 8 queries of
    // chunk c (queries 16 (c/2) + {4(c%2)..+3, 8+4(c%2)..+3}, the vt_pos
    // order of a 16-query group). Written by the dK/dV kernel when set, read
    // by bwd_dq_ds_kernel; null: the dQ kernel forms dS itself.
    bf16* ds;
    const float* lse2;   // (BH,Sp) LSE * log2(e); +inf on pad rows
    const float* delta;  // (BH,Sp) rowsum(dO * O); 0 on pad rows
    float* dq;           // (BH,S,D)
    float* dk;           // (BH,Sk,D)
    float* dv;
    int BH, S, Sp;       // S: query rows, Sp: S padded (lse2 / delta rows)
    int Sk, Skp;         // key rows and padded (equal to S, Sp except in the
                         // fp32 kernels' cross-attention backward)
    float scale;       // signed scale (fp32 kernels)
    float scale_log2;  // scale * log2(e) (fp32 kernels)
    // bf16 kernels: Q is packed times sign(scale) * c2 with
    // c2 = (scale ? |scale| : 1) * log2(e) (sign 0 for a zero scale), as the
    // bf16 forward packs it, so the exponent scale is c2b = 1; outputs
    // dQ = dqs * acc, dK = dks * acc with dqs = scale, dks = |scale| / c2.
    float c2b, dqs, dks;
    // Optional per-sequence key counts (device int32[BH / H]): keys
    // t >= kv_len[bh / H] of slice bh are padded (ForwardMasked key padding);
    // their dK, dV rows are zero and they add nothing to dQ.
    const int* kv_len;
    int H;
    // Optional additive mask, as in FwdParams.
    const float* mask;
    long long mask_sb, mask_sh;
    // Key-block chunk of the dS-store path (nkb = 0: every key block, the
    // whole call). The bf16 dK/dV kernel covers the 128-key blocks
    // [kb0, kb0 + nkb) and stores their dS, each slice's chunk from block
    // bh * ds_chunk_blocks(..) on, key block kb's part at ds_block_base(kb)
    // - ds_block_base(kb0); bwd_dq_ds_kernel adds the chunk's key tiles to
    // dQ. dq_mode: 0 the whole sum (start from 0, store dqs * sum); 1 a first
    // partial (start from 0, store the sum); 2 a middle one (start from the
    // stored partial, store the sum); 3 the last (start from the stored
    // partial, store dqs * sum). The partials pass through memory as fp32
    // unchanged, so a chunked call gives the same bits as a whole one.
    int kb0, nkb, dq_mode;
};

// Exact fp64 attention (attn_f64.hip): fp64 (BH, rows, d) buffers.
struct F64Params {
    const double* q;      // (BH, Sq, d)
    const double* k;      // (BH, Sk, d)
    const double* v;
    double* out_o;        // forward: O (BH, Sq, d)
    double* out_lse;      // forward: LSE (BH, Sq), natural log; may be null
    const double* o;      // backward inputs: O, dO (BH, Sq, d), LSE (BH, Sq)
    const double* dO;
    const double* lse;
    double* delta;        // backward workspace (BH, Sq)
    double* dq;           // backward outputs
    double* dk;
    double* dv;
    const int* kv_len;    // optional device int[B]: keys >= kv_len[b] are padded
    const double* mask;   // optional additive mask, element (b, h, i, j) at
    long long mask_sb, mask_sh;  // b * mask_sb + h * mask_sh + i * Sk + j
    int B, H, Sq, Sk, d;  // d <= 128
    double scale;
    int causal;           // top-left: key j > query i is masked
    // Causal forward split (fwd_f64_mfma_kernel; null items: none): rank r of
    // the grid (blockIdx / BH) runs item items[r] = 4 qb + part + 1, q-block
    // qb whole (part -1) or one half of its key range (part 0, 1). Q-blocks
    // from split_q0 on are split; each half writes its partial (per row: O
    // unnormalised, m, l) to `part`, and fwd_f64_combine_kernel, launched
    // after it, writes their O and LSE.
    const int* items;
    int nitems, split_q0;
    double* part;
    // Causal backward split, the same scheme in both kernels: the dQ kernel
    // halves the later q-blocks' key ranges (items, split_q0), the dK/dV
    // kernel the first key blocks' query ranges (items_k = 4 kb + part + 1,
    // key blocks before split_k1; those are the longest). Half 0 writes dQ
    // (dK, dV) itself and half 1 its partial to part (part_k), which
    // bwd_f64_combine_kernel, launched after both, adds in.
    const int* items_k;
    int nitems_k, split_k1;
    double* part_k;
};
// The causal split plan of the fp64 MFMA forward for these parameters: the
// item table (empty: no split), its first split q-block, and the bytes of
// the partials it needs.
struct F64FwdSplit {
    std::vector<int> items;
    int split_q0 = 0;
    size_t part_bytes = 0;
};
F64FwdSplit f64_fwd_split_plan(const F64Params& p);
// The causal split plan of the fp64 MFMA backward (empty tables: none).
struct F64BwdSplit {
    std::vector<int> items, items_k;
    int split_q0 = 0, split_k1 = 0;
    size_t part_bytes = 0, part_k_bytes = 0;
};
F64BwdSplit f64_bwd_split_plan(const F64Params& p);
hipError_t launch_f64_fwd(const F64Params& p, hipStream_t s);
hipError_t launch_f64_bwd(const F64Params& p, hipStream_t s);

// Additive mask (WithAttnMask) in the bf16 kernels whose lanes each own one
// query and whose S^T tiles hold 64 keys (the forwards and the dQ
// backward): one lane's row of one (b,h) slice, read 4 consecutive keys at a
// time through a raw buffer resource (a read past the slice returns 0; keys
// past the key end read whatever follows and are set to -inf by the key-end
// mask afterwards). Values are added to completed S^T tiles in log2 units
// (m log2 e), the units of the bf16 kernels' scores, before their masks.
struct MaskRow {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t row;  // byte offset of this lane's row
    GONN_DEV void init(const float* mask, long long sb, long long sh, int H, int Sq, int Sk, int bh,
                       int qi) {
        const float* base = mask + (size_t)(bh / H) * sb + (size_t)(bh % H) * sh;
        rs = make_rsrc(base, (uint32_t)((size_t)Sq * Sk * 4));
        row = (uint32_t)((qi < Sq ? qi : Sq - 1) * Sk) * 4u;
    }
    // The 32 mask values of this lane's scores in 64-key tile kt: register
    // 4j + e of S^T block mt holds key kt*64 + mt*32 + 8j + 4g + e.
    GONN_DEV void load(int kt, int g, f32x4* m) const {
        for (int mt = 0; mt < 2; mt++)
            for (int j = 0; j < 4; j++) {
                const uint32_t key0 = (uint32_t)(kt * 64 + mt * 32 + 8 * j + 4 * g);
                m[mt * 4 + j] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, row + key0 * 4u, 0, 0));
            }
    }
    GONN_DEV static void add(const f32x4* m, f32x16* s) {
        for (int mt = 0; mt < 2; mt++)
            for (int j = 0; j < 4; j++)
                for (int e = 0; e < 4; e++)
                    s[mt][4 * j + e] = __builtin_fmaf(m[mt * 4 + j][e], kLog2e, s[mt][4 * j + e]);
    }
};

// The same mask for the bf16 dK/dV backward, whose lanes each own one key and
// whose S tiles hold 64 queries: register 4j + e of S block mt of query tile
// qb is query qb*64 + mt*32 + 8j + 4g + e. One 4-byte read per score (a read
// past the slice returns 0; rows past the last query have P = 0).
struct MaskCol {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t col;  // byte offset of this lane's key in row 0
    uint32_t rowb;  // bytes per row
    GONN_DEV void init(const float* mask, long long sb, long long sh, int H, int Sq, int Sk, int bh,
                       int kj) {
        const float* base = mask + (size_t)(bh / H) * sb + (size_t)(bh % H) * sh;
        rs = make_rsrc(base, (uint32_t)((size_t)Sq * Sk * 4));
        col = (uint32_t)(kj < Sk ? kj : Sk - 1) * 4u;
        rowb = (uint32_t)Sk * 4u;
    }
    GONN_DEV void load(int qb, int g, f32x4* m) const {
        for (int mt = 0; mt < 2; mt++)
            for (int j = 0; j < 4; j++)
                for (int e = 0; e < 4; e++) {
                    const uint32_t q = (uint32_t)(qb * 64 + mt * 32 + 8 * j + 4 * g + e);
                    m[mt * 4 + j][e] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rs, col + q * rowb, 0, 0));
                }
    }
};

// Keys of slice bh that take part in the backward: Sk, or the sequence's
// kv_len clamped to [0, Sk]. Wave-uniform.
GONN_DEV int bwd_keys(const BwdParams& p, int bh) {
    if (!p.kv_len) return p.Sk;
    int l = p.kv_len[bh / p.H];
    l = l < 0 ? 0 : (l > p.Sk ? p.Sk : l);
    return __builtin_amdgcn_readfirstlane(l);
}

// Zero rows r0 .. r0 + rows - 1 (those below S) of the (BH, S, D) output
// `out` for slice bh, with every thread of the workgroup.
template <int D>
GONN_DEV void bwd_zero_rows(float* out, int S, int bh, int r0, int rows) {
    const int r1 = r0 + rows < S ? r0 + rows : S;
    if (r1 <= r0) return;
    f32x4* o = (f32x4*)(out + ((size_t)bh * S + r0) * D);
    for (int i = threadIdx.x; i < (r1 - r0) * D / 4; i += blockDim.x) o[i] = f32x4{};
}

hipError_t launch_pack(const PackParams& p, int nsrc, int in_bf16, int BH, int D, hipStream_t s);
hipError_t launch_fwd(const FwdParams& p, int mode, int D, int causal, int q_bf16,
                      hipStream_t s);
hipError_t launch_decode_split(const DecodeParams& p, int D, int q_bf16, hipStream_t s);
hipError_t launch_decode_combine(const DecodeParams& p, int D, hipStream_t s);
// Causal multi-token attend over the cache (attn_decode.hip): the split and
// combine kernels for p.T new queries per (b,h), kDecodeGroup queries per
// workgroup sharing each K/V row read.
constexpr int kDecodeGroup = 4;
hipError_t launch_decode_causal_split(const DecodeParams& p, int D, hipStream_t s);
hipError_t launch_decode_causal_combine(const DecodeParams& p, int D, hipStream_t s);
// KV-cache append (attn_decode.hip): row t < cnt[b] of the (B,H,T,D) sources
// (f32, or bf16 when src_bf16) to position pos[b] + t of the bf16 cache
// (B,H,Lmax,D). pos and cnt are device int32[B].
hipError_t launch_kv_append(const void* ks, const void* vs, int src_bf16, void* kc, void* vc,
                            const int* pos, const int* cnt, int B, int H, int T, int Lmax,
                            int D, hipStream_t s);
// Backward stages: prep (lse2, delta), then dK/dV (one workgroup per key
// block) and dQ (one workgroup per query block), both deterministic.
hipError_t launch_bwd_prep(const float* O, const float* dO, const float* lse, float* lse2,
                           float* delta, int BH, int S, int Sp, int D, int round_do,
                           hipStream_t s);
hipError_t launch_bwd_dkdv(const BwdParams& p, int mode, int D, int causal, hipStream_t s);
hipError_t launch_bwd_dq(const BwdParams& p, int mode, int D, int causal, hipStream_t s);
// bf16 dQ (attn_bwd_dq.hip); launch_bwd_dq dispatches mode 1 here.
hipError_t launch_bwd_dq_bf16(const BwdParams& p, int D, int causal, hipStream_t s);
// bf16 dQ from the stored dS (attn_bwd_dqds.hip): p.ds and p.kt set.
hipError_t launch_bwd_dq_ds(const BwdParams& p, int D, int causal, hipStream_t s);
// Sequence padding of the backward's workspace layouts.
constexpr int kBwdPad = 128;
// bf16 elements of one (128-key block, 64-query tile) block of stored dS.
constexpr int kDsTileElems = 128 * 64;
// Placement of the stored dS blocks of one (b,h) slice with nqt = Sp/64
// query tiles. A causal (top-left) key block kb reaches query tiles 2 kb
// and later only, and only those blocks are stored: key block kb's blocks
// start after sum_{k<kb} max(0, nqt - 2k) blocks, which for k < ceil(nqt/2)
// is kb nqt - kb (kb - 1) (key blocks past every query store none).
__host__ __device__ inline int ds_first_qt(int kb, int causal) { return causal ? 2 * kb : 0; }
__host__ __device__ inline long long ds_block_base(int kb, int nqt, int causal) {
    if (!causal) return (long long)kb * nqt;
    const int half = (nqt + 1) / 2;
    const long long kc = kb < half ? kb : half;
    return kc * nqt - kc * (kc - 1);
}
__host__ __device__ inline long long ds_slice_blocks(int nkb, int nqt, int causal) {
    return ds_block_base(nkb, nqt, causal);
}
// Stored dS blocks of key blocks [kb0, kb0 + nkb) of one slice.
__host__ __device__ inline long long ds_chunk_blocks(int kb0, int nkb, int nqt, int causal) {
    return ds_block_base(kb0 + nkb, nqt, causal) - ds_block_base(kb0, nqt, causal);
}

// f64 <-> f32/bf16 conversion with optional head-dim padding:
// dst (rows, dpad) <- src (rows, d); pad columns are zero.
hipError_t launch_convert_from_f64(const double* src, void* dst, int dst_bf16, size_t rows,
                                   int d, int dpad, hipStream_t s);
hipError_t launch_convert_to_f64(const void* src, int src_bf16, double* dst, size_t rows, int d,
                                 int dpad, hipStream_t s);
hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t s);

int selftest_mfma();

}  // namespace gonn
