// attn_f64.hip -- exact fp64 attention for the reference-named f64 entry
// points (GONN_ATTN_FP64 mode).
//
// GoNN's CUDA seam computes attention in fp64 end to end
// (backend/cuda/gonn_cuda.cu:302-450, driven by :466-529), and its own
// checking programs hold the fused path to that: max abs diff <= 1e-9
// against refAttn (benchmark/flashattn/main.go:114), the same against the
// unfused MHA (benchmark/mha/main.go:64), and a central-difference
// gradcheck with eps 1e-6 (benchmark/flashbwd/main.go:56-90). These kernels
// give the f64 entries that precision on the GPU: every product, sum, exp
// and log is a double (exp and log from the device math library, accurate
// to about 1 ulp), so results agree with a CPU fp64 evaluation to rounding.
//
// The math is the same as the other modes' (and GoNN's CPU chain,
// nn/attention.go:136-146 plus tensor/ops_activation.go:455-461):
//   s_ij = scale * q_i . k_j (+ m_ij, the additive mask), masked keys -inf
//   (causal top-left key j > query i; keys j >= kv_len[b]);
//   forward: online softmax over 32-key tiles (row max, exp(s - max),
//   rescale of l and O when the max moves); O_i = sum_j p_ij v_j / l_i,
//   LSE_i = max + log l (natural log; -inf and O = 0 for a row without keys);
//   backward from O and LSE: p_ij = exp(s_ij - LSE_i),
//   D_i = dO_i . O_i, dS_ij = p_ij (dO_i . v_j - D_i),
//   dV_j = sum_i p_ij dO_i, dK_j = scale sum_i dS_ij q_i,
//   dQ_i = scale sum_j dS_ij k_j (backend/cuda/gonn_cuda.cu:333-340).
//
// Layout: fp64 (BH, rows, d) row-major, as the f64 entries receive them.
// Two kernel families:
//  * the default, on v_mfma_f64_16x16x4f64 (fwd_f64_mfma_kernel,
//    dq_f64_mfma_kernel, dkdv_f64_mfma_kernel): a wave owns 16 rows, and
//    the score tiles are formed in the orientation whose register layout is
//    the next product's operand layout, so P and dS feed the MFMAs from
//    registers and each score's exp is computed once (the kernels' own
//    comments give the layouts);
//  * the team kernels (GONN_HIP_F64_FWD / GONN_HIP_F64_BWD = "valu"): a row
//    (query or key) is owned by a team of 8 lanes; lane u of the team holds
//    elements 8t + u (t < DP/8) of the row's vectors, so a team reads 64
//    contiguous bytes per t and dot products end in a 3-step lane
//    reduction; the streamed rows sit in LDS tiles of 32 rows that every
//    team reads in the same order (broadcasts).
// Every backward kernel owns its outputs: no atomics, deterministic.
#include <cmath>
#include <cstdlib>

#include <algorithm>
#include <utility>

#include "common.h"
#include "kernels.h"

namespace gonn {

namespace {

constexpr int kTeam = 8;     // lanes per row
constexpr int kRowsWG = 32;  // rows owned per workgroup (256 threads)
constexpr int kTile = 32;    // streamed rows per LDS tile

__device__ __forceinline__ double team_sum(double x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    return x;
}

// Keys [0, kend) of slice bh are real (kv_len key padding).
__device__ __forceinline__ int keys_of(const F64Params& p, int bh) {
    if (!p.kv_len) return p.Sk;
    const int n = p.kv_len[bh / p.H];
    return n < 0 ? 0 : (n < p.Sk ? n : p.Sk);
}

__device__ __forceinline__ double mask_at(const F64Params& p, int bh, int i, int j) {
    if (!p.mask) return 0.0;
    const long long b = bh / p.H, h = bh % p.H;
    return p.mask[b * p.mask_sb + h * p.mask_sh + (long long)i * p.Sk + j];
}

// Loads rows [r0, r0 + kTile) of a (rows, d) slice into an LDS tile of
// stride DP (rows past nrows and columns past d are zero).
template <int DP>
__device__ __forceinline__ void load_tile(double (*dst)[DP + 1], const double* src, int r0,
                                          int nrows, int d) {
    for (int e = threadIdx.x; e < kTile * DP; e += blockDim.x) {
        const int r = e / DP, c = e % DP;
        const int row = r0 + r;
        dst[r][c] = (row < nrows && c < d) ? src[(size_t)row * d + c] : 0.0;
    }
}

}  // namespace

// Forward: 32 queries per workgroup.
template <int DP>
__global__ __launch_bounds__(256) void fwd_f64_kernel(F64Params p) {
    constexpr int DQ = DP / kTeam;
    __shared__ double sK[kTile][DP + 1], sV[kTile][DP + 1];
    const int bh = blockIdx.y, team = threadIdx.x / kTeam, u = threadIdx.x % kTeam;
    const int q0 = blockIdx.x * kRowsWG, i = q0 + team;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int kend_b = keys_of(p, bh);
    // Keys any query of the block can see (top-left causal: j <= i).
    int kend = kend_b;
    if (p.causal && q0 + kRowsWG < kend) kend = q0 + kRowsWG;
    const int kend_i = p.causal ? (i + 1 < kend_b ? i + 1 : kend_b) : kend_b;

    double qd[DQ], od[DQ];
    const double* qrow = p.q + ((size_t)bh * Sq + (i < Sq ? i : 0)) * d;
    for (int t = 0; t < DQ; t++) {
        const int c = kTeam * t + u;
        qd[t] = (i < Sq && c < d) ? qrow[c] : 0.0;
        od[t] = 0.0;
    }
    double m = -INFINITY, l = 0.0;
    const double* kg = p.k + (size_t)bh * Sk * d;
    const double* vg = p.v + (size_t)bh * Sk * d;
    for (int j0 = 0; j0 < kend; j0 += kTile) {
        __syncthreads();  // the previous tile is consumed
        load_tile<DP>(sK, kg, j0, Sk, d);
        load_tile<DP>(sV, vg, j0, Sk, d);
        __syncthreads();
        double s[kTile];
        double tmax = -INFINITY;
        for (int j = 0; j < kTile; j++) {
            double acc = 0.0;
            for (int t = 0; t < DQ; t++) acc = fma(qd[t], sK[j][kTeam * t + u], acc);
            acc = team_sum(acc);
            const int key = j0 + j;
            const bool off = key >= kend_i || i >= Sq;
            s[j] = off ? -INFINITY
                       : p.scale * acc + mask_at(p, bh, i < Sq ? i : 0, key < Sk ? key : 0);
            tmax = fmax(tmax, s[j]);
        }
        const double mnew = fmax(m, tmax);
        if (mnew == -INFINITY) continue;  // no visible key yet (lane-uniform per team)
        const double alpha = m == -INFINITY ? 0.0 : exp(m - mnew);
        l *= alpha;
        for (int t = 0; t < DQ; t++) od[t] *= alpha;
        for (int j = 0; j < kTile; j++) {
            const double pj = exp(s[j] - mnew);
            l += pj;
            for (int t = 0; t < DQ; t++) od[t] = fma(pj, sV[j][kTeam * t + u], od[t]);
        }
        m = mnew;
    }
    if (i < Sq) {
        double* orow = p.out_o + ((size_t)bh * Sq + i) * d;
        const double inv = l > 0.0 ? 1.0 / l : 0.0;
        for (int t = 0; t < DQ; t++) {
            const int c = kTeam * t + u;
            if (c < d) orow[c] = od[t] * inv;
        }
        if (p.out_lse && u == 0) p.out_lse[(size_t)bh * Sq + i] = l > 0.0 ? m + log(l) : -INFINITY;
    }
}

// Forward on v_mfma_f64_16x16x4f64 (fp64 in, fp64 accumulate). Layout of
// that instruction (probed on gfx950, as in gemm.hip): the A operand (16 x 4)
// is element (l % 16, l / 16) of lane l, B (4 x 16) element (l / 16, l % 16),
// and register r of the 16 x 16 result holds row 4 r + l / 16, column l % 16.
//
// A wave owns 16 queries (workgroup: 4 waves, 64 queries). Per 16-key tile
// it forms S^T = K Q^T (rows: keys, columns: queries; Q^T is the B operand,
// kept in registers), so register r of a lane holds the score of key
// 4 r + l / 16 for query l % 16. That is exactly the B operand of the PV
// product's k-step r: O^T (d x queries) += V^T (d x keys) P^T, with k-slot
// l / 16 of step r standing for key 4 r + l / 16. P goes from the score
// registers into the PV MFMAs without moving, and the exponential of every
// score is taken once (the VALU kernel above takes it on all 8 lanes of a
// team). A query's scores sit in the 4 lanes l % 16 = c; its row max and
// sum are in-lane plus two cross-lane steps.
//
// K and V stages (32 keys, 16 at d = 128) are staged through registers into
// LDS in the order the A operands are read, so every MFMA operand read is 64
// doubles in lane order:
//   sK[t][s][j][q] = K[16 t + j][4 s + q]               (S^T k-step s)
//   sV[t][r][dt][q][j] = V[16 t + 4 r + q][16 dt + j]   (PV k-step r, d tile dt)
// Causal grids put the longest q-blocks first. From 16 q-blocks on, the later
// half of a causal grid's q-blocks is split into two key ranges run by two
// workgroups (F64Params::items), and fwd_f64_combine_kernel merges their
// partials: a grid that is one round of workgroups then lasts about half the
// longest q-block instead of all of it.
typedef double f64x4_t __attribute__((ext_vector_type(4)));
typedef double f64x2_t __attribute__((ext_vector_type(2)));
constexpr int kMWaveQ = 16;                   // queries per wave
constexpr int kMRows = 4 * kMWaveQ;           // queries per workgroup
// Keys per LDS stage: 32 at d <= 64; 16 at d = 128, where the register
// staging of a 32-key stage would not fit beside the Q fragment and O.
constexpr int mstage(int DP) { return DP <= 64 ? 32 : 16; }

__device__ __forceinline__ f64x4_t mfma_f64(double a, double b, f64x4_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Value of lane l combined with lanes l ^ 16 and l ^ 32 (the 4 lanes that
// hold one query's keys).
__device__ __forceinline__ double quad_max(double x) {
    x = fmax(x, __shfl_xor(x, 16));
    return fmax(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ double quad_sum(double x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

template <int DP>
__global__ __launch_bounds__(256, 2) void fwd_f64_mfma_kernel(F64Params p) {
    constexpr int NS = DP / 4;    // S^T k-steps (d)
    constexpr int NDT = DP / 16;  // 16-row d tiles of O^T
    constexpr int kMStage = mstage(DP), kMTiles = kMStage / 16;
    constexpr int NCH = kMStage * DP / 2 / 256;  // 16-byte chunks per thread per stage (K, V each)
    static_assert(NCH * 256 * 2 == kMStage * DP, "whole chunks per stage");
    __shared__ double sK[kMTiles * NS * 64];
    __shared__ double sV[kMTiles * 4 * NDT * 64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, quad = lane >> 4;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int nqb = (Sq + kMRows - 1) / kMRows, BH = p.B * p.H;
    const int rank = blockIdx.x / BH;
    const int bh = blockIdx.x - rank * BH;
    // Causal grids run the longest work first: whole q-blocks from the last,
    // or the items of the split plan (halves of the long q-blocks' key
    // ranges, which even out a grid that is a single round of workgroups).
    int qb = p.causal ? nqb - 1 - rank : rank, part = -1;
    if (p.items) {
        const int c = p.items[rank];
        qb = c >> 2;
        part = (c & 3) - 1;
    }
    const int q0 = qb * kMRows, qw = q0 + wave * kMWaveQ, qi = qw + col;
    const int kend_b = keys_of(p, bh);
    int kend = kend_b, kbeg = 0;
    if (p.causal && q0 + kMRows < kend) kend = q0 + kMRows;
    if (part >= 0) {  // keys [0, mid) or [mid, kend), mid on a stage boundary
        const int mid = (kend / 2) / kMStage * kMStage;
        if (part == 0) kend = mid;
        else kbeg = mid;
    }

    // Q^T fragment: qf[s] = Q[qi][4 s + quad].
    double qf[NS];
    {
        const double* qrow = p.q + ((size_t)bh * Sq + (qi < Sq ? qi : 0)) * d;
        for (int s = 0; s < NS; s++) {
            const int c = 4 * s + quad;
            qf[s] = (qi < Sq && c < d) ? qrow[c] : 0.0;
        }
    }
    f64x4_t oacc[NDT];
    for (int t = 0; t < NDT; t++) oacc[t] = f64x4_t{0.0, 0.0, 0.0, 0.0};
    double m = -INFINITY, l = 0.0;

    const double* kg = p.k + (size_t)bh * Sk * d;
    const double* vg = p.v + (size_t)bh * Sk * d;
    // Chunk i of thread tid: key (i*256 + tid) / (DP/2), columns 2 ((i*256 +
    // tid) % (DP/2)) and the next (coalesced rows).
    f64x2_t kst[NCH], vst[NCH];
    auto load_stage = [&](int j0) {
        for (int i = 0; i < NCH; i++) {
            const int c = i * 256 + tid, key = j0 + c / (DP / 2), dd = 2 * (c % (DP / 2));
            const bool in = key < Sk && dd < d;  // d even or dd + 1 < d handled below
            f64x2_t kv{0.0, 0.0}, vv{0.0, 0.0};
            if (in) {
                const size_t off = (size_t)key * d + dd;
                kv[0] = kg[off];
                vv[0] = vg[off];
                if (dd + 1 < d) {
                    kv[1] = kg[off + 1];
                    vv[1] = vg[off + 1];
                }
            }
            kst[i] = kv;
            vst[i] = vv;
        }
    };
    auto store_stage = [&]() {
        for (int i = 0; i < NCH; i++) {
            const int c = i * 256 + tid, kr = c / (DP / 2), dd = 2 * (c % (DP / 2));
            const int t = kr >> 4, j = kr & 15;
            // K: (t, s = dd / 4, j, q = dd % 4 and + 1)
            *(f64x2_t*)&sK[((t * NS + (dd >> 2)) * 16 + j) * 4 + (dd & 3)] = kst[i];
            // V: (t, r = j / 4, dt = dd / 16, q = j % 4, jj = dd % 16 and + 1)
            *(f64x2_t*)&sV[(((t * 4 + (j >> 2)) * NDT + (dd >> 4)) * 4 + (j & 3)) * 16 + (dd & 15)] =
                vst[i];
        }
    };

    if (kend > kbeg) load_stage(kbeg);
    for (int j0 = kbeg; j0 < kend; j0 += kMStage) {
        __syncthreads();  // the previous stage is consumed
        store_stage();
        __syncthreads();
        if (j0 + kMStage < kend) load_stage(j0 + kMStage);  // lands during this stage
        // Tiles of this stage this wave sees at all (causal: keys <= its last query).
        f64x4_t sacc[kMTiles];
        double smax = -INFINITY;
        for (int t = 0; t < kMTiles; t++) {
            const int kt0 = j0 + 16 * t;
            sacc[t] = f64x4_t{0.0, 0.0, 0.0, 0.0};
            if (kt0 >= kend || (p.causal && kt0 > qw + kMWaveQ - 1)) {
                sacc[t] = f64x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
                continue;
            }
            for (int s = 0; s < NS; s++)
                sacc[t] = mfma_f64(sK[((t * NS + s) * 16 + col) * 4 + quad], qf[s], sacc[t]);
            for (int r = 0; r < 4; r++) {
                const int key = kt0 + 4 * r + quad;
                const bool off = key >= kend_b || qi >= Sq || (p.causal && key > qi);
                const double sc = off ? -INFINITY
                                      : p.scale * sacc[t][r] +
                                            mask_at(p, bh, qi < Sq ? qi : 0, key < Sk ? key : 0);
                sacc[t][r] = sc;
                smax = fmax(smax, sc);
            }
        }
        smax = quad_max(smax);
        // No branch on a query column's state around the MFMAs (they read
        // operands from every lane): a column that has seen no key yet keeps
        // m = -inf, gets offset 0 (so P = exp(-inf) = 0) and alpha = 0.
        const double mnew = fmax(m, smax);
        const double mref = mnew == -INFINITY ? 0.0 : mnew;
        const double alpha = m == -INFINITY ? 0.0 : exp(m - mref);
        l *= alpha;
        for (int t = 0; t < NDT; t++) oacc[t] *= alpha;
        m = mnew;
        for (int t = 0; t < kMTiles; t++) {
            const int kt0 = j0 + 16 * t;
            if (kt0 >= kend || (p.causal && kt0 > qw + kMWaveQ - 1)) continue;  // wave-uniform
            for (int r = 0; r < 4; r++) {
                const double pr = exp(sacc[t][r] - mref);  // once per score
                l += pr;
                for (int dt = 0; dt < NDT; dt++)
                    oacc[dt] = mfma_f64(sV[(((t * 4 + r) * NDT + dt) * 4 + quad) * 16 + col], pr,
                                        oacc[dt]);
            }
        }
    }
    const double lt = quad_sum(l);
    if (part >= 0) {
        // A half's partial, per row of the q-block: O unnormalised (DP
        // columns), then m and l; fwd_f64_combine_kernel merges the halves.
        const int si = bh * (nqb - p.split_q0) + (qb - p.split_q0);
        double* row = p.part + (((size_t)si * 2 + part) * kMRows + wave * kMWaveQ + col) * (DP + 2);
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) row[16 * dt + 4 * r + quad] = oacc[dt][r];
        if (quad == 0) {
            row[DP] = m;
            row[DP + 1] = lt;
        }
        return;
    }
    if (qi < Sq) {
        double* orow = p.out_o + ((size_t)bh * Sq + qi) * d;
        const double inv = lt > 0.0 ? 1.0 / lt : 0.0;
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) {
                const int c = 16 * dt + 4 * r + quad;
                if (c < d) orow[c] = oacc[dt][r] * inv;
            }
        if (p.out_lse && quad == 0)
            p.out_lse[(size_t)bh * Sq + qi] = lt > 0.0 ? m + log(lt) : -INFINITY;
    }
}

// The two halves of each split q-block (fwd_f64_mfma_kernel): one thread per
// (row, column) of a split q-block, O = (o0 a0 + o1 a1) / (l0 a0 + l1 a1)
// with a = exp(m - max(m0, m1)), LSE = max(m0, m1) + log(l); a row no key
// reaches gets O = 0 and LSE = -inf, as in the whole kernel.
template <int DP>
__global__ __launch_bounds__(256) void fwd_f64_combine_kernel(F64Params p) {
    const int nqb = (p.Sq + kMRows - 1) / kMRows, ns = nqb - p.split_q0;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per = (size_t)kMRows * DP;  // threads per split q-block
    if (i >= (size_t)p.B * p.H * ns * per) return;
    const int si = (int)(i / per), rc = (int)(i % per), r = rc / DP, c = rc % DP;
    const int bh = si / ns, qb = p.split_q0 + si % ns, qi = qb * kMRows + r;
    if (qi >= p.Sq || c >= p.d) return;
    const double* h0 = p.part + (((size_t)si * 2 + 0) * kMRows + r) * (DP + 2);
    const double* h1 = h0 + (size_t)kMRows * (DP + 2);
    const double m0 = h0[DP], l0 = h0[DP + 1], m1 = h1[DP], l1 = h1[DP + 1];
    const double mm = fmax(m0, m1);
    const double a0 = m0 == -INFINITY ? 0.0 : exp(m0 - mm);
    const double a1 = m1 == -INFINITY ? 0.0 : exp(m1 - mm);
    const double l = l0 * a0 + l1 * a1;
    p.out_o[((size_t)bh * p.Sq + qi) * p.d + c] = l > 0.0 ? (h0[c] * a0 + h1[c] * a1) / l : 0.0;
    if (p.out_lse && c == 0) p.out_lse[(size_t)bh * p.Sq + qi] = l > 0.0 ? mm + log(l) : -INFINITY;
}

// Backward on v_mfma_f64_16x16x4f64, the forward's layout applied to the
// backward identities (P = exp(s - L), dS = P (dP - D) scale):
//  dQ: a wave owns 16 queries; per 16-key tile S^T = K Q^T and dP^T = V dO^T
//      (Q^T, dO^T fragments in registers), then dQ^T (d x queries) += K^T
//      dS^T with dS^T straight from the score registers (register r = key
//      4 r + l / 16, the k-slot of step r).
//  dK/dV: a wave owns 16 keys; per 16-query tile S = Q K^T and dP = dO V^T
//      (K^T, V^T fragments in registers; register r = query 4 r + l / 16),
//      then dV^T += dO^T P and dK^T += Q^T dS from those registers.
// The streamed rows go into LDS in both operand orders they are read in:
//   "rows"  X[t][s][j][q] = X[16 t + j][4 s + q]   (A of S, dP: rows x d)
//   "cols"  X[t][r][dt][q][j] = X[16 t + 4 r + q][16 dt + j]  (A of the
//           output products: d x rows)
// Each kernel owns its outputs (no atomics), so results are deterministic.
// d = 128 runs one wave per SIMD (the four register fragments and
// accumulators need more than half the register file).
constexpr int mb_waves(int DP) { return DP <= 64 ? 2 : 1; }  // workgroups per CU

// Stage `srcA` (and `srcB`) rows [r0, r0 + ROWS) of a (nrows, d) slice into
// LDS in the rows order (la, lb) and the cols order (ta, tb); rows past
// nrows and columns past d are zero. Chunk i of thread tid is row (i*256 +
// tid) / (DP/2), columns 2 ((i*256 + tid) % (DP/2)) and the next.
template <int DP, int ROWS>
struct F64Stage {
    static constexpr int NS = DP / 4, NDT = DP / 16;
    static constexpr int NCH = ROWS * DP / 2 / 256;
    static_assert(NCH * 512 == ROWS * DP, "whole chunks per stage");
    f64x2_t a[NCH], b[NCH];
    __device__ __forceinline__ void load(const double* srcA, const double* srcB, int r0, int nrows,
                                         int d) {
        for (int i = 0; i < NCH; i++) {
            const int c = i * 256 + threadIdx.x, row = r0 + c / (DP / 2), dd = 2 * (c % (DP / 2));
            f64x2_t va{0.0, 0.0}, vb{0.0, 0.0};
            if (row < nrows && dd < d) {
                const size_t off = (size_t)row * d + dd;
                va[0] = srcA[off];
                vb[0] = srcB[off];
                if (dd + 1 < d) {
                    va[1] = srcA[off + 1];
                    vb[1] = srcB[off + 1];
                }
            }
            a[i] = va;
            b[i] = vb;
        }
    }
    // la/lb: rows order (or null), ta/tb: cols order (or null).
    __device__ __forceinline__ void store(double* la, double* lb, double* ta, double* tb) const {
        for (int i = 0; i < NCH; i++) {
            const int c = i * 256 + threadIdx.x, kr = c / (DP / 2), dd = 2 * (c % (DP / 2));
            const int t = kr >> 4, j = kr & 15;
            const int ro = ((t * NS + (dd >> 2)) * 16 + j) * 4 + (dd & 3);
            const int co = (((t * 4 + (j >> 2)) * NDT + (dd >> 4)) * 4 + (j & 3)) * 16 + (dd & 15);
            if (la) *(f64x2_t*)&la[ro] = a[i];
            if (lb) *(f64x2_t*)&lb[ro] = b[i];
            if (ta) *(f64x2_t*)&ta[co] = a[i];
            if (tb) *(f64x2_t*)&tb[co] = b[i];
        }
    }
};

template <int DP>
__global__ __launch_bounds__(256, mb_waves(DP)) void dq_f64_mfma_kernel(F64Params p) {
    constexpr int NS = DP / 4, NDT = DP / 16;
    constexpr int STG = mstage(DP), NT16 = STG / 16;
    __shared__ double sK[NT16 * NS * 64];             // K, rows order (A of S^T)
    __shared__ double sV[NT16 * NS * 64];             // V, rows order (A of dP^T)
    __shared__ double sKt[NT16 * 4 * NDT * 64];       // K, cols order (A of dQ^T)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, quad = lane >> 4;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int nqb = (Sq + kMRows - 1) / kMRows, BH = p.B * p.H;
    const int rank = blockIdx.x / BH, bh = blockIdx.x - rank * BH;
    int qb = p.causal ? nqb - 1 - rank : rank, part = -1;
    if (p.items) {  // the causal split (F64Params::items)
        const int c = p.items[rank];
        qb = c >> 2;
        part = (c & 3) - 1;
    }
    const int q0 = qb * kMRows, qw = q0 + wave * kMWaveQ, qi = qw + col;
    const int kend_b = keys_of(p, bh);
    int kend = kend_b, kbeg = 0;
    if (p.causal && q0 + kMRows < kend) kend = q0 + kMRows;
    if (part >= 0) {  // keys [0, mid) or [mid, kend), mid on a stage boundary
        const int mid = (kend / 2) / STG * STG;
        if (part == 0) kend = mid;
        else kbeg = mid;
    }
    const int ic = qi < Sq ? qi : 0;
    const size_t row = ((size_t)bh * Sq + ic) * d;
    double qf[NS], gf[NS];
    for (int s = 0; s < NS; s++) {
        const int c = 4 * s + quad;
        qf[s] = (qi < Sq && c < d) ? p.q[row + c] : 0.0;
        gf[s] = (qi < Sq && c < d) ? p.dO[row + c] : 0.0;
    }
    const double L = p.lse[(size_t)bh * Sq + ic];
    const double Di = p.delta[(size_t)bh * Sq + ic];
    const bool live = qi < Sq && L != -INFINITY;
    f64x4_t dqacc[NDT];
    for (int t = 0; t < NDT; t++) dqacc[t] = f64x4_t{0.0, 0.0, 0.0, 0.0};
    const double* kg = p.k + (size_t)bh * Sk * d;
    const double* vg = p.v + (size_t)bh * Sk * d;
    F64Stage<DP, STG> st;
    if (kend > kbeg) st.load(kg, vg, kbeg, Sk, d);
    for (int j0 = kbeg; j0 < kend; j0 += STG) {
        __syncthreads();
        st.store(sK, sV, sKt, nullptr);
        __syncthreads();
        if (j0 + STG < kend) st.load(kg, vg, j0 + STG, Sk, d);
        for (int t = 0; t < NT16; t++) {
            const int kt0 = j0 + 16 * t;
            if (kt0 >= kend || (p.causal && kt0 > qw + kMWaveQ - 1)) continue;  // wave-uniform
            f64x4_t sacc{0.0, 0.0, 0.0, 0.0}, pacc{0.0, 0.0, 0.0, 0.0};
            for (int s2 = 0; s2 < NS; s2++) {
                const int a = ((t * NS + s2) * 16 + col) * 4 + quad;
                sacc = mfma_f64(sK[a], qf[s2], sacc);
                pacc = mfma_f64(sV[a], gf[s2], pacc);
            }
            for (int r = 0; r < 4; r++) {
                const int key = kt0 + 4 * r + quad;
                const bool on = live && key < kend_b && !(p.causal && key > qi);
                const double sc = p.scale * sacc[r] + mask_at(p, bh, ic, key < Sk ? key : 0);
                const double ds = on ? exp(sc - L) * (pacc[r] - Di) * p.scale : 0.0;
                for (int dt = 0; dt < NDT; dt++)
                    dqacc[dt] = mfma_f64(sKt[(((t * 4 + r) * NDT + dt) * 4 + quad) * 16 + col], ds,
                                         dqacc[dt]);
            }
        }
    }
    if (part == 1) {  // the second half's partial, all DP columns of its rows
        const int si = bh * (nqb - p.split_q0) + (qb - p.split_q0);
        double* pr = p.part + ((size_t)si * kMRows + wave * kMWaveQ + col) * DP;
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) pr[16 * dt + 4 * r + quad] = dqacc[dt][r];
        return;
    }
    if (qi < Sq) {
        double* dqr = p.dq + row;
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) {
                const int c = 16 * dt + 4 * r + quad;
                if (c < d) dqr[c] = dqacc[dt][r];
            }
    }
}

template <int DP>
__global__ __launch_bounds__(256, mb_waves(DP)) void dkdv_f64_mfma_kernel(F64Params p) {
    constexpr int NS = DP / 4, NDT = DP / 16;
    constexpr int STG = mstage(DP), NT16 = STG / 16;
    __shared__ double sQ[NT16 * NS * 64];        // Q, rows order (A of S)
    __shared__ double sG[NT16 * NS * 64];        // dO, rows order (A of dP)
    __shared__ double sQt[NT16 * 4 * NDT * 64];  // Q, cols order (A of dK^T)
    __shared__ double sGt[NT16 * 4 * NDT * 64];  // dO, cols order (A of dV^T)
    __shared__ double sL[STG], sD[STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, quad = lane >> 4;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int nkb = (Sk + kMRows - 1) / kMRows, BH = p.B * p.H;
    const int rank = blockIdx.x / BH, bh = blockIdx.x - rank * BH;
    // Causal key blocks see queries from their first key on: the first
    // blocks are the longest.
    int kb = rank, part = -1;
    if (p.items_k) {  // the causal split (F64Params::items_k)
        const int c = p.items_k[rank];
        kb = c >> 2;
        part = (c & 3) - 1;
    }
    const int k0 = kb * kMRows, kw = k0 + wave * kMWaveQ, kj = kw + col;
    const int kend_b = keys_of(p, bh);
    const int jc = kj < Sk ? kj : 0;
    const size_t row = ((size_t)bh * Sk + jc) * d;
    double kf[NS], vf[NS];
    for (int s = 0; s < NS; s++) {
        const int c = 4 * s + quad;
        kf[s] = (kj < Sk && c < d) ? p.k[row + c] : 0.0;
        vf[s] = (kj < Sk && c < d) ? p.v[row + c] : 0.0;
    }
    const bool klive = kj < kend_b;
    f64x4_t dkacc[NDT], dvacc[NDT];
    for (int t = 0; t < NDT; t++) dkacc[t] = dvacc[t] = f64x4_t{0.0, 0.0, 0.0, 0.0};
    int i_start = (p.causal ? k0 : 0) / STG * STG, i_end = Sq;
    if (part >= 0) {  // queries [i_start, mid) or [mid, Sq), mid on a stage boundary
        const int mid = i_start + (Sq > i_start ? (Sq - i_start) / 2 / STG * STG : 0);
        if (part == 0) i_end = mid;
        else i_start = mid;
    }
    const double* qg = p.q + (size_t)bh * Sq * d;
    const double* gg = p.dO + (size_t)bh * Sq * d;
    F64Stage<DP, STG> st;
    if (k0 < kend_b && i_start < i_end) st.load(qg, gg, i_start, Sq, d);
    for (int i0 = i_start; k0 < kend_b && i0 < i_end; i0 += STG) {
        __syncthreads();
        st.store(sQ, sG, sQt, sGt);
        if (tid < STG) {
            const int ii = i0 + tid;
            sL[tid] = ii < Sq ? p.lse[(size_t)bh * Sq + ii] : -INFINITY;
            sD[tid] = ii < Sq ? p.delta[(size_t)bh * Sq + ii] : 0.0;
        }
        __syncthreads();
        if (i0 + STG < i_end) st.load(qg, gg, i0 + STG, Sq, d);
        for (int t = 0; t < NT16; t++) {
            const int it0 = i0 + 16 * t;
            if (it0 >= Sq || (p.causal && it0 + 15 < kw)) continue;  // wave-uniform
            f64x4_t sacc{0.0, 0.0, 0.0, 0.0}, pacc{0.0, 0.0, 0.0, 0.0};
            for (int s2 = 0; s2 < NS; s2++) {
                const int a = ((t * NS + s2) * 16 + col) * 4 + quad;
                sacc = mfma_f64(sQ[a], kf[s2], sacc);
                pacc = mfma_f64(sG[a], vf[s2], pacc);
            }
            for (int r = 0; r < 4; r++) {
                const int qr = 16 * t + 4 * r + quad, i = i0 + qr;
                const double Li = sL[qr];
                const bool on = klive && i < Sq && Li != -INFINITY && !(p.causal && kj > i);
                const double sc = p.scale * sacc[r] + mask_at(p, bh, i < Sq ? i : 0, jc);
                const double pr = on ? exp(sc - Li) : 0.0;
                const double ds = pr * (pacc[r] - sD[qr]) * p.scale;
                for (int dt = 0; dt < NDT; dt++) {
                    const int a = (((t * 4 + r) * NDT + dt) * 4 + quad) * 16 + col;
                    dvacc[dt] = mfma_f64(sGt[a], pr, dvacc[dt]);
                    dkacc[dt] = mfma_f64(sQt[a], ds, dkacc[dt]);
                }
            }
        }
    }
    if (part == 1) {  // the second half's partials, all DP columns of its keys
        const int sk = bh * p.split_k1 + kb;
        double* pr = p.part_k + ((size_t)sk * kMRows + wave * kMWaveQ + col) * 2 * DP;
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) {
                pr[16 * dt + 4 * r + quad] = dkacc[dt][r];
                pr[DP + 16 * dt + 4 * r + quad] = dvacc[dt][r];
            }
        return;
    }
    if (kj < Sk) {
        double* dkr = p.dk + row;
        double* dvr = p.dv + row;
        for (int dt = 0; dt < NDT; dt++)
            for (int r = 0; r < 4; r++) {
                const int c = 16 * dt + 4 * r + quad;
                if (c < d) {
                    dkr[c] = dkacc[dt][r];
                    dvr[c] = dvacc[dt][r];
                }
            }
    }
}

// Adds the second halves' partials of the causal backward split: dQ rows of
// the split q-blocks, then dK and dV rows of the split key blocks; one thread
// per (row, column).
template <int DP>
__global__ __launch_bounds__(256) void bwd_f64_combine_kernel(F64Params p) {
    const int nqb = (p.Sq + kMRows - 1) / kMRows, nsq = nqb - p.split_q0;
    const size_t per = (size_t)kMRows * DP, BH = (size_t)p.B * p.H;
    const size_t nq = p.items ? BH * nsq * per : 0, nk = p.items_k ? BH * p.split_k1 * per : 0;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nq) {
        const int si = (int)(i / per), rc = (int)(i % per), r = rc / DP, c = rc % DP;
        const int bh = si / nsq, qi = (p.split_q0 + si % nsq) * kMRows + r;
        if (qi < p.Sq && c < p.d)
            p.dq[((size_t)bh * p.Sq + qi) * p.d + c] += p.part[((size_t)si * kMRows + r) * DP + c];
        return;
    }
    i -= nq;
    if (i >= nk) return;
    const int sk = (int)(i / per), rc = (int)(i % per), r = rc / DP, c = rc % DP;
    const int bh = sk / p.split_k1, kj = (sk % p.split_k1) * kMRows + r;
    if (kj >= p.Sk || c >= p.d) return;
    const double* pr = p.part_k + ((size_t)sk * kMRows + r) * 2 * DP;
    const size_t o = ((size_t)bh * p.Sk + kj) * p.d + c;
    p.dk[o] += pr[c];
    p.dv[o] += pr[DP + c];
}

// D_i = dO_i . O_i, one team per row.
template <int DP>
__global__ __launch_bounds__(256) void prep_f64_kernel(F64Params p) {
    constexpr int DQ = DP / kTeam;
    const int bh = blockIdx.y, team = threadIdx.x / kTeam, u = threadIdx.x % kTeam;
    const int i = blockIdx.x * kRowsWG + team;
    const int Sq = p.Sq, d = p.d;
    const size_t row = ((size_t)bh * Sq + (i < Sq ? i : 0)) * d;
    double acc = 0.0;
    for (int t = 0; t < DQ; t++) {
        const int c = kTeam * t + u;
        if (c < d) acc = fma(p.dO[row + c], p.o[row + c], acc);
    }
    acc = team_sum(acc);
    if (i < Sq && u == 0) p.delta[(size_t)bh * Sq + i] = acc;
}

// dQ: 32 queries per workgroup, keys streamed.
template <int DP>
__global__ __launch_bounds__(256) void dq_f64_kernel(F64Params p) {
    constexpr int DQ = DP / kTeam;
    __shared__ double sK[kTile][DP + 1], sV[kTile][DP + 1];
    const int bh = blockIdx.y, team = threadIdx.x / kTeam, u = threadIdx.x % kTeam;
    const int q0 = blockIdx.x * kRowsWG, i = q0 + team;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int kend_b = keys_of(p, bh);
    int kend = kend_b;
    if (p.causal && q0 + kRowsWG < kend) kend = q0 + kRowsWG;
    const int kend_i = p.causal ? (i + 1 < kend_b ? i + 1 : kend_b) : kend_b;
    const int ic = i < Sq ? i : 0;
    const size_t row = ((size_t)bh * Sq + ic) * d;
    double qd[DQ], gd[DQ], dqd[DQ];
    for (int t = 0; t < DQ; t++) {
        const int c = kTeam * t + u;
        qd[t] = (i < Sq && c < d) ? p.q[row + c] : 0.0;
        gd[t] = (i < Sq && c < d) ? p.dO[row + c] : 0.0;
        dqd[t] = 0.0;
    }
    const double L = p.lse[(size_t)bh * Sq + ic];
    const double Di = p.delta[(size_t)bh * Sq + ic];
    const bool live = i < Sq && L != -INFINITY;
    const double* kg = p.k + (size_t)bh * Sk * d;
    const double* vg = p.v + (size_t)bh * Sk * d;
    for (int j0 = 0; j0 < kend; j0 += kTile) {
        __syncthreads();
        load_tile<DP>(sK, kg, j0, Sk, d);
        load_tile<DP>(sV, vg, j0, Sk, d);
        __syncthreads();
        for (int j = 0; j < kTile; j++) {
            double sd = 0.0, dp = 0.0;
            for (int t = 0; t < DQ; t++) {
                sd = fma(qd[t], sK[j][kTeam * t + u], sd);
                dp = fma(gd[t], sV[j][kTeam * t + u], dp);
            }
            sd = team_sum(sd);
            dp = team_sum(dp);
            const int key = j0 + j;
            if (!live || key >= kend_i) continue;
            const double s = p.scale * sd + mask_at(p, bh, ic, key);
            const double ds = exp(s - L) * (dp - Di) * p.scale;
            for (int t = 0; t < DQ; t++) dqd[t] = fma(ds, sK[j][kTeam * t + u], dqd[t]);
        }
    }
    if (i < Sq) {
        double* dqr = p.dq + row;
        for (int t = 0; t < DQ; t++) {
            const int c = kTeam * t + u;
            if (c < d) dqr[c] = dqd[t];
        }
    }
}

// dK, dV: 32 keys per workgroup, queries streamed.
template <int DP>
__global__ __launch_bounds__(256) void dkdv_f64_kernel(F64Params p) {
    constexpr int DQ = DP / kTeam;
    __shared__ double sQ[kTile][DP + 1], sG[kTile][DP + 1];
    __shared__ double sL[kTile], sD[kTile];
    const int bh = blockIdx.y, team = threadIdx.x / kTeam, u = threadIdx.x % kTeam;
    const int k0 = blockIdx.x * kRowsWG, j = k0 + team;
    const int Sq = p.Sq, Sk = p.Sk, d = p.d;
    const int kend_b = keys_of(p, bh);
    const int jc = j < Sk ? j : 0;
    const size_t row = ((size_t)bh * Sk + jc) * d;
    double kd[DQ], vd[DQ], dkd[DQ], dvd[DQ];
    for (int t = 0; t < DQ; t++) {
        const int c = kTeam * t + u;
        kd[t] = (j < Sk && c < d) ? p.k[row + c] : 0.0;
        vd[t] = (j < Sk && c < d) ? p.v[row + c] : 0.0;
        dkd[t] = dvd[t] = 0.0;
    }
    const bool live = j < kend_b;
    // Top-left causal: key j is seen by queries i >= j.
    const int i_start = (p.causal ? k0 : 0) / kTile * kTile;
    const double* qg = p.q + (size_t)bh * Sq * d;
    const double* gg = p.dO + (size_t)bh * Sq * d;
    if (k0 < kend_b) {
        for (int i0 = i_start; i0 < Sq; i0 += kTile) {
            __syncthreads();
            load_tile<DP>(sQ, qg, i0, Sq, d);
            load_tile<DP>(sG, gg, i0, Sq, d);
            if (threadIdx.x < kTile) {
                const int ii = i0 + threadIdx.x;
                sL[threadIdx.x] = ii < Sq ? p.lse[(size_t)bh * Sq + ii] : -INFINITY;
                sD[threadIdx.x] = ii < Sq ? p.delta[(size_t)bh * Sq + ii] : 0.0;
            }
            __syncthreads();
            for (int r = 0; r < kTile; r++) {
                double sd = 0.0, dp = 0.0;
                for (int t = 0; t < DQ; t++) {
                    sd = fma(sQ[r][kTeam * t + u], kd[t], sd);
                    dp = fma(sG[r][kTeam * t + u], vd[t], dp);
                }
                sd = team_sum(sd);
                dp = team_sum(dp);
                const int i = i0 + r;
                const double L = sL[r];
                if (!live || i >= Sq || L == -INFINITY || (p.causal && j > i)) continue;
                const double s = p.scale * sd + mask_at(p, bh, i, j);
                const double pij = exp(s - L);
                const double ds = pij * (dp - sD[r]) * p.scale;
                for (int t = 0; t < DQ; t++) {
                    dvd[t] = fma(pij, sG[r][kTeam * t + u], dvd[t]);
                    dkd[t] = fma(ds, sQ[r][kTeam * t + u], dkd[t]);
                }
            }
        }
    }
    if (j < Sk) {
        double* dkr = p.dk + row;
        double* dvr = p.dv + row;
        for (int t = 0; t < DQ; t++) {
            const int c = kTeam * t + u;
            if (c < d) {
                dkr[c] = dkd[t];
                dvr[c] = dvd[t];
            }
        }
    }
}

namespace {

int dp_of(int d) { return d <= 32 ? 32 : (d <= 64 ? 64 : 128); }

bool f64_args_ok(const F64Params& p) {
    return p.B > 0 && p.H > 0 && p.Sq > 0 && p.Sk > 0 && p.d > 0 && p.d <= 128 && p.q && p.k &&
           p.v;
}

}  // namespace

F64FwdSplit f64_fwd_split_plan(const F64Params& p) {
    F64FwdSplit r;
    // From 16 q-blocks on: at 8 (GoNN's BH 64, S 512 shape) the combine launch
    // and the extra workgroups cost more than the balance gains (22.97
    // against 23.98 TFLOP/s; at S 1024 27.06 against 25.23, at S 2048 28.70
    // against 25.84).
    const int nqb = (p.Sq + kMRows - 1) / kMRows;
    if (!p.causal || nqb < 16) return r;
    const int stage = mstage(dp_of(p.d) <= 64 ? 64 : 128);
    // Keys of q-block qb (top-left causal, at most Sk); the later half of
    // the q-blocks is split into two key ranges at a stage boundary.
    auto keys = [&](int qb) { return std::min(p.Sk, (qb + 1) * kMRows); };
    r.split_q0 = nqb / 2;
    std::vector<std::pair<int, int>> it;  // (keys, code)
    for (int qb = 0; qb < nqb; qb++) {
        const int k = keys(qb);
        if (qb < r.split_q0) {
            it.push_back({k, 4 * qb});
        } else {
            const int mid = (k / 2) / stage * stage;
            it.push_back({mid, 4 * qb + 1});
            it.push_back({k - mid, 4 * qb + 2});
        }
    }
    std::stable_sort(it.begin(), it.end(), [](const std::pair<int, int>& a,
                                              const std::pair<int, int>& b) {
        return a.first > b.first || (a.first == b.first && a.second > b.second);
    });
    for (const auto& x : it) r.items.push_back(x.second);
    const int dp = dp_of(p.d) <= 64 ? 64 : 128;
    const size_t bh = (size_t)p.B * p.H;
    r.part_bytes = bh * (size_t)(nqb - r.split_q0) * 2 * kMRows * (dp + 2) * sizeof(double);
    return r;
}

hipError_t launch_f64_fwd(const F64Params& p, hipStream_t s) {
    if (!f64_args_ok(p) || !p.out_o) return hipErrorInvalidValue;
    if (p.items && (!p.causal || !p.part || p.nitems <= 0 || p.split_q0 < 0 ||
                    p.split_q0 >= (p.Sq + kMRows - 1) / kMRows))
        return hipErrorInvalidValue;
    const char* e = std::getenv("GONN_HIP_F64_FWD");
    if (!(e && e[0] == 'v')) {  // "valu": the team kernel (kept for comparison)
        const int nqb = (p.Sq + kMRows - 1) / kMRows;
        const int ranks = p.items ? p.nitems : nqb;
        const dim3 grid(ranks * p.B * p.H);
        // the split q-blocks' halves, then their combine
        const size_t nc = p.items ? (size_t)p.B * p.H * (nqb - p.split_q0) * kMRows *
                                        (dp_of(p.d) <= 64 ? 64 : 128)
                                  : 0;
        const dim3 gc((unsigned)((nc + 255) / 256));
        switch (dp_of(p.d)) {
        case 32:
        case 64:
            fwd_f64_mfma_kernel<64><<<grid, 256, 0, s>>>(p);
            if (nc) fwd_f64_combine_kernel<64><<<gc, 256, 0, s>>>(p);
            break;
        default:
            fwd_f64_mfma_kernel<128><<<grid, 256, 0, s>>>(p);
            if (nc) fwd_f64_combine_kernel<128><<<gc, 256, 0, s>>>(p);
            break;
        }
        return hipGetLastError();
    }
    const dim3 grid((p.Sq + kRowsWG - 1) / kRowsWG, p.B * p.H);
    switch (dp_of(p.d)) {
    case 32: fwd_f64_kernel<32><<<grid, 256, 0, s>>>(p); break;
    case 64: fwd_f64_kernel<64><<<grid, 256, 0, s>>>(p); break;
    default: fwd_f64_kernel<128><<<grid, 256, 0, s>>>(p); break;
    }
    return hipGetLastError();
}

// Items (4 b + part + 1) of a split grid, longest first: blocks whose
// range is keys(b) long, the blocks `split(b)` halved at a stage boundary
// (mid = lo(b) + (n / 2) / stage * stage for n = keys(b) - lo(b)).
template <typename K, typename L, typename P>
static std::vector<int> f64_split_items(int nb, int stage, K keys, L lo, P split) {
    std::vector<std::pair<int, int>> it;  // (length, code)
    for (int b = 0; b < nb; b++) {
        const int n = keys(b) - lo(b);
        if (!split(b)) {
            it.push_back({n, 4 * b});
        } else {
            const int mid = (n / 2) / stage * stage;
            it.push_back({mid, 4 * b + 1});
            it.push_back({n - mid, 4 * b + 2});
        }
    }
    std::stable_sort(it.begin(), it.end(), [](const std::pair<int, int>& a,
                                              const std::pair<int, int>& b) {
        return a.first > b.first || (a.first == b.first && a.second > b.second);
    });
    std::vector<int> r;
    for (const auto& x : it) r.push_back(x.second);
    return r;
}

F64BwdSplit f64_bwd_split_plan(const F64Params& p) {
    F64BwdSplit r;
    const int nqb = (p.Sq + kMRows - 1) / kMRows, nkb = (p.Sk + kMRows - 1) / kMRows;
    if (!p.causal) return r;
    const int dp = dp_of(p.d) <= 64 ? 64 : 128, stage = mstage(dp);
    const size_t bh = (size_t)p.B * p.H;
    if (nqb >= 16) {  // dQ: the later q-blocks' key ranges (top-left causal)
        r.split_q0 = nqb / 2;
        r.items = f64_split_items(
            nqb, stage, [&](int qb) { return std::min(p.Sk, (qb + 1) * kMRows); },
            [](int) { return 0; }, [&](int qb) { return qb >= r.split_q0; });
        r.part_bytes = bh * (size_t)(nqb - r.split_q0) * kMRows * dp * sizeof(double);
    }
    if (nkb >= 16) {  // dK/dV: the first key blocks' query ranges
        r.split_k1 = nkb / 2;
        r.items_k = f64_split_items(
            nkb, stage, [&](int) { return p.Sq; },
            [&](int kb) { return std::min(p.Sq, kb * kMRows / stage * stage); },
            [&](int kb) { return kb < r.split_k1; });
        r.part_k_bytes = bh * (size_t)r.split_k1 * kMRows * 2 * dp * sizeof(double);
    }
    return r;
}

hipError_t launch_f64_bwd(const F64Params& p, hipStream_t s) {
    if (!f64_args_ok(p) || !p.o || !p.dO || !p.lse || !p.delta || !p.dq || !p.dk || !p.dv)
        return hipErrorInvalidValue;
    const int nqb = (p.Sq + kMRows - 1) / kMRows, nkb = (p.Sk + kMRows - 1) / kMRows;
    if (p.items && (!p.causal || !p.part || p.nitems <= 0 || p.split_q0 < 0 || p.split_q0 >= nqb))
        return hipErrorInvalidValue;
    if (p.items_k &&
        (!p.causal || !p.part_k || p.nitems_k <= 0 || p.split_k1 <= 0 || p.split_k1 > nkb))
        return hipErrorInvalidValue;
    const char* e = std::getenv("GONN_HIP_F64_BWD");
    if (!(e && e[0] == 'v')) {  // "valu": the team kernels (kept for comparison)
        const dim3 gp((p.Sq + kRowsWG - 1) / kRowsWG, p.B * p.H);
        const dim3 gq((p.items ? p.nitems : nqb) * p.B * p.H);
        const dim3 gk((p.items_k ? p.nitems_k : nkb) * p.B * p.H);
        const size_t dp = dp_of(p.d) <= 64 ? 64 : 128, bh = (size_t)p.B * p.H;
        const size_t nc = (p.items ? bh * (nqb - p.split_q0) * kMRows * dp : 0) +
                          (p.items_k ? bh * p.split_k1 * kMRows * dp : 0);
        const dim3 gc((unsigned)((nc + 255) / 256));
        if (dp == 64) {
            prep_f64_kernel<64><<<gp, 256, 0, s>>>(p);
            dq_f64_mfma_kernel<64><<<gq, 256, 0, s>>>(p);
            dkdv_f64_mfma_kernel<64><<<gk, 256, 0, s>>>(p);
            if (nc) bwd_f64_combine_kernel<64><<<gc, 256, 0, s>>>(p);
        } else {
            prep_f64_kernel<128><<<gp, 256, 0, s>>>(p);
            dq_f64_mfma_kernel<128><<<gq, 256, 0, s>>>(p);
            dkdv_f64_mfma_kernel<128><<<gk, 256, 0, s>>>(p);
            if (nc) bwd_f64_combine_kernel<128><<<gc, 256, 0, s>>>(p);
        }
        return hipGetLastError();
    }
    const dim3 gq((p.Sq + kRowsWG - 1) / kRowsWG, p.B * p.H);
    const dim3 gk((p.Sk + kRowsWG - 1) / kRowsWG, p.B * p.H);
    switch (dp_of(p.d)) {
    case 32:
        prep_f64_kernel<32><<<gq, 256, 0, s>>>(p);
        dq_f64_kernel<32><<<gq, 256, 0, s>>>(p);
        dkdv_f64_kernel<32><<<gk, 256, 0, s>>>(p);
        break;
    case 64:
        prep_f64_kernel<64><<<gq, 256, 0, s>>>(p);
        dq_f64_kernel<64><<<gq, 256, 0, s>>>(p);
        dkdv_f64_kernel<64><<<gk, 256, 0, s>>>(p);
        break;
    default:
        prep_f64_kernel<128><<<gq, 256, 0, s>>>(p);
        dq_f64_kernel<128><<<gq, 256, 0, s>>>(p);
        dkdv_f64_kernel<128><<<gk, 256, 0, s>>>(p);
        break;
    }
    return hipGetLastError();
}

}  // namespace gonn
