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
// A row (query or key) is owned by a team of 8 lanes; lane u of the team
// holds elements 8t + u (t < DP/8) of the row's vectors, so a team reads 64
// contiguous bytes per t and dot products end in a 3-step lane reduction.
// The streamed rows (K/V for the forward and dQ, Q/dO for dK/dV) sit in LDS
// tiles of 32 rows that every team reads in the same order (broadcasts).
// The two backward kernels each own their outputs: no atomics,
// deterministic.
#include <cmath>

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

hipError_t launch_f64_fwd(const F64Params& p, hipStream_t s) {
    if (!f64_args_ok(p) || !p.out_o) return hipErrorInvalidValue;
    const dim3 grid((p.Sq + kRowsWG - 1) / kRowsWG, p.B * p.H);
    switch (dp_of(p.d)) {
    case 32: fwd_f64_kernel<32><<<grid, 256, 0, s>>>(p); break;
    case 64: fwd_f64_kernel<64><<<grid, 256, 0, s>>>(p); break;
    default: fwd_f64_kernel<128><<<grid, 256, 0, s>>>(p); break;
    }
    return hipGetLastError();
}

hipError_t launch_f64_bwd(const F64Params& p, hipStream_t s) {
    if (!f64_args_ok(p) || !p.o || !p.dO || !p.lse || !p.delta || !p.dq || !p.dk || !p.dv)
        return hipErrorInvalidValue;
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
