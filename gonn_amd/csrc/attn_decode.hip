// attn_decode.hip -- split-KV decode over a bf16 KV cache, plus the combine.
//
// New relative to the reference (GoNN has no KV cache); the result is pinned
// to MultiHeadAttention.ForwardMasked with a key-padding mask
// (nn/attention.go:305-341, :261-272): query 1 x D per (b,h), keys
// 0..kv_len[b]-1 of the cache, no causal mask. A padded key gets weight
// exactly 0 in the reference, so it is never read here.
//
// One query row per (b,h) makes this a pair of GEMVs; the bound is HBM
// bandwidth over the valid K/V rows, so the kernel is built for streaming:
//  * split kernel: a (b,h) of len keys takes ns = ceil(len / split_keys)
//    workgroups, which split [0, len) evenly (each gets floor or ceil of
//    len / ns keys, never a sliver), so only valid rows are ever fetched;
//    the 1-D grid is split-major (every sequence's split 0, then split 1,
//    ...), so the workgroups that exit at once (s >= ns) gather at the end
//    of the grid instead of sitting between the working ones;
//  * a row of 16 lanes covers one key (D=128: 8 bf16 = 16 bytes per lane), so
//    one wave instruction reads 4 whole consecutive rows (1 KB contiguous);
//    each lane keeps 8 keys' K and V loads in flight per iteration; the cache
//    is read once, so the loads are non-temporal (streamed past the caches:
//    5.4 -> 5.8 TB/s on C4);
//  * q.k is reduced across the 16 lanes of a row with DPP row_ror adds;
//  * each lane row runs its own online softmax in log2 units (scale*log2e is
//    folded into q); the 16 lane rows of a workgroup merge through LDS and
//    write one partial (m, l, o[D]) per split;
//  * combine kernel: per (b,h), O = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s;
//  * kv_append kernel: writes new K/V rows (f32 or bf16) into the bf16 cache
//    at each sequence's current length (the KV-cache handle of the C ABI).
#include "common.h"
#include "kernels.h"

namespace gonn {

template <int D, typename QT>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeParams p) {
    constexpr int EPL = D / 16;  // elements per lane
    constexpr int U = 8;         // keys per lane row per iteration
    constexpr int NROWS = 16;    // lane rows per workgroup
    __shared__ float pm[NROWS], pl[NROWS];
    __shared__ float po[NROWS][D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = lane >> 4, dc = lane & 15, d0 = dc * EPL;
    const int BH = p.B * p.H;
    const int s = blockIdx.x / BH, bh = blockIdx.x - s * BH, b = bh / p.H;
    int len = p.kv_len[b];
    len = len < 0 ? 0 : (len > p.Lmax ? p.Lmax : len);
    const int ns = (len + p.split_keys - 1) / p.split_keys;
    if (s >= ns) return;  // uniform for the workgroup
    // [k0, k1): split s of ns even parts of [0, len), non-empty as ns <= len
    const int k0 = (int)((long long)s * len / ns);
    const int k1 = (int)((long long)(s + 1) * len / ns);

    float q[EPL];
    {
        const QT* qp = (const QT*)p.q + (size_t)bh * D + d0;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            float v;
            if constexpr (sizeof(QT) == 4) v = qp[e];
            else v = bf16_to_f32(*(const uint16_t*)(qp + e));
            q[e] = v * p.scale_log2;
        }
    }
    const bf16* Kb = (const bf16*)p.kc + (size_t)bh * p.Lmax * D + d0;
    const bf16* Vb = (const bf16*)p.vc + (size_t)bh * p.Lmax * D + d0;

    float m = -INFINITY, l = 0.f, o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.f;

    typedef uint16_t ld_t __attribute__((ext_vector_type(EPL)));
    for (int base = k0 + wave * (4 * U); base < k1; base += 4 * 4 * U) {
        // Keys past k1 are clamped to k1-1 (a valid row) and masked below, so
        // every load is in bounds and the loop body has no branches.
        ld_t kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            int key = base + u * 4 + rr;
            key = key < k1 ? key : k1 - 1;
            kr[u] = __builtin_nontemporal_load((const ld_t*)(Kb + (size_t)key * D));
            vr[u] = __builtin_nontemporal_load((const ld_t*)(Vb + (size_t)key * D));
        }
        float sc[U];
        float mb = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; u++) {
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) a = __builtin_fmaf(q[e], bf16_to_f32(kr[u][e]), a);
            a = row_sum16(a);
            sc[u] = (base + u * 4 + rr < k1) ? a : -INFINITY;
            mb = fmaxf(mb, sc[u]);
        }
        const float mnew = fmaxf(m, mb);
        // A lane row that has seen no valid key keeps m = -inf and l = o = 0.
        const float mref = (mnew == -INFINITY) ? 0.f : mnew;
        const float alpha = fast_exp2(m - mref);
        float rs = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float pu = fast_exp2(sc[u] - mref);
            rs += pu;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[e] = __builtin_fmaf(pu, bf16_to_f32(vr[u][e]), o[e]);
        }
        l = l * alpha + rs;
        m = mnew;
    }

    const int row = wave * 4 + rr;
    if (dc == 0) {
        pm[row] = m;
        pl[row] = l;
    }
#pragma unroll
    for (int e = 0; e < EPL; e++) po[row][d0 + e] = o[e];
    __syncthreads();
    if (tid < D) {
        float M = -INFINITY;
        for (int i = 0; i < NROWS; i++) M = fmaxf(M, pm[i]);
        float L = 0.f, O = 0.f;
        for (int i = 0; i < NROWS; i++) {
            const float w = (pm[i] == -INFINITY) ? 0.f : fast_exp2(pm[i] - M);
            L = __builtin_fmaf(w, pl[i], L);
            O = __builtin_fmaf(w, po[i][tid], O);
        }
        const size_t part = (size_t)bh * p.nsplit + s;
        p.part_o[part * D + tid] = O;
        if (tid == 0) {
            p.part_ml[part * 2 + 0] = M;
            p.part_ml[part * 2 + 1] = L;
        }
    }
}

// One workgroup of D threads per (b,h). The partial (m, l) pairs are read by
// all threads at once into LDS (one memory round trip), their max and
// weights formed there, and each thread then sums its column of the partial
// outputs with independent loads, CH splits at a time.
template <int D>
__global__ __launch_bounds__(D) void decode_combine_kernel(DecodeParams p) {
    constexpr int CH = D;  // splits per LDS chunk
    __shared__ float sm[CH], sw[CH], sl[CH];
    const int bh = blockIdx.x, b = bh / p.H, tid = threadIdx.x;
    int len = p.kv_len[b];
    len = len < 0 ? 0 : (len > p.Lmax ? p.Lmax : len);
    const int ns = (len + p.split_keys - 1) / p.split_keys;
    const float* ml = p.part_ml + (size_t)bh * p.nsplit * 2;
    const float* po = p.part_o + (size_t)bh * p.nsplit * D;
    float M = -INFINITY, L = 0.f, O = 0.f;
    for (int c0 = 0; c0 < ns; c0 += CH) {
        const int nc = ns - c0 < CH ? ns - c0 : CH;
        __syncthreads();
        if (tid < nc) {
            sm[tid] = ml[2 * (c0 + tid)];
            sl[tid] = ml[2 * (c0 + tid) + 1];
        }
        __syncthreads();
        float mc = M;
        for (int i = 0; i < nc; i++) mc = fmaxf(mc, sm[i]);
        if (tid < nc) sw[tid] = fast_exp2(sm[tid] - mc);
        const float a = (M == -INFINITY) ? 0.f : fast_exp2(M - mc);
        L *= a;
        O *= a;
        M = mc;
        __syncthreads();
        int i = 0;
        for (; i + 4 <= nc; i += 4) {
            float v[4];
            for (int u = 0; u < 4; u++) v[u] = po[(size_t)(c0 + i + u) * D + tid];
            for (int u = 0; u < 4; u++) {
                L = __builtin_fmaf(sw[i + u], sl[i + u], L);
                O = __builtin_fmaf(sw[i + u], v[u], O);
            }
        }
        for (; i < nc; i++) {
            L = __builtin_fmaf(sw[i], sl[i], L);
            O = __builtin_fmaf(sw[i], po[(size_t)(c0 + i) * D + tid], O);
        }
    }
    p.o[(size_t)bh * D + tid] = ns > 0 ? O / L : 0.f;
}

// ---------------------------------------------------------------------------
// Causal multi-token attend over the cache: T new queries per (b,h) whose own
// K/V rows are the last T cached positions of their sequence (chunked
// prefill into a cache, several tokens of one decoding step). Query t sees
// keys [0, lim_t), lim_t = kv_len[b] - (T - 1 - t): the top-left causal mask
// of nn/attention.go:185-196 aligned at the sequence's end, which is what
// decoding one position at a time over the cache computes.
//
// Queries go in groups of G = kDecodeGroup: a workgroup takes one split of
// the group's key range [0, lim of its last query) and scores each key it
// loads against all G queries, so the cache is read once per group. The key
// range, its even splits and the lane-row layout are the decode kernel's;
// each lane keeps G online-softmax states. Key j of the split counts for
// query t only when j < lim_t; a query with no key in a split leaves the
// partial (m, l) = (-inf, 0), which the combine weights by zero.
// ---------------------------------------------------------------------------
GONN_DEV int causal_group_keys(int len, int T, int t_last) { return len - (T - 1 - t_last); }

template <int D>
__global__ __launch_bounds__(256) void decode_causal_split_kernel(DecodeParams p) {
    constexpr int G = kDecodeGroup;
    constexpr int EPL = D / 16;  // elements per lane
    constexpr int U = 4;         // keys per lane row per iteration
    constexpr int NROWS = 16;    // lane rows per workgroup
    __shared__ float pm[G][NROWS], pl[G][NROWS];
    __shared__ float po[G][NROWS][D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = lane >> 4, dc = lane & 15, d0 = dc * EPL;
    const int BH = p.B * p.H, T = p.T, NG = (T + G - 1) / G;
    const int per = BH * NG;
    const int s = blockIdx.x / per, rem = blockIdx.x - s * per;
    const int gr = rem / BH, bh = rem - gr * BH, b = bh / p.H;
    int len = p.kv_len[b];
    len = len < 0 ? 0 : (len > p.Lmax ? p.Lmax : len);
    const int t0 = gr * G, ng = T - t0 < G ? T - t0 : G;
    const int kmax = causal_group_keys(len, T, t0 + ng - 1);
    const int ns = kmax > 0 ? (kmax + p.split_keys - 1) / p.split_keys : 0;
    if (s >= ns) return;  // uniform for the workgroup
    const int k0 = (int)((long long)s * kmax / ns);
    const int k1 = (int)((long long)(s + 1) * kmax / ns);

    float q[G][EPL];
    int lim[G];
#pragma unroll
    for (int i = 0; i < G; i++) {
        const bool on = i < ng;
        const float* qp = (const float*)p.q + ((size_t)bh * T + t0 + (on ? i : 0)) * D + d0;
#pragma unroll
        for (int e = 0; e < EPL; e++) q[i][e] = on ? qp[e] * p.scale_log2 : 0.f;
        lim[i] = on ? causal_group_keys(len, T, t0 + i) : 0;
    }
    const bf16* Kb = (const bf16*)p.kc + (size_t)bh * p.Lmax * D + d0;
    const bf16* Vb = (const bf16*)p.vc + (size_t)bh * p.Lmax * D + d0;

    float m[G], l[G], o[G][EPL];
#pragma unroll
    for (int i = 0; i < G; i++) {
        m[i] = -INFINITY;
        l[i] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[i][e] = 0.f;
    }

    typedef uint16_t ld_t __attribute__((ext_vector_type(EPL)));
    for (int base = k0 + wave * (4 * U); base < k1; base += 4 * 4 * U) {
        // Keys past k1 are clamped to k1-1 (a valid row) and masked below.
        ld_t kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            int key = base + u * 4 + rr;
            key = key < k1 ? key : k1 - 1;
            kr[u] = __builtin_nontemporal_load((const ld_t*)(Kb + (size_t)key * D));
            vr[u] = __builtin_nontemporal_load((const ld_t*)(Vb + (size_t)key * D));
        }
        float kf[U][EPL];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int e = 0; e < EPL; e++) kf[u][e] = bf16_to_f32(kr[u][e]);
#pragma unroll
        for (int i = 0; i < G; i++) {
            float sc[U];
            float mb = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; u++) {
                float a = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) a = __builtin_fmaf(q[i][e], kf[u][e], a);
                a = row_sum16(a);
                const int key = base + u * 4 + rr;
                sc[u] = (key < k1 && key < lim[i]) ? a : -INFINITY;
                mb = fmaxf(mb, sc[u]);
            }
            const float mnew = fmaxf(m[i], mb);
            // A state that has seen no valid key keeps m = -inf, l = o = 0.
            const float mref = (mnew == -INFINITY) ? 0.f : mnew;
            const float alpha = fast_exp2(m[i] - mref);
            float rs = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[i][e] *= alpha;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float pu = fast_exp2(sc[u] - mref);
                rs += pu;
#pragma unroll
                for (int e = 0; e < EPL; e++)
                    o[i][e] = __builtin_fmaf(pu, bf16_to_f32(vr[u][e]), o[i][e]);
            }
            l[i] = l[i] * alpha + rs;
            m[i] = mnew;
        }
    }

    const int row = wave * 4 + rr;
#pragma unroll
    for (int i = 0; i < G; i++) {
        if (dc == 0) {
            pm[i][row] = m[i];
            pl[i][row] = l[i];
        }
#pragma unroll
        for (int e = 0; e < EPL; e++) po[i][row][d0 + e] = o[i][e];
    }
    __syncthreads();
    if (tid < D) {
        for (int i = 0; i < ng; i++) {
            float M = -INFINITY;
            for (int r = 0; r < NROWS; r++) M = fmaxf(M, pm[i][r]);
            float L = 0.f, O = 0.f;
            for (int r = 0; r < NROWS; r++) {
                const float w = (pm[i][r] == -INFINITY) ? 0.f : fast_exp2(pm[i][r] - M);
                L = __builtin_fmaf(w, pl[i][r], L);
                O = __builtin_fmaf(w, po[i][r][tid], O);
            }
            const size_t part = ((size_t)bh * T + t0 + i) * p.nsplit + s;
            p.part_o[part * D + tid] = O;
            if (tid == 0) {
                p.part_ml[part * 2 + 0] = M;
                p.part_ml[part * 2 + 1] = L;
            }
        }
    }
}

// One workgroup of D threads per (b,h,t): the combine of decode_combine_kernel
// over the splits of query t's group. A split in which query t saw no key
// has M = -inf and weight 0; every query sees at least its own key.
template <int D>
__global__ __launch_bounds__(D) void decode_causal_combine_kernel(DecodeParams p) {
    constexpr int G = kDecodeGroup;
    const int T = p.T;
    const int bht = blockIdx.x, bh = bht / T, t = bht - bh * T, b = bh / p.H, tid = threadIdx.x;
    int len = p.kv_len[b];
    len = len < 0 ? 0 : (len > p.Lmax ? p.Lmax : len);
    const int t0 = t / G * G, ng = T - t0 < G ? T - t0 : G;
    const int kmax = causal_group_keys(len, T, t0 + ng - 1);
    const int ns = kmax > 0 ? (kmax + p.split_keys - 1) / p.split_keys : 0;
    const float* ml = p.part_ml + (size_t)bht * p.nsplit * 2;
    const float* po = p.part_o + (size_t)bht * p.nsplit * D;
    float M = -INFINITY;
    for (int i = 0; i < ns; i++) M = fmaxf(M, ml[2 * i]);
    float L = 0.f, O = 0.f;
    for (int i = 0; i < ns; i++) {
        const float w = (ml[2 * i] == -INFINITY) ? 0.f : fast_exp2(ml[2 * i] - M);
        L = __builtin_fmaf(w, ml[2 * i + 1], L);
        O = __builtin_fmaf(w, po[(size_t)i * D + tid], O);
    }
    p.o[(size_t)bht * D + tid] = L > 0.f ? O / L : 0.f;
}

// KV-cache append: row t < cnt[b] of (b, h) in the sources (B,H,T,D), f32 or
// bf16, goes to position pos[b] + t of the bf16 cache (B,H,Lmax,D); rows at
// or past Lmax are dropped (the host rejects such appends beforehand). One
// thread per 8 elements of K and of V (one 16-byte store each).
template <typename ST>
__global__ __launch_bounds__(256) void kv_append_kernel(const ST* __restrict__ ks,
                                                        const ST* __restrict__ vs, bf16* kc,
                                                        bf16* vc, const int* __restrict__ pos,
                                                        const int* __restrict__ cnt, int H,
                                                        int T, int Lmax, int D, size_t nchunk) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nchunk) return;
    const int cpr = D / 8;  // 16-byte chunks per row
    const size_t row = c / cpr;
    const int e0 = (int)(c % cpr) * 8;
    const int t = (int)(row % T);
    const size_t bh = row / T;
    const int b = (int)(bh / H);
    if (t >= cnt[b]) return;
    const int dst_t = pos[b] + t;
    if (dst_t < 0 || dst_t >= Lmax) return;
    const size_t src = row * D + e0, dst = (bh * Lmax + dst_t) * D + e0;
    bf16x8 kk, vv;
    if constexpr (sizeof(ST) == 4) {
        const f32x4 k0 = *(const f32x4*)(ks + src), k1 = *(const f32x4*)(ks + src + 4);
        const f32x4 v0 = *(const f32x4*)(vs + src), v1 = *(const f32x4*)(vs + src + 4);
        kk = pack8(k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]);
        vv = pack8(v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]);
    } else {
        kk = *(const bf16x8*)(ks + src);
        vv = *(const bf16x8*)(vs + src);
    }
    *(bf16x8*)(kc + dst) = kk;
    *(bf16x8*)(vc + dst) = vv;
}

hipError_t launch_kv_append(const void* ks, const void* vs, int src_bf16, void* kc, void* vc,
                            const int* pos, const int* cnt, int B, int H, int T, int Lmax,
                            int D, hipStream_t s) {
    if (D % 8 != 0 || B <= 0 || H <= 0 || T <= 0) return hipErrorInvalidValue;
    const size_t nchunk = (size_t)B * H * T * (D / 8);
    const unsigned grid = (unsigned)((nchunk + 255) / 256);
    if (src_bf16)
        kv_append_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)ks, (const bf16*)vs, (bf16*)kc,
                                                    (bf16*)vc, pos, cnt, H, T, Lmax, D, nchunk);
    else
        kv_append_kernel<float><<<grid, 256, 0, s>>>((const float*)ks, (const float*)vs, (bf16*)kc,
                                                     (bf16*)vc, pos, cnt, H, T, Lmax, D, nchunk);
    return hipGetLastError();
}

hipError_t launch_decode_split(const DecodeParams& p, int D, int q_bf16, hipStream_t s) {
    const unsigned grid = (unsigned)p.nsplit * (unsigned)(p.B * p.H);
    if (D == 128) {
        if (q_bf16) decode_split_kernel<128, bf16><<<grid, 256, 0, s>>>(p);
        else decode_split_kernel<128, float><<<grid, 256, 0, s>>>(p);
    } else if (D == 64) {
        if (q_bf16) decode_split_kernel<64, bf16><<<grid, 256, 0, s>>>(p);
        else decode_split_kernel<64, float><<<grid, 256, 0, s>>>(p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_decode_causal_split(const DecodeParams& p, int D, hipStream_t s) {
    if (p.T <= 0) return hipErrorInvalidValue;
    const unsigned groups = (unsigned)((p.T + kDecodeGroup - 1) / kDecodeGroup);
    const unsigned grid = (unsigned)p.nsplit * groups * (unsigned)(p.B * p.H);
    if (D == 128) decode_causal_split_kernel<128><<<grid, 256, 0, s>>>(p);
    else if (D == 64) decode_causal_split_kernel<64><<<grid, 256, 0, s>>>(p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_decode_causal_combine(const DecodeParams& p, int D, hipStream_t s) {
    if (p.T <= 0) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(p.B * p.H) * (unsigned)p.T;
    if (D == 128) decode_causal_combine_kernel<128><<<grid, 128, 0, s>>>(p);
    else if (D == 64) decode_causal_combine_kernel<64><<<grid, 64, 0, s>>>(p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_decode_combine(const DecodeParams& p, int D, hipStream_t s) {
    if (D == 128) decode_combine_kernel<128><<<p.B * p.H, 128, 0, s>>>(p);
    else if (D == 64) decode_combine_kernel<64><<<p.B * p.H, 64, 0, s>>>(p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace gonn
