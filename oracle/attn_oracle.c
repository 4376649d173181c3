/*
 * attn_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A CPU fp64 restatement of GoNN's pure-Go attention core, used only as the
 * checker of the HIP kernels (by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py). Nothing in the gonn_amd package links or
 * calls it.
 *
 * What it restates, op by op, in the reference's order:
 *   MultiHeadAttention.Forward core      nn/attention.go:135-146
 *     scores = qp @ kp^T                 tensor/ops_matmul.go:72-105 (batched),
 *                                        backend/cpu.go:20-48 (one GEMM per
 *                                        (b,h), sequential over batches); the
 *                                        K^T operand is a Permute copy,
 *                                        tensor/ops_shape.go:53-107
 *     .MulScalar(scale)                  tensor/ops_binary.go:32-56
 *     .Add(causalMaskAdd)                nn/attention.go:185-196 (-1e30, j > i)
 *     .Add(keyPaddingMaskAdd)            nn/attention.go:261-272 (ForwardMasked,
 *                                        :330-332)
 *     .Softmax(3) = MaxAxis, Sub, Exp,   tensor/ops_activation.go:455-461,
 *                   SumAxis, Div         tensor/ops_reduce.go:110-112, :172-271,
 *                                        tensor/ops_unary.go:12-14
 *     attn @ vp                          nn/attention.go:144
 *   Linear.Forward  y = x @ W^T + b      nn/linear.go:40-59
 *   autograd of the core                 tensor/autograd.go:52-151 with the
 *                                        per-op backward closures:
 *     MatMul  dA = g B^T, dB = A^T g     tensor/ops_matmul.go:93-100
 *     Mul/Div/Add/Sub                    tensor/ops_binary.go:63-90
 *     MaxAxis scatter to argmax          tensor/ops_reduce.go:261-266
 *     SumAxis broadcast                  tensor/ops_reduce.go:200-214
 *     Exp     g * y                      tensor/ops_unary.go:12-14
 *   LSE  L = m + log(l) over the scaled, masked scores, the quantity the
 *        reference CUDA kernel saves (backend/cuda/gonn_cuda.cu:330, :448).
 *   closed-form backward identities      backend/cuda/gonn_cuda.cu:333-340
 *
 * GEMM: gonum blas64.Gemm (gonum v0.14.0, go.mod:5) is not vendored; the
 * reference pins it to a naive triple loop at 1e-12
 * (backend/backend_test.go:47-86), so a naive loop stands in for it.
 *
 * Every function is deterministic: threads split rows, and each element's
 * arithmetic order does not depend on the thread count.
 * Build: oracle/build.py (gcc -O3 -ffp-contract=off -fopenmp -shared).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdint.h>

#define MASK_NEG (-1e30)

/* Planted mistakes, used only by the oracle's own mutation tests to show that
 * the pinning checks catch them. 0 = none. */
static int g_mutation = 0;
void oracle_set_mutation(int m) { g_mutation = m; }
enum {
    MUT_NONE = 0,
    MUT_NO_SCALE = 1,      /* drop the 1/sqrt(D) scale                   */
    MUT_CAUSAL_GE = 2,     /* mask j >= i instead of j > i               */
    MUT_TRANSPOSE_V = 3,   /* use V^T in the context product (D == Sk)   */
    MUT_NO_MAX_SUB = 4,    /* skip the max subtraction (changes LSE only
                              through overflow; detectable by huge inputs) */
    MUT_DS_SIGN = 5,       /* flip the sign of D_i in the backward       */
    MUT_LSE_LOG2 = 6       /* store LSE in log2 units                    */
};

/* C = A(m,k) @ B(k,n), row-major, sum over k in ascending order. */
static void gemm_nn(const double* A, const double* B, double* C, int m, int k, int n) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < m; i++) {
        double* c = C + (size_t)i * n;
        for (int j = 0; j < n; j++) c[j] = 0.0;
        for (int t = 0; t < k; t++) {
            const double a = A[(size_t)i * k + t];
            const double* b = B + (size_t)t * n;
            for (int j = 0; j < n; j++) c[j] += a * b[j];
        }
    }
}

/* Permute copy of a (r, c) matrix into (c, r). */
static void transpose(const double* A, double* T, int r, int c) {
    #pragma omp parallel for schedule(static)
    for (int j = 0; j < c; j++)
        for (int i = 0; i < r; i++) T[(size_t)j * r + i] = A[(size_t)i * c + j];
}

/* Softmax of one row (MaxAxis, Sub, Exp, SumAxis, Div), in place. Returns the
 * max and the sum so callers can form LSE = max + log(sum). */
static void softmax_row(double* x, int n, double* mx_out, double* sum_out) {
    double mx = -INFINITY;
    for (int j = 0; j < n; j++)
        if (x[j] > mx) mx = x[j];
    double sum = 0.0;
    for (int j = 0; j < n; j++) {
        const double sh = (g_mutation == MUT_NO_MAX_SUB) ? x[j] : x[j] - mx;
        x[j] = exp(sh);
        sum += x[j];
    }
    for (int j = 0; j < n; j++) x[j] = x[j] / sum;
    if (mx_out) *mx_out = (g_mutation == MUT_NO_MAX_SUB) ? 0.0 : mx;
    if (sum_out) *sum_out = sum;
}

static inline int masked(int i, int j, int causal, int len) {
    if (causal) {
        if (g_mutation == MUT_CAUSAL_GE ? (j >= i && j > 0) : (j > i)) return 1;
    }
    if (j >= len) return 1;
    return 0;
}

/*
 * Scores of one (b,h) slice for the listed query rows, after scale and masks:
 * out (nrows, Sk). rows == NULL means rows 0..Sq-1. The additive masks are
 * added exactly like the reference (x + (-1e30)), not by assignment, in the
 * reference's order (nn/attention.go:321-330): causal, the user's additive
 * mask amask (this slice's (Sq, Sk) rows, or NULL), key padding.
 */
static void scores_rows(const double* Qb, const double* KTb, int Sk, int D,
                        const int* rows, int nrows, double scale, int causal,
                        const double* amask, int len, double* out) {
    const double sc = (g_mutation == MUT_NO_SCALE) ? 1.0 : scale;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < nrows; r++) {
        const int i = rows ? rows[r] : r;
        double* s = out + (size_t)r * Sk;
        for (int j = 0; j < Sk; j++) s[j] = 0.0;
        for (int t = 0; t < D; t++) {
            const double a = Qb[(size_t)i * D + t];
            const double* b = KTb + (size_t)t * Sk;
            for (int j = 0; j < Sk; j++) s[j] += a * b[j];
        }
        for (int j = 0; j < Sk; j++) s[j] = s[j] * sc;
        if (causal)
            for (int j = 0; j < Sk; j++) s[j] = s[j] + (masked(i, j, 1, Sk) ? MASK_NEG : 0.0);
        if (amask)  /* WithAttnMask: the user's additive mask, row i */
            for (int j = 0; j < Sk; j++) s[j] = s[j] + amask[(size_t)i * Sk + j];
        if (len < Sk)
            for (int j = 0; j < Sk; j++) s[j] = s[j] + (j >= len ? MASK_NEG : 0.0);
    }
}

/*
 * Forward of the attention core over BH = B*H slices.
 *   Q (BH,Sq,D), K/V (BH,Sk,D), O (BH,Sq,D), LSE (BH,Sq) or NULL.
 *   kv_len: NULL, or per-batch valid key counts (length BH/H), applied as the
 *   key padding mask of every head of that batch.
 *   amask: NULL, or the additive mask of WithAttnMask (nn/attention.go:212-
 *   257): slice bh = b*H + h reads (Sq, Sk) rows at amask + b*mask_sb +
 *   h*mask_sh (strides 0 broadcast, as expandAttnMask's shapes do).
 *   rows/nrows: NULL/0 for all query rows, else only these rows are computed
 *   (and only those rows of O/LSE are written); each row's arithmetic is the
 *   same as in the full computation.
 */
int oracle_attn_fwd_ex(const double* Q, const double* K, const double* V, double* O,
                       double* LSE, int BH, int H, int Sq, int Sk, int D, double scale,
                       int causal, const int* kv_len, const double* amask, long mask_sb,
                       long mask_sh, const int* rows, int nrows) {
    if (BH <= 0 || Sq <= 0 || Sk <= 0 || D <= 0 || H <= 0 || BH % H) return -1;
    const int nr = rows ? nrows : Sq;
    double* KT = (double*)malloc(sizeof(double) * (size_t)D * Sk);
    double* P = (double*)malloc(sizeof(double) * (size_t)nr * Sk);
    double* Vu = (double*)malloc(sizeof(double) * (size_t)Sk * D);
    if (!KT || !P || !Vu) { free(KT); free(P); free(Vu); return -2; }
    for (int bh = 0; bh < BH; bh++) {
        const double* Qb = Q + (size_t)bh * Sq * D;
        const double* Kb = K + (size_t)bh * Sk * D;
        const double* Vb = V + (size_t)bh * Sk * D;
        const int len = kv_len ? kv_len[bh / H] : Sk;
        transpose(Kb, KT, Sk, D);
        const double* am = amask ? amask + (size_t)(bh / H) * mask_sb + (size_t)(bh % H) * mask_sh
                                 : NULL;
        scores_rows(Qb, KT, Sk, D, rows, nr, scale, causal, am, len, P);
        double* mx = (double*)malloc(sizeof(double) * nr);
        double* sm = (double*)malloc(sizeof(double) * nr);
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < nr; r++) softmax_row(P + (size_t)r * Sk, Sk, &mx[r], &sm[r]);
        const double* Vuse = Vb;
        if (g_mutation == MUT_TRANSPOSE_V && D == Sk) {
            transpose(Vb, Vu, Sk, D);
            Vuse = Vu;
        }
        /* context rows: attn (nr, Sk) @ V (Sk, D) */
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < nr; r++) {
            const int i = rows ? rows[r] : r;
            double* o = O + ((size_t)bh * Sq + i) * D;
            for (int t = 0; t < D; t++) o[t] = 0.0;
            for (int j = 0; j < Sk; j++) {
                const double a = P[(size_t)r * Sk + j];
                const double* v = Vuse + (size_t)j * D;
                for (int t = 0; t < D; t++) o[t] += a * v[t];
            }
            if (LSE) {
                double L = mx[r] + log(sm[r]);
                if (g_mutation == MUT_LSE_LOG2) L = L / log(2.0);
                LSE[(size_t)bh * Sq + i] = L;
            }
        }
        free(mx);
        free(sm);
    }
    free(KT);
    free(P);
    free(Vu);
    return 0;
}

int oracle_attn_fwd(const double* Q, const double* K, const double* V, double* O,
                    double* LSE, int BH, int H, int Sq, int Sk, int D, double scale,
                    int causal, const int* kv_len, const int* rows, int nrows) {
    return oracle_attn_fwd_ex(Q, K, V, O, LSE, BH, H, Sq, Sk, D, scale, causal, kv_len, NULL, 0,
                              0, rows, nrows);
}

/*
 * Backward of the core by the reference's autograd chain, one (b,h) slice at a
 * time, materialising every intermediate the Go graph holds:
 *   raw = qp @ kp^T; scaled = raw * scale; masked = scaled + mask;
 *   mx = MaxAxis(masked); sh = masked - mx; e = Exp(sh); se = SumAxis(e);
 *   attn = e / se; ctx = attn @ vp.
 * Given g = dL/dctx: walks the nodes in reverse topological order, summing
 * the two gradient contributions into e (Div numerator and SumAxis) and into
 * masked (Sub and MaxAxis scatter) as tensor/autograd.go:52-99 accumulates
 * them. Q, dO, dQ are (BH,Sq,D), K, V, dK, dV (BH,Sk,D) (Sq != Sk for
 * cross-attention, top-left causal). kv_len: NULL, or per-batch valid key
 * counts (length BH/H): the key
 * padding mask ForwardMasked adds (nn/attention.go:261-272, :321-330), one
 * more additive -1e30 term of `mask`; amask / mask_sb / mask_sh: the user's
 * additive mask as in oracle_attn_fwd_ex (a constant: its gradient is not
 * needed, the chain passes through the addition unchanged).
 */
int oracle_attn_bwd_autograd_x(const double* Q, const double* K, const double* V,
                               const double* dO, double* dQ, double* dK, double* dV, int BH,
                               int H, int Sq, int Sk, int D, double scale, int causal,
                               const int* kv_len, const double* amask, long mask_sb,
                               long mask_sh) {
    if (BH <= 0 || Sq <= 0 || Sk <= 0 || D <= 0 || H <= 0 || BH % H != 0) return -1;
    const size_t QK = (size_t)Sq * Sk;
    double* KT = (double*)malloc(sizeof(double) * (size_t)D * Sk);
    double* msk = (double*)malloc(sizeof(double) * QK);  /* masked scores */
    double* e = (double*)malloc(sizeof(double) * QK);
    double* attn = (double*)malloc(sizeof(double) * QK);
    double* g_attn = (double*)malloc(sizeof(double) * QK);
    double* g_e = (double*)malloc(sizeof(double) * QK);
    double* g_m = (double*)malloc(sizeof(double) * QK);
    double* VT = (double*)malloc(sizeof(double) * (size_t)D * Sk);
    double* AT = (double*)malloc(sizeof(double) * QK);
    double* GT = (double*)malloc(sizeof(double) * QK);
    if (!KT || !msk || !e || !attn || !g_attn || !g_e || !g_m || !VT || !AT || !GT) {
        free(KT); free(msk); free(e); free(attn); free(g_attn); free(g_e); free(g_m);
        free(VT); free(AT); free(GT);
        return -2;
    }
    const double sc = (g_mutation == MUT_NO_SCALE) ? 1.0 : scale;
    for (int bh = 0; bh < BH; bh++) {
        const double* Qb = Q + (size_t)bh * Sq * D;
        const double* Kb = K + (size_t)bh * Sk * D;
        const double* Vb = V + (size_t)bh * Sk * D;
        const double* G = dO + (size_t)bh * Sq * D;
        double* dQb = dQ + (size_t)bh * Sq * D;
        double* dKb = dK + (size_t)bh * Sk * D;
        double* dVb = dV + (size_t)bh * Sk * D;
        /* forward, keeping the graph's tensors */
        transpose(Kb, KT, Sk, D);
        int len = Sk;
        if (kv_len) {
            len = kv_len[bh / H];
            len = len < 0 ? 0 : (len > Sk ? Sk : len);
        }
        const double* am = amask ? amask + (size_t)(bh / H) * mask_sb + (size_t)(bh % H) * mask_sh
                                 : NULL;
        scores_rows(Qb, KT, Sk, D, NULL, Sq, scale, causal, am, len, msk);
        int* amax = (int*)malloc(sizeof(int) * Sq);
        double* se = (double*)malloc(sizeof(double) * Sq);
        double* g_se = (double*)malloc(sizeof(double) * Sq);
        double* g_mx = (double*)malloc(sizeof(double) * Sq);
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < Sq; i++) {
            const double* x = msk + (size_t)i * Sk;
            double best = -INFINITY;
            int bi = 0;
            for (int j = 0; j < Sk; j++)
                if (x[j] > best) { best = x[j]; bi = j; }
            amax[i] = bi;
            double s = 0.0;
            for (int j = 0; j < Sk; j++) {
                e[(size_t)i * Sk + j] = exp(x[j] - best);
                s += e[(size_t)i * Sk + j];
            }
            se[i] = s;
            for (int j = 0; j < Sk; j++) attn[(size_t)i * Sk + j] = e[(size_t)i * Sk + j] / s;
        }
        /* ctx = attn @ V: dattn = g @ V^T, dV = attn^T @ g */
        transpose(Vb, VT, Sk, D);
        gemm_nn(G, VT, g_attn, Sq, D, Sk);
        transpose(attn, AT, Sq, Sk);
        gemm_nn(AT, G, dVb, Sk, Sq, D);
        /* attn = e / se (broadcast): ga = g / se, gb = -g * e / se^2 summed */
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < Sq; i++) {
            double acc = 0.0;
            for (int j = 0; j < Sk; j++) {
                const double g = g_attn[(size_t)i * Sk + j];
                g_e[(size_t)i * Sk + j] = g / se[i];
                acc += -g * e[(size_t)i * Sk + j] / (se[i] * se[i]);
            }
            g_se[i] = acc;
        }
        /* se = SumAxis(e): broadcast back and accumulate into g_e */
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < Sq; i++)
            for (int j = 0; j < Sk; j++) g_e[(size_t)i * Sk + j] += g_se[i];
        /* e = Exp(sh): g_sh = g_e * e; sh = masked - mx */
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < Sq; i++) {
            double acc = 0.0;
            for (int j = 0; j < Sk; j++) {
                const double gs = g_e[(size_t)i * Sk + j] * e[(size_t)i * Sk + j];
                g_m[(size_t)i * Sk + j] = gs;
                acc += -gs;
            }
            g_mx[i] = acc;
        }
        /* mx = MaxAxis(masked): scatter to the argmax */
        for (int i = 0; i < Sq; i++) g_m[(size_t)i * Sk + amax[i]] += g_mx[i];
        /* masked = scaled + mask: identity; scaled = raw * scale */
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < Sq; i++)
            for (int j = 0; j < Sk; j++) g_m[(size_t)i * Sk + j] = g_m[(size_t)i * Sk + j] * sc;
        /* raw = Q @ K^T: dQ = g_raw @ K, d(K^T) = Q^T @ g_raw -> dK = g_raw^T @ Q */
        gemm_nn(g_m, Kb, dQb, Sq, Sk, D);
        transpose(g_m, GT, Sq, Sk);
        gemm_nn(GT, Qb, dKb, Sk, Sq, D);
        free(amax); free(se); free(g_se); free(g_mx);
    }
    free(KT); free(msk); free(e); free(attn); free(g_attn); free(g_e); free(g_m);
    free(VT); free(AT); free(GT);
    return 0;
}

/* The square form (S x S) of oracle_attn_bwd_autograd_x. */
int oracle_attn_bwd_autograd_ex(const double* Q, const double* K, const double* V,
                                const double* dO, double* dQ, double* dK, double* dV,
                                int BH, int H, int S, int D, double scale, int causal,
                                const int* kv_len, const double* amask, long mask_sb,
                                long mask_sh) {
    return oracle_attn_bwd_autograd_x(Q, K, V, dO, dQ, dK, dV, BH, H, S, S, D, scale, causal,
                                      kv_len, amask, mask_sb, mask_sh);
}

/* The reference backward's signature (no key padding). */
int oracle_attn_bwd_autograd(const double* Q, const double* K, const double* V,
                             const double* dO, double* dQ, double* dK, double* dV,
                             int BH, int S, int D, double scale, int causal) {
    return oracle_attn_bwd_autograd_ex(Q, K, V, dO, dQ, dK, dV, BH, 1, S, D, scale, causal, NULL,
                                       NULL, 0, 0);
}

/*
 * Backward by the closed-form identities the reference kernel documents
 * (backend/cuda/gonn_cuda.cu:333-340), for selected rows of one or more
 * (b,h) slices, so that full-size configurations can be checked on samples:
 *   p_ij = exp(scale q_i.k_j - L_i), D_i = dO_i . O_i,
 *   dV_j = sum_i p_ij dO_i, dS_ij = p_ij (dO_i.v_j - D_i) scale,
 *   dQ_i = sum_j dS_ij k_j, dK_j = sum_i dS_ij q_i.
 * Inputs O and LSE are the oracle's own forward (oracle_attn_fwd, all rows).
 * qrows: query rows whose dQ is computed; krows: key rows whose dK, dV are
 * computed. Either may be NULL with count 0 to skip.
 */
int oracle_attn_bwd_rows(const double* Q, const double* K, const double* V,
                         const double* O, const double* LSE, const double* dO,
                         double* dQ, double* dK, double* dV, int BH, int S, int D,
                         double scale, int causal, const int* qrows, int nq,
                         const int* krows, int nk) {
    if (BH <= 0 || S <= 0 || D <= 0) return -1;
    const double dsign = (g_mutation == MUT_DS_SIGN) ? -1.0 : 1.0;
    for (int bh = 0; bh < BH; bh++) {
        const double* Qb = Q + (size_t)bh * S * D;
        const double* Kb = K + (size_t)bh * S * D;
        const double* Vb = V + (size_t)bh * S * D;
        const double* Ob = O + (size_t)bh * S * D;
        const double* Gb = dO + (size_t)bh * S * D;
        const double* Lb = LSE + (size_t)bh * S;
        double* Dd = (double*)malloc(sizeof(double) * S);
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < S; i++) {
            double a = 0.0;
            for (int t = 0; t < D; t++) a += Gb[(size_t)i * D + t] * Ob[(size_t)i * D + t];
            Dd[i] = dsign * a;
        }
        #pragma omp parallel for schedule(dynamic, 1)
        for (int r = 0; r < nq; r++) {
            const int i = qrows[r];
            double* dq = dQ + ((size_t)bh * S + i) * D;
            for (int t = 0; t < D; t++) dq[t] = 0.0;
            const int jmax = causal ? i + 1 : S;
            for (int j = 0; j < jmax; j++) {
                double s = 0.0, dp = 0.0;
                for (int t = 0; t < D; t++) {
                    s += Qb[(size_t)i * D + t] * Kb[(size_t)j * D + t];
                    dp += Gb[(size_t)i * D + t] * Vb[(size_t)j * D + t];
                }
                const double p = exp(s * scale - Lb[i]);
                const double ds = p * (dp - Dd[i]) * scale;
                for (int t = 0; t < D; t++) dq[t] += ds * Kb[(size_t)j * D + t];
            }
        }
        #pragma omp parallel for schedule(dynamic, 1)
        for (int r = 0; r < nk; r++) {
            const int j = krows[r];
            double* dk = dK + ((size_t)bh * S + j) * D;
            double* dv = dV + ((size_t)bh * S + j) * D;
            for (int t = 0; t < D; t++) { dk[t] = 0.0; dv[t] = 0.0; }
            const int i0 = causal ? j : 0;
            for (int i = i0; i < S; i++) {
                double s = 0.0, dp = 0.0;
                for (int t = 0; t < D; t++) {
                    s += Qb[(size_t)i * D + t] * Kb[(size_t)j * D + t];
                    dp += Gb[(size_t)i * D + t] * Vb[(size_t)j * D + t];
                }
                const double p = exp(s * scale - Lb[i]);
                const double ds = p * (dp - Dd[i]) * scale;
                for (int t = 0; t < D; t++) {
                    dv[t] += p * Gb[(size_t)i * D + t];
                    dk[t] += ds * Qb[(size_t)i * D + t];
                }
            }
        }
        free(Dd);
    }
    return 0;
}

/* Linear.Forward: y (N,out) = x (N,in) @ W^T + b, W (out,in), b (out) or NULL.
 * W^T is a Permute copy, then the GEMM, then the bias Add (nn/linear.go:53-57). */
int oracle_linear(const double* x, const double* W, const double* b, double* y,
                  int N, int in, int out) {
    double* WT = (double*)malloc(sizeof(double) * (size_t)in * out);
    if (!WT) return -2;
    transpose(W, WT, out, in);
    gemm_nn(x, WT, y, N, in, out);
    if (b)
        for (int n = 0; n < N; n++)
            for (int o = 0; o < out; o++) y[(size_t)n * out + o] = y[(size_t)n * out + o] + b[o];
    free(WT);
    return 0;
}

/* (B, T, H, D) -> (B, H, T, D) Permute copy (nn/attention.go:120-122) and back
 * (nn/attention.go:146). dir 0: split heads, dir 1: merge heads. */
void oracle_heads(const double* in, double* out, int B, int T, int H, int D, int dir) {
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                for (int d = 0; d < D; d++) {
                    const size_t a = (((size_t)b * T + t) * H + h) * D + d;
                    const size_t s = (((size_t)b * H + h) * T + t) * D + d;
                    if (dir == 0) out[s] = in[a]; else out[a] = in[s];
                }
}

/*
 * GoNN's CPU forward core with GoNN's own pass structure and threading, for
 * the cpu_baseline leg of bench.py (timing only; O equals oracle_attn_fwd's
 * bit for bit, which tests/test_oracle.py checks). Each tensor op of
 * nn/attention.go:135-146 is one pass over the whole (BH, S, S) score tensor
 * into a freshly allocated result, as the tensor package does:
 *   MatMul            one GEMM per slice in sequence (backend/cpu.go:38-45),
 *                     the GEMM itself threaded, as gonum's Dgemm is; the K^T
 *                     operand a Permute copy (tensor/ops_shape.go:53-107)
 *   MulScalar(scale)  Scalar(scale) broadcast to the full shape by expandTo
 *                     (tensor/broadcast.go:35-80, a copy), then the binary loop
 *                     (tensor/ops_binary.go:32-56)
 *   Add(causal mask)  causalMaskAdd (1,1,S,S) built (nn/attention.go:185-196),
 *                     expanded to (BH,S,S), then the binary loop
 *   Softmax(3)        MaxAxis; Sub with the max expanded; Exp; SumAxis; Div
 *                     with the sum expanded (tensor/ops_activation.go:455-461)
 *   MatMul with V     as above.
 * The elementwise loops and reductions run on one thread: the CPU backend has
 * no Elementwiser (backend/cpu.go:9-11), so they are plain Go loops.
 */
static double* g_alloc(size_t n) { return (double*)malloc(n * sizeof(double)); }
int oracle_attn_fwd_goflow(const double* Q, const double* K, const double* V, double* O,
                           int BH, int S, int D, double scale, int causal) {
    const size_t SS = (size_t)S * S, N = (size_t)BH * SS;
    double* KT = g_alloc((size_t)BH * D * S);
    double* sc = g_alloc(N);
    if (!KT || !sc) { free(KT); free(sc); return -2; }
    for (int bh = 0; bh < BH; bh++)  /* Permute copy (single-threaded loop) */
        for (int j = 0; j < D; j++)
            for (int i = 0; i < S; i++)
                KT[((size_t)bh * D + j) * S + i] = K[((size_t)bh * S + i) * D + j];
    for (int bh = 0; bh < BH; bh++)
        gemm_nn(Q + (size_t)bh * S * D, KT + (size_t)bh * D * S, sc + (size_t)bh * SS, S, D, S);
    free(KT);
    /* MulScalar */
    double* ex = g_alloc(N);
    double* t1 = g_alloc(N);
    if (!ex || !t1) { free(ex); free(t1); free(sc); return -2; }
    for (size_t i = 0; i < N; i++) ex[i] = scale;
    for (size_t i = 0; i < N; i++) t1[i] = sc[i] * ex[i];
    free(sc);
    double* t2 = t1;
    if (causal) {
        double* m = g_alloc(SS);
        t2 = g_alloc(N);
        if (!m || !t2) { free(m); free(t2); free(ex); free(t1); return -2; }
        for (int i = 0; i < S; i++)
            for (int j = 0; j < S; j++) m[(size_t)i * S + j] = j > i ? MASK_NEG : 0.0;
        for (size_t i = 0; i < N; i++) ex[i] = m[i % SS];
        for (size_t i = 0; i < N; i++) t2[i] = t1[i] + ex[i];
        free(m);
        free(t1);
    }
    /* Softmax(3) */
    const size_t R = (size_t)BH * S;
    double* mx = g_alloc(R);
    double* sm = g_alloc(R);
    double* t3 = g_alloc(N);
    if (!mx || !sm || !t3) { free(mx); free(sm); free(t3); free(ex); free(t2); return -2; }
    for (size_t r = 0; r < R; r++) {
        double v = -INFINITY;
        for (int j = 0; j < S; j++) if (t2[r * S + j] > v) v = t2[r * S + j];
        mx[r] = v;
    }
    for (size_t i = 0; i < N; i++) ex[i] = mx[i / S];
    for (size_t i = 0; i < N; i++) t3[i] = t2[i] - ex[i];
    free(t2);
    double* t4 = g_alloc(N);
    if (!t4) { free(mx); free(sm); free(t3); free(ex); return -2; }
    for (size_t i = 0; i < N; i++) t4[i] = exp(t3[i]);
    free(t3);
    for (size_t r = 0; r < R; r++) {
        double v = 0.0;
        for (int j = 0; j < S; j++) v += t4[r * S + j];
        sm[r] = v;
    }
    double* at = g_alloc(N);
    if (!at) { free(mx); free(sm); free(t4); free(ex); return -2; }
    for (size_t i = 0; i < N; i++) ex[i] = sm[i / S];
    for (size_t i = 0; i < N; i++) at[i] = t4[i] / ex[i];
    free(t4);
    free(ex);
    free(mx);
    free(sm);
    for (int bh = 0; bh < BH; bh++)
        gemm_nn(at + (size_t)bh * SS, V + (size_t)bh * S * D, O + (size_t)bh * S * D, S, S, D);
    free(at);
    return 0;
}

/* Timing helper for the CPU baseline: the forward core over `nslices` (b,h)
 * slices with OpenMP threads `threads` (0 = runtime default). */
#ifdef _OPENMP
#include <omp.h>
#endif
void oracle_set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}
int oracle_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
