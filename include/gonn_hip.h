/*
 * gonn_hip.h -- C ABI of the MI355X (gfx950) attention core for GoNN.
 *
 * This library replaces the fused flash-attention seam of GoNN
 * (nn/flashattn_cuda.go -> backend/cuda/cuda.go -> backend/cuda/gonn_cuda.cu).
 * Every entry point is plain C: scalar arguments, raw pointers and sizes.
 * Nothing here needs HIP or PyTorch headers; a hipStream_t is passed as an
 * opaque pointer (NULL = the legacy default stream).
 *
 * Layouts (all dense row-major, exactly the reference's layout after the head
 * split at nn/attention.go:120-122 and nn/attention.go:170-176):
 *   Q        (B*H, Sq, D)          K, V   (B*H, Sk, D)
 *   O        (B*H, Sq, D) fp32     LSE    (B*H, Sq) fp32, natural-log units:
 *            LSE[i] = max_j s_ij + ln(sum_j exp(s_ij - max_j s_ij)) with
 *            s_ij = scale * q_i . k_j over the unmasked keys, the quantity
 *            the reference kernel stores as L = m + log(l)
 *            (backend/cuda/gonn_cuda.cu:330 and :448).
 *   decode   q (B, H, D), cache (B, H, Lmax, D) bf16, o (B, H, D) fp32.
 *
 * Masking semantics follow the reference CPU path bit-for-bit in which keys
 * carry weight:
 *   causal   key j is masked for query i when j > i, top-left aligned even
 *            when Sq != Sk (causalMaskAdd, nn/attention.go:185-196);
 *   kv_len   keys t >= kv_len[b] are masked for every head and query
 *            (keyPaddingMaskAdd, nn/attention.go:261-272). A -1e30 additive
 *            mask gives an exactly-zero weight in fp64, so skipping the key
 *            is the same result. The kernels never read a key >= kv_len[b].
 *
 * Return values: 0 on success; a negative GONN_E_* code for argument and
 * library errors (checked on the host before any GPU work is queued); a
 * positive value is a hipError_t from the runtime.
 *
 * Threading: every call is reentrant. Entry points that take a workspace keep
 * no hidden global state; calls on the same stream are ordered, calls on
 * different streams may run concurrently as long as their buffers do not
 * alias. The f64 compatibility shims allocate per call, like the reference.
 */
#ifndef GONN_HIP_H
#define GONN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ------------------------------------------------------- */
enum {
    GONN_OK = 0,
    GONN_E_INVALID = -1,     /* bad shape, null pointer, short buffer, bad enum  */
    GONN_E_UNSUPPORTED = -2, /* valid request the kernels do not cover (e.g. D) */
    GONN_E_WORKSPACE = -3,   /* workspace missing or smaller than required      */
    GONN_E_NOMEM = -4,       /* device allocation failed                        */
    GONN_E_NODEVICE = -5,    /* no usable gfx950 device                         */
    GONN_E_INJECTED = -6,    /* failure forced by GONN_HIP_FAIL_ALLOC=1         */
    GONN_E_BLAS = -7         /* a rocBLAS call failed (GEMM)                    */
};

/* ---- element types and arithmetic modes --------------------------------- */
typedef enum { GONN_F32 = 0, GONN_BF16 = 1, GONN_F64 = 2, GONN_I32 = 3 } gonn_dtype;

/* The two dense contractions (QK^T and PV, and the five backward products)
 * run on MFMA in one of two modes, accumulating in fp32; the f64 entry
 * points can instead run fp64 kernels throughout (the precision of the
 * reference's fp64 CUDA seam).                                             */
typedef enum {
    GONN_ATTN_FP32_MFMA = 0, /* fp32 operands (v_mfma_f32_32x32x2_f32)        */
    GONN_ATTN_BF16_MFMA = 1, /* bf16 operands (v_mfma_f32_32x32x16_bf16)      */
    GONN_ATTN_FP64 = 2       /* fp64 throughout, exact to rounding: the f64
                                entry points only (the device entries take
                                modes 0 and 1)                              */
} gonn_attn_mode;

/* A device buffer handle: a device pointer, its size in bytes and the type
 * of its elements. The library checks `bytes` against the shape it needs.  */
typedef struct {
    void* ptr;
    size_t bytes;
    int dtype; /* gonn_dtype */
} gonn_buf;

/* Forward: O = softmax(scale * Q K^T + mask) V, plus LSE.
 * q, k, v: GONN_F32 or GONN_BF16. o: GONN_F32. lse: GONN_F32 or ptr NULL.
 * kv_len: optional GONN_I32 device array [B] (ptr NULL = none): keys
 * t >= kv_len[b] are masked for every head and query of sequence b (a
 * prefix key-padding mask, nn/attention.go:261-272), combined with the
 * causal mask as ForwardMasked adds both (nn/attention.go:321-330). Values
 * are clamped to [0, Sk]; a sequence with kv_len 0 gets O = 0 and
 * LSE = -inf. That is this ABI's own definition: GoNN gives such a row the
 * uniform average of the -1e30-absorbed scores, which the kernels do not
 * compute; the host mirrors (nn.py, nn_attention.cpp) and the Go gate
 * refuse or decline such calls instead of passing kv_len 0. */
typedef struct {
    gonn_buf q, k, v, o, lse;
    int B, H, Sq, Sk, D;
    double scale;
    int causal;
    int mode; /* gonn_attn_mode */
    gonn_buf kv_len;
    /* Optional additive mask (WithAttnMask, nn/attention.go:212-257):
     * GONN_F32 device data, ptr NULL = none. Slice b*H + h adds
     * attn_mask[b*mask_stride_b + h*mask_stride_h + i*Sk + j] to the scaled
     * score of query i and key j, after the causal mask and before the key
     * padding, as ForwardMasked orders them. Strides (elements, >= 0) of 0
     * broadcast: (Sq,Sk) -> 0, 0; (B,Sq,Sk) -> Sq*Sk, 0; (B*H,Sq,Sk) and
     * (B,H,Sq,Sk) -> H*Sq*Sk, Sq*Sk. A masked forward runs in the
     * requested mode (bf16 mode: Sq*Sk*4 bytes must stay below 4 GiB, else
     * GONN_E_UNSUPPORTED); the fp32 mode needs GONN_F32 q, k, v. Values
     * are added in fp32: -1e30 blocks a key (weight exactly 0 when the row
     * keeps another key), also when it blocks whole leading key tiles. A row
     * whose every key is blocked (no unblocked key within its causal window
     * and kv_len) is outside this ABI's definition, as kv_len 0 is; the host
     * mirrors and the Go gate refuse or decline it. They also shift each
     * mask row by its maximum, so a large common offset costs no fp32
     * precision; callers of this entry with such masks should do the same. */
    gonn_buf attn_mask;
    int64_t mask_stride_b, mask_stride_h;
} gonn_attn_fwd_args;

/* Backward from the saved forward tensors: dQ, dK, dV (all GONN_F32).
 * q, k, v, o, dO: GONN_F32; lse: GONN_F32 from gonn_hip_attn_fwd.
 * S is the query (and, unless Sk is set, key) count.
 * deterministic: accepted for API completeness; every mode of this library
 * is deterministic (no floating-point atomics), so 0 and 1 give
 * bit-identical results.
 * kv_len: optional GONN_I32 device array [B] (ptr NULL = none), the same as
 * the forward's: keys t >= kv_len[b] are padded, so their dK and dV rows are
 * 0 and they add nothing to dQ; o and lse must come from the forward with
 * the same kv_len. A sequence with kv_len 0 gets dQ = dK = dV = 0.         */
typedef struct {
    gonn_buf q, k, v, o, lse, dO, dq, dk, dv;
    int B, H, S, D;
    double scale;
    int causal;
    int mode;
    int deterministic;
    gonn_buf kv_len;
    /* The forward's additive mask (layout as in gonn_attn_fwd_args with
     * Sq = S), read in the requested mode's kernels (bf16 mode: S*Sk*4
     * bytes must stay below 4 GiB, else GONN_E_UNSUPPORTED).               */
    gonn_buf attn_mask;
    int64_t mask_stride_b, mask_stride_h;
    /* Key rows when they differ from the S query rows (cross-attention with
     * the forward's top-left causal mask): k, v, dk, dv are (B*H, Sk, D).
     * 0 means Sk = S. Cross-attention runs in the requested mode.          */
    int Sk;
} gonn_attn_bwd_args;

/* KV-cache decode, one query per (b, h): o[b,h] = attention of q[b,h] over
 * the first kv_len[b] rows of kcache[b,h] / vcache[b,h], non-causal.
 * q: GONN_F32 or GONN_BF16 (B,H,D); kcache, vcache: GONN_BF16 (B,H,Lmax,D);
 * kv_len: GONN_I32 device array [B], values clamped to [0, Lmax];
 * o: GONN_F32 (B,H,D). A sequence with kv_len 0 gets o = 0.
 * split_keys: keys per split-KV work item (multiple of 64, 0 = automatic). */
typedef struct {
    gonn_buf q, kcache, vcache, kv_len, o;
    int B, H, Lmax, D;
    double scale;
    int split_keys;
} gonn_attn_decode_args;

enum { GONN_OP_FWD = 0, GONN_OP_BWD = 1, GONN_OP_DECODE = 2 };

/* ---- library ----------------------------------------------------------- */

/* Version string of the library build. */
const char* gonn_hip_version(void);

/* Human-readable text for a return code (GONN_E_* or hipError_t). */
const char* gonn_hip_strerror(int code);

/* 1 when a gfx950 device is present and usable, else 0. Replaces
 * fusedAttnAvailable (nn/flashattn_cuda.go:13) as a runtime query.        */
int gonn_hip_available(void);

/* 1 when the fused kernels cover head dim D with Sq x Sk, else 0. The
 * reference hard-codes D == 64 && Tq == Tk at nn/attention.go:129 and :165;
 * this predicate replaces that gate.                                       */
int gonn_hip_attn_supports(int D, int Sq, int Sk);

/* Default arithmetic mode used by the f64 compatibility shims. Initialised
 * from the environment variable GONN_HIP_ATTN_MODE ("fp32", "bf16" or
 * "f64"), default fp32-MFMA. GONN_ATTN_FP64 makes the f64 entries compute
 * in fp64 (agreeing with an fp64 CPU evaluation to rounding, as the
 * reference's CUDA seam does); the MFMA modes convert their host fp64 data
 * to fp32. The resident MHA layer (gonn_hip_mha_*) runs its core in this
 * mode on its fp32 intermediates, fp32-MFMA when the mode is
 * GONN_ATTN_FP64. Returns GONN_E_INVALID for an unknown mode.              */
int gonn_hip_set_attn_mode(int mode);
int gonn_hip_get_attn_mode(void);

/* ---- device-resident API ---------------------------------------------- */

/* Workspace bytes a call with these arguments needs (0 if none).
 * op: GONN_OP_FWD / GONN_OP_BWD / GONN_OP_DECODE with the matching struct. */
size_t gonn_hip_attn_workspace_bytes(int op, const void* args);

/* Flash forward. Replaces gonn_flash_attn_f64_fwd
 * (backend/cuda/gonn_cuda.h:67-69, gonn_cuda.cu:483-498) for device buffers.
 * ws: device workspace of gonn_hip_attn_workspace_bytes(GONN_OP_FWD) bytes. */
int gonn_hip_attn_fwd(const gonn_attn_fwd_args* a, void* ws, size_t ws_bytes, void* stream);

/* Flash backward. Replaces gonn_flash_attn_f64_bwd
 * (backend/cuda/gonn_cuda.h:71-74, gonn_cuda.cu:501-529) for device buffers.
 * ws: gonn_hip_attn_workspace_bytes(GONN_OP_BWD) bytes. In bf16 mode it holds
 * the dS that dQ is formed from, at most 16 GiB; a call with up to twice that
 * runs in two key-block chunks (same results), a larger one forms dS again in
 * the dQ kernel (no dS buffer). Environment, read by each call and by the
 * workspace query alike: GONN_HIP_BWD_DS_MB=<MB> sets the dS budget and always
 * chunks within it; GONN_HIP_BWD_DQ=recompute forms dS again.               */
int gonn_hip_attn_bwd(const gonn_attn_bwd_args* a, void* ws, size_t ws_bytes, void* stream);

/* Split-KV decode plus combine. New: the reference has no KV cache; the
 * semantics are ForwardMasked with WithKeyPaddingMask (nn/attention.go:305-341,
 * :261-272) on the post-projection core with pad[b][t] = (t >= kv_len[b]).  */
int gonn_hip_attn_decode(const gonn_attn_decode_args* a, void* ws, size_t ws_bytes, void* stream);

/* No-allocation split-KV decode. No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The same kernels and
 * result as gonn_hip_attn_decode, with the split partials kept in a
 * library-owned device array of GONN_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends) instead of a caller workspace; calls no
 * hipMalloc/hipFree. A call whose partials need more than that
 * (gonn_hip_attn_workspace_bytes(GONN_OP_DECODE) > GONN_NOALLOC_SCRATCH_BYTES)
 * returns GONN_E_WORKSPACE before any GPU work is queued. Every call on one
 * GPU shares that array: calls that overlap on one GPU (different streams or
 * threads) race and must be serialised by the caller.                     */
#define GONN_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int gonn_hip_attn_decode_noalloc(const gonn_attn_decode_args* a, void* stream);

/* ---- KV cache for incremental decoding ----------------------------------
 * New: the reference has no KV cache (its decoder recomputes attention over
 * the whole prefix through MultiHeadAttention.Forward). A handle owns one
 * attention layer's device cache: K and V of B sequences x H heads, up to
 * Lmax positions of head dim D, bf16 (B,H,Lmax,D), and the number of cached
 * positions of each sequence. Appending writes new positions at each
 * sequence's length; attending runs the split-KV decode of one query per
 * (b, h) over the cached positions, i.e. ForwardMasked with a key-padding
 * mask (nn/attention.go:305-341, :261-272) on the post-projection core; a
 * sequence with no cached position gets o = 0. Calls on one handle are not
 * reentrant; different handles are independent. For callers that cannot
 * hold device pointers (cgo), the _f64 variants take host arrays.
 * A failed call leaves the lengths as they were. If putting the device copy
 * of the lengths back fails as well, the handle is stale: every append and
 * attend on it (and the incremental MHA forward) returns GONN_E_INVALID
 * until gonn_hip_kvcache_reset succeeds.                                 */
typedef struct gonn_kvcache gonn_kvcache;

/* D must be 64 or 128 (GONN_E_UNSUPPORTED otherwise); GONN_E_NODEVICE
 * without a gfx950 device. *out is NULL on failure.                       */
int gonn_hip_kvcache_create(gonn_kvcache** out, int B, int H, int Lmax, int D);
/* Frees the handle and its device memory (NULL is allowed).              */
int gonn_hip_kvcache_free(gonn_kvcache* c);
/* Drops every cached position (lengths back to 0); clears a stale handle. */
int gonn_hip_kvcache_reset(gonn_kvcache* c);
/* Copies the B current lengths into len[B].                              */
int gonn_hip_kvcache_lengths(const gonn_kvcache* c, int* len);
/* Appends new positions: k, v are (B,H,T,D) device buffers, GONN_F32 or
 * GONN_BF16 (both the same, 16-byte aligned); sequence b takes its first
 * counts[b] rows (host int[B]; NULL = T for every sequence). An append that
 * would take a sequence past Lmax returns GONN_E_INVALID and writes nothing.
 * Synchronous with respect to `stream`.                                   */
int gonn_hip_kvcache_append(gonn_kvcache* c, const gonn_buf* k, const gonn_buf* v, int T,
                            const int* counts, void* stream);
/* As gonn_hip_kvcache_append with host fp64 (B,H,T,D) arrays.            */
int gonn_hip_kvcache_append_f64(gonn_kvcache* c, const double* k, const double* v, int T,
                                const int* counts);
/* o (B,H,D) = softmax(scale q . K^T) V over each sequence's cached
 * positions; q: GONN_F32 or GONN_BF16 (B,H,D), o: GONN_F32 (B,H,D).      */
int gonn_hip_kvcache_attend(gonn_kvcache* c, const gonn_buf* q, gonn_buf* o, double scale,
                            void* stream);
/* As gonn_hip_kvcache_attend with host fp64 q and o (B,H,D); synchronous. */
int gonn_hip_kvcache_attend_f64(gonn_kvcache* c, const double* q, double* o, double scale);
/* Causal multi-token attend (no counterpart in the reference, which has no
 * KV cache; the result is nn/attention.go:185-196's top-left causal mask
 * over the whole sequence): T new queries per (b,h), q and o GONN_F32
 * (B,H,T,D) device buffers, whose own K/V rows are the last T cached
 * positions of their sequence; query t attends cached positions
 * [0, len_b - T + t]. Every length must be >= T (GONN_E_INVALID otherwise).
 * Workspace: gonn_hip_kvcache_attend_causal_workspace_bytes(c, T) bytes; on
 * `stream`, allocates nothing. T = 1 is gonn_hip_kvcache_attend.          */
size_t gonn_hip_kvcache_attend_causal_workspace_bytes(const gonn_kvcache* c, int T);
int gonn_hip_kvcache_attend_causal(gonn_kvcache* c, const gonn_buf* q, gonn_buf* o, int T,
                                   double scale, void* ws, size_t ws_bytes, void* stream);

/* ---- fp64 GEMM of the backend -------------------------------------------
 * backend.Backend.Gemm (backend/backend.go:61-78) on the device: row-major
 * batched C = op(A) op(B); op(A) (m,k) stored (m,k), or (k,m) when transA;
 * op(B) (k,n) stored (k,n), or (n,k) when transB; C (m,n); `batch`
 * contiguous pairs. Replaces gonn_gemm (backend/cuda/gonn_cuda.h:36,
 * gonn_cuda.cu:147-177): host fp64 in and out, synchronous, serialised on
 * an internal workspace like the reference's. The _dev variant takes
 * GONN_F64 device buffers and a stream.                                   */
int gonn_hip_gemm_f64(const double* A, const double* B, double* C, int batch, int m, int k, int n,
                      int transA, int transB);
int gonn_hip_gemm_f64_dev(const gonn_buf* A, const gonn_buf* B, gonn_buf* C, int batch, int m,
                          int k, int n, int transA, int transB, void* stream);

/* ---- fp64 elementwise ops of the backend --------------------------------
 * backend.Elementwiser (backend/backend.go:80-92). The kind values are the
 * reference's append-only ABI (backend.go:26-58, gonn_cuda.h:13-28).       */
enum {
    GONN_UN_RELU = 0,
    GONN_UN_SIGMOID = 1,
    GONN_UN_TANH = 2,
    GONN_UN_EXP = 3,
    GONN_UN_LOG = 4,
    GONN_UN_GELU = 5,       /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
    GONN_UN_SILU = 6,       /* x sigmoid(x)                                     */
    GONN_UN_GELU_EXACT = 7  /* 0.5 x (1 + erf(x / sqrt(2)))                     */
};
enum { GONN_BIN_ADD = 0, GONN_BIN_SUB = 1, GONN_BIN_MUL = 2, GONN_BIN_DIV = 3 };

/* C[i] = f_kind(A[i]), i < n; replaces gonn_unary (gonn_cuda.h:39-40): host
 * fp64 in and out, synchronous, serialised on an internal workspace. An
 * unknown kind returns GONN_E_INVALID (the Go wrapper then declines).      */
int gonn_hip_unary_f64(int kind, const double* A, double* C, long n);
/* C[i] = A[i] op_kind B[i]; replaces gonn_binary (gonn_cuda.h:42-43).      */
int gonn_hip_binary_f64(int kind, const double* A, const double* B, double* C, long n);
/* The same on GONN_F64 device buffers (16-byte aligned) on a stream; no
 * copies, no allocation.                                                   */
int gonn_hip_unary_f64_dev(int kind, const gonn_buf* A, gonn_buf* C, long n, void* stream);
int gonn_hip_binary_f64_dev(int kind, const gonn_buf* A, const gonn_buf* B, gonn_buf* C, long n,
                            void* stream);

/* ---- device-resident multi-head attention -------------------------------
 * nn.MultiHeadAttention's forward (nn/attention.go:107-148) with its weights
 * in HBM: projections (rocBLAS fp64), head split into fp32 (B, H, T, dp),
 * the fused core in the current MFMA mode with scale 1/sqrt(E/H), head merge,
 * output projection. New: the reference copies across PCIe around every GEMM
 * (tensor/dispatch.go:111-113) and around the core (gonn_cuda.cu:466-529).
 * Weights W* are (E, in) row-major fp64 with in = E (q, out), kdim (k), vdim
 * (v); a null bias is zero. E % H == 0 and E/H <= 128.                      */
typedef struct gonn_mha gonn_mha;
int gonn_hip_mha_create(gonn_mha** out, int E, int H, int kdim, int vdim, const double* Wq,
                        const double* bq, const double* Wk, const double* bk, const double* Wv,
                        const double* bv, const double* Wo, const double* bo);
int gonn_hip_mha_free(gonn_mha* m);
/* q (B, Tq, E), k (B, Tk, kdim), v (B, Tk, vdim) host fp64 -> out (B, Tq, E).
 * kv_len: optional host int32[B], keys t >= kv_len[b] ignored (ForwardMasked
 * key padding, nn/attention.go:261-272); causal is top-left (j > i masked).
 * Synchronous; one upload of the inputs (once when k == q and v == k), one
 * download. Calls on one handle are serialised on its workspace.            */
int gonn_hip_mha_forward_f64(gonn_mha* m, const double* q, const double* k, const double* v,
                             double* out, int B, int Tq, int Tk, int causal, const int* kv_len);
/* The same on GONN_F64 device buffers (kv_len: GONN_I32 device buffer or
 * null) with a caller workspace of gonn_hip_mha_workspace_bytes bytes, on
 * `stream`; allocates nothing. Calls that share a workspace must not overlap.
 * Where both projections take the library's skinny fp64 GEMM (B*Tq <= 256
 * rows, E a multiple of 128, as at C1), the call only launches kernels and
 * can be captured in a HIP graph once an eager call has run on the device
 * (it creates the GEMM handle); replays are bit-identical to eager calls.   */
size_t gonn_hip_mha_workspace_bytes(const gonn_mha* m, int B, int Tq, int Tk);
int gonn_hip_mha_forward_dev(gonn_mha* m, const gonn_buf* q, const gonn_buf* k, const gonn_buf* v,
                             gonn_buf* out, int B, int Tq, int Tk, int causal,
                             const gonn_buf* kv_len, void* ws, size_t ws_bytes, void* stream);
/* Incremental self-attention on the device (no counterpart in the reference,
 * which has no KV cache): x (B, T, E) GONN_F64 device -> out (B, T, E), the
 * last T rows of a causal Forward(seq, seq, seq) over every position the
 * cache holds plus these. One stream: the stacked q/k/v projection, head
 * split, append of the T new K/V rows to the cache, the causal multi-token
 * attend, head merge and output projection; one host synchronisation per
 * call, after which the cache lengths advance by T (they stay as they were
 * on failure). The cache must be (B, H, *, dp) with dp = 64 or 128 (E/H
 * zero-padded) and the layer a self-attention with kdim = vdim = E. The
 * workspace is gonn_hip_mha_incremental_workspace_bytes(m, c, T) bytes (0:
 * the handles do not fit together).                                       */
size_t gonn_hip_mha_incremental_workspace_bytes(const gonn_mha* m, const gonn_kvcache* c, int T);
int gonn_hip_mha_forward_incremental_dev(gonn_mha* m, gonn_kvcache* c, const gonn_buf* x,
                                         gonn_buf* out, int T, void* ws, size_t ws_bytes,
                                         void* stream);

/* ---- device buffers ------------------------------------------------------
 * Replace gonn_dev_alloc / gonn_dev_free / gonn_dev_upload / gonn_dev_download
 * (backend/cuda/gonn_cuda.h:77-80) for the attention path. The f64 transfer
 * helpers convert on the device (f64 <-> f32 or bf16, round to nearest even). */
int gonn_hip_alloc(gonn_buf* b, size_t n_elems, int dtype);
int gonn_hip_free(gonn_buf* b);
int gonn_hip_upload_from_f64(gonn_buf* dst, const double* src, size_t n_elems, void* stream);
int gonn_hip_download_to_f64(double* dst, const gonn_buf* src, size_t n_elems, void* stream);
int gonn_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int gonn_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int gonn_hip_stream_sync(void* stream);

/* ---- f64 host compatibility shims (reference signatures, synchronous) ----
 * Same arguments and meaning as the reference entry points; they upload the
 * host fp64 arrays, convert on the device, run the kernels in the current
 * mode and download fp64 results. Any 1 <= d <= 128 is accepted: head dims
 * other than 64/128 are zero-padded on the device, which leaves every score
 * and every kept output column unchanged. Unlike the reference, which
 * returns void and ignores CUDA errors, they return a status code.        */

/* backend/cuda/gonn_cuda.h:60-61, gonn_cuda.cu:466-480 */
int gonn_hip_flash_attn_f64(const double* Q, const double* K, const double* V,
                            double* O, int BH, int S, int d, double scale, int causal);
/* backend/cuda/gonn_cuda.h:67-69, gonn_cuda.cu:483-498 */
int gonn_hip_flash_attn_f64_fwd(const double* Q, const double* K, const double* V,
                                double* O, double* L, int BH, int S, int d,
                                double scale, int causal);
/* backend/cuda/gonn_cuda.h:71-74, gonn_cuda.cu:501-529 */
int gonn_hip_flash_attn_f64_bwd(const double* Q, const double* K, const double* V,
                                const double* O, const double* L, const double* dO,
                                double* dQ, double* dK, double* dV,
                                int BH, int S, int d, double scale, int causal);
/* General fp64 backward (new): B sequences x H heads of S x S, with the
 * forward's optional host kv_len[B] (ForwardMasked key padding, see
 * gonn_attn_bwd_args); O and L from gonn_hip_flash_attn_f64_ex with the same
 * kv_len. gonn_hip_flash_attn_f64_bwd is this with B = BH, H = 1, no kv_len. */
int gonn_hip_flash_attn_f64_bwd_ex(const double* Q, const double* K, const double* V,
                                   const double* O, const double* L, const double* dO, double* dQ,
                                   double* dK, double* dV, int B, int H, int S, int d,
                                   double scale, int causal, const int* kv_len);

/* Additive-mask forms of the two general fp64 entries (new): mask is host
 * fp64 data read as in gonn_attn_fwd_args.attn_mask with element strides
 * mask_sb (sequence) and mask_sh (head) and rows Sk apart; NULL = none. The
 * backward also takes cross-attention (Sq != Sk: K, V, dK, dV are
 * (B*H, Sk, d)). Both run in the current mode.                           */
int gonn_hip_flash_attn_f64_masked(const double* Q, const double* K, const double* V, double* O,
                                   double* L, int B, int H, int Sq, int Sk, int d, double scale,
                                   int causal, const int* kv_len, const double* mask,
                                   long mask_sb, long mask_sh);
int gonn_hip_flash_attn_f64_bwd_masked(const double* Q, const double* K, const double* V,
                                       const double* O, const double* L, const double* dO,
                                       double* dQ, double* dK, double* dV, int B, int H, int Sq,
                                       int Sk, int d, double scale, int causal,
                                       const int* kv_len, const double* mask, long mask_sb,
                                       long mask_sh);
/* New (the reference's fused seam is Tq == Tk, causal-or-not only): the
 * general forward on host fp64 arrays for the wider fused gate, i.e.
 * cross-attention (Sq != Sk, top-left causal mask when causal) and
 * ForwardMasked with a prefix key-padding mask (nn/attention.go:305-341):
 * Q (B*H, Sq, d), K, V (B*H, Sk, d), O (B*H, Sq, d); L (B*H, Sq) natural-log
 * LSE or NULL; kv_len host int[B] (keys t >= kv_len[b] masked) or NULL.   */
int gonn_hip_flash_attn_f64_ex(const double* Q, const double* K, const double* V, double* O,
                               double* L, int B, int H, int Sq, int Sk, int d, double scale,
                               int causal, const int* kv_len);
/* backend/cuda/gonn_cuda.h:63, gonn_cuda.cu:532-560: device-resident,
 * event-timed forward; returns mean ms per launch, or a negative value on
 * error. Inputs are zero-filled like the reference's benchmark.           */
double gonn_hip_bench_flash_attn_f64(int BH, int S, int d, int iters, int causal);
/* New (the reference times no backward: benchmark/flashbwd/main.go only
 * gradchecks FlashAttnF64Bwd): the exact-mode backward timed like the
 * forward above (zero-filled device fp64 inputs, 5 warm-ups, one event pair
 * around `iters` calls, mean ms per call). Only in mode GONN_ATTN_FP64;
 * other modes return GONN_E_INVALID (their backward is gonn_hip_attn_bwd).*/
double gonn_hip_bench_flash_attn_f64_bwd(int BH, int S, int d, int iters, int causal);

/* ---- diagnostics ---------------------------------------------------------- */

/* Per-kernel event profiler. While enabled, every kernel stage this library
 * launches ("pack_kv", "fwd_bf16", "fwd_f32", "decode_split",
 * "decode_combine", "bwd_prep", "bwd_dkdv", "bwd_dq") is bracketed by two HIP
 * events on its own stream. profile_read synchronises on the recorded events
 * and returns the summed milliseconds and launch count of one stage. No
 * reference counterpart: the reference times whole launches with CUDA events
 * (backend/cuda/gonn_cuda.cu:548-559).                                    */
int gonn_hip_profile_enable(int on);
int gonn_hip_profile_reset(void);
int gonn_hip_profile_read(const char* kernel, double* total_ms, int* count);

/* Box calibration for benchmarks (no reference counterpart: GoNN's
 * benchmark reports raw times, backend/cuda/gonn_cuda.cu:532-560).
 * calib_mfma: TFLOP/s of a fixed loop of v_mfma_f32_32x32x16_bf16 over
 * the whole device (two waves per SIMD, eight independent chains each, no
 * memory traffic), and the mean shader clock (GHz) over the loop; operands
 * constant (random = 0) or distinct uniform [-1, 1) values per lane and
 * chain (random = 1: the switching of real data, whose power sets the
 * clock); synchronous.
 * calib_clock_start: enqueues on `stream` a one-wave probe that reads the
 * shader clock against the fixed 100 MHz counter for `ms` milliseconds
 * (0 < ms <= 60000), for running beside other work on another stream.
 * calib_clock_read: the probe's shader clock in GHz; call it after that
 * stream has been synchronised.                                          */
int gonn_hip_calib_mfma(int random, double* tflops, double* ghz);
int gonn_hip_calib_clock_start(double ms, void* stream);
int gonn_hip_calib_clock_read(double* ghz);

/* Runs one v_mfma_f32_32x32x16_bf16 and one v_mfma_f32_32x32x2_f32 on known
 * inputs and compares every output element with a host matrix product; the
 * kernels rely on that operand/result lane layout. Returns the number of
 * mismatching elements (0 = layout as assumed) or a negative error.       */
int gonn_hip_selftest_mfma(void);

#ifdef __cplusplus
}
#endif

#endif /* GONN_HIP_H */
