// gonn_host.hpp -- C++ host mirror of GoNN's attention seam over the C ABI.
//
// GoNN's host side for this path is Go: the cgo wrappers backend/cuda/cuda.go
// (flash entry points :125-194) and the build-tagged nn seam
// nn/flashattn_cuda.go:13-38, called from MultiHeadAttention.Forward /
// ForwardFused (nn/attention.go:107-180). This header restates that layer in
// C++ on top of include/gonn_hip.h, with the same names, argument meaning and
// error behaviour:
//
//   gonn::hip  (backend/hip, the counterpart of backend/cuda/cuda.go)
//     Available, Supports, SetMode, FlashAttnF64, FlashAttnF64Fwd,
//     FlashAttnF64Bwd, BenchFlashAttnF64, KVCache (new)
//   gonn::backend  (backend/backend.go:61-118: Backend, NewCPU, Use, Current;
//     NewHIP is the counterpart of backend/cuda's Backend(), cuda.go:30-67)
//   gonn::nn   (nn/flashattn_hip.go + the fused branch of nn/attention.go)
//     Tensor, Linear, fusedAttnAvailable, fusedAttnSupports, fusedAttnF64,
//     fusedAttnDiff, MultiHeadAttention::{Forward, ForwardFused,
//     NewCache, ForwardIncremental (new)}
//
// Where the Go code panics (slice length mismatch, checkQKVDims, a failed
// device call surfaced by the new ABI's status codes) these throw:
// std::invalid_argument for argument errors, gonn::hip::Error for a non-zero
// ABI status. Tensors hold host float64 data, like tensor.Tensor
// (tensor/tensor.go:22-23). The attention core only runs on the device: with
// no library or no gfx950 device the fused calls throw, there is no CPU
// attention path in this library.
#pragma once

#include <array>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace gonn {
namespace hip {

// A non-zero status from the C ABI (GONN_E_* or a hipError_t value).
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& where);
};

// cuda.go has no Available(): the Go cuda build returns true at compile time
// (nn/flashattn_cuda.go:13). This is a runtime device query.
bool Available();
// Head-dim / shape predicate replacing the D == 64 gate of nn/attention.go:129.
bool Supports(int D, int Tq, int Tk);
// 0 = fp32-MFMA (default), 1 = bf16-MFMA, for the f64 entry points.
void SetMode(int mode);
int Mode();

// cuda.go:128-140: O = softmax(scale Q K^T + causal mask) V on flat
// (BH, S, d) float64 data; O is caller-allocated.
void FlashAttnF64(const std::vector<double>& Q, const std::vector<double>& K,
                  const std::vector<double>& V, std::vector<double>& O, int BH, int S, int d,
                  double scale, bool causal);

struct FwdOut {
    std::vector<double> O;  // (BH, S, d)
    std::vector<double> L;  // (BH, S) log-sum-exp, natural log
};
// cuda.go:144-160.
FwdOut FlashAttnF64Fwd(const std::vector<double>& Q, const std::vector<double>& K,
                       const std::vector<double>& V, int BH, int S, int d, double scale,
                       bool causal);

struct BwdOut {
    std::vector<double> dQ, dK, dV;
};
// cuda.go:162-184.
BwdOut FlashAttnF64Bwd(const std::vector<double>& Q, const std::vector<double>& K,
                       const std::vector<double>& V, const std::vector<double>& O,
                       const std::vector<double>& L, const std::vector<double>& dO, int BH,
                       int S, int d, double scale, bool causal);

// cuda.go:188-194: mean milliseconds of `iters` device-resident forwards.
double BenchFlashAttnF64(int BH, int S, int d, int iters, bool causal);

// New (the reference seam is Tq == Tk only): the general fused forward for
// the wider gate, cross-attention (Sq != Sk, top-left causal) and a prefix
// key-padding mask kvLen[B] (empty = none). Q (B*H,Sq,d), K/V (B*H,Sk,d);
// returns O (B*H,Sq,d).
std::vector<double> FlashAttnF64Ex(const std::vector<double>& Q, const std::vector<double>& K,
                                   const std::vector<double>& V, int B, int H, int Sq, int Sk,
                                   int d, double scale, bool causal,
                                   const std::vector<int>& kvLen = {});
// The same forward returning O and L (B*H,Sq), for a backward.
FwdOut FlashAttnF64ExFwd(const std::vector<double>& Q, const std::vector<double>& K,
                         const std::vector<double>& V, int B, int H, int Sq, int Sk, int d,
                         double scale, bool causal, const std::vector<int>& kvLen = {});
// New: forward and backward with an additive mask (WithAttnMask) as well:
// mask is host fp64 read at b*maskSB + h*maskSH + i*Sk + j (rows S apart in
// the backward); empty = none. They run in the current mode.
FwdOut FlashAttnF64Masked(const std::vector<double>& Q, const std::vector<double>& K,
                          const std::vector<double>& V, int B, int H, int Sq, int Sk, int d,
                          double scale, bool causal, const std::vector<int>& kvLen,
                          const std::vector<double>& mask, long maskSB, long maskSH);
// The backward also takes cross-attention: K, V, dK, dV are (B*H,Sk,d).
BwdOut FlashAttnF64BwdMasked(const std::vector<double>& Q, const std::vector<double>& K,
                             const std::vector<double>& V, const std::vector<double>& O,
                             const std::vector<double>& L, const std::vector<double>& dO, int B,
                             int H, int Sq, int Sk, int d, double scale, bool causal,
                             const std::vector<int>& kvLen, const std::vector<double>& mask,
                             long maskSB, long maskSH);
// New: the backward of a square (S x S) forward with key padding kvLen[B]
// (empty = none); O and L from FlashAttnF64ExFwd with the same kvLen.
BwdOut FlashAttnF64BwdEx(const std::vector<double>& Q, const std::vector<double>& K,
                         const std::vector<double>& V, const std::vector<double>& O,
                         const std::vector<double>& L, const std::vector<double>& dO, int B,
                         int H, int S, int d, double scale, bool causal,
                         const std::vector<int>& kvLen = {});

// Device KV cache of one attention layer (gonn_hip_kvcache_*). New: the
// reference has no KV cache. Attend is ForwardMasked with a key-padding mask
// (nn/attention.go:305-341) over each sequence's cached positions; a sequence
// with none gets zeros. Move-only; frees its device memory on destruction.
class KVCache {
  public:
    KVCache(int B, int H, int Lmax, int D);
    ~KVCache();
    KVCache(KVCache&& o) noexcept;
    KVCache& operator=(KVCache&& o) noexcept;
    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;

    // k, v: flat (B,H,T,D) fp64; sequence b takes its first counts[b] rows
    // (all T when counts is empty). Past Lmax: throws Error, nothing written.
    void Append(const std::vector<double>& k, const std::vector<double>& v, int T,
                const std::vector<int>& counts = {});
    // q: flat (B,H,D) fp64 -> o (B,H,D).
    std::vector<double> Attend(const std::vector<double>& q, double scale) const;
    std::vector<int> Lengths() const;
    void Reset();
    // The C handle (gonn_kvcache*), for entries that take the cache.
    void* Handle() const { return h_; }
    int B() const { return B_; }
    int H() const { return H_; }
    int Lmax() const { return Lmax_; }
    int D() const { return D_; }

  private:
    void* h_ = nullptr;
    int B_, H_, Lmax_, D_;
};

// Device-resident multi-head attention (gonn_hip_mha_*): the forward of
// nn.MultiHeadAttention (nn/attention.go:107-148) with the four projections'
// weights in HBM. New: the reference copies across PCIe around every GEMM
// and around the fused core. W* are (E, in) row-major; an empty bias is
// zero. Move-only; frees its device memory on destruction.
class DeviceMHA {
  public:
    DeviceMHA(int E, int H, int kdim, int vdim, const std::vector<double>& Wq,
              const std::vector<double>& bq, const std::vector<double>& Wk,
              const std::vector<double>& bk, const std::vector<double>& Wv,
              const std::vector<double>& bv, const std::vector<double>& Wo,
              const std::vector<double>& bo);
    ~DeviceMHA();
    DeviceMHA(DeviceMHA&& o) noexcept;
    DeviceMHA& operator=(DeviceMHA&& o) noexcept;
    DeviceMHA(const DeviceMHA&) = delete;
    DeviceMHA& operator=(const DeviceMHA&) = delete;

    // q (B,Tq,E), k (B,Tk,kdim), v (B,Tk,vdim) flat fp64 -> (B,Tq,E); kvLen
    // (B entries or empty): keys t >= kvLen[b] are ignored. One upload (once
    // for self-attention, when k and v are q itself) and one download.
    std::vector<double> Forward(const std::vector<double>& q, const std::vector<double>& k,
                                const std::vector<double>& v, int B, int Tq, int Tk, bool causal,
                                const std::vector<int>& kvLen = {}) const;
    // Incremental self-attention over `cache` (gonn_hip_mha_forward_incremental_dev;
    // new, the reference has no KV cache): x flat (B,T,E) fp64, the T new
    // positions of every sequence -> (B,T,E), the last T rows of the causal
    // forward over everything the cache then holds. One upload, one download.
    std::vector<double> ForwardIncremental(const std::vector<double>& x, int B, int T,
                                           KVCache& cache) const;

  private:
    void* h_ = nullptr;
    int E_, H_, kdim_, vdim_;
};

}  // namespace hip

namespace backend {

// backend/backend.go:61-78: row-major batched C = op(A) op(B) of `batch`
// contiguous matrix pairs; op(A) is (m,k) (stored (k,m) when transA), op(B)
// (k,n) (stored (n,k) when transB); returns the batch*m*n result.
class Backend {
public:
    virtual ~Backend() = default;
    virtual std::string Name() const = 0;
    virtual std::vector<double> Gemm(const std::vector<double>& a, const std::vector<double>& b,
                                     int batch, int m, int k, int n, bool transA,
                                     bool transB) const = 0;
    virtual void Synchronize() const = 0;
};

// backend.UnaryKind / BinaryKind (backend/backend.go:26-58); the values are
// the C ABI's GONN_UN_* / GONN_BIN_*.
enum UnaryKind : int {
    UnaryNone = -1,
    UnaryReLU = 0,
    UnarySigmoid,
    UnaryTanh,
    UnaryExp,
    UnaryLog,
    UnaryGELU,
    UnarySiLU,
    UnaryGELUExact
};
enum BinaryKind : int { BinaryAdd = 0, BinarySub, BinaryMul, BinaryDiv };

// Optional capability (backend.go:80-92): write out and return true, or
// return false to decline (the caller runs its own loop). The HIP backend
// declines only kinds it has no kernel for; a device error throws
// gonn::hip::Error instead of falling back. The CPU backend does not
// implement it (backend_test.go:117-126).
class Elementwiser {
public:
    virtual ~Elementwiser() = default;
    virtual bool Unary(UnaryKind kind, const std::vector<double>& a,
                       std::vector<double>& out) const = 0;
    virtual bool Binary(BinaryKind kind, const std::vector<double>& a,
                        const std::vector<double>& b, std::vector<double>& out) const = 0;
};

// The host loop backend (backend/cpu.go), the default.
std::shared_ptr<Backend> NewCPU();
// The device GEMM (gonn_hip_gemm_f64). Throws gonn::hip::Error with
// GONN_E_NODEVICE when no gfx950 device is present; a failed device GEMM
// throws gonn::hip::Error (cuda.go:62-64 panics).
std::shared_ptr<Backend> NewHIP();
// Swap the process-wide backend and return the previous one (backend.go:108-118).
// Safe for concurrent use.
std::shared_ptr<Backend> Use(std::shared_ptr<Backend> b);
std::shared_ptr<Backend> Current();

}  // namespace backend

namespace nn {

// Host float64 tensor, row-major (tensor/tensor.go:22-23).
struct Tensor {
    std::vector<double> Data;
    std::vector<int> Shape;

    static Tensor New(std::vector<double> data, std::vector<int> shape);
    static Tensor Zeros(std::vector<int> shape);
    size_t Numel() const;
    // Reshape keeps the data (tensor/ops_shape.go:5-51).
    Tensor Reshape(std::vector<int> shape) const;
    // Permute(0, 2, 1, 3) of a 4-D tensor, materialised as a copy the way
    // tensor/ops_shape.go:64-107 does.
    Tensor Permute0213() const;
};

// y = x W^T + b (nn/linear.go:40-59); W is (out, in), b (out) or empty. The
// product runs on backend::Current(), as tensor.MatMul dispatches its GEMM
// (tensor/dispatch.go:111-113).
struct Linear {
    Tensor W;
    std::vector<double> B;
    Tensor Forward(const Tensor& x) const;
};

bool fusedAttnAvailable();
bool fusedAttnSupports(int D, int Tq, int Tk);
// nn/flashattn_cuda.go:17-21.
std::vector<double> fusedAttnF64(const std::vector<double>& Q, const std::vector<double>& K,
                                 const std::vector<double>& V, int BH, int S, int D,
                                 double scale, bool causal);

// What nn/flashattn_cuda.go:26-38 returns: the output tensor and the custom
// autograd node tensor.MakeNode(out, "FlashAttn", ...) attaches to it. The
// node keeps the inputs, O and L, and maps the upstream gradient to
// (dQ, dK, dV) with the device backward.
struct FlashAttnNode {
    std::string Op = "FlashAttn";
    std::function<std::array<Tensor, 3>(const Tensor& grad)> Backward;
};
struct DiffOut {
    Tensor Out;
    FlashAttnNode Node;
};
// kvLen (new, BH / H entries or empty): the key padding of ForwardMasked;
// attnMask (new, empty = none): its additive mask in one of expandAttnMask's
// shapes for B = BH / H; Sk (new, 0 = S): key rows of kp and vp for
// cross-attention (top-left causal mask); all in the forward and in the
// node's backward.
DiffOut fusedAttnDiff(const Tensor& qp, const Tensor& kp, const Tensor& vp, int BH, int S, int D,
                      double scale, bool causal, const std::vector<int>& kvLen = {}, int H = 1,
                      const Tensor& attnMask = Tensor{}, int Sk = 0);

// expandAttnMask (nn/attention.go:242-257): the (sequence, head) element
// strides of an additive mask of shape (Tq,Tk), (B*H,Tq,Tk), (B,Tq,Tk) or
// (B,H,Tq,Tk); throws std::invalid_argument with the reference's message
// for any other shape.
std::array<long, 2> maskStrides(const std::vector<int>& shape, int B, int H, int Tq, int Tk);

// nn.MultiHeadAttention with the fused core (nn/attention.go:38-180).
// Weights are given explicitly: GoNN draws them from Go's math/rand stream
// (nn/linear.go:20-36).
class MultiHeadAttention {
  public:
    int EmbedDim, NumHeads, HeadDim, KDim, VDim;
    Linear QProj, KProj, VProj, OutProj;

    MultiHeadAttention(int embedDim, int numHeads, Linear q, Linear k, Linear v, Linear out);

    // Forward (nn/attention.go:107-148) through the differentiable fused core,
    // Tq != Tk included (cross-attention); the node of the last call is kept
    // in LastNode for a backward pass.
    Tensor Forward(const Tensor& q, const Tensor& k, const Tensor& v, bool causal);
    // ForwardFused (nn/attention.go:159-180): inference core, no node. Also
    // takes Tq != Tk (cross-attention), which the reference's gate sends to
    // its CPU path.
    Tensor ForwardFused(const Tensor& q, const Tensor& k, const Tensor& v, bool causal);
    // ForwardMasked (nn/attention.go:305-341) on the fused core with causal,
    // a (B, Tk) key-padding mask (nonzero = ignore; suffix-form masks run as
    // per-sequence key counts, others are added as -1e30) and an additive
    // attnMask in any of expandAttnMask's shapes, in the current mode. Empty
    // tensors mean none. A query row with no unblocked key throws
    // std::invalid_argument (GoNN gives it a uniform average; the fused core
    // does not define it). Inference; the differentiable form is
    // fusedAttnDiff with kvLen and attnMask.
    Tensor ForwardMasked(const Tensor& q, const Tensor& k, const Tensor& v, bool causal,
                         const Tensor& keyPad, const Tensor& attnMask = Tensor{});

    FlashAttnNode LastNode;

    // Incremental decoding (new: the reference has no KV cache). A cache of
    // `batch` sequences and `maxLen` positions for this layer.
    hip::KVCache NewCache(int batch, int maxLen) const;
    // Causal self-attention of new tokens x (B, T, E) over the cached tokens
    // plus themselves, one position at a time; row t equals row (cached + t)
    // of Forward(seq, seq, seq, causal=true) over the whole sequence.
    Tensor ForwardIncremental(const Tensor& x, hip::KVCache& cache);

    // This layer with its weights uploaded once (new): Forward / ForwardMasked
    // of the result run projections, core and output projection on the
    // device with one upload and one download per call.
    class ResidentMultiHeadAttention ToDevice() const;

  private:
    friend class ResidentMultiHeadAttention;
    void checkQKVDims(const Tensor& q, const Tensor& k, const Tensor& v) const;
    void requireFused(int D, int Tq, int Tk) const;
    Tensor fusedGeneral(const Tensor& q, const Tensor& k, const Tensor& v, bool causal,
                        const std::vector<int>& kvLen, const Tensor& attnMask = Tensor{});
};

// MultiHeadAttention::Forward / ForwardMasked on a hip::DeviceMHA; the same
// shape checks and mask rules as the host-projection path.
class ResidentMultiHeadAttention {
  public:
    explicit ResidentMultiHeadAttention(const MultiHeadAttention& m);
    Tensor Forward(const Tensor& q, const Tensor& k, const Tensor& v, bool causal) const;
    Tensor ForwardMasked(const Tensor& q, const Tensor& k, const Tensor& v, bool causal,
                         const Tensor& keyPad) const;
    // A KV cache for ForwardIncremental: heads at the padded head dim (64 or 128).
    hip::KVCache NewCache(int batch, int maxLen) const;
    // MultiHeadAttention::ForwardIncremental on the device: the T new
    // positions are projected, appended and attended in one device pass
    // (one host synchronisation per call, none per position).
    Tensor ForwardIncremental(const Tensor& x, hip::KVCache& cache) const;

  private:
    MultiHeadAttention layer_;
    hip::DeviceMHA dev_;
};

}  // namespace nn
}  // namespace gonn
