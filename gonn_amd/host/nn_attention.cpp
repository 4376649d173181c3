// nn_attention.cpp -- gonn::nn: the fused attention seam and the fused branch
// of MultiHeadAttention, mirroring nn/flashattn_cuda.go:13-38 and
// nn/attention.go:83-180 over gonn::hip.
#include <algorithm>
#include <cmath>
#include <memory>
#include <string>
#include <utility>

#include "gonn_host.hpp"

namespace gonn {
namespace nn {

namespace {

std::string shape_str(const std::vector<int>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) r += (i ? " " : "") + std::to_string(s[i]);
    return r + "]";
}

size_t prod(const std::vector<int>& s) {
    size_t n = 1;
    for (int x : s) {
        if (x < 0) throw std::invalid_argument("tensor: negative dimension");
        n *= (size_t)x;
    }
    return n;
}

}  // namespace

Tensor Tensor::New(std::vector<double> data, std::vector<int> shape) {
    if (data.size() != prod(shape))
        throw std::invalid_argument("tensor.New: data length " + std::to_string(data.size()) +
                                    " does not match shape " + shape_str(shape));
    Tensor t;
    t.Data = std::move(data);
    t.Shape = std::move(shape);
    return t;
}

Tensor Tensor::Zeros(std::vector<int> shape) {
    const size_t n = prod(shape);
    return New(std::vector<double>(n, 0.0), std::move(shape));
}

size_t Tensor::Numel() const { return Data.size(); }

Tensor Tensor::Reshape(std::vector<int> shape) const {
    if (prod(shape) != Data.size())
        throw std::invalid_argument("Reshape: cannot reshape " + shape_str(Shape) + " to " +
                                    shape_str(shape));
    return New(Data, std::move(shape));
}

Tensor Tensor::Permute0213() const {
    if (Shape.size() != 4) throw std::invalid_argument("Permute: need a 4-D tensor");
    const int A = Shape[0], B = Shape[1], C = Shape[2], D = Shape[3];
    std::vector<double> out(Data.size());
    for (int a = 0; a < A; a++)
        for (int b = 0; b < B; b++)
            for (int c = 0; c < C; c++) {
                const double* src = &Data[(((size_t)a * B + b) * C + c) * D];
                double* dst = &out[(((size_t)a * C + c) * B + b) * D];
                for (int d = 0; d < D; d++) dst[d] = src[d];
            }
    return New(std::move(out), {A, C, B, D});
}

Tensor Linear::Forward(const Tensor& x) const {
    if (W.Shape.size() != 2) throw std::invalid_argument("Linear: W must be (out, in)");
    const int out = W.Shape[0], in = W.Shape[1];
    if (x.Shape.empty() || x.Shape.back() != in)
        throw std::invalid_argument("Linear: input shape " + shape_str(x.Shape) +
                                    ", want (..., " + std::to_string(in) + ")");
    if (!B.empty() && (int)B.size() != out) throw std::invalid_argument("Linear: bias length");
    const size_t N = x.Numel() / (size_t)in;
    // x (N, in) @ W^T: op(B) is W stored (out, in), so transB.
    std::vector<double> y = backend::Current()->Gemm(x.Data, W.Data, 1, (int)N, in, out, false, true);
    if (!B.empty())
        for (size_t n = 0; n < N; n++)
            for (int o = 0; o < out; o++) y[n * out + o] += B[o];
    std::vector<int> shape = x.Shape;
    shape.back() = out;
    return Tensor::New(std::move(y), std::move(shape));
}

bool fusedAttnAvailable() { return hip::Available(); }

bool fusedAttnSupports(int D, int Tq, int Tk) { return hip::Supports(D, Tq, Tk); }

std::vector<double> fusedAttnF64(const std::vector<double>& Q, const std::vector<double>& K,
                                 const std::vector<double>& V, int BH, int S, int D,
                                 double scale, bool causal) {
    std::vector<double> O(Q.size(), 0.0);
    hip::FlashAttnF64(Q, K, V, O, BH, S, D, scale, causal);
    return O;
}

DiffOut fusedAttnDiff(const Tensor& qp, const Tensor& kp, const Tensor& vp, int BH, int S, int D,
                      double scale, bool causal, const std::vector<int>& kvLen, int H,
                      const Tensor& attnMask, int Sk) {
    if (H <= 0 || BH % H != 0) throw std::invalid_argument("fusedAttnDiff: BH must be a multiple of H");
    if (Sk <= 0) Sk = S;
    const bool masked = !attnMask.Data.empty();
    // The reference seam's entry points (square, no mask, no padding), else
    // the general ones of the wider gate.
    const bool plain = !masked && kvLen.empty() && Sk == S;
    std::array<long, 2> st{0, 0};
    if (masked) st = maskStrides(attnMask.Shape, BH / H, H, S, Sk);
    auto mask = std::make_shared<std::vector<double>>(attnMask.Data);
    hip::FwdOut f = plain ? hip::FlashAttnF64Fwd(qp.Data, kp.Data, vp.Data, BH, S, D, scale, causal)
                          : hip::FlashAttnF64Masked(qp.Data, kp.Data, vp.Data, BH / H, H, S, Sk, D,
                                                    scale, causal, kvLen, *mask, st[0], st[1]);
    DiffOut r;
    r.Out = Tensor::New(f.O, qp.Shape);
    // The node's closure holds the inputs and the saved O and L, as the Go
    // closure captures them (nn/flashattn_cuda.go:29-37).
    auto saved = std::make_shared<std::array<Tensor, 3>>(std::array<Tensor, 3>{qp, kp, vp});
    auto O = std::make_shared<std::vector<double>>(std::move(f.O));
    auto L = std::make_shared<std::vector<double>>(std::move(f.L));
    r.Node.Backward = [saved, O, L, BH, S, Sk, D, scale, causal, kvLen, H, plain, mask,
                       st](const Tensor& grad) {
        const Tensor &q = (*saved)[0], &k = (*saved)[1], &v = (*saved)[2];
        hip::BwdOut b =
            plain ? hip::FlashAttnF64Bwd(q.Data, k.Data, v.Data, *O, *L, grad.Data, BH, S, D, scale,
                                         causal)
                  : hip::FlashAttnF64BwdMasked(q.Data, k.Data, v.Data, *O, *L, grad.Data, BH / H, H,
                                               S, Sk, D, scale, causal, kvLen, *mask, st[0], st[1]);
        return std::array<Tensor, 3>{Tensor::New(std::move(b.dQ), q.Shape),
                                     Tensor::New(std::move(b.dK), k.Shape),
                                     Tensor::New(std::move(b.dV), v.Shape)};
    };
    return r;
}

MultiHeadAttention::MultiHeadAttention(int embedDim, int numHeads, Linear q, Linear k, Linear v,
                                       Linear out)
    : EmbedDim(embedDim), NumHeads(numHeads), HeadDim(0), KDim(0), VDim(0),
      QProj(std::move(q)), KProj(std::move(k)), VProj(std::move(v)), OutProj(std::move(out)) {
    // nn/attention.go:45-58
    if (numHeads <= 0 || embedDim % numHeads != 0)
        throw std::invalid_argument("MultiHeadAttention: embedDim must be divisible by numHeads");
    HeadDim = embedDim / numHeads;
    KDim = KProj.W.Shape.size() == 2 ? KProj.W.Shape[1] : 0;
    VDim = VProj.W.Shape.size() == 2 ? VProj.W.Shape[1] : 0;
}

// nn/attention.go:83-103
void MultiHeadAttention::checkQKVDims(const Tensor& q, const Tensor& k, const Tensor& v) const {
    const int kd = KDim ? KDim : EmbedDim, vd = VDim ? VDim : EmbedDim;
    if (q.Shape.size() != 3 || q.Shape[2] != EmbedDim)
        throw std::invalid_argument("MultiHeadAttention: q shape " + shape_str(q.Shape) +
                                    ", want (B, Tq, " + std::to_string(EmbedDim) + ")");
    if (k.Shape.size() != 3 || k.Shape[2] != kd)
        throw std::invalid_argument("MultiHeadAttention: k shape " + shape_str(k.Shape) +
                                    ", want (B, Tk, kdim=" + std::to_string(kd) + ")");
    if (v.Shape.size() != 3 || v.Shape[2] != vd)
        throw std::invalid_argument("MultiHeadAttention: v shape " + shape_str(v.Shape) +
                                    ", want (B, Tk, vdim=" + std::to_string(vd) + ")");
    if (k.Shape[1] != v.Shape[1])
        throw std::invalid_argument("MultiHeadAttention: k and v sequence lengths differ (" +
                                    std::to_string(k.Shape[1]) + " vs " +
                                    std::to_string(v.Shape[1]) + ")");
}

// The reference takes its CPU core when the gate at nn/attention.go:129 is
// false; this library has no CPU attention core, so the gate failing is an
// error here.
void MultiHeadAttention::requireFused(int D, int Tq, int Tk) const {
    if (!fusedAttnAvailable())
        throw hip::Error(-5, "nn: fused attention needs libgonn_hip.so and a gfx950 device");
    if (!fusedAttnSupports(D, Tq, Tk))
        throw std::invalid_argument("nn: the fused core needs D in {64, 128}, got D=" +
                                    std::to_string(D) + " Tq=" + std::to_string(Tq) +
                                    " Tk=" + std::to_string(Tk));
}

Tensor MultiHeadAttention::Forward(const Tensor& q, const Tensor& k, const Tensor& v,
                                   bool causal) {
    checkQKVDims(q, k, v);
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1], H = NumHeads, D = HeadDim;
    requireFused(D, Tq, Tk);
    // project; (B, T, H, D) -> (B, H, T, D)   nn/attention.go:115-122
    const Tensor qp = QProj.Forward(q).Reshape({B, Tq, H, D}).Permute0213();
    const Tensor kp = KProj.Forward(k).Reshape({B, Tk, H, D}).Permute0213();
    const Tensor vp = VProj.Forward(v).Reshape({B, Tk, H, D}).Permute0213();
    const double scale = 1.0 / std::sqrt((double)D);
    // Cross-attention (Tq != Tk, TransformerDecoderLayer's Forward(x, memory,
    // memory, false), nn/transformer.go:234) takes the same differentiable
    // node with Tk key rows.
    DiffOut f = fusedAttnDiff(qp, kp, vp, B * H, Tq, D, scale, causal, {}, H, Tensor{}, Tk);
    LastNode = f.Node;
    const Tensor ctx = f.Out.Permute0213().Reshape({B, Tq, EmbedDim});  // :130-131
    return OutProj.Forward(ctx);                                         // :132
}

std::array<long, 2> maskStrides(const std::vector<int>& s, int B, int H, int Tq, int Tk) {
    const long qk = (long)Tq * Tk;
    if (s.size() == 2 && s[0] == Tq && s[1] == Tk) return {0, 0};
    if (s.size() == 3 && s[0] == B * H && s[1] == Tq && s[2] == Tk) return {H * qk, qk};
    if (s.size() == 3 && s[0] == B && s[1] == Tq && s[2] == Tk) return {qk, 0};
    if (s.size() == 4 && s[0] == B && s[1] == H && s[2] == Tq && s[3] == Tk) return {H * qk, qk};
    throw std::invalid_argument("MultiHeadAttention: attn mask shape " + shape_str(s) +
                                " incompatible with (Tq,Tk)=(" + std::to_string(Tq) + "," +
                                std::to_string(Tk) + "), (B,Tq,Tk) B=" + std::to_string(B) +
                                ", (B*H,Tq,Tk) B*H=" + std::to_string(B * H) +
                                ", or (B,H,Tq,Tk)");
}

Tensor MultiHeadAttention::fusedGeneral(const Tensor& q, const Tensor& k, const Tensor& v,
                                        bool causal, const std::vector<int>& kvLen,
                                        const Tensor& attnMask) {
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1], H = NumHeads, D = HeadDim;
    if (!fusedAttnAvailable())
        throw hip::Error(-5, "nn: fused attention needs libgonn_hip.so and a gfx950 device");
    if (!fusedAttnSupports(D, Tq, Tk))
        throw std::invalid_argument("nn: the fused core needs D in {64, 128}, got D=" +
                                    std::to_string(D));
    const Tensor qp = QProj.Forward(q).Reshape({B, Tq, H, D}).Permute0213();
    const Tensor kp = KProj.Forward(k).Reshape({B, Tk, H, D}).Permute0213();
    const Tensor vp = VProj.Forward(v).Reshape({B, Tk, H, D}).Permute0213();
    const double scale = 1.0 / std::sqrt((double)D);
    std::vector<double> O;
    if (attnMask.Data.empty()) {
        O = hip::FlashAttnF64Ex(qp.Data, kp.Data, vp.Data, B, H, Tq, Tk, D, scale, causal, kvLen);
    } else {
        const auto st = maskStrides(attnMask.Shape, B, H, Tq, Tk);
        O = hip::FlashAttnF64Masked(qp.Data, kp.Data, vp.Data, B, H, Tq, Tk, D, scale, causal,
                                    kvLen, attnMask.Data, st[0], st[1])
                .O;
    }
    const Tensor ctx = Tensor::New(std::move(O), {B, H, Tq, D}).Permute0213().Reshape({B, Tq, EmbedDim});
    return OutProj.Forward(ctx);
}

// A query row whose best in-window additive mask value is at or below
// kNoKeyLevel has no unblocked key. GoNN adds its masks as fp64 -1e30
// constants (nn/attention.go:185-196, :261-272), which absorb the scores, so
// such a row is a uniform average over the keys whose summed mask is the
// row's maximum, future keys included (their causal -1e30). The fused core
// reproduces it when that maximum is at or below kUniformLevel: the scores
// vanish next to it in fp32 as in fp64, so the row is passed unshifted. A
// blocked row between the two levels (fp64 keeps part of the score there,
// fp32 does not) or of -inf keys only (NaN in GoNN) is refused.
constexpr double kNoKeyLevel = -1e15;
constexpr double kUniformLevel = -1e25;
static const char* kNoKeyMsg =
    "nn: a query row has no unblocked key (every key it may attend is padded or masked); "
    "the fused core does not define such rows";
static const char* kBlockedMsg =
    "nn: a query row has no unblocked key and its best mask value lies between -1e25 and "
    "-1e15 (or is -inf); the fused core does not define such rows";

// keyPaddingMaskAdd's shape check (nn/attention.go:262-264) and the mask's
// form: kvLen (B entries) when every row's padded keys (nonzero = ignore) are
// a suffix that leaves a key, else kpAdd, the (B, Tk) 0 / -1e30 values
// GoNN adds. Both empty for no mask.
static void key_padding(const Tensor& keyPad, int B, int Tk, std::vector<int>& kvLen,
                        std::vector<double>& kpAdd) {
    kvLen.clear();
    kpAdd.clear();
    if (keyPad.Data.empty()) return;
    if (keyPad.Shape.size() != 2 || keyPad.Shape[0] != B || keyPad.Shape[1] != Tk)
        throw std::invalid_argument("MultiHeadAttention: key padding mask shape " +
                                    shape_str(keyPad.Shape) + ", want (B, Tk) = (" +
                                    std::to_string(B) + ", " + std::to_string(Tk) + ")");
    bool suffix = true;
    kvLen.assign(B, Tk);
    for (int b = 0; b < B && suffix; b++) {
        const double* row = &keyPad.Data[(size_t)b * Tk];
        int n = 0;
        while (n < Tk && row[n] == 0) n++;
        for (int t = n; t < Tk; t++)
            if (row[t] == 0) suffix = false;
        if (n == 0) suffix = false;
        kvLen[b] = n;
    }
    if (suffix) return;
    kvLen.clear();
    kpAdd.assign(keyPad.Data.size(), 0.0);
    for (size_t i = 0; i < kpAdd.size(); i++)
        if (keyPad.Data[i] != 0) kpAdd[i] = -1e30;
}

// kvLen of a suffix-form key-padding mask whose rows keep a key (the
// resident layer takes no other).
static std::vector<int> kv_len_from_mask(const Tensor& keyPad, int B, int Tk) {
    std::vector<int> kvLen;
    std::vector<double> kpAdd;
    key_padding(keyPad, B, Tk, kvLen, kpAdd);
    if (!kpAdd.empty()) {
        for (int b = 0; b < B; b++) {
            bool any = false;
            for (int t = 0; t < Tk; t++) any |= keyPad.Data[(size_t)b * Tk + t] == 0;
            if (!any) throw std::invalid_argument(kNoKeyMsg);
        }
        throw std::invalid_argument(
            "nn: this path takes key padding masks whose padded keys are a suffix of the row");
    }
    return kvLen;
}

// ForwardMasked's masks (nn/attention.go:318-330) in the form the fused core
// takes them. A suffix-form padding mask becomes kvLen (the kernels skip the
// padded keys); any other is added as keyPaddingMaskAdd's -1e30. Each row of
// the additive mask is shifted by its maximum over the keys the row attends
// (causal window, kvLen): softmax is unchanged, and the fp32 scores the
// kernels form keep full precision under a large common offset.
//
// When some row has no unblocked key, the call takes the whole-row form: the
// causal mask and the key padding become GoNN's -1e30 terms, added in its
// order (causal, attn mask, key padding) over every key; `causal` is cleared
// and kvLen emptied; rows with an unblocked key are shifted by their maximum
// and blocked rows stay as they are (kUniformLevel). Blocked rows the core
// cannot reproduce throw.
static void core_masks(const Tensor& keyPad, const Tensor& attnMask, int B, int H, int Tq,
                       int Tk, bool& causal, std::vector<int>& kvLen, Tensor& mask) {
    std::vector<double> kpAdd;
    key_padding(keyPad, B, Tk, kvLen, kpAdd);
    mask = Tensor{};
    if (attnMask.Data.empty() && kpAdd.empty()) return;  // a suffix kvLen leaves every row a key
    int Bu = 1, Hu = 1;
    if (!attnMask.Data.empty()) {
        const auto st = maskStrides(attnMask.Shape, B, H, Tq, Tk);  // expandAttnMask's check
        Bu = st[0] ? B : 1;
        Hu = st[1] ? H : 1;
    }
    const size_t QK = (size_t)Tq * Tk;
    auto user = [&](int b, int h, int i) {
        return attnMask.Data.empty()
                   ? nullptr
                   : &attnMask.Data[((size_t)(b % Bu) * Hu + h) * QK + (size_t)i * Tk];
    };
    std::vector<double> full((size_t)B * Hu * QK);
    bool shifted = !kpAdd.empty(), blocked = false;
    for (int b = 0; b < B && !blocked; b++)
        for (int h = 0; h < Hu && !blocked; h++)
            for (int i = 0; i < Tq; i++) {
                const double* src = user(b, h, i);
                double* dst = &full[((size_t)b * Hu + h) * QK + (size_t)i * Tk];
                for (int j = 0; j < Tk; j++)
                    dst[j] = (src ? src[j] : 0.0) + (kpAdd.empty() ? 0.0 : kpAdd[(size_t)b * Tk + j]);
                int n = kvLen.empty() ? Tk : kvLen[b];
                if (causal && i + 1 < n) n = i + 1;
                double mx = -INFINITY;
                for (int j = 0; j < n; j++) mx = std::max(mx, dst[j]);
                if (!(mx > kNoKeyLevel)) {
                    blocked = true;
                    break;
                }
                if (mx != 0) {
                    shifted = true;
                    for (int j = 0; j < Tk; j++) dst[j] -= mx;
                }
            }
    if (!blocked) {
        if (!shifted) {
            mask = attnMask;
            return;
        }
        mask = Hu == 1 ? Tensor::New(std::move(full), {B, Tq, Tk})
                       : Tensor::New(std::move(full), {B, H, Tq, Tk});
        return;
    }
    // whole-row form, in GoNN's order of additions
    for (int b = 0; b < B; b++)
        for (int h = 0; h < Hu; h++)
            for (int i = 0; i < Tq; i++) {
                const double* src = user(b, h, i);
                double* dst = &full[((size_t)b * Hu + h) * QK + (size_t)i * Tk];
                for (int j = 0; j < Tk; j++) {
                    double x = 0.0;
                    if (causal) x = x + (j > i ? -1e30 : 0.0);
                    x = x + (src ? src[j] : 0.0);
                    if (!kvLen.empty()) x = x + (j >= kvLen[b] ? -1e30 : 0.0);
                    if (!kpAdd.empty()) x = x + kpAdd[(size_t)b * Tk + j];
                    dst[j] = x;
                }
                double mx = -INFINITY;
                for (int j = 0; j < Tk; j++) mx = std::max(mx, dst[j]);
                if (mx > kNoKeyLevel) {
                    for (int j = 0; j < Tk; j++) dst[j] -= mx;
                } else if (!(mx <= kUniformLevel && mx > -INFINITY)) {
                    throw std::invalid_argument(kBlockedMsg);
                }
            }
    causal = false;
    kvLen.clear();
    mask = Hu == 1 ? Tensor::New(std::move(full), {B, Tq, Tk})
                   : Tensor::New(std::move(full), {B, H, Tq, Tk});
}

Tensor MultiHeadAttention::ForwardMasked(const Tensor& q, const Tensor& k, const Tensor& v,
                                         bool causal, const Tensor& keyPad,
                                         const Tensor& attnMask) {
    checkQKVDims(q, k, v);
    const int B = q.Shape[0], Tk = k.Shape[1];
    std::vector<int> kvLen;
    Tensor mask;
    core_masks(keyPad, attnMask, B, NumHeads, q.Shape[1], Tk, causal, kvLen, mask);
    return fusedGeneral(q, k, v, causal, kvLen, mask);
}

Tensor MultiHeadAttention::ForwardFused(const Tensor& q, const Tensor& k, const Tensor& v,
                                        bool causal) {
    checkQKVDims(q, k, v);
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1], H = NumHeads, D = HeadDim;
    if (Tq != Tk) return fusedGeneral(q, k, v, causal, {});
    requireFused(D, Tq, Tk);
    const Tensor qp = QProj.Forward(q).Reshape({B, Tq, H, D}).Permute0213();
    const Tensor kp = KProj.Forward(k).Reshape({B, Tk, H, D}).Permute0213();
    const Tensor vp = VProj.Forward(v).Reshape({B, Tk, H, D}).Permute0213();
    const double scale = 1.0 / std::sqrt((double)D);
    std::vector<double> O = fusedAttnF64(qp.Data, kp.Data, vp.Data, B * H, Tq, D, scale, causal);
    const Tensor ctx = Tensor::New(std::move(O), {B, H, Tq, D}).Permute0213().Reshape({B, Tq, EmbedDim});
    return OutProj.Forward(ctx);
}

hip::KVCache MultiHeadAttention::NewCache(int batch, int maxLen) const {
    return hip::KVCache(batch, NumHeads, maxLen, HeadDim);
}

Tensor MultiHeadAttention::ForwardIncremental(const Tensor& x, hip::KVCache& cache) {
    if (x.Shape.size() != 3 || x.Shape[2] != EmbedDim)
        throw std::invalid_argument("MultiHeadAttention: x shape " + shape_str(x.Shape) +
                                    ", want (B, T, " + std::to_string(EmbedDim) + ")");
    const int B = x.Shape[0], T = x.Shape[1], H = NumHeads, D = HeadDim;
    if (cache.B() != B || cache.H() != H || cache.D() != D)
        throw std::invalid_argument("MultiHeadAttention: cache shape does not match (B, H, D)");
    // project all new tokens, (B, T, H, D) -> (B, H, T, D)
    const Tensor qp = QProj.Forward(x).Reshape({B, T, H, D}).Permute0213();
    const Tensor kp = KProj.Forward(x).Reshape({B, T, H, D}).Permute0213();
    const Tensor vp = VProj.Forward(x).Reshape({B, T, H, D}).Permute0213();
    const double scale = 1.0 / std::sqrt((double)D);
    std::vector<double> ctx((size_t)B * H * T * D);
    std::vector<double> kt((size_t)B * H * D), vt(kt.size()), qt(kt.size());
    for (int t = 0; t < T; t++) {
        for (size_t bh = 0; bh < (size_t)B * H; bh++)
            for (int d = 0; d < D; d++) {
                const size_t src = (bh * T + t) * D + d;
                kt[bh * D + d] = kp.Data[src];
                vt[bh * D + d] = vp.Data[src];
                qt[bh * D + d] = qp.Data[src];
            }
        cache.Append(kt, vt, 1);
        const std::vector<double> o = cache.Attend(qt, scale);
        for (size_t bh = 0; bh < (size_t)B * H; bh++)
            for (int d = 0; d < D; d++) ctx[(bh * T + t) * D + d] = o[bh * D + d];
    }
    const Tensor merged = Tensor::New(std::move(ctx), {B, H, T, D}).Permute0213().Reshape({B, T, EmbedDim});
    return OutProj.Forward(merged);
}

ResidentMultiHeadAttention MultiHeadAttention::ToDevice() const {
    return ResidentMultiHeadAttention(*this);
}

ResidentMultiHeadAttention::ResidentMultiHeadAttention(const MultiHeadAttention& m)
    : layer_(m),
      dev_(m.EmbedDim, m.NumHeads, m.KDim, m.VDim, m.QProj.W.Data, m.QProj.B, m.KProj.W.Data,
           m.KProj.B, m.VProj.W.Data, m.VProj.B, m.OutProj.W.Data, m.OutProj.B) {}

Tensor ResidentMultiHeadAttention::Forward(const Tensor& q, const Tensor& k, const Tensor& v,
                                           bool causal) const {
    layer_.checkQKVDims(q, k, v);
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1];
    const std::vector<double>& kd = &k == &q ? q.Data : k.Data;
    const std::vector<double>& vd = &v == &k ? kd : v.Data;
    return Tensor::New(dev_.Forward(q.Data, kd, vd, B, Tq, Tk, causal), {B, Tq, layer_.EmbedDim});
}

Tensor ResidentMultiHeadAttention::ForwardMasked(const Tensor& q, const Tensor& k,
                                                 const Tensor& v, bool causal,
                                                 const Tensor& keyPad) const {
    layer_.checkQKVDims(q, k, v);
    const int B = q.Shape[0], Tq = q.Shape[1], Tk = k.Shape[1];
    const std::vector<int> kvLen = kv_len_from_mask(keyPad, B, Tk);
    const std::vector<double>& kd = &k == &q ? q.Data : k.Data;
    const std::vector<double>& vd = &v == &k ? kd : v.Data;
    return Tensor::New(dev_.Forward(q.Data, kd, vd, B, Tq, Tk, causal, kvLen),
                       {B, Tq, layer_.EmbedDim});
}

hip::KVCache ResidentMultiHeadAttention::NewCache(int batch, int maxLen) const {
    return hip::KVCache(batch, layer_.NumHeads, maxLen, layer_.HeadDim <= 64 ? 64 : 128);
}

Tensor ResidentMultiHeadAttention::ForwardIncremental(const Tensor& x, hip::KVCache& cache) const {
    if (x.Shape.size() != 3 || x.Shape[2] != layer_.EmbedDim)
        throw std::invalid_argument("MultiHeadAttention: x shape " + shape_str(x.Shape) +
                                    ", want (B, T, " + std::to_string(layer_.EmbedDim) + ")");
    const int B = x.Shape[0], T = x.Shape[1];
    return Tensor::New(dev_.ForwardIncremental(x.Data, B, T, cache), {B, T, layer_.EmbedDim});
}

}  // namespace nn
}  // namespace gonn
