// int8_ext.cpp — PyTorch binding `int8_ext` over the libint8k C ABI.
//
// Drop-in for the reference's pybind11 module of the same name
// (kernels/int8_ext.cu:458-479): same op names, positional signatures,
// overloads, return types and argument checks (TORCH_CHECK -> RuntimeError).
// Differences a caller can observe are deliberate and listed where they occur:
// launches go to torch's current HIP stream (the reference used the legacy
// default stream), workspaces come from torch's caching allocator, and the
// library holds no global scratch.
//
// This file is plain C++: it includes only torch's HIP stream/guard headers and
// int8k.h, and calls the C ABI; no kernel code lives here.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/hip/HIPGuard.h>

#include <cstdint>
#include <string>
#include <tuple>

#include "int8k.h"

namespace {

void* current_stream(const torch::Tensor& t) {
    return reinterpret_cast<void*>(
        c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

void check_status(int st, const char* op) {
    if (st == INT8K_OK) return;
    const char* detail = int8k_last_error();
    TORCH_CHECK(false, op, " failed: ", int8k_status_string(st),
                (detail && detail[0]) ? std::string(" — ") + detail : std::string());
}

torch::Tensor workspace(size_t bytes, const torch::Device& dev) {
    return torch::empty({(int64_t)std::max<size_t>(bytes, 1)},
                        torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

bool aligned16(const torch::Tensor& t) {
    return (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0;
}

// The kernels load 16-byte vectors; a view whose storage offset breaks that
// alignment is copied to a fresh (aligned) allocation instead of failing.
torch::Tensor aligned_i8(const torch::Tensor& t) {
    return aligned16(t) ? t : t.clone();
}

}  // namespace

// ── prefill attention (seq_q == seq_kv) ───────────────────────────────────
// Mirrors int8_attention_forward_torch (kernels/int8_ext.cu:83-129): Q/K/V int8
// (batch, heads, seq_len, head_dim), all the same shape; per-token fp32 scales
// with batch*heads*seq_len elements; returns fp16 of Q's shape.  `is_causal`
// is a new optional trailing argument (default false = the reference's math).
// With `quant` the output is the per-token int8 of those fp16 rows: {int8 of
// Q's shape, fp32 scales (batch, heads, seq_len)}.  With `out_bshd` the rows
// come out in (batch, seq_len, heads, ...) order instead, the layout the
// output projection reads.
static std::vector<torch::Tensor> attention_impl(torch::Tensor Q, torch::Tensor K,
                                                 torch::Tensor V, torch::Tensor scale_Q,
                                                 torch::Tensor scale_K, torch::Tensor scale_V,
                                                 bool is_causal, bool out_bshd, bool quant) {
    TORCH_CHECK(Q.device().is_cuda(), "Q must be a CUDA tensor");
    TORCH_CHECK(Q.dtype() == torch::kInt8, "Q must be int8");
    TORCH_CHECK(K.dtype() == torch::kInt8, "K must be int8");
    TORCH_CHECK(V.dtype() == torch::kInt8, "V must be int8");
    TORCH_CHECK(Q.is_contiguous(), "Q must be contiguous");
    TORCH_CHECK(K.is_contiguous(), "K must be contiguous");
    TORCH_CHECK(V.is_contiguous(), "V must be contiguous");
    TORCH_CHECK(Q.dim() == 4, "expected (batch, heads, seq_len, head_dim)");
    TORCH_CHECK(Q.sizes() == K.sizes() && Q.sizes() == V.sizes(), "Q/K/V shape mismatch");
    TORCH_CHECK(scale_Q.dtype() == torch::kFloat32, "scale_Q must be float32");
    TORCH_CHECK(scale_K.dtype() == torch::kFloat32, "scale_K must be float32");
    TORCH_CHECK(scale_V.dtype() == torch::kFloat32, "scale_V must be float32");
    TORCH_CHECK(scale_Q.device().is_cuda(), "scale_Q must be CUDA");
    TORCH_CHECK(K.device() == Q.device() && V.device() == Q.device() &&
                    scale_Q.device() == Q.device() && scale_K.device() == Q.device() &&
                    scale_V.device() == Q.device(),
                "all inputs must be on Q's device");
    const int64_t batch = Q.size(0), heads = Q.size(1), seq_len = Q.size(2),
                  head_dim = Q.size(3);
    TORCH_CHECK(head_dim >= 1 && head_dim <= 512,
                "prefill attention supports head_dim 1..512");
    TORCH_CHECK(seq_len >= 1 && batch * heads * seq_len <= INT32_MAX, "seq_len out of range");
    const int64_t n_tokens = batch * heads * seq_len;
    auto sQ = scale_Q.contiguous().view({n_tokens});
    auto sK = scale_K.contiguous().view({n_tokens});
    auto sV = scale_V.contiguous().view({n_tokens});
    auto q = aligned_i8(Q), k = aligned_i8(K), v = aligned_i8(V);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(Q.device());
    const int flags = (is_causal ? INT8K_ATTN_CAUSAL : 0) | (out_bshd ? INT8K_ATTN_OUT_BSHD : 0);
    const std::vector<int64_t> rows = out_bshd ? std::vector<int64_t>{batch, seq_len, heads}
                                               : std::vector<int64_t>{batch, heads, seq_len};
    std::vector<int64_t> shape = rows;
    shape.push_back(head_dim);
    if (quant) {
        auto oq = torch::empty(shape, torch::TensorOptions().dtype(torch::kInt8).device(Q.device()));
        auto os = torch::empty(rows,
                               torch::TensorOptions().dtype(torch::kFloat32).device(Q.device()));
        check_status(int8k_attention_forward_quant(
                         q.data_ptr<int8_t>(), k.data_ptr<int8_t>(), v.data_ptr<int8_t>(),
                         oq.data_ptr<int8_t>(), os.data_ptr<float>(), sQ.data_ptr<float>(),
                         sK.data_ptr<float>(), sV.data_ptr<float>(), (int)batch, (int)heads,
                         (int)seq_len, (int)head_dim, flags, current_stream(Q)),
                     "int8_attention_forward_quant");
        return {oq, os};
    }
    auto out =
        torch::empty(shape, torch::TensorOptions().dtype(torch::kFloat16).device(Q.device()));
    const int st = int8k_attention_forward(
        q.data_ptr<int8_t>(), k.data_ptr<int8_t>(), v.data_ptr<int8_t>(),
        reinterpret_cast<uint16_t*>(out.data_ptr<at::Half>()), sQ.data_ptr<float>(),
        sK.data_ptr<float>(), sV.data_ptr<float>(), (int)batch, (int)heads, (int)seq_len,
        (int)head_dim, flags, current_stream(Q));
    check_status(st, "int8_attention_forward");
    return {out};
}

torch::Tensor int8_attention_forward_torch(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                           torch::Tensor scale_Q, torch::Tensor scale_K,
                                           torch::Tensor scale_V, bool is_causal, bool out_bshd) {
    return attention_impl(Q, K, V, scale_Q, scale_K, scale_V, is_causal, out_bshd, false)[0];
}

std::tuple<torch::Tensor, torch::Tensor> int8_attention_forward_quant_torch(
    torch::Tensor Q, torch::Tensor K, torch::Tensor V, torch::Tensor scale_Q,
    torch::Tensor scale_K, torch::Tensor scale_V, bool is_causal, bool out_bshd) {
    auto r = attention_impl(Q, K, V, scale_Q, scale_K, scale_V, is_causal, out_bshd, true);
    return {r[0], r[1]};
}

// ── decode attention (seq_q == 1) ─────────────────────────────────────────
// Mirrors int8_decode_attention_forward_torch (kernels/int8_ext.cu:136-178).
// Q : (batch, heads, head_dim) int8; K, V : (batch, heads, seq_kv, head_dim)
// int8; scale_Q numel batch*heads; scale_K/V numel batch*heads*seq_kv (fp32).
// Returns (batch, heads, head_dim) fp16.
// With `quant`: {int8 (batch, heads, head_dim), fp32 scales (batch, heads)}.
static std::vector<torch::Tensor> decode_impl(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                              torch::Tensor scale_Q, torch::Tensor scale_K,
                                              torch::Tensor scale_V, bool quant) {
    TORCH_CHECK(Q.device().is_cuda(), "Q must be a CUDA tensor");
    TORCH_CHECK(Q.dtype() == torch::kInt8, "Q must be int8");
    TORCH_CHECK(K.dtype() == torch::kInt8 && V.dtype() == torch::kInt8, "K, V must be int8");
    TORCH_CHECK(Q.is_contiguous() && K.is_contiguous() && V.is_contiguous(),
                "Q/K/V must be contiguous");
    TORCH_CHECK(Q.dim() == 3, "expected Q (batch, heads, head_dim) — seq_q == 1");
    TORCH_CHECK(K.dim() == 4, "expected K (batch, heads, seq_kv, head_dim)");
    TORCH_CHECK(K.sizes() == V.sizes(), "K/V shape mismatch");

    const int64_t batch = Q.size(0);
    const int64_t heads = Q.size(1);
    const int64_t head_dim = Q.size(2);
    const int64_t seq_kv = K.size(2);
    TORCH_CHECK(K.size(0) == batch && K.size(1) == heads && K.size(3) == head_dim,
                "Q/K head/batch/dim mismatch");
    TORCH_CHECK(head_dim == 64 || head_dim == 128,
                "decode kernel v1 supports head_dim 64 or 128");
    TORCH_CHECK(seq_kv >= 1, "decode needs seq_kv >= 1");
    TORCH_CHECK(K.device() == Q.device() && V.device() == Q.device(),
                "Q/K/V must be on the same device");
    TORCH_CHECK(scale_Q.dtype() == torch::kFloat32 && scale_K.dtype() == torch::kFloat32 &&
                    scale_V.dtype() == torch::kFloat32,
                "scales must be float32");
    TORCH_CHECK(scale_Q.device() == Q.device() && scale_K.device() == Q.device() &&
                    scale_V.device() == Q.device(),
                "scales must be on Q's device");

    const int64_t BH = batch * heads;
    TORCH_CHECK(BH <= INT32_MAX && seq_kv <= INT32_MAX, "decode shape too large");
    auto sQ = scale_Q.contiguous().view({BH});
    auto sK = scale_K.contiguous().view({BH * seq_kv});
    auto sV = scale_V.contiguous().view({BH * seq_kv});
    auto q = aligned_i8(Q), k = aligned_i8(K), v = aligned_i8(V);

    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(Q.device());
    const size_t ws_bytes =
        int8k_decode_attention_workspace_bytes((int)BH, (int)seq_kv, (int)head_dim, 0);
    auto ws = workspace(ws_bytes, Q.device());
    if (quant) {
        auto oq = torch::empty({batch, heads, head_dim},
                               torch::TensorOptions().dtype(torch::kInt8).device(Q.device()));
        auto os = torch::empty({batch, heads},
                               torch::TensorOptions().dtype(torch::kFloat32).device(Q.device()));
        check_status(int8k_decode_attention_forward_quant(
                         q.data_ptr<int8_t>(), k.data_ptr<int8_t>(), v.data_ptr<int8_t>(),
                         oq.data_ptr<int8_t>(), os.data_ptr<float>(), sQ.data_ptr<float>(),
                         sK.data_ptr<float>(), sV.data_ptr<float>(), (int)BH, (int)seq_kv,
                         (int)head_dim, 0, ws.data_ptr(), ws_bytes, current_stream(Q)),
                     "int8_decode_attention_forward_quant");
        return {oq, os};
    }
    auto out = torch::empty({batch, heads, head_dim},
                            torch::TensorOptions().dtype(torch::kFloat16).device(Q.device()));
    const int st = int8k_decode_attention_forward(
        q.data_ptr<int8_t>(), k.data_ptr<int8_t>(), v.data_ptr<int8_t>(),
        reinterpret_cast<uint16_t*>(out.data_ptr<at::Half>()), sQ.data_ptr<float>(),
        sK.data_ptr<float>(), sV.data_ptr<float>(), (int)BH, (int)seq_kv, (int)head_dim, 0,
        ws.data_ptr(), ws_bytes, current_stream(Q));
    check_status(st, "int8_decode_attention_forward");
    return {out};
}

torch::Tensor int8_decode_attention_forward_torch(torch::Tensor Q, torch::Tensor K,
                                                  torch::Tensor V, torch::Tensor scale_Q,
                                                  torch::Tensor scale_K, torch::Tensor scale_V) {
    return decode_impl(Q, K, V, scale_Q, scale_K, scale_V, false)[0];
}

std::tuple<torch::Tensor, torch::Tensor> int8_decode_attention_forward_quant_torch(
    torch::Tensor Q, torch::Tensor K, torch::Tensor V, torch::Tensor scale_Q,
    torch::Tensor scale_K, torch::Tensor scale_V) {
    auto r = decode_impl(Q, K, V, scale_Q, scale_K, scale_V, true);
    return {r[0], r[1]};
}

// ── INT8 MLP ────────────────────────────────────────────────────────────────
// Mirrors the four MLP bindings of kernels/int8_ext.cu:188-455.  One C ABI
// entry point (int8k_mlp_forward) serves all of them through its flags.

namespace {

struct MlpDims {
    int64_t batch, seq_len, d_model, d_ff, T;
};

MlpDims check_mlp_args(const torch::Tensor& x, const torch::Tensor& W1, const torch::Tensor& W2,
                       bool prepacked) {
    TORCH_CHECK(x.device().is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.dtype() == torch::kInt8, "x must be int8");
    const char* n1 = prepacked ? "W1T" : "W1";
    const char* n2 = prepacked ? "W2T" : "W2";
    TORCH_CHECK(W1.dtype() == torch::kInt8, n1, " must be int8");
    TORCH_CHECK(W2.dtype() == torch::kInt8, n2, " must be int8");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(W1.is_contiguous(), n1, " must be contiguous");
    TORCH_CHECK(W2.is_contiguous(), n2, " must be contiguous");
    TORCH_CHECK(x.dim() == 3, "x must be 3-D (batch, seq_len, d_model)");
    TORCH_CHECK(W1.dim() == 2, prepacked ? "W1T must be 2-D (d_ff, d_model)"
                                         : "W1 must be 2-D (d_model, d_ff)");
    TORCH_CHECK(W2.dim() == 2, prepacked ? "W2T must be 2-D (d_model, d_ff)"
                                         : "W2 must be 2-D (d_ff, d_model)");
    TORCH_CHECK(W1.device() == x.device() && W2.device() == x.device(),
                "x/W1/W2 must be on the same device");
    MlpDims d;
    d.batch = x.size(0);
    d.seq_len = x.size(1);
    d.d_model = x.size(2);
    d.T = d.batch * d.seq_len;
    if (prepacked) {
        d.d_ff = W1.size(0);
        TORCH_CHECK(W1.size(1) == d.d_model, "W1T shape mismatch (expected d_model cols)");
        TORCH_CHECK(W2.size(0) == d.d_model, "W2T shape mismatch (expected d_model rows)");
        TORCH_CHECK(W2.size(1) == d.d_ff, "W2T shape mismatch (expected d_ff cols)");
    } else {
        d.d_ff = W1.size(1);
        TORCH_CHECK(W1.size(0) == d.d_model, "W1 shape mismatch");
        TORCH_CHECK(W2.size(0) == d.d_ff, "W2 shape mismatch");
        TORCH_CHECK(W2.size(1) == d.d_model, "W2 shape mismatch");
    }
    TORCH_CHECK(d.d_model % 16 == 0 && d.d_ff % 16 == 0,
                "int8 MLP needs d_model and d_ff to be multiples of 16");
    TORCH_CHECK(d.T > 0 && d.T <= INT32_MAX && d.d_ff <= INT32_MAX, "MLP shape out of range");
    return d;
}

torch::Tensor scalar_scale(double v, const torch::Device& dev) {
    return torch::full({1}, (float)v, torch::TensorOptions().dtype(torch::kFloat32).device(dev));
}

void check_scale(const torch::Tensor& s, int64_t n, const char* nm, const torch::Device& dev) {
    TORCH_CHECK(s.dtype() == torch::kFloat32, nm, " must be float32");
    TORCH_CHECK(s.device().is_cuda(), nm, " must be CUDA");
    TORCH_CHECK(s.device() == dev, nm, " must be on x's device");
    TORCH_CHECK(s.numel() == n || s.numel() == 1, nm, " must have ", n, " (or 1) elements");
}

// Runs the MLP; returns (out int8 like x, out_scale fp32 [T] or [1]).
std::tuple<torch::Tensor, torch::Tensor> run_mlp(const torch::Tensor& x, const torch::Tensor& W1,
                                                 const torch::Tensor& W2, const torch::Tensor& sx,
                                                 const torch::Tensor& sw1,
                                                 const torch::Tensor& sw2,
                                                 const c10::optional<torch::Tensor>& bias1,
                                                 const MlpDims& d, int flags) {
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto xa = aligned_i8(x), w1 = aligned_i8(W1), w2 = aligned_i8(W2);
    auto out = torch::empty_like(x);
    const bool per_tensor = (flags & INT8K_MLP_OUT_PER_TENSOR) != 0;
    auto out_scale = torch::empty({per_tensor ? 1 : d.T},
                                  torch::TensorOptions().dtype(torch::kFloat32).device(x.device()));
    const size_t ws_bytes =
        int8k_mlp_workspace_bytes((int)d.T, (int)d.d_model, (int)d.d_ff, flags);
    auto ws = workspace(ws_bytes, x.device());
    const int st = int8k_mlp_forward(
        xa.data_ptr<int8_t>(), w1.data_ptr<int8_t>(), w2.data_ptr<int8_t>(),
        out.data_ptr<int8_t>(), sx.data_ptr<float>(), (int)sx.numel(), sw1.data_ptr<float>(),
        (int)sw1.numel(), sw2.data_ptr<float>(), (int)sw2.numel(),
        bias1 ? bias1->data_ptr<float>() : nullptr, out_scale.data_ptr<float>(), (int)d.T,
        (int)d.d_model, (int)d.d_ff, flags, ws.data_ptr(), ws_bytes, current_stream(x));
    check_status(st, "int8_mlp_forward");
    return {out, out_scale};
}

}  // namespace

// Per-tensor scales (kernels/int8_ext.cu:188-233): returns (int8 out, float out_scale).
// Reading the scale back is the only host synchronisation.
std::tuple<torch::Tensor, double> int8_mlp_forward_torch(torch::Tensor x, torch::Tensor W1,
                                                         torch::Tensor W2, double scale_x,
                                                         double scale_W1, double scale_W2) {
    const MlpDims d = check_mlp_args(x, W1, W2, false);
    auto r = run_mlp(x, W1, W2, scalar_scale(scale_x, x.device()),
                     scalar_scale(scale_W1, x.device()), scalar_scale(scale_W2, x.device()),
                     c10::nullopt, d, INT8K_MLP_OUT_PER_TENSOR);
    return {std::get<0>(r), (double)std::get<1>(r).item<float>()};
}

// Per-token activation + per-channel weight scales (kernels/int8_ext.cu:246-300):
// scale_x [T] (or [1]), scale_W1 [d_ff] (or [1]), scale_W2 [d_model] (or [1]);
// returns (int8 out, fp32 out_scale [T]) — the output is quantized per token.
std::tuple<torch::Tensor, torch::Tensor> int8_mlp_forward_pc_torch(
    torch::Tensor x, torch::Tensor W1, torch::Tensor W2, torch::Tensor scale_x,
    torch::Tensor scale_W1, torch::Tensor scale_W2) {
    const MlpDims d = check_mlp_args(x, W1, W2, false);
    check_scale(scale_x, d.T, "scale_x", x.device());
    check_scale(scale_W1, d.d_ff, "scale_W1", x.device());
    check_scale(scale_W2, d.d_model, "scale_W2", x.device());
    return run_mlp(x, W1, W2, scale_x.contiguous(), scale_W1.contiguous(), scale_W2.contiguous(),
                   c10::nullopt, d, 0);
}

// As above plus a per-channel pre-GELU bias b1 [d_ff] (kernels/int8_ext.cu:306-365).
std::tuple<torch::Tensor, torch::Tensor> int8_mlp_forward_pc_bias_torch(
    torch::Tensor x, torch::Tensor W1, torch::Tensor W2, torch::Tensor scale_x,
    torch::Tensor scale_W1, torch::Tensor scale_W2, torch::Tensor bias1) {
    const MlpDims d = check_mlp_args(x, W1, W2, false);
    check_scale(scale_x, d.T, "scale_x", x.device());
    check_scale(scale_W1, d.d_ff, "scale_W1", x.device());
    check_scale(scale_W2, d.d_model, "scale_W2", x.device());
    TORCH_CHECK(bias1.dtype() == torch::kFloat32, "bias1 must be float32");
    TORCH_CHECK(bias1.device().is_cuda(), "bias1 must be CUDA");
    TORCH_CHECK(bias1.device() == x.device(), "bias1 must be on x's device");
    TORCH_CHECK(bias1.numel() == d.d_ff, "bias1 must have d_ff elements");
    return run_mlp(x, W1, W2, scale_x.contiguous(), scale_W1.contiguous(), scale_W2.contiguous(),
                   bias1.contiguous(), d, 0);
}

// W1 (d_model, d_ff) -> W1T (d_ff, d_model); W2 (d_ff, d_model) -> W2T (d_model, d_ff)
// (kernels/int8_ext.cu:372-399).
std::tuple<torch::Tensor, torch::Tensor> transpose_int8_weights_torch(torch::Tensor W1,
                                                                      torch::Tensor W2) {
    TORCH_CHECK(W1.device().is_cuda(), "W1 must be a CUDA tensor");
    TORCH_CHECK(W1.dtype() == torch::kInt8, "W1 must be int8");
    TORCH_CHECK(W2.dtype() == torch::kInt8, "W2 must be int8");
    TORCH_CHECK(W1.is_contiguous(), "W1 must be contiguous");
    TORCH_CHECK(W2.is_contiguous(), "W2 must be contiguous");
    TORCH_CHECK(W1.dim() == 2, "W1 must be 2-D (d_model, d_ff)");
    TORCH_CHECK(W2.dim() == 2, "W2 must be 2-D (d_ff, d_model)");
    const int64_t d_model = W1.size(0), d_ff = W1.size(1);
    TORCH_CHECK(W2.size(0) == d_ff, "W2 shape mismatch (expected d_ff rows)");
    TORCH_CHECK(W2.size(1) == d_model, "W2 shape mismatch (expected d_model cols)");
    TORCH_CHECK(W2.device() == W1.device(), "W1/W2 must be on the same device");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(W1.device());
    auto opts = torch::TensorOptions().dtype(torch::kInt8).device(W1.device());
    auto W1T = torch::empty({d_ff, d_model}, opts);
    auto W2T = torch::empty({d_model, d_ff}, opts);
    const int st = int8k_transpose_int8_weights(W1.data_ptr<int8_t>(), W2.data_ptr<int8_t>(),
                                                W1T.data_ptr<int8_t>(), W2T.data_ptr<int8_t>(),
                                                (int)d_model, (int)d_ff, current_stream(W1));
    check_status(st, "transpose_int8_weights");
    return {W1T, W2T};
}

// Per-tensor MLP on pre-transposed weights (kernels/int8_ext.cu:407-455).  The
// reference also demands T, d_model, d_ff % 128 == 0 (its WMMA tiles); these
// kernels handle any T and need only d_model, d_ff % 16 == 0.
std::tuple<torch::Tensor, double> int8_mlp_forward_prepacked_torch(torch::Tensor x,
                                                                   torch::Tensor W1T,
                                                                   torch::Tensor W2T,
                                                                   double scale_x,
                                                                   double scale_W1,
                                                                   double scale_W2) {
    const MlpDims d = check_mlp_args(x, W1T, W2T, true);
    auto r = run_mlp(x, W1T, W2T, scalar_scale(scale_x, x.device()),
                     scalar_scale(scale_W1, x.device()), scalar_scale(scale_W2, x.device()),
                     c10::nullopt, d, INT8K_MLP_WEIGHTS_PREPACKED | INT8K_MLP_OUT_PER_TENSOR);
    return {std::get<0>(r), (double)std::get<1>(r).item<float>()};
}

// New overload (not in the reference): per-token / per-channel scales on
// pre-transposed weights, for static-weight inference on the per-channel path.
// Same results as int8_mlp_forward's tensor overload on the untransposed weights.
std::tuple<torch::Tensor, torch::Tensor> int8_mlp_forward_prepacked_pc_torch(
    torch::Tensor x, torch::Tensor W1T, torch::Tensor W2T, torch::Tensor scale_x,
    torch::Tensor scale_W1, torch::Tensor scale_W2) {
    const MlpDims d = check_mlp_args(x, W1T, W2T, true);
    check_scale(scale_x, d.T, "scale_x", x.device());
    check_scale(scale_W1, d.d_ff, "scale_W1", x.device());
    check_scale(scale_W2, d.d_model, "scale_W2", x.device());
    return run_mlp(x, W1T, W2T, scale_x.contiguous(), scale_W1.contiguous(),
                   scale_W2.contiguous(), c10::nullopt, d, INT8K_MLP_WEIGHTS_PREPACKED);
}

// ── quantization and the INT8 KV cache (new ops; the reference exposes its
// quant utils only as C++ functions, kernels/int8_common.cuh:51-59) ─────────

namespace {

int dtype_code(const torch::Tensor& t) {
    if (t.dtype() == torch::kFloat16) return INT8K_DTYPE_F16;
    if (t.dtype() == torch::kBFloat16) return INT8K_DTYPE_BF16;
    if (t.dtype() == torch::kFloat32) return INT8K_DTYPE_F32;
    TORCH_CHECK(false, "expected a float16, bfloat16 or float32 tensor");
    return -1;
}

}  // namespace

// Per-tensor fp16 -> int8 (kernels/quant_utils.cu:56-69): returns (int8, scale [1]).
std::tuple<torch::Tensor, torch::Tensor> quantize_fp16_to_int8_torch(torch::Tensor x) {
    TORCH_CHECK(x.device().is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.dtype() == torch::kFloat16, "x must be float16");
    TORCH_CHECK(x.numel() > 0, "x must not be empty");
    auto xc = x.contiguous();
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty(x.sizes(), torch::TensorOptions().dtype(torch::kInt8).device(x.device()));
    auto s = torch::empty({1}, torch::TensorOptions().dtype(torch::kFloat32).device(x.device()));
    check_status(int8k_quantize_fp16_to_int8(
                     reinterpret_cast<const uint16_t*>(xc.data_ptr<at::Half>()), q.data_ptr<int8_t>(),
                     s.data_ptr<float>(), xc.numel(), current_stream(x)),
                 "quantize_fp16_to_int8");
    return {q, s};
}

// int8 -> fp16 with a host scale (kernels/quant_utils.cu:72-77).
torch::Tensor dequantize_int8_to_fp16_torch(torch::Tensor q, double scale) {
    TORCH_CHECK(q.device().is_cuda(), "q must be a CUDA tensor");
    TORCH_CHECK(q.dtype() == torch::kInt8, "q must be int8");
    TORCH_CHECK(q.numel() > 0, "q must not be empty");
    auto qc = q.contiguous();
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
    auto y = torch::empty(q.sizes(), torch::TensorOptions().dtype(torch::kFloat16).device(q.device()));
    check_status(int8k_dequantize_int8_to_fp16(qc.data_ptr<int8_t>(),
                                               reinterpret_cast<uint16_t*>(y.data_ptr<at::Half>()),
                                               (float)scale, qc.numel(), current_stream(q)),
                 "dequantize_int8_to_fp16");
    return y;
}

// Per-token (last-dim) symmetric quantization: returns (int8 like x, fp32 x.shape[:-1]).
std::tuple<torch::Tensor, torch::Tensor> quantize_per_token_torch(torch::Tensor x) {
    TORCH_CHECK(x.device().is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.dim() >= 1 && x.numel() > 0, "x must be a non-empty tensor");
    const int code = dtype_code(x);
    auto xc = x.contiguous();
    const int64_t cols = x.size(-1);
    TORCH_CHECK(cols <= INT32_MAX, "rows too long");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty(x.sizes(), torch::TensorOptions().dtype(torch::kInt8).device(x.device()));
    auto s = torch::empty(x.sizes().slice(0, x.dim() - 1),
                          torch::TensorOptions().dtype(torch::kFloat32).device(x.device()));
    check_status(int8k_quantize_per_token(xc.data_ptr(), code, q.data_ptr<int8_t>(),
                                          s.data_ptr<float>(), xc.numel() / cols, (int)cols,
                                          current_stream(x)),
                 "quantize_per_token");
    return {q, s};
}

// Per-token dequantization: y = (q.float() * s[..., None]).to(dtype), or with a
// residual r: r + that (in r's dtype, which then sets the output dtype).
torch::Tensor dequantize_per_token_torch(torch::Tensor q, torch::Tensor s,
                                         c10::optional<torch::Tensor> residual,
                                         c10::optional<at::ScalarType> dtype) {
    TORCH_CHECK(q.device().is_cuda(), "q must be a CUDA tensor");
    TORCH_CHECK(q.dtype() == torch::kInt8, "q must be int8");
    TORCH_CHECK(q.dim() >= 1 && q.numel() > 0, "q must be a non-empty tensor");
    const int64_t cols = q.size(-1);
    TORCH_CHECK(cols <= INT32_MAX, "rows too long");
    const int64_t rows = q.numel() / cols;
    TORCH_CHECK(s.numel() == rows, "scales must have one element per row of q");
    TORCH_CHECK(s.device() == q.device(), "scales must be on q's device");
    torch::ScalarType out_t = torch::kFloat16;
    torch::Tensor r;
    if (residual.has_value() && residual->defined()) {
        r = residual->contiguous();
        TORCH_CHECK(r.sizes() == q.sizes(), "residual must have q's shape");
        TORCH_CHECK(r.device() == q.device(), "residual must be on q's device");
        out_t = r.scalar_type();
        TORCH_CHECK(!dtype.has_value() || *dtype == out_t,
                    "dtype must match the residual's dtype, which sets the output dtype");
    } else if (dtype.has_value()) {
        out_t = *dtype;
    }
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
    auto y = torch::empty(q.sizes(), torch::TensorOptions().dtype(out_t).device(q.device()));
    const int code = dtype_code(y);
    auto qc = q.contiguous();
    auto sc = s.to(torch::kFloat32).contiguous();
    check_status(int8k_dequantize_per_token(qc.data_ptr<int8_t>(), sc.data_ptr<float>(), code,
                                            r.defined() ? r.data_ptr() : nullptr, y.data_ptr(),
                                            rows, (int)cols, current_stream(q)),
                 "dequantize_per_token");
    return y;
}

// LayerNorm over the last dim, rounded to x's dtype, then per-token int8:
// returns (q, scales).  weight/bias optional (any float dtype; used as fp32).
std::tuple<torch::Tensor, torch::Tensor> layernorm_quantize_per_token_torch(
    torch::Tensor x, c10::optional<torch::Tensor> weight, c10::optional<torch::Tensor> bias,
    double eps) {
    TORCH_CHECK(x.device().is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.dim() >= 1 && x.numel() > 0, "x must be a non-empty tensor");
    const int code = dtype_code(x);
    auto xc = x.contiguous();
    const int64_t cols = x.size(-1);
    TORCH_CHECK(cols <= INT32_MAX, "rows too long");
    torch::Tensor g, b;
    if (weight.has_value() && weight->defined()) {
        TORCH_CHECK(weight->numel() == cols, "weight must have size(-1) elements");
        g = weight->to(x.device(), torch::kFloat32).contiguous();
    }
    if (bias.has_value() && bias->defined()) {
        TORCH_CHECK(bias->numel() == cols, "bias must have size(-1) elements");
        b = bias->to(x.device(), torch::kFloat32).contiguous();
    }
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty(x.sizes(), torch::TensorOptions().dtype(torch::kInt8).device(x.device()));
    auto s = torch::empty(x.sizes().slice(0, x.dim() - 1),
                          torch::TensorOptions().dtype(torch::kFloat32).device(x.device()));
    check_status(int8k_layernorm_quantize_per_token(
                     xc.data_ptr(), code, g.defined() ? g.data_ptr<float>() : nullptr,
                     b.defined() ? b.data_ptr<float>() : nullptr, (float)eps,
                     q.data_ptr<int8_t>(), s.data_ptr<float>(), nullptr, xc.numel() / cols,
                     (int)cols, current_stream(x)),
                 "layernorm_quantize_per_token");
    return {q, s};
}

// x (batch, seq, parts * heads * head_dim) -> [q_0, s_0, q_1, s_1, ...] with
// q_p int8 (batch, heads, seq, head_dim) and s_p fp32 (batch, heads, seq).
std::vector<torch::Tensor> quantize_heads_torch(torch::Tensor x, int64_t heads, int64_t parts) {
    TORCH_CHECK(x.device().is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.dim() == 3, "x must be (batch, seq, parts * heads * head_dim)");
    TORCH_CHECK(parts >= 1 && parts <= 3 && heads >= 1, "parts must be 1..3, heads >= 1");
    TORCH_CHECK(x.size(2) % (parts * heads) == 0, "last dim must be parts * heads * head_dim");
    const int code = dtype_code(x);
    auto xc = x.contiguous();
    const int64_t B = x.size(0), S = x.size(1), Dh = x.size(2) / (parts * heads);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    std::vector<torch::Tensor> outs;
    for (int64_t p = 0; p < parts; ++p) {
        outs.push_back(torch::empty({B, heads, S, Dh},
                                    torch::TensorOptions().dtype(torch::kInt8).device(x.device())));
        outs.push_back(torch::empty({B, heads, S},
                                    torch::TensorOptions().dtype(torch::kFloat32).device(x.device())));
    }
    auto qp = [&](int64_t p) { return p < parts ? outs[2 * p].data_ptr<int8_t>() : nullptr; };
    auto sp = [&](int64_t p) { return p < parts ? outs[2 * p + 1].data_ptr<float>() : nullptr; };
    check_status(int8k_quantize_heads(xc.data_ptr(), code, (int)parts, qp(0), sp(0), qp(1), sp(1),
                                      qp(2), sp(2), (int)B, (int)S, (int)heads, (int)Dh,
                                      current_stream(x)),
                 "quantize_heads");
    return outs;
}

// Quantize k_new/v_new (batch, heads, n_new, head_dim) per token into positions
// pos .. pos+n_new-1 of the int8 caches (batch, heads, capacity, head_dim) and
// their fp32 scales (batch, heads, capacity).  In place.
void kv_cache_append_torch(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor K_cache,
                           torch::Tensor V_cache, torch::Tensor sK_cache, torch::Tensor sV_cache,
                           int64_t pos) {
    TORCH_CHECK(k_new.device().is_cuda(), "k_new must be a CUDA tensor");
    TORCH_CHECK(k_new.dim() == 4 && k_new.sizes() == v_new.sizes(),
                "k_new/v_new must be (batch, heads, n_new, head_dim) of one shape");
    TORCH_CHECK(k_new.dtype() == v_new.dtype(), "k_new/v_new dtype mismatch");
    const int code = dtype_code(k_new);
    TORCH_CHECK(K_cache.dtype() == torch::kInt8 && V_cache.dtype() == torch::kInt8,
                "caches must be int8");
    TORCH_CHECK(sK_cache.dtype() == torch::kFloat32 && sV_cache.dtype() == torch::kFloat32,
                "cache scales must be float32");
    TORCH_CHECK(K_cache.is_contiguous() && V_cache.is_contiguous() && sK_cache.is_contiguous() &&
                    sV_cache.is_contiguous(),
                "caches must be contiguous");
    TORCH_CHECK(K_cache.dim() == 4 && K_cache.sizes() == V_cache.sizes(),
                "caches must be (batch, heads, capacity, head_dim) of one shape");
    const int64_t B = k_new.size(0), H = k_new.size(1), n = k_new.size(2), D = k_new.size(3);
    const int64_t cap = K_cache.size(2);
    TORCH_CHECK(K_cache.size(0) == B && K_cache.size(1) == H && K_cache.size(3) == D,
                "cache/new-token shape mismatch");
    TORCH_CHECK(sK_cache.numel() == B * H * cap && sV_cache.numel() == B * H * cap,
                "cache scales must have batch*heads*capacity elements");
    TORCH_CHECK(pos >= 0 && pos + n <= cap, "append past the cache capacity");
    for (const auto* t : {&v_new, &K_cache, &V_cache, &sK_cache, &sV_cache})
        TORCH_CHECK(t->device() == k_new.device(), "all tensors must be on one device");
    auto kc = k_new.contiguous(), vc = v_new.contiguous();
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(k_new.device());
    check_status(int8k_kv_cache_append(kc.data_ptr(), vc.data_ptr(), code, K_cache.data_ptr<int8_t>(),
                                       V_cache.data_ptr<int8_t>(), sK_cache.data_ptr<float>(),
                                       sV_cache.data_ptr<float>(), (int)(B * H), (int)n, (int)pos,
                                       (int)cap, (int)D, current_stream(k_new)),
                 "kv_cache_append");
}

// Decode over the first seq_len positions of a preallocated cache
// (batch, heads, capacity, head_dim); Q (batch, heads, head_dim) int8.
static std::vector<torch::Tensor> decode_cache_impl(torch::Tensor Q, torch::Tensor K_cache,
                                                    torch::Tensor V_cache, torch::Tensor scale_Q,
                                                    torch::Tensor sK_cache,
                                                    torch::Tensor sV_cache, int64_t seq_len,
                                                    bool quant) {
    TORCH_CHECK(Q.device().is_cuda(), "Q must be a CUDA tensor");
    TORCH_CHECK(Q.dtype() == torch::kInt8 && K_cache.dtype() == torch::kInt8 &&
                    V_cache.dtype() == torch::kInt8,
                "Q/K/V must be int8");
    TORCH_CHECK(Q.is_contiguous() && K_cache.is_contiguous() && V_cache.is_contiguous(),
                "Q/K/V must be contiguous");
    TORCH_CHECK(Q.dim() == 3 && K_cache.dim() == 4 && K_cache.sizes() == V_cache.sizes(),
                "expected Q (batch, heads, head_dim), caches (batch, heads, capacity, head_dim)");
    const int64_t B = Q.size(0), H = Q.size(1), D = Q.size(2), cap = K_cache.size(2);
    TORCH_CHECK(K_cache.size(0) == B && K_cache.size(1) == H && K_cache.size(3) == D,
                "Q/K head/batch/dim mismatch");
    TORCH_CHECK(D == 64 || D == 128, "decode kernel v1 supports head_dim 64 or 128");
    TORCH_CHECK(seq_len >= 1 && seq_len <= cap, "seq_len must be in [1, capacity]");
    TORCH_CHECK(scale_Q.dtype() == torch::kFloat32 && sK_cache.dtype() == torch::kFloat32 &&
                    sV_cache.dtype() == torch::kFloat32,
                "scales must be float32");
    TORCH_CHECK(sK_cache.numel() == B * H * cap && sV_cache.numel() == B * H * cap &&
                    scale_Q.numel() == B * H,
                "scale sizes mismatch");
    auto sQ = scale_Q.contiguous();
    auto sK = sK_cache.contiguous();
    auto sV = sV_cache.contiguous();
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(Q.device());
    const int BH = (int)(B * H);
    const size_t ws_bytes = int8k_decode_attention_workspace_bytes(BH, (int)seq_len, (int)D, 0);
    auto ws = workspace(ws_bytes, Q.device());
    if (quant) {
        auto oq = torch::empty({B, H, D}, torch::TensorOptions().dtype(torch::kInt8).device(Q.device()));
        auto os = torch::empty({B, H}, torch::TensorOptions().dtype(torch::kFloat32).device(Q.device()));
        check_status(int8k_decode_attention_forward_cache_quant(
                         Q.data_ptr<int8_t>(), K_cache.data_ptr<int8_t>(),
                         V_cache.data_ptr<int8_t>(), oq.data_ptr<int8_t>(), os.data_ptr<float>(),
                         sQ.data_ptr<float>(), sK.data_ptr<float>(), sV.data_ptr<float>(), BH,
                         (int)seq_len, (int)cap, (int)D, 0, ws.data_ptr(), ws_bytes,
                         current_stream(Q)),
                     "int8_decode_attention_forward_cache_quant");
        return {oq, os};
    }
    auto out = torch::empty({B, H, D}, torch::TensorOptions().dtype(torch::kFloat16).device(Q.device()));
    const int st = int8k_decode_attention_forward_cache(
        Q.data_ptr<int8_t>(), K_cache.data_ptr<int8_t>(), V_cache.data_ptr<int8_t>(),
        reinterpret_cast<uint16_t*>(out.data_ptr<at::Half>()), sQ.data_ptr<float>(),
        sK.data_ptr<float>(), sV.data_ptr<float>(), BH, (int)seq_len, (int)cap, (int)D, 0,
        ws.data_ptr(), ws_bytes, current_stream(Q));
    check_status(st, "int8_decode_attention_forward_cache");
    return {out};
}

torch::Tensor int8_decode_attention_forward_cache_torch(torch::Tensor Q, torch::Tensor K_cache,
                                                        torch::Tensor V_cache, torch::Tensor scale_Q,
                                                        torch::Tensor sK_cache,
                                                        torch::Tensor sV_cache, int64_t seq_len) {
    return decode_cache_impl(Q, K_cache, V_cache, scale_Q, sK_cache, sV_cache, seq_len, false)[0];
}

std::tuple<torch::Tensor, torch::Tensor> int8_decode_attention_forward_cache_quant_torch(
    torch::Tensor Q, torch::Tensor K_cache, torch::Tensor V_cache, torch::Tensor scale_Q,
    torch::Tensor sK_cache, torch::Tensor sV_cache, int64_t seq_len) {
    auto r = decode_cache_impl(Q, K_cache, V_cache, scale_Q, sK_cache, sV_cache, seq_len, true);
    return {r[0], r[1]};
}

// Decode over a paged int8 KV cache (no reference counterpart): K/V pages
// [num_pages, H, page, D], scale pages [num_pages, H, page], block_tables
// [B, max_pages] int32, context_lens [B] int32 (each in [1, max_context]).
static std::vector<torch::Tensor> decode_paged_impl(
    torch::Tensor Q, torch::Tensor K_pages, torch::Tensor V_pages, torch::Tensor scale_Q,
    torch::Tensor sK_pages, torch::Tensor sV_pages, torch::Tensor block_tables,
    torch::Tensor context_lens, int64_t max_context, bool quant) {
    TORCH_CHECK(Q.device().is_cuda(), "Q must be a CUDA tensor");
    TORCH_CHECK(Q.dtype() == torch::kInt8 && K_pages.dtype() == torch::kInt8 &&
                    V_pages.dtype() == torch::kInt8,
                "Q/K/V must be int8");
    TORCH_CHECK(Q.is_contiguous() && K_pages.is_contiguous() && V_pages.is_contiguous(),
                "Q/K/V must be contiguous");
    TORCH_CHECK(Q.dim() == 3 && K_pages.dim() == 4 && K_pages.sizes() == V_pages.sizes(),
                "expected Q (batch, heads, head_dim), pages (num_pages, heads, page, head_dim)");
    const int64_t B = Q.size(0), H = Q.size(1), D = Q.size(2);
    const int64_t NP = K_pages.size(0), P = K_pages.size(2);
    TORCH_CHECK(K_pages.size(1) == H && K_pages.size(3) == D, "Q/K head/dim mismatch");
    TORCH_CHECK(D == 64 || D == 128, "decode kernel supports head_dim 64 or 128");
    TORCH_CHECK(block_tables.dtype() == torch::kInt32 && context_lens.dtype() == torch::kInt32,
                "block_tables and context_lens must be int32");
    TORCH_CHECK(block_tables.dim() == 2 && block_tables.size(0) == B && context_lens.numel() == B,
                "block_tables (batch, max_pages) / context_lens (batch,) shape mismatch");
    TORCH_CHECK(scale_Q.dtype() == torch::kFloat32 && sK_pages.dtype() == torch::kFloat32 &&
                    sV_pages.dtype() == torch::kFloat32,
                "scales must be float32");
    TORCH_CHECK(scale_Q.numel() == B * H && sK_pages.numel() == NP * H * P &&
                    sV_pages.numel() == NP * H * P,
                "scale sizes mismatch");
    const int64_t max_pages = block_tables.size(1);
    TORCH_CHECK(max_context >= 1 && max_context <= max_pages * P,
                "max_context must be in [1, max_pages * page_size]");
    auto sQ = scale_Q.contiguous();
    auto sK = sK_pages.contiguous();
    auto sV = sV_pages.contiguous();
    auto bt = block_tables.contiguous();
    auto cl = context_lens.contiguous();
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(Q.device());
    const size_t ws_bytes = int8k_decode_attention_paged_workspace_bytes(
        (int)B, (int)H, (int)max_context, (int)D, 0);
    auto ws = workspace(ws_bytes, Q.device());
    if (quant) {
        auto oq = torch::empty({B, H, D}, torch::TensorOptions().dtype(torch::kInt8).device(Q.device()));
        auto os = torch::empty({B, H}, torch::TensorOptions().dtype(torch::kFloat32).device(Q.device()));
        check_status(int8k_decode_attention_forward_paged_quant(
                         Q.data_ptr<int8_t>(), K_pages.data_ptr<int8_t>(),
                         V_pages.data_ptr<int8_t>(), oq.data_ptr<int8_t>(), os.data_ptr<float>(),
                         sQ.data_ptr<float>(), sK.data_ptr<float>(), sV.data_ptr<float>(),
                         bt.data_ptr<int32_t>(), cl.data_ptr<int32_t>(), (int)B, (int)H, (int)D,
                         (int)NP, (int)P, (int)max_pages, (int)max_context, 0, ws.data_ptr(),
                         ws_bytes, current_stream(Q)),
                     "int8_decode_attention_forward_paged_quant");
        return {oq, os};
    }
    auto out = torch::empty({B, H, D}, torch::TensorOptions().dtype(torch::kFloat16).device(Q.device()));
    const int st = int8k_decode_attention_forward_paged(
        Q.data_ptr<int8_t>(), K_pages.data_ptr<int8_t>(), V_pages.data_ptr<int8_t>(),
        reinterpret_cast<uint16_t*>(out.data_ptr<at::Half>()), sQ.data_ptr<float>(),
        sK.data_ptr<float>(), sV.data_ptr<float>(), bt.data_ptr<int32_t>(),
        cl.data_ptr<int32_t>(), (int)B, (int)H, (int)D, (int)NP, (int)P, (int)max_pages,
        (int)max_context, 0, ws.data_ptr(), ws_bytes, current_stream(Q));
    check_status(st, "int8_decode_attention_forward_paged");
    return {out};
}

torch::Tensor int8_decode_attention_forward_paged_torch(
    torch::Tensor Q, torch::Tensor K_pages, torch::Tensor V_pages, torch::Tensor scale_Q,
    torch::Tensor sK_pages, torch::Tensor sV_pages, torch::Tensor block_tables,
    torch::Tensor context_lens, int64_t max_context) {
    return decode_paged_impl(Q, K_pages, V_pages, scale_Q, sK_pages, sV_pages, block_tables,
                             context_lens, max_context, false)[0];
}

std::tuple<torch::Tensor, torch::Tensor> int8_decode_attention_forward_paged_quant_torch(
    torch::Tensor Q, torch::Tensor K_pages, torch::Tensor V_pages, torch::Tensor scale_Q,
    torch::Tensor sK_pages, torch::Tensor sV_pages, torch::Tensor block_tables,
    torch::Tensor context_lens, int64_t max_context) {
    auto r = decode_paged_impl(Q, K_pages, V_pages, scale_Q, sK_pages, sV_pages, block_tables,
                               context_lens, max_context, true);
    return {r[0], r[1]};
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("int8_attention_forward", &int8_attention_forward_torch,
          "INT8 attention with per-token quantization — returns FP16 (optional is_causal; "
          "out_bshd: output as (batch, seq_len, heads, head_dim))",
          py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("scale_Q"), py::arg("scale_K"),
          py::arg("scale_V"), py::arg("is_causal") = false, py::arg("out_bshd") = false);
    m.def("int8_decode_attention_forward", &int8_decode_attention_forward_torch,
          "INT8 flash-decoding attention (seq_q==1, INT8 KV cache) — returns FP16");
    // Two overloads: scalar scales (per-tensor) and tensor scales (per-token
    // activation + per-channel weight); pybind11 dispatches by argument type.
    m.def("int8_mlp_forward", &int8_mlp_forward_torch,
          "INT8 MLP, per-tensor scales — returns (int8_out, out_scale)");
    m.def("int8_mlp_forward", &int8_mlp_forward_pc_torch,
          "INT8 MLP, per-token/per-channel scales — returns (int8_out, out_scale[T])");
    m.def("int8_mlp_forward_per_channel_bias", &int8_mlp_forward_pc_bias_torch,
          "INT8 MLP, per-token/per-channel scales + per-channel pre-GELU bias b1 — "
          "returns (int8_out, out_scale[T])");
    m.def("transpose_int8_weights", &transpose_int8_weights_torch,
          "Pre-transpose INT8 W1/W2 to [N][K] for the prepacked MLP path — returns (W1T, W2T)");
    m.def("int8_mlp_forward_prepacked", &int8_mlp_forward_prepacked_torch,
          "INT8 MLP, per-tensor scales, pre-transposed weights — returns (int8_out, out_scale)");
    m.def("int8_mlp_forward_prepacked", &int8_mlp_forward_prepacked_pc_torch,
          "INT8 MLP, per-token/per-channel scales, pre-transposed weights — "
          "returns (int8_out, out_scale[T])");
    // Not in the reference's module: quant utils it keeps C++-only, the
    // per-token quantizer every caller runs in PyTorch, and the KV cache.
    m.def("quantize_fp16_to_int8", &quantize_fp16_to_int8_torch,
          "Per-tensor fp16 -> int8 — returns (int8, scale[1])");
    m.def("dequantize_int8_to_fp16", &dequantize_int8_to_fp16_torch,
          "int8 -> fp16 with a scalar scale");
    m.def("quantize_per_token", &quantize_per_token_torch,
          "Per-token (last dim) int8 quantization — returns (int8, fp32 scales)");
    m.def("dequantize_per_token", &dequantize_per_token_torch,
          "Per-token int8 -> float (q * s[..., None]) rounded to dtype, plus an optional "
          "residual (whose dtype then sets the output's)",
          py::arg("q"), py::arg("scales"), py::arg("residual") = py::none(),
          py::arg("dtype") = py::none());
    m.def("layernorm_quantize_per_token", &layernorm_quantize_per_token_torch,
          "LayerNorm (last dim) then per-token int8 — returns (int8, fp32 scales)",
          py::arg("x"), py::arg("weight") = py::none(), py::arg("bias") = py::none(),
          py::arg("eps") = 1e-5);
    m.def("quantize_heads", &quantize_heads_torch,
          "Split (batch, seq, parts*heads*head_dim) into heads and quantize per token — "
          "returns [q_0, s_0, q_1, s_1, ...]",
          py::arg("x"), py::arg("heads"), py::arg("parts") = 3);
    m.def("kv_cache_append", &kv_cache_append_torch,
          "Quantize new K/V tokens into an int8 KV cache at position pos (in place)");
    m.def("int8_decode_attention_forward_paged", &int8_decode_attention_forward_paged_torch,
          "INT8 decode attention over a paged KV cache (block tables, per-sequence lengths)");
    m.def("int8_decode_attention_forward_cache", &int8_decode_attention_forward_cache_torch,
          "INT8 decode attention over the first seq_len positions of a KV cache — returns FP16");
    // The attention output emitted as int8 + per-token scales (the per-token
    // quantization of the fp16 rows the ops above return).
    m.def("int8_attention_forward_quant", &int8_attention_forward_quant_torch,
          "INT8 attention emitting per-token int8 — returns (int8, fp32 scales)",
          py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("scale_Q"), py::arg("scale_K"),
          py::arg("scale_V"), py::arg("is_causal") = false, py::arg("out_bshd") = false);
    m.def("int8_decode_attention_forward_quant", &int8_decode_attention_forward_quant_torch,
          "INT8 decode attention emitting per-token int8 — returns (int8, fp32 scales)");
    m.def("int8_decode_attention_forward_cache_quant",
          &int8_decode_attention_forward_cache_quant_torch,
          "INT8 decode over a KV cache emitting per-token int8 — returns (int8, fp32 scales)");
    m.def("int8_decode_attention_forward_paged_quant",
          &int8_decode_attention_forward_paged_quant_torch,
          "INT8 paged decode emitting per-token int8 — returns (int8, fp32 scales)");
    m.attr("abi_version") = int8k_abi_version();
}
