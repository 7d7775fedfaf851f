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

// ── decode attention (seq_q == 1) ─────────────────────────────────────────
// Mirrors int8_decode_attention_forward_torch (kernels/int8_ext.cu:136-178).
// Q : (batch, heads, head_dim) int8; K, V : (batch, heads, seq_kv, head_dim)
// int8; scale_Q numel batch*heads; scale_K/V numel batch*heads*seq_kv (fp32).
// Returns (batch, heads, head_dim) fp16.
torch::Tensor int8_decode_attention_forward_torch(torch::Tensor Q, torch::Tensor K,
                                                  torch::Tensor V, torch::Tensor scale_Q,
                                                  torch::Tensor scale_K, torch::Tensor scale_V) {
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
    auto out = torch::empty({batch, heads, head_dim},
                            torch::TensorOptions().dtype(torch::kFloat16).device(Q.device()));
    const size_t ws_bytes =
        int8k_decode_attention_workspace_bytes((int)BH, (int)seq_kv, (int)head_dim, 0);
    auto ws = workspace(ws_bytes, Q.device());
    const int st = int8k_decode_attention_forward(
        q.data_ptr<int8_t>(), k.data_ptr<int8_t>(), v.data_ptr<int8_t>(),
        reinterpret_cast<uint16_t*>(out.data_ptr<at::Half>()), sQ.data_ptr<float>(),
        sK.data_ptr<float>(), sV.data_ptr<float>(), (int)BH, (int)seq_kv, (int)head_dim, 0,
        ws.data_ptr(), ws_bytes, current_stream(Q));
    check_status(st, "int8_decode_attention_forward");
    return out;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("int8_decode_attention_forward", &int8_decode_attention_forward_torch,
          "INT8 flash-decoding attention (seq_q==1, INT8 KV cache) — returns FP16");
    m.attr("abi_version") = int8k_abi_version();
}
