"""Pre-LN transformer block with the INT8 kernels, beside its FP16 form.

The block of the reference's bench/bench_block.py:73-151:

    h = x + Wo . Attn(split_heads(LN1(x) . Wqkv))
    y = h + MLP(LN2(h)),   MLP = Linear -> GELU(tanh) -> Linear

The INT8 form runs the attention core and the MLP on this library, with its
producer-fused quantizers: the QKV projection output is split into heads and
quantized per token in one pass (`quantize_heads`), LN2 and the MLP input's
per-token quantization are one pass (`layernorm_quantize_per_token`), the
prefill attention writes its rows in the output projection's [B, S, H, Dh]
order, and the MLP output's dequantization is fused with the residual add
(`dequantize_per_token`).  LayerNorm 1, the QKV / output projections and the
first residual add stay FP16 in both forms, as in the reference.

`capture`, when given a dict, receives every intermediate of the INT8 form
(the tests check each stage against the CPU oracle's piece).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

import int8_ext as ext
import workloads


class TransformerBlock:
    """Random-init weights (seeded) of one block: d_model = heads * head_dim."""

    def __init__(self, d_model: int, heads: int, d_ff: int, device, seed: int = 0):
        if d_model % heads:
            raise ValueError("d_model must be a multiple of heads")
        self.d, self.H, self.Dh, self.dff = d_model, heads, d_model // heads, d_ff
        g = torch.Generator(device=device).manual_seed(seed)

        def rn(*shape):
            return torch.randn(*shape, generator=g, device=device, dtype=torch.float16)

        self.Wqkv = rn(d_model, 3 * d_model) * (d_model ** -0.5)
        self.Wo = rn(d_model, d_model) * (d_model ** -0.5)
        self.W1 = rn(d_model, d_ff) * (d_model ** -0.5)
        self.W2 = rn(d_ff, d_model) * (d_ff ** -0.5)
        self.W1i, self.sW1 = workloads.quantize_per_channel_w(self.W1)
        self.W2i, self.sW2 = workloads.quantize_per_channel_w(self.W2)
        self.W1T, self.W2T = ext.transpose_int8_weights(self.W1i, self.W2i)

    # -- MLP sub-block ------------------------------------------------------
    def mlp_int8_residual(self, h, capture=None):
        """h + MLP(LN2(h)) on the INT8 MLP; the output's dequantization and the
        residual add are one pass (the reference: h + (out.float() * out_scale).half())."""
        B, S, d = h.shape
        xi, sx = ext.layernorm_quantize_per_token(h)
        o, so = ext.int8_mlp_forward_prepacked(xi.view(B, S, d), self.W1T, self.W2T,
                                               sx.reshape(-1), self.sW1, self.sW2)
        y = ext.dequantize_per_token(o.view(B, S, d), so.view(B, S), residual=h)
        if capture is not None:
            capture.update(h=h, xi=xi, sx=sx, o=o, so=so, y=y)
        return y

    def mlp_fp16(self, h):
        return F.gelu(F.layer_norm(h, (self.d,)) @ self.W1, approximate="tanh") @ self.W2

    # -- prefill --------------------------------------------------------------
    def prefill(self, x, int8: bool, capture=None):
        """x [B, S, d_model] fp16 -> y [B, S, d_model]; non-causal attention, as the
        reference block (F.scaled_dot_product_attention without a mask)."""
        B, S, _ = x.shape
        qkv = F.layer_norm(x, (self.d,)) @ self.Wqkv
        if int8:
            qi, sq, ki, sk, vi, sv = ext.quantize_heads(qkv, self.H)
            # rows come out as [B, S, H, Dh], the projection's order: no transpose copy
            a = ext.int8_attention_forward(qi, ki, vi, sq, sk, sv, out_bshd=True)
            if capture is not None:
                capture.update(qkv=qkv, qi=qi, sq=sq, ki=ki, sk=sk, vi=vi, sv=sv, attn=a)
            a = a.view(B, S, self.d)
        else:
            q, k, v = (t.view(B, S, self.H, self.Dh).transpose(1, 2).contiguous()
                       for t in qkv.split(self.d, dim=-1))
            a = F.scaled_dot_product_attention(q, k, v)
            a = a.transpose(1, 2).contiguous().view(B, S, self.d)
        h = x + a @ self.Wo
        return self.mlp_int8_residual(h, capture) if int8 else h + self.mlp_fp16(h)

    # -- decode ---------------------------------------------------------------
    def decode(self, x, kv, int8: bool, capture=None):
        """One new token per sequence, x [B, 1, d_model], against a KV cache:
        int8 (Ki, Vi [B,H,S,Dh], sK, sV [B,H,S]) or fp16 (Kf, Vf [B,H,S,Dh])."""
        B = x.size(0)
        q = (F.layer_norm(x, (self.d,)) @ self.Wqkv)[..., :self.d]
        if int8:
            Ki, Vi, sK, sV = kv
            qi, sq = ext.quantize_per_token(q.reshape(B, self.H, self.Dh))
            a = ext.int8_decode_attention_forward(qi, Ki, Vi, sq, sK, sV)
            if capture is not None:
                capture.update(q=q, qi=qi, sq=sq, attn=a)
            a = a.view(B, 1, self.d)
        else:
            Kf, Vf = kv
            a = F.scaled_dot_product_attention(q.view(B, self.H, 1, self.Dh), Kf, Vf)
            a = a.transpose(1, 2).contiguous().view(B, 1, self.d)
        h = x + a @ self.Wo
        return self.mlp_int8_residual(h, capture) if int8 else h + self.mlp_fp16(h)
