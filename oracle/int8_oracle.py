"""CPU oracle for the INT8 kernels — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.  The product path (libint8k + int8_ext)
never calls it and has no CPU fallback.

Each function restates, from scratch in numpy, the math of one reference
function (cited file:line, relative to the reference checkout).  Integer work
is exact (int64 accumulation); fp32 steps keep the reference's operation order
in float32 so rounding-sensitive outputs (fp16 hidden, int8 requant) land
within one LSB of the kernels; attention is evaluated in float64 (the
reference's oracle is dequant -> fp32 SDPA, common/baseline.py:7-22).

How each function is pinned (tests/test_oracle.py):
  quantize_per_token / per_channel_w / per_tensor : closed-form KATs (zeros,
      constant rows, codes +-127/126 on boundary data, round-half-even ties),
      reconstruction bound |x - q*s| <= s/2.
  decode_attention / prefill_attention : pure-Python brute force on tiny
      shapes, S=1 -> V row, constant K -> mean of V, permutation invariance,
      causal row 0 -> V[0], agreement with torch's own SDPA (an independent
      library routine) on dequantized inputs, and the C restatement.
  gemm_i8_i32 : pure-Python triple loop on small shapes, identity/permutation
      matrices, the C restatement, extreme values (-128*-128*K).
  gelu_tanh_f32 : closed-form points and torch.nn.functional.gelu(approximate
      ="tanh") as an independent routine.
  mlp_forward : stage-by-stage against the pieces above on small shapes plus
      KATs (zero input -> zero output codes; constant input -> one code).
  quantize_fp16_per_tensor / dequantize_int8_to_fp16 : closed form + KATs.
  dequantize_per_token_residual : PyTorch's own ops on the CPU (the reference block
      runs exactly those) for fp16/bf16/fp32 with and without a residual, and
      crafted (q, s) pairs whose fp32 product double-rounds to a different fp16
      than the exact product (the two-step rounding is what is pinned).
  layernorm_quantize_per_token : torch.nn.functional.layer_norm (an independent
      library routine) on the same inputs, then quantize_per_token; closed
      form for a two-valued row (y = +-1 -> codes +-127).
  quantize_heads : a pure-Python loop over (b, s, part, h) rows on small shapes.
  gather_paged_kv / decode_attention_paged : identity block tables over a
      contiguous cache reproduce decode_attention exactly; a permuted table
      with permuted pages gives the same result; positions past a sequence's
      length never enter (changing them changes nothing).
No function is left "parity unpinned".
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
F16 = np.float16

# ----------------------------------------------------------------------------
# Quantizers
# ----------------------------------------------------------------------------


def quantize_per_token(x):
    """Per-token (last-dim) symmetric int8 quantization.

    Reference: validation/check_decode.py:42-47, validation/validate_int8.py:63-66,
    tests/test_int8.py:47-63 — s = max(amax_row, 1e-8)/127 (fp32),
    q = clamp(round_half_even(x / s), -128, 127).
    Returns (q int8 [..., D], s float32 [...]).
    """
    xf = np.asarray(x, dtype=F32)
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    amax = np.maximum(amax, F32(1e-8))
    s = (amax / F32(127.0)).astype(F32)
    q = np.clip(np.rint(xf / s), -128, 127).astype(np.int8)
    return q, s[..., 0].copy()


def quantize_per_channel_w(w):
    """Per-output-channel weight quant, w [in, out] -> (int8 [in,out], s [out]).

    Reference: validation/validate_int8.py:75-81 (amax over dim 0).
    """
    wf = np.asarray(w, dtype=F32)
    amax = np.maximum(np.abs(wf).max(axis=0), F32(1e-8))
    s = (amax / F32(127.0)).astype(F32)
    q = np.clip(np.rint(wf / s[None, :]), -128, 127).astype(np.int8)
    return q, s


def quantize_per_tensor(x):
    """Per-tensor symmetric quant: validation/validate_int8.py:58-61."""
    xf = np.asarray(x, dtype=F32)
    s = F32(max(float(np.abs(xf).max()) if xf.size else 0.0, 1e-8)) / F32(127.0)
    s = F32(s)
    q = np.clip(np.rint(xf / s), -128, 127).astype(np.int8)
    return q, s


def dequantize(q, s):
    """q * s broadcast over the last dim (per-token) — float32."""
    return np.asarray(q, dtype=F32) * np.asarray(s, dtype=F32)[..., None]


# ----------------------------------------------------------------------------
# Attention
# ----------------------------------------------------------------------------


def decode_attention(Qi, Ki, Vi, sQ, sK, sV):
    """Single-query attention over an int8 KV cache, float64.

    Reference: the contract of int8_decode_attention_forward
    (kernels/int8_decode_attention.cu:333, 361, 415-425, 448) and its checker
    validation/check_decode.py:65-68 (SDPA on dequantized Q/K/V).
    Shapes: Qi [BH, D], Ki/Vi [BH, S, D] int8; sQ [BH]; sK/sV [BH, S].
    Returns float64 [BH, D].
    """
    Qi = np.asarray(Qi)
    BH, D = Qi.shape
    S = np.asarray(Ki).shape[1]
    q = Qi.astype(np.float64) * np.asarray(sQ, np.float64).reshape(BH, 1)
    k = np.asarray(Ki).astype(np.float64) * np.asarray(sK, np.float64).reshape(BH, S, 1)
    v = np.asarray(Vi).astype(np.float64) * np.asarray(sV, np.float64).reshape(BH, S, 1)
    scores = np.einsum("bd,bsd->bs", q, k) / math.sqrt(D)
    scores -= scores.max(axis=1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("bs,bsd->bd", p, v)


def gather_paged_kv(pages, block_tables, context_len, b, page_size):
    """Positions 0 .. context_len-1 of sequence b from a paged array
    [num_pages, H, page_size, ...]: position j is pages[block_tables[b][j // page_size], :,
    j % page_size].  Returns [H, context_len, ...].  No reference counterpart (its decode is
    contiguous only, kernels/int8_decode_attention.cu:443-547); this is the layout contract of
    int8k_decode_attention_forward_paged."""
    pages = np.asarray(pages)
    j = np.arange(context_len)
    pg = np.asarray(block_tables)[b][j // page_size]
    return np.moveaxis(pages[pg, :, j % page_size], 0, 1)


def decode_attention_paged(Qi, K_pages, V_pages, sQ, sK_pages, sV_pages, block_tables,
                           context_lens):
    """decode_attention per sequence over its gathered pages.
    Qi [B, H, D]; K/V_pages [num_pages, H, P, D]; sQ [B, H]; sK/sV_pages [num_pages, H, P];
    block_tables [B, max_pages]; context_lens [B].  Returns float64 [B, H, D]."""
    Qi = np.asarray(Qi)
    B, H, D = Qi.shape
    P = np.asarray(K_pages).shape[2]
    out = np.zeros((B, H, D))
    for b in range(B):
        n = int(context_lens[b])
        if n <= 0:
            continue
        k = gather_paged_kv(K_pages, block_tables, n, b, P)
        v = gather_paged_kv(V_pages, block_tables, n, b, P)
        sk = gather_paged_kv(sK_pages, block_tables, n, b, P)
        sv = gather_paged_kv(sV_pages, block_tables, n, b, P)
        out[b] = decode_attention(Qi[b], k, v, np.asarray(sQ)[b], sk, sv)
    return out


def prefill_attention(Qi, Ki, Vi, sQ, sK, sV, causal=False):
    """Full (seq_q == seq_kv) attention on per-token int8 inputs, float64.

    Reference: int8_attention_forward (kernels/int8_attention.cu:926-1028;
    scores kernels/int8_attention.cu:292-298, 467-488; softmax 489-506;
    P.V 530-572; normalisation 622-643) checked in tests/test_int8.py:109-123
    against common/baseline.py:18-22 on dequantized inputs.  The reference is
    non-causal only; causal=True applies the standard lower-triangular mask
    (query i sees keys 0..i), which the reference cannot pin.
    Shapes: [BH, S, D] int8; scales [BH, S].  Returns float64 [BH, S, D].
    """
    Qi = np.asarray(Qi)
    BH, S, D = Qi.shape
    def deq64(a, s):
        return np.asarray(a).astype(np.float64) * np.asarray(s, np.float64).reshape(BH, S, 1)

    q, k, v = deq64(Qi, sQ), deq64(Ki, sK), deq64(Vi, sV)
    scores = np.einsum("bid,bjd->bij", q, k) / math.sqrt(D)
    if causal:
        mask = np.triu(np.ones((S, S), dtype=bool), k=1)
        scores = np.where(mask[None], -np.inf, scores)
    scores -= scores.max(axis=2, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=2, keepdims=True)
    return np.einsum("bij,bjd->bid", p, v)


# ----------------------------------------------------------------------------
# GEMM + MLP
# ----------------------------------------------------------------------------


def gemm_i8_i32(A, B):
    """Exact int8 x int8 -> int32 matmul, A [M,K] @ B [K,N].

    Reference: the s8 x s8 -> s32 mainloop of kernels/int8_mlp.cu:242-310.
    Raises if a sum leaves int32 (the kernels accumulate in int32).
    """
    acc = np.asarray(A, np.int64) @ np.asarray(B, np.int64)
    if acc.size and (acc.max() > 2**31 - 1 or acc.min() < -(2**31)):
        raise OverflowError("int32 accumulator overflow")
    return acc.astype(np.int32)


def gelu_tanh_f32(x):
    """GELU, tanh form, in float32: kernels/int8_common.cuh:8-13."""
    x = np.asarray(x, F32)
    kC = F32(0.7978845608028654)
    kA = F32(0.044715)
    inner = kC * (x + kA * x * x * x)
    return (F32(0.5) * x * (F32(1.0) + np.tanh(inner).astype(F32))).astype(F32)


def requant_rows_f16(h16, amax):
    """Per-row requant of an fp16 matrix given per-row fp32 absmax.

    Reference: quantize_rows_kernel (kernels/int8_mlp.cu:768-795):
    amax' = max(amax, 1e-8); inv = 127/amax'; q = rn(clamp(h*inv)); s = amax'/127.
    """
    amax = np.maximum(np.asarray(amax, F32), F32(1e-8))
    inv = (F32(127.0) / amax).astype(F32)
    hf = np.asarray(h16, F16).astype(F32)
    q = np.rint(np.clip(hf * inv[:, None], F32(-128.0), F32(127.0))).astype(np.int8)
    return q, (amax / F32(127.0)).astype(F32)


def requant_tensor_f16(o16, amax):
    """Per-tensor requant: quantize_tensor_kernel (kernels/int8_mlp.cu:799-825)."""
    amax = F32(max(float(amax), 1e-8))
    inv = F32(F32(127.0) / amax)
    of = np.asarray(o16, F16).astype(F32)
    q = np.rint(np.clip(of * inv, F32(-128.0), F32(127.0))).astype(np.int8)
    return q, F32(amax / F32(127.0))


def _as_scale(s, n):
    s = np.asarray(s, F32).reshape(-1)
    if s.size == 1:
        return np.full(n, s[0], F32)
    assert s.size == n, (s.size, n)
    return s


def mlp_forward(x, W1, W2, sx, sW1, sW2, bias1=None, per_token_out=True, return_stages=False,
                gemm=None):
    """Two-GEMM int8 MLP with dynamic per-token hidden requant.

    Reference: int8_mlp_forward_impl dynamic path (kernels/int8_mlp.cu:999-1191):
      GEMM1 epilogue (kernels/int8_mlp.cu:441-449): v = (f32(acc1)*sA)*sB (+b1),
        v = GELU(v), hidden = fp16(v), row absmax over |v| in fp32;
      quantize_rows (kernels/int8_mlp.cu:768-795) -> int8 hidden + sh[t];
      GEMM2 epilogue: o = (f32(acc2)*sh[t])*sW2 -> fp16, absmax of |o|;
      output quant per token (per-channel entry, kernels/int8_mlp.cu:1165-1173)
      or per tensor (scalar entry, kernels/int8_mlp.cu:1176-1190).
    x [T, dm] int8; W1 [dm, dff] int8; W2 [dff, dm] int8; sx [T] or [1];
    sW1 [dff] or [1]; sW2 [dm] or [1]; bias1 [dff] or None.
    Returns (out int8 [T, dm], out_scale [T] or scalar) and, when asked, the
    intermediate stages.  `gemm` may supply another exact int8 GEMM (the C
    restatement) for speed.
    """
    gemm = gemm or gemm_i8_i32
    x = np.asarray(x, np.int8)
    T, dm = x.shape
    dff = np.asarray(W1).shape[1]
    sxv = _as_scale(sx, T)
    s1 = _as_scale(sW1, dff)
    s2 = _as_scale(sW2, dm)

    acc1 = gemm(x, W1)
    v = (acc1.astype(F32) * sxv[:, None]).astype(F32) * s1[None, :]
    v = v.astype(F32)
    if bias1 is not None:
        v = (v + np.asarray(bias1, F32)[None, :]).astype(F32)
    v = gelu_tanh_f32(v)
    h16 = v.astype(F16)
    h_amax = np.abs(v).max(axis=1).astype(F32) if dff else np.zeros(T, F32)
    hq, sh = requant_rows_f16(h16, h_amax)

    acc2 = gemm(hq, W2)
    o = ((acc2.astype(F32) * sh[:, None]).astype(F32) * s2[None, :]).astype(F32)
    o16 = o.astype(F16)
    if per_token_out:
        o_amax = np.abs(o).max(axis=1).astype(F32)
        out, out_scale = requant_rows_f16(o16, o_amax)
    else:
        out, out_scale = requant_tensor_f16(o16, np.abs(o).max() if o.size else 0.0)
    if return_stages:
        return out, out_scale, dict(acc1=acc1, v=v, h16=h16, h_amax=h_amax, hq=hq, sh=sh,
                                    acc2=acc2, o=o, o16=o16)
    return out, out_scale


def mlp_dequant_reference(x, W1, W2, sx, sW1, sW2, bias1=None):
    """Float64 Linear -> GELU(tanh) -> Linear on dequantized inputs.

    Reference: common/baseline.py:25-37 (mlp_baseline) fed dequantized
    operands, as tests/test_int8.py:130-154 and validate_int8.py do.
    """
    x = np.asarray(x)
    T, dm = x.shape
    dff = np.asarray(W1).shape[1]
    xd = x.astype(np.float64) * _as_scale(sx, T).astype(np.float64)[:, None]
    w1 = np.asarray(W1).astype(np.float64) * _as_scale(sW1, dff).astype(np.float64)[None, :]
    w2 = np.asarray(W2).astype(np.float64) * _as_scale(sW2, dm).astype(np.float64)[None, :]
    h = xd @ w1
    if bias1 is not None:
        h = h + np.asarray(bias1, np.float64)[None, :]
    h = 0.5 * h * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (h + 0.044715 * h ** 3)))
    return h @ w2


# ----------------------------------------------------------------------------
# quant utils (per-tensor fp16 <-> int8)
# ----------------------------------------------------------------------------


def quantize_fp16_per_tensor(x16):
    """Per-tensor fp16 -> int8 with a device-computed scale.

    Reference: quantize_fp16_to_int8 (kernels/quant_utils.cu:56-69):
    amax over |x| (fp32), scale = amax/127, q = rn(clamp(x / scale)).
    Deliberate fix: amax is clamped to 1e-8 first, as every Python quantizer
    of the reference does; the reference kernel returns scale 0 and code -128
    on all-zero input (kernels/quant_utils.cu:29-31, 39-40).
    """
    xf = np.asarray(x16, F16).astype(F32)
    amax = F32(np.abs(xf).max()) if xf.size else F32(0.0)
    scale = F32(max(amax, F32(1e-8)) / F32(127.0))
    q = np.rint(np.clip(xf / scale, F32(-128.0), F32(127.0))).astype(np.int8)
    return q, scale


def dequantize_int8_to_fp16(q, scale):
    """half(q * scale): kernels/quant_utils.cu:44-49, 72-77."""
    return (np.asarray(q, F32) * F32(scale)).astype(F16)


def _round_to(y, dtype):
    """Round float values to the storage dtype ("f16", "bf16", "f32") and back to float32."""
    y = np.asarray(y, np.float32)
    if dtype == "f16":
        return y.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = y.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        return r.view(np.float32)
    return y


def dequantize_per_token_residual(q, s, dtype="f16", residual=None):
    """Consumer side of the block's INT8 MLP: (q.float() * s[..., None]).to(dtype), then
    residual + that in the residual's dtype (bench/bench_block.py:107-113, 126-127).
    Every step rounds on its own: the fp32 product, then `dtype`; with a residual the
    fp32 sum of the two `dtype` values, then `dtype` again.  Returns float32 values."""
    y = _round_to(np.asarray(q, F32) * np.asarray(s, F32)[..., None], dtype)
    if residual is not None:
        y = _round_to(np.asarray(residual, F32) + y, dtype)
    return y


def layernorm_quantize_per_token(x, gamma=None, beta=None, eps=1e-5, dtype="f16"):
    """LayerNorm over the last dim (float64 statistics, biased variance, eps inside the
    sqrt, optional affine), rounded to `dtype` as F.layer_norm's output would be, then
    quantize_per_token.  Producer fusion of the reference block's LN -> _q_per_token
    (bench/bench_block.py:59-63, 94-95, 119-121).  Returns (q int8, scales fp32, y fp32)."""
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)
    if beta is not None:
        y = y + np.asarray(beta, np.float64)
    y = _round_to(y.astype(np.float32), dtype)
    q, s = quantize_per_token(y)
    return q, s, y


def quantize_heads(x, heads, parts=3):
    """x [B, S, parts*heads*Dh] -> per part (q [B, H, S, Dh] int8, s [B, H, S] fp32): the
    reference block's split_heads + .contiguous() + _q_per_token on Q, K and V
    (bench/bench_block.py:97-102, 119-120)."""
    x = np.asarray(x, np.float32)
    B, S, W = x.shape
    Dh = W // (parts * heads)
    v = x.reshape(B, S, parts, heads, Dh).transpose(2, 0, 3, 1, 4)  # [P, B, H, S, Dh]
    return [quantize_per_token(np.ascontiguousarray(v[p])) for p in range(parts)]
