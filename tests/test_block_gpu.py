"""The end-to-end pre-LN block (block.TransformerBlock, the reference's
bench/bench_block.py:73-151) as a tested component (GPU tests).

Each stage of the INT8 block is checked against the CPU oracle's piece fed the
block's own input to that stage:
  * split-heads + per-token quantization of the QKV projection: bit-exact;
  * prefill / decode attention: max-abs <= 2e-2, cos >= 0.9999 (float64 oracle);
  * LayerNorm 2 + per-token quantization: codes within 1 LSB, scales 1e-3 relative
    (the kernel's fp32 statistics may round y to a neighbouring fp16);
  * the INT8 MLP: codes within 1 LSB, at most 2% of them off by one;
  * the output's dequantization + residual add: bit-exact;
and the whole block against the FP16 block: cos >= 0.9999.
"""
import numpy as np
import pytest
import torch

import int8_ext as ext
from block import TransformerBlock
from helpers import assert_attn_close, cosine
from oracle import int8_oracle as O
from oracle import oracle_c

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def _check_mlp_stages(blk, cap, T):
    d = blk.d
    h = cap["h"].reshape(T, d)
    # LayerNorm 2 + per-token quantization
    rq, rs, _ = O.layernorm_quantize_per_token(_np(h), None, None, 1e-5, "f16")
    q = _np(cap["xi"]).reshape(T, d).astype(np.int32)
    assert np.abs(q - rq.astype(np.int32)).max() <= 1
    np.testing.assert_allclose(_np(cap["sx"]).reshape(T), rs, rtol=1e-3)
    # the INT8 MLP on the block's own codes
    ref, rsc = O.mlp_forward(_np(cap["xi"]).reshape(T, d), _np(blk.W1i), _np(blk.W2i),
                             _np(cap["sx"]).reshape(T), _np(blk.sW1), _np(blk.sW2),
                             gemm=oracle_c.gemm_i8_i32)
    o = _np(cap["o"]).reshape(T, d).astype(np.int32)
    diff = np.abs(o - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff != 0).mean() <= 0.02
    np.testing.assert_allclose(_np(cap["so"]).reshape(T), rsc, rtol=2e-3)
    # dequantization of the block's own output codes + the residual add
    y = O.dequantize_per_token_residual(_np(cap["o"]).reshape(T, d), _np(cap["so"]).reshape(T),
                                        "f16", residual=_np(h))
    np.testing.assert_array_equal(_np(cap["y"]).reshape(T, d), y)


@pytest.mark.parametrize("B,S,d,H,dff", [(2, 128, 256, 4, 1024), (1, 300, 512, 8, 2048)])
def test_block_prefill_stages_and_end_to_end(gpu, B, S, d, H, dff):
    blk = TransformerBlock(d, H, dff, gpu, seed=3)
    g = torch.Generator(device=gpu).manual_seed(S)
    x = torch.randn(B, S, d, generator=g, device=gpu, dtype=torch.float16)
    cap = {}
    y8 = blk.prefill(x, True, capture=cap)
    y16 = blk.prefill(x, False)
    torch.cuda.synchronize()
    Dh = d // H
    # split-heads + per-token quantization: bit-exact
    for (rq, rs), qn, sn in zip(O.quantize_heads(_np(cap["qkv"]), H),
                                ("qi", "ki", "vi"), ("sq", "sk", "sv")):
        np.testing.assert_array_equal(_np(cap[qn]), rq)
        np.testing.assert_array_equal(_np(cap[sn]), rs)
    # attention (non-causal, as the reference block) on the block's own codes
    BH = B * H
    ref = oracle_c.prefill_attention(*(_np(cap[k]).reshape(BH, S, Dh) for k in ("qi", "ki", "vi")),
                                     *(_np(cap[k]).reshape(BH, S) for k in ("sq", "sk", "sv")))
    ref = ref.reshape(B, H, S, Dh).transpose(0, 2, 1, 3)  # the block keeps [B, S, H, Dh]
    assert_attn_close(_np(cap["attn"]), ref, "block prefill attention")
    _check_mlp_stages(blk, cap, B * S)
    c = cosine(_np(y8), _np(y16))
    assert c >= 0.9999, c


@pytest.mark.parametrize("B,Skv,d,H,dff", [(4, 512, 256, 4, 1024), (16, 2048, 1024, 16, 4096)])
def test_block_decode_stages_and_end_to_end(gpu, B, Skv, d, H, dff):
    blk = TransformerBlock(d, H, dff, gpu, seed=5)
    g = torch.Generator(device=gpu).manual_seed(Skv)
    Dh = d // H
    x = torch.randn(B, 1, d, generator=g, device=gpu, dtype=torch.float16)
    Kf = torch.randn(B, H, Skv, Dh, generator=g, device=gpu, dtype=torch.float16)
    Vf = torch.randn(B, H, Skv, Dh, generator=g, device=gpu, dtype=torch.float16)
    Ki, sK = ext.quantize_per_token(Kf)
    Vi, sV = ext.quantize_per_token(Vf)
    cap = {}
    y8 = blk.decode(x, (Ki, Vi, sK, sV), True, capture=cap)
    y16 = blk.decode(x, (Kf, Vf), False)
    torch.cuda.synchronize()
    # the cache and the query quantized per token: bit-exact against the oracle
    rq, rs = O.quantize_per_token(_np(Kf))
    np.testing.assert_array_equal(_np(Ki), rq)
    np.testing.assert_array_equal(_np(sK), rs)
    rq, rs = O.quantize_per_token(_np(cap["q"]).reshape(B, H, Dh))
    np.testing.assert_array_equal(_np(cap["qi"]), rq)
    np.testing.assert_array_equal(_np(cap["sq"]), rs)
    BH = B * H
    ref = oracle_c.decode_attention(_np(cap["qi"]).reshape(BH, Dh), _np(Ki).reshape(BH, Skv, Dh),
                                    _np(Vi).reshape(BH, Skv, Dh), _np(cap["sq"]).reshape(BH),
                                    _np(sK).reshape(BH, Skv), _np(sV).reshape(BH, Skv))
    assert_attn_close(_np(cap["attn"]).reshape(BH, Dh), ref, "block decode attention")
    _check_mlp_stages(blk, cap, B)
    c = cosine(_np(y8), _np(y16))
    assert c >= 0.9999, c
