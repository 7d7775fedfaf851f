"""Producer-fused quantizers (GPU tests): LayerNorm -> per-token int8 and split-heads ->
per-token int8, against the CPU oracle (whose LayerNorm is pinned to
torch.nn.functional.layer_norm) and against the two-step torch path they replace.

Bars: int8 codes within 1 LSB and scales within 1e-3 relative for the LayerNorm path
(the kernel's fp32 statistics may round y to a neighbouring fp16/bf16 value), bit-exact
for split-heads (same quantizer on the same values).
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from oracle import int8_oracle as O

pytestmark = pytest.mark.gpu

_DT = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
# (37, 1000) and fp32 rows of 8192 take the block-per-row kernel; the others spread a row
# over 8..64 lanes with 1..16 chunks of 16 bytes per lane.
@pytest.mark.parametrize("rows,cols", [(1, 64), (37, 1000), (19, 1024), (5, 3072), (256, 4096),
                                       (3, 8192)])
@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_quantize(gpu, dtype, rows, cols, affine):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 2 + 0.5).to(dtype)
    gamma = torch.rand(cols, generator=g) + 0.5 if affine else None
    beta = torch.rand(cols, generator=g) - 0.5 if affine else None
    q, s, y = capi.layernorm_quantize_per_token(
        x.to(gpu), gamma.to(gpu) if affine else None, beta.to(gpu) if affine else None,
        1e-5, want_y=True)
    torch.cuda.synchronize()
    rq, rs, ry = O.layernorm_quantize_per_token(
        x.float().numpy(), gamma.numpy() if affine else None, beta.numpy() if affine else None,
        1e-5, _DT[dtype])
    # one storage ulp (fp16, bf16); for fp32 output the fp32 row statistics themselves differ
    # from the float64 oracle by ~sqrt(cols) roundings
    ulp = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -17}[dtype]
    yd = np.abs(y.float().cpu().numpy() - ry)
    assert np.all(yd <= ulp * np.maximum(np.abs(ry), 2.0 ** -14) + 1e-7), yd.max()
    assert np.abs(q.cpu().numpy().astype(np.int32) - rq).max() <= 1
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-3)


def test_layernorm_quantize_unaligned_source(gpu):
    # a source that is not 16-byte aligned takes the block-per-row kernel
    rows, cols = 6, 1024
    base = torch.randn(rows * cols + 1, generator=torch.Generator().manual_seed(4)).half().to(gpu)
    x = base[1:].view(rows, cols)
    q, s, y = capi.layernorm_quantize_per_token(x, None, None, 1e-5, want_y=True)
    torch.cuda.synchronize()
    rq, rs, ry = O.layernorm_quantize_per_token(x.float().cpu().numpy(), None, None, 1e-5, "f16")
    yd = np.abs(y.float().cpu().numpy() - ry)
    assert np.all(yd <= 2.0 ** -10 * np.maximum(np.abs(ry), 2.0 ** -14) + 1e-7), yd.max()
    assert np.abs(q.cpu().numpy().astype(np.int32) - rq).max() <= 1
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-3)


def test_layernorm_quantize_torch_op_matches_two_step(ext, gpu):
    # the reference block's LN2 -> _q_per_token (bench/bench_block.py:59-63, 94-95, 121)
    x = torch.randn(8, 128, 1024, generator=torch.Generator().manual_seed(1)).half().to(gpu)
    q, s = ext.layernorm_quantize_per_token(x)
    y = torch.nn.functional.layer_norm(x, (1024,))
    rq, rs = workloads.quantize_per_token(y.float().cpu())
    assert q.shape == x.shape and s.shape == x.shape[:-1]
    assert int((q.cpu().int() - rq.int()).abs().max()) <= 1
    torch.testing.assert_close(s.cpu(), rs, rtol=1e-3, atol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
# Dh 48 (and fp32 Dh 512) take the one-element-per-lane kernel, the others one 16-byte chunk
# per lane.
@pytest.mark.parametrize("B,S,H,Dh,parts", [(1, 1, 1, 64, 1), (2, 37, 4, 64, 3), (2, 512, 16, 128, 3),
                                             (3, 5, 2, 128, 2), (2, 9, 3, 48, 3), (1, 7, 2, 256, 3),
                                             (1, 3, 1, 512, 2)])
def test_quantize_heads(ext, gpu, dtype, B, S, H, Dh, parts):
    g = torch.Generator().manual_seed(B * S + H)
    x = (torch.randn(B, S, parts * H * Dh, generator=g) * 3).to(dtype)
    outs = ext.quantize_heads(x.to(gpu), H, parts)
    torch.cuda.synchronize()
    ref = O.quantize_heads(x.float().numpy(), H, parts)
    assert len(outs) == 2 * parts
    for p in range(parts):
        np.testing.assert_array_equal(outs[2 * p].cpu().numpy(), ref[p][0])
        np.testing.assert_array_equal(outs[2 * p + 1].cpu().numpy(), ref[p][1])
    # the same result as the reference block's split_heads + _q_per_token
    qkv = x.float().view(B, S, parts, H, Dh)
    for p in range(parts):
        rq, rs = workloads.quantize_per_token(qkv[:, :, p].transpose(1, 2).contiguous())
        assert torch.equal(outs[2 * p].cpu(), rq) and torch.equal(outs[2 * p + 1].cpu(), rs)


def test_quantize_heads_feeds_attention(ext, gpu):
    B, S, H, Dh = 2, 256, 4, 64
    x = torch.randn(B, S, 3 * H * Dh, generator=torch.Generator().manual_seed(2)).half().to(gpu)
    qi, sq, ki, sk, vi, sv = ext.quantize_heads(x, H)
    out = ext.int8_attention_forward(qi, ki, vi, sq, sk, sv, True)
    torch.cuda.synchronize()
    assert out.shape == (B, H, S, Dh) and torch.isfinite(out.float()).all()
