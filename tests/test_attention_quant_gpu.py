"""Attention outputs emitted as per-token int8 (GPU tests).

The `_quant` entry points must give, byte for byte, the per-token quantization
(int8k_quantize_per_token) of the fp16 rows their fp16 counterparts return: the same
fp16 values, their row absmax, the per-token quantizer's scale and codes.  The
per-token quantizer itself is pinned bit-exactly against the CPU oracle in
test_quant_gpu.py; here the fused output is also checked end to end against the
oracle quantizer applied to the fp16 kernel output, and its dequantized values against
the attention oracle.  Cases: prefill causal and non-causal for every head_dim,
ragged sequence lengths; decode contiguous with the automatic and forced split counts
(one split takes the fp16 path's in-kernel final write, the int8 path the combine
pass), over a cache and over pages.
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from helpers import assert_attn_close
from oracle import int8_oracle as O

pytestmark = pytest.mark.gpu


def _two_step(ext, out16):
    return ext.quantize_per_token(out16)


def _assert_same(q, s, rq, rs, label):
    assert q.dtype == torch.int8 and s.dtype == torch.float32, label
    assert q.shape == rq.shape and s.shape == rs.shape, label
    assert torch.equal(s, rs), f"{label}: scales differ"
    assert torch.equal(q, rq), f"{label}: codes differ ({int((q != rq).sum())} elements)"


@pytest.mark.parametrize("D,S,causal", [(64, 300, False), (64, 129, True), (128, 200, True),
                                        (128, 64, False), (256, 77, True)])
def test_prefill_quant_equals_quantized_fp16(ext, gpu, D, S, causal):
    c = workloads.prefill_case(2, 2, S, D, seed=D + S, device=gpu)
    args = (c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"])
    out16 = ext.int8_attention_forward(*args, is_causal=causal)
    q, s = ext.int8_attention_forward_quant(*args, is_causal=causal)
    rq, rs = _two_step(ext, out16)
    torch.cuda.synchronize()
    _assert_same(q, s, rq, rs, f"prefill D{D} S{S} causal={causal}")
    # the C ABI directly, and the oracle's quantizer on the fp16 output
    q2, s2 = capi.attention_forward_quant(*args, causal=causal)
    torch.cuda.synchronize()
    _assert_same(q2, s2, rq, rs, "prefill C ABI")
    oq, os_ = O.quantize_per_token(out16.float().cpu().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), oq)
    np.testing.assert_array_equal(s.cpu().numpy(), os_)
    # dequantized, against the attention oracle (a half step of the scale on top)
    BH = 4
    flat = [t.reshape(BH, S, D) if t.dim() == 4 else t.reshape(BH, S) for t in args]
    ref = O.prefill_attention(*(t.cpu().numpy() for t in flat), causal=causal)
    deq = (q.float() * s.unsqueeze(-1)).reshape(BH, S, D).cpu().numpy()
    assert np.abs(deq - ref).max() <= 2e-2 + 0.5 * float(s.max())


@pytest.mark.parametrize("D,S,causal", [(64, 300, False), (128, 513, True), (256, 77, False)])
def test_prefill_bshd_output_is_the_transpose(ext, gpu, D, S, causal):
    # [B, S, H, D] rows (the output projection's order) are the [B, H, S, D] rows,
    # byte for byte, for the fp16 and the int8 outputs
    B, H = 2, 3
    c = workloads.prefill_case(B, H, S, D, seed=7 * D + S, device=gpu)
    args = (c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"])
    ref = ext.int8_attention_forward(*args, is_causal=causal)
    got = ext.int8_attention_forward(*args, is_causal=causal, out_bshd=True)
    rq, rs = ext.int8_attention_forward_quant(*args, is_causal=causal)
    q, s = ext.int8_attention_forward_quant(*args, is_causal=causal, out_bshd=True)
    got2 = capi.attention_forward(*args, causal=causal, out_bshd=True)
    q2, s2 = capi.attention_forward_quant(*args, causal=causal, out_bshd=True)
    torch.cuda.synchronize()
    assert got.shape == (B, S, H, D) and q.shape == (B, S, H, D) and s.shape == (B, S, H)
    want = ref.transpose(1, 2)
    assert torch.equal(got, want) and torch.equal(got2, want)
    _assert_same(q, s, rq.transpose(1, 2), rs.transpose(1, 2), f"bshd D{D} S{S}")
    _assert_same(q2, s2, rq.transpose(1, 2), rs.transpose(1, 2), "bshd C ABI")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nsplit", [0, 1, 5])
def test_decode_quant_equals_quantized_fp16(ext, gpu, D, nsplit):
    B, H, S = 3, 4, 333
    c = workloads.decode_case(B, H, D, S, seed=D + nsplit, device=gpu)
    BH = B * H
    flat = (c["Qi"].reshape(BH, D), c["Ki"].reshape(BH, S, D), c["Vi"].reshape(BH, S, D),
            c["sQ"].reshape(-1), c["sK"].reshape(-1), c["sV"].reshape(-1))
    out16 = capi.decode_attention(*flat, nsplit=nsplit)
    q, s = capi.decode_attention_quant(*flat, nsplit=nsplit)
    rq, rs = _two_step(ext, out16)
    torch.cuda.synchronize()
    _assert_same(q, s, rq, rs, f"decode D{D} nsplit={nsplit}")
    ref = O.decode_attention(*(t.cpu().numpy() for t in flat))
    assert_attn_close((q.float() * s.unsqueeze(-1)).cpu().numpy(), ref, "decode quant")


def test_decode_quant_torch_ops(ext, gpu):
    B, H, D, S, cap = 2, 3, 128, 500, 640
    c = workloads.decode_case(B, H, D, S, seed=21, device=gpu)
    args = (c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"])
    q, s = ext.int8_decode_attention_forward_quant(*args)
    rq, rs = _two_step(ext, ext.int8_decode_attention_forward(*args))
    torch.cuda.synchronize()
    assert q.shape == (B, H, D) and s.shape == (B, H)
    _assert_same(q, s, rq, rs, "decode op")
    # the same rows through a larger cache
    Kc = torch.zeros((B, H, cap, D), dtype=torch.int8, device=gpu)
    Vc = torch.zeros_like(Kc)
    sKc = torch.ones((B, H, cap), dtype=torch.float32, device=gpu)
    sVc = torch.ones_like(sKc)
    Kc[:, :, :S] = c["Ki"]
    Vc[:, :, :S] = c["Vi"]
    sKc[:, :, :S] = c["sK"]
    sVc[:, :, :S] = c["sV"]
    qc, sc = ext.int8_decode_attention_forward_cache_quant(c["Qi"], Kc, Vc, c["sQ"], sKc, sVc, S)
    rqc, rsc = _two_step(ext, ext.int8_decode_attention_forward_cache(c["Qi"], Kc, Vc, c["sQ"],
                                                                      sKc, sVc, S))
    torch.cuda.synchronize()
    _assert_same(qc, sc, rqc, rsc, "decode cache op")
    _assert_same(qc, sc, q, s, "cache vs contiguous")


@pytest.mark.parametrize("nsplit", [0, 1])
def test_paged_decode_quant(ext, gpu, nsplit):
    lens = [1, 15, 17, 300, 1024]
    c = workloads.paged_case(len(lens), 4, 64, 16, lens, seed=30 + nsplit, device=gpu)
    args = (c["Qi"], c["K_pages"], c["V_pages"], c["sQ"], c["sK_pages"], c["sV_pages"],
            c["block_tables"], c["context_lens"], c["max_context"])
    q, s = capi.decode_attention_paged_quant(*args, nsplit=nsplit)
    rq, rs = _two_step(ext, capi.decode_attention_paged(*args, nsplit=nsplit))
    torch.cuda.synchronize()
    _assert_same(q, s, rq, rs, f"paged nsplit={nsplit}")
    qo, so = ext.int8_decode_attention_forward_paged_quant(*args)
    torch.cuda.synchronize()
    _assert_same(qo, so, *_two_step(ext, ext.int8_decode_attention_forward_paged(*args)),
                 "paged op")


def test_quant_entry_validation(gpu):
    lib = capi.load()
    c = workloads.prefill_case(1, 1, 64, 64, seed=1, device=gpu)
    q = torch.empty((1, 1, 64, 64), dtype=torch.int8, device=gpu)
    s = torch.empty((1, 1, 64), dtype=torch.float32, device=gpu)
    p = capi._ptr
    base = (p(c["Qi"]), p(c["Ki"]), p(c["Vi"]))
    sc = (p(c["sQ"]), p(c["sK"]), p(c["sV"]))
    # a missing scale output is an invalid argument, an unaligned one misaligned
    assert lib.int8k_attention_forward_quant(*base, p(q), None, *sc, 1, 1, 64, 64, 0,
                                             capi._stream(q)) == capi.INT8K_ERR_INVALID_ARGUMENT
    s_bytes = torch.empty(64 * 4 + 4, dtype=torch.uint8, device=gpu)
    bad = capi.ctypes.c_void_p(s_bytes.data_ptr() + 2)
    assert lib.int8k_attention_forward_quant(*base, p(q), bad, *sc, 1, 1, 64, 64, 0,
                                             capi._stream(q)) == capi.INT8K_ERR_MISALIGNED
    assert lib.int8k_decode_attention_forward_quant(
        p(c["Qi"]), p(c["Ki"]), p(c["Vi"]), None, p(s), *sc, 1, 64, 64, 0, None, 0,
        capi._stream(q)) == capi.INT8K_ERR_INVALID_ARGUMENT
