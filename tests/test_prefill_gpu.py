"""Parity of INT8 prefill attention against the CPU oracle (GPU tests).

Shapes: the reference's attention configs (tests/test_int8.py:78-86: batch 2,
heads 8, seq 512/1024, head_dim 64/128/256) non-causal as the reference, plus
the causal mask this build adds, ragged lengths, every other head_dim up to
512, known-answer cases, a large-V-scale case and the BASELINE config 5 (B4 H32
S4096 D128 causal) at full size, every head.
Bar: max-abs <= 2e-2 and cosine >= 0.9999 against dequant -> float64 SDPA.
"""

import numpy as np
import pytest
import torch

import workloads
from helpers import assert_attn_close
from oracle import oracle_c

pytestmark = pytest.mark.gpu

REFERENCE_CONFIGS = [(2, 8, 512, 64), (2, 8, 512, 128), (2, 8, 512, 256),
                     (2, 8, 1024, 64), (2, 8, 1024, 128), (2, 8, 1024, 256)]


def _cpu(case):
    return {k: v.cpu().numpy() for k, v in case.items()}


def _oracle(case, causal):
    n = _cpu(case)
    B, H, S, D = n["Qi"].shape
    BH = B * H
    return oracle_c.prefill_attention(n["Qi"].reshape(BH, S, D), n["Ki"].reshape(BH, S, D),
                                      n["Vi"].reshape(BH, S, D), n["sQ"].reshape(BH, S),
                                      n["sK"].reshape(BH, S), n["sV"].reshape(BH, S),
                                      causal=causal).reshape(B, H, S, D)


def _run(ext, case, causal):
    out = ext.int8_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                     case["sK"], case["sV"], causal)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("B,H,S,D", REFERENCE_CONFIGS)
def test_prefill_reference_configs(ext, gpu, B, H, S, D):
    case = workloads.prefill_case(B, H, S, D, seed=42, device=gpu, gen_device="cpu")
    out = _run(ext, case, False)
    assert_attn_close(out, _oracle(case, False), f"B{B} H{H} S{S} D{D}")


@pytest.mark.parametrize("S,D", [(1, 64), (31, 128), (100, 64), (200, 128), (257, 128),
                                 (513, 128), (767, 128), (1000, 256), (1024, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_ragged_and_causal(ext, gpu, S, D, causal):
    case = workloads.prefill_case(1, 3, S, D, seed=S + D, device=gpu, gen_device="cpu")
    out = _run(ext, case, causal)
    assert_attn_close(out, _oracle(case, causal), f"S{S} D{D} causal={causal}")


# Head dims besides 64/128/256: multiples of 16 run the MFMA kernel padded to the
# next of those sizes; the rest (and 320, 512) run the generic kernel, as the
# reference's scalar fallback takes every head_dim (kernels/int8_attention.cu:65-157).
OTHER_HEAD_DIMS = [16, 32, 48, 80, 96, 112, 160, 192, 240, 8, 33, 40, 72, 100, 130, 320, 512]


@pytest.mark.parametrize("D", OTHER_HEAD_DIMS)
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_other_head_dims(ext, gpu, D, causal):
    S = 200 if D <= 256 else 100
    case = workloads.prefill_case(2, 2, S, D, seed=D, device=gpu, gen_device="cpu")
    out = _run(ext, case, causal)
    assert out.shape == (2, 2, S, D)
    assert_attn_close(out, _oracle(case, causal), f"D{D} S{S} causal={causal}")


@pytest.mark.parametrize("D", [80, 72])
def test_prefill_other_head_dims_quant_and_bshd(ext, gpu, D):
    # int8 output = per-token quantization of the fp16 output, byte for byte; [B,S,H,D] rows
    case = workloads.prefill_case(2, 3, 150, D, seed=D + 1, device=gpu, gen_device="cpu")
    a = [case[k] for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")]
    o16 = ext.int8_attention_forward(*a, True)
    oq, osc = ext.int8_attention_forward_quant(*a, True)
    rq, rs = ext.quantize_per_token(o16)
    torch.cuda.synchronize()
    assert torch.equal(oq, rq) and torch.equal(osc, rs)
    ob = ext.int8_attention_forward(*a, True, True)
    assert torch.equal(ob, o16.transpose(1, 2).contiguous())


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,key,D", [(192, 150, 64), (193, 192, 64), (195, 194, 128),
                                     (4097, 4096, 128)])
def test_prefill_large_v_scale_stays_finite(ext, gpu, causal, S, key, D):
    # A V row of absmax 635000 (sV = 5000, legal for fp32/bf16 sources) in a later
    # tile whose best key beats the running max by 3.9 log2 units: a fast path that
    # allowed p up to 16 would form P' = fp16(14.9 * 5000) = inf.  The reference keeps
    # p <= 1 there (kernels/int8_attention.cu:489-506, 530-572) and stays finite.
    # The large row also sits at the last key of ragged lengths (S % 4 = 1, 3), where the
    # kernel's V-scale exponent must still see it.
    B, H = 1, 2
    g = torch.Generator().manual_seed(11)
    Qf = torch.ones(B, H, S, D)
    Kf = torch.zeros(B, H, S, D)
    Kf[:, :, key] = 2.70 / D ** 0.5     # score 2.70 nats for every query; all others 0
    Vf = torch.randn(B, H, S, D, generator=g)
    Vf[:, :, key] *= 635000.0 / Vf[:, :, key].abs().amax(-1, keepdim=True)
    c = {}
    for name, x in (("Q", Qf), ("K", Kf), ("V", Vf)):
        q, s = workloads.quantize_per_token(x)
        c[name + "i"], c["s" + name] = q.to(gpu), s.to(gpu)
    assert 4094 < float(c["sV"][0, 0, key]) < 5001
    out = _run(ext, c, causal)
    ref = _oracle(c, causal)
    assert np.isfinite(out).all()
    scale = np.abs(ref).max()
    assert scale > 1e3  # the large row dominates the rows that see it (else |out| ~ 1)
    rel = np.abs(out - ref).max() / scale
    assert rel < 2e-3, rel
    from helpers import cosine
    assert cosine(out, ref) >= 0.9999


def test_prefill_capi_matches_ext(capi, ext, gpu):
    case = workloads.prefill_case(2, 2, 300, 128, seed=9, device=gpu, gen_device="cpu")
    a = ext.int8_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"], case["sK"],
                                   case["sV"])
    b = capi.attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"].reshape(-1),
                               case["sK"].reshape(-1), case["sV"].reshape(-1))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_prefill_kats(ext, gpu):
    B, H, S, D = 1, 2, 200, 128
    case = workloads.prefill_case(B, H, S, D, seed=4, device=gpu, gen_device="cpu")
    # constant keys: uniform softmax -> every (non-causal) row is the mean of V
    c = dict(case)
    c["Ki"] = case["Ki"][:, :, :1].expand(B, H, S, D).contiguous()
    c["sK"] = case["sK"][:, :, :1].expand(B, H, S).contiguous()
    out = _run(ext, c, False)
    vd = case["Vi"].float().cpu().numpy() * case["sV"].cpu().numpy()[..., None]
    assert np.abs(out - vd.mean(axis=2, keepdims=True)).max() < 2e-3
    # causal: query 0 sees only key 0
    out = _run(ext, case, True)
    np.testing.assert_allclose(out[:, :, 0], vd[:, :, 0], atol=2e-3)
    # zeros dataset
    z = {k: torch.zeros_like(v) for k, v in case.items()}
    for k in ("sQ", "sK", "sV"):
        z[k] = torch.full_like(case[k], 1e-8 / 127)
    out = _run(ext, z, False)
    assert np.isfinite(out).all() and np.abs(out).max() == 0.0


def test_prefill_argument_errors(ext, gpu):
    case = workloads.prefill_case(1, 1, 64, 64, seed=1, device=gpu, gen_device="cpu")
    args = [case[k] for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")]
    with pytest.raises(RuntimeError, match="Q/K/V shape mismatch"):
        ext.int8_attention_forward(args[0], args[1][:, :, :32].contiguous(), *args[2:])
    with pytest.raises(RuntimeError, match="head_dim 1..512"):
        x = torch.zeros(1, 1, 8, 520, dtype=torch.int8, device=gpu)
        s = torch.ones(8, device=gpu)
        ext.int8_attention_forward(x, x, x, s, s, s)
    with pytest.raises(RuntimeError, match="scale_K must be float32"):
        ext.int8_attention_forward(*args[:4], args[4].double(), args[5])


def test_prefill_baseline_cfg5_full_size(ext, gpu):
    # B=4 H=32 S=4096 D=128, causal; every head against the C oracle
    # (float64 attention on the dequantized inputs).
    B, H, S, D = 4, 32, 4096, 128
    case = workloads.prefill_case(B, H, S, D, seed=5, device=gpu)
    out = ext.int8_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                     case["sK"], case["sV"], True)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = _oracle(case, True)
    for b in range(B):
        assert_attn_close(got[b], ref[b], f"cfg5 b{b}")
