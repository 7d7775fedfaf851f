"""Parity of INT8 prefill attention against the CPU oracle (GPU tests).

Shapes: the reference's attention configs (tests/test_int8.py:78-86: batch 2,
heads 8, seq 512/1024, head_dim 64/128/256) non-causal as the reference, plus
the causal mask this build adds, ragged lengths, known-answer cases and the
BASELINE config 5 (B4 H32 S4096 D128 causal) at full size with sampled rows.
Bar: max-abs <= 2e-2 and cosine >= 0.9999 against dequant -> float64 SDPA.
"""
import math

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
    with pytest.raises(RuntimeError, match="head_dim 64, 128 or 256"):
        x = torch.zeros(1, 1, 8, 96, dtype=torch.int8, device=gpu)
        s = torch.ones(8, device=gpu)
        ext.int8_attention_forward(x, x, x, s, s, s)
    with pytest.raises(RuntimeError, match="scale_K must be float32"):
        ext.int8_attention_forward(*args[:4], args[4].double(), args[5])


def test_prefill_baseline_cfg5_full_size_sampled(ext, gpu):
    # B=4 H=32 S=4096 D=128, causal.  Sampled rows of two
    # heads against float64 attention on the dequantized inputs.
    B, H, S, D = 4, 32, 4096, 128
    case = workloads.prefill_case(B, H, S, D, seed=5, device=gpu)
    out = ext.int8_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                     case["sK"], case["sV"], True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    rng = np.random.default_rng(0)
    for b, hh in ((0, 0), (3, 31)):
        q = case["Qi"][b, hh].cpu().numpy().astype(np.float64) * case["sQ"][b, hh].cpu().numpy()[:, None]
        k = case["Ki"][b, hh].cpu().numpy().astype(np.float64) * case["sK"][b, hh].cpu().numpy()[:, None]
        v = case["Vi"][b, hh].cpu().numpy().astype(np.float64) * case["sV"][b, hh].cpu().numpy()[:, None]
        rows = np.concatenate([[0, 1, 127, 128, S - 1], rng.choice(S, 59, replace=False)])
        ref = np.empty((len(rows), D))
        for n, i in enumerate(rows):
            sc = k[: i + 1] @ q[i] / math.sqrt(D)
            p = np.exp(sc - sc.max())
            ref[n] = p @ v[: i + 1] / p.sum()
        got = out[b, hh].float().cpu().numpy()[rows]
        assert_attn_close(got, ref, f"cfg5 b{b} h{hh}")
