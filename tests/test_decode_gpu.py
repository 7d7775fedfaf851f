"""Parity of the split-KV decode kernel against the CPU oracle (GPU tests).

Cases mirror the reference's decode checker (validation/check_decode.py:50-53:
S tails, nsplit = 1, empty chunks, deep combines) plus the BASELINE configs.
The kernel is driven through the C ABI (int8k_capi) and through the drop-in
torch op (int8_ext.int8_decode_attention_forward).
"""
import numpy as np
import pytest
import torch

import workloads
from helpers import assert_attn_close
from oracle import int8_oracle, oracle_c

pytestmark = pytest.mark.gpu

CHECK_DECODE_CASES = [(1, 1, 64, 1), (1, 1, 64, 31), (2, 2, 64, 33), (1, 2, 64, 127),
                      (2, 2, 64, 128), (3, 5, 64, 1000), (8, 8, 64, 4096), (64, 16, 64, 8192),
                      (1, 1, 128, 1), (1, 1, 128, 31), (2, 2, 128, 33), (1, 2, 128, 127),
                      (2, 2, 128, 128), (3, 5, 128, 1000), (8, 8, 128, 4096),
                      (64, 16, 128, 8192)]


def _flat(case):
    B, H = case["Qi"].shape[:2]
    D = case["Qi"].shape[-1]
    S = case["Ki"].shape[2]
    BH = B * H
    return (case["Qi"].reshape(BH, D), case["Ki"].reshape(BH, S, D),
            case["Vi"].reshape(BH, S, D), case["sQ"].reshape(BH), case["sK"].reshape(BH * S),
            case["sV"].reshape(BH * S))


def _oracle(case, rows=None):
    Q, K, V, sQ, sK, sV = (t.cpu().numpy() for t in _flat(case))
    BH, D = Q.shape
    S = K.shape[1]
    sK, sV = sK.reshape(BH, S), sV.reshape(BH, S)
    if rows is not None:
        Q, K, V, sQ, sK, sV = Q[rows], K[rows], V[rows], sQ[rows], sK[rows], sV[rows]
    return oracle_c.decode_attention(Q, K, V, sQ, sK, sV)


def _run_capi(capi, case, nsplit=0):
    out = capi.decode_attention(*_flat(case), nsplit=nsplit)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("B,H,D,S", CHECK_DECODE_CASES)
def test_decode_check_cases(capi, gpu, B, H, D, S):
    big = B * H * S * D > (1 << 26)
    case = workloads.decode_case(B, H, D, S, seed=1234 + S, device=gpu,
                                 gen_device=gpu if big else "cpu")
    out = _run_capi(capi, case)
    ref = _oracle(case)
    assert_attn_close(out, ref, f"B{B} H{H} D{D} S{S}")


@pytest.mark.parametrize("D", [64, 128])
def test_decode_split_invariance(capi, gpu, D):
    # up to 16 chunks per (b,h) run as one launch (chunks merged in LDS), more as the
    # split + combine pair: the result does not depend on the split count either way
    case = workloads.decode_case(3, 5, D, 3000, seed=7, device=gpu, gen_device="cpu")
    ref = _oracle(case)
    outs = []
    for ns in (1, 2, 3, 5, 8, 16, 17, 24, 100):
        got = capi.decode_num_splits(15, 3000, D, ns)
        assert 1 <= got <= ns
        out = _run_capi(capi, case, nsplit=ns)
        assert_attn_close(out, ref, f"nsplit={ns}")
        outs.append(out)
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() <= 2e-3


@pytest.mark.parametrize("D", [64, 128])
def test_decode_chunk_iteration_counts(capi, gpu, D):
    # chunks of 0..9 whole wave iterations plus masked tails, at 1, 2, 3 and 8 chunks
    # per (b,h): at D=64 these take the one-launch kernel's two-register-set loop
    # (every parity of the iteration count, the rotated start, the last pair)
    rows = 64  # rows per wave iteration at the default slots, both head dims
    for S in (1, 40, rows, rows + 9, 2 * rows, 3 * rows - 1, 3 * rows, 5 * rows + 17, 9 * rows,
              19 * rows + 3):
        case = workloads.decode_case(2, 3, D, S, seed=S, device=gpu, gen_device="cpu")
        ref = _oracle(case)
        for ns in (1, 2, 3, 8):
            out = _run_capi(capi, case, nsplit=ns)
            assert_attn_close(out, ref, f"D{D} S{S} nsplit={ns}")


@pytest.mark.parametrize("D", [64, 128])
def test_decode_few_heads_long_context(capi, gpu, D):
    # few (b,h) and a long context: the automatic plan has more than 16 chunks per
    # (b,h), so it runs the split kernel and the combine kernel
    case = workloads.decode_case(1, 2, D, 40000, seed=17, outlier_frac=0.01, device=gpu)
    assert capi.decode_num_splits(2, 40000, D, 0) > 16
    out = _run_capi(capi, case)
    assert_attn_close(out, _oracle(case), f"B1 H2 D{D} S40000")


@pytest.mark.parametrize("D", [64, 128])
def test_decode_single_position_returns_v_row(capi, gpu, D):
    # S = 1: softmax over one key is 1, so out = V[0] * sV[0] exactly (fp16-rounded).
    case = workloads.decode_case(4, 3, D, 1, seed=11, device=gpu, gen_device="cpu")
    out = _run_capi(capi, case)
    Q, K, V, sQ, sK, sV = (t.cpu().numpy() for t in _flat(case))
    expect = (V[:, 0, :].astype(np.float32) * sV.reshape(-1, 1)).astype(np.float16)
    np.testing.assert_array_equal(out.astype(np.float16), expect)


@pytest.mark.parametrize("D", [64, 128])
def test_decode_constant_keys_average_values(capi, gpu, D):
    # Identical keys give uniform softmax weights: out = mean_j V[j]*sV[j].
    case = workloads.decode_case(2, 2, D, 777, seed=3, device=gpu, gen_device="cpu")
    case["Ki"][:] = case["Ki"][:, :, :1, :]
    case["sK"][:] = case["sK"][:, :, :1]
    out = _run_capi(capi, case)
    V = case["Vi"].reshape(4, 777, D).cpu().numpy().astype(np.float64)
    sV = case["sV"].reshape(4, 777, 1).cpu().numpy().astype(np.float64)
    expect = (V * sV).mean(axis=1)
    assert np.abs(out - expect).max() <= 2e-3


def test_decode_zero_inputs(capi, gpu):
    # The reference's `zeros` dataset: all-zero codes -> all-zero output, no NaN.
    B, H, D, S = 2, 4, 128, 300
    z = dict(Qi=torch.zeros(B, H, D, dtype=torch.int8, device=gpu),
             Ki=torch.zeros(B, H, S, D, dtype=torch.int8, device=gpu),
             Vi=torch.zeros(B, H, S, D, dtype=torch.int8, device=gpu),
             sQ=torch.full((B, H), 1e-8 / 127, device=gpu),
             sK=torch.full((B, H, S), 1e-8 / 127, device=gpu),
             sV=torch.full((B, H, S), 1e-8 / 127, device=gpu))
    out = _run_capi(capi, z)
    assert np.isfinite(out).all() and np.abs(out).max() == 0.0


def test_decode_position_permutation_invariance(capi, gpu):
    case = workloads.decode_case(2, 3, 128, 513, seed=5, device=gpu, gen_device="cpu")
    out = _run_capi(capi, case)
    perm = torch.randperm(513, generator=torch.Generator().manual_seed(1)).to(gpu)
    pcase = dict(case)
    pcase["Ki"] = case["Ki"][:, :, perm].contiguous()
    pcase["Vi"] = case["Vi"][:, :, perm].contiguous()
    pcase["sK"] = case["sK"][:, :, perm].contiguous()
    pcase["sV"] = case["sV"][:, :, perm].contiguous()
    pout = _run_capi(capi, pcase)
    assert np.abs(out - pout).max() <= 2e-3


def test_decode_baseline_cfg1(capi, ext, gpu):
    # B=1 H=12 D=64 ctx=1024, checked in full.
    case = workloads.decode_case(1, 12, 64, 1024, seed=2024, device=gpu, gen_device="cpu")
    out = ext.int8_decode_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                            case["sK"], case["sV"])
    assert out.dtype == torch.float16 and tuple(out.shape) == (1, 12, 64)
    ref = _oracle(case).reshape(1, 12, 64)
    assert_attn_close(out.float().cpu().numpy(), ref, "cfg1")
    # the numpy restatement agrees with the C one on this case
    Q, K, V, sQ, sK, sV = (t.cpu().numpy() for t in _flat(case))
    ref_np = int8_oracle.decode_attention(Q, K, V, sQ, sK.reshape(12, 1024), sV.reshape(12, 1024))
    assert np.abs(ref_np - ref.reshape(12, 64)).max() < 1e-9


@pytest.mark.parametrize("B,H,D,S", [(32, 32, 128, 8192), (8, 32, 64, 32768),
                                     (8, 32, 64, 2048), (8, 32, 64, 4096), (8, 32, 64, 8192),
                                     (8, 32, 64, 16384)])
def test_decode_baseline_full_size(capi, ext, gpu, B, H, D, S):
    # BASELINE configs 2 and 3 and config 3's ctx sweep at full size, 1% outlier
    # channels x8: every (b,h) row against the C oracle, plus finiteness and the
    # |out| <= max|V_deq| convexity bound.
    print(f"decode full size B{B} H{H} D{D} S{S}", flush=True)
    case = workloads.decode_case(B, H, D, S, seed=99, outlier_frac=0.01, device=gpu)
    out = ext.int8_decode_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                            case["sK"], case["sV"])
    torch.cuda.synchronize()
    o = out.float().reshape(B * H, D)
    assert torch.isfinite(o).all()
    vmax = (case["Vi"].abs().float().amax(dim=-1) * case["sV"]).amax(dim=-1).reshape(B * H)
    assert (o.abs().amax(dim=-1) <= vmax * (1 + 1e-3) + 1e-6).all()
    ref = _oracle(case)
    assert_attn_close(o.cpu().numpy(), ref, f"full B{B} H{H} D{D} S{S}")


def test_decode_ext_scale_shapes_and_views(ext, gpu):
    case = workloads.decode_case(2, 3, 128, 200, seed=8, device=gpu, gen_device="cpu")
    a = ext.int8_decode_attention_forward(case["Qi"], case["Ki"], case["Vi"], case["sQ"],
                                          case["sK"], case["sV"])
    # flat scale tensors are accepted (numel is what matters)
    b = ext.int8_decode_attention_forward(case["Qi"], case["Ki"], case["Vi"],
                                          case["sQ"].reshape(-1), case["sK"].reshape(-1),
                                          case["sV"].reshape(-1))
    assert torch.equal(a, b)
    # a contiguous view whose storage offset breaks 16-byte alignment still works
    buf = torch.empty(case["Ki"].numel() + 1, dtype=torch.int8, device=gpu)
    kview = buf[1:].view_as(case["Ki"])
    kview.copy_(case["Ki"])
    c = ext.int8_decode_attention_forward(case["Qi"], kview, case["Vi"], case["sQ"],
                                          case["sK"], case["sV"])
    assert torch.equal(a, c)


def test_decode_ext_argument_errors(ext, gpu):
    case = workloads.decode_case(1, 2, 128, 16, seed=1, device=gpu, gen_device="cpu")
    args = [case["Qi"], case["Ki"], case["Vi"], case["sQ"], case["sK"], case["sV"]]
    with pytest.raises(RuntimeError, match="head_dim 64 or 128"):
        q = torch.zeros(1, 2, 96, dtype=torch.int8, device=gpu)
        k = torch.zeros(1, 2, 16, 96, dtype=torch.int8, device=gpu)
        ext.int8_decode_attention_forward(q, k, k, *args[3:])
    with pytest.raises(RuntimeError, match="Q must be int8"):
        ext.int8_decode_attention_forward(args[0].float(), *args[1:])
    with pytest.raises(RuntimeError, match="K/V shape mismatch"):
        ext.int8_decode_attention_forward(args[0], args[1], args[2][:, :, :8].contiguous(),
                                          *args[3:])
    with pytest.raises(RuntimeError, match="seq_q == 1"):
        ext.int8_decode_attention_forward(args[1], *args[1:])
    with pytest.raises(RuntimeError, match="contiguous"):
        ext.int8_decode_attention_forward(args[0], args[1].transpose(2, 3), *args[2:])
