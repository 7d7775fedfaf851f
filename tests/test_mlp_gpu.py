"""Parity of the INT8 MLP (and its raw GEMM core) against the CPU oracle (GPU tests).

Bar: int32 accumulators bit-exact; int8 outputs within +-1 LSB of the oracle
(the oracle keeps the reference's fp32 epilogue order — kernels/int8_mlp.cu:441-449,
768-795 — so only transcendental/FMA rounding can differ); output scales to
fp32 rounding.  Shapes cover the reference's per-tensor MLP check
(tests/test_int8.py:130-154: 2x512, 512 -> 2048), ragged tiles, bias, the
prepacked path and the BASELINE config 4 at full size (sampled rows — each
output row depends only on its own input row).
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from oracle import int8_oracle as O
from oracle import oracle_c

pytestmark = pytest.mark.gpu

# Largest tolerated share of +-1 LSB disagreements between kernel and oracle.
MAX_FLIP_FRACTION = 0.02


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (512, 768, 256), (300, 200, 64),
                                   (1, 16, 16), (257, 513, 4112), (1000, 256, 128)])
def test_gemm_i32_bit_exact(gpu, M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    Bt = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    C = capi.gemm_i8_i32(A.to(gpu), Bt.to(gpu))
    torch.cuda.synchronize()
    ref = oracle_c.gemm_i8_i32(A.numpy(), Bt.numpy().T.copy())
    np.testing.assert_array_equal(_np(C), ref)


def test_gemm_i32_extreme_values(gpu):
    # |acc| = 16384 * 128 * 128 = 2^28: the deepest MLP reduction, all -128 codes
    M, N, K = 256, 256, 16384
    A = torch.full((M, K), -128, dtype=torch.int8, device=gpu)
    Bt = torch.full((N, K), -128, dtype=torch.int8, device=gpu)
    C = capi.gemm_i8_i32(A, Bt)
    torch.cuda.synchronize()
    assert int(C.min()) == int(C.max()) == K * 128 * 128


def _compare_mlp(out, out_scale, ref_out, ref_scale, label):
    out = np.asarray(out, np.int32)
    ref_out = np.asarray(ref_out, np.int32)
    diff = np.abs(out - ref_out)
    assert diff.max() <= 1, f"{label}: int8 output off by {diff.max()} LSB"
    flips = float((diff != 0).mean())
    assert flips <= MAX_FLIP_FRACTION, f"{label}: {flips:.4f} of codes differ by 1 LSB"
    np.testing.assert_allclose(np.asarray(out_scale, np.float64),
                               np.asarray(ref_scale, np.float64), rtol=2e-3)
    return flips


def _mlp_case(T, dm, dff, seed, gpu):
    c = workloads.mlp_case(T, dm, dff, seed=seed, device=gpu, gen_device="cpu")
    return c, {k: _np(v) for k, v in c.items()}


@pytest.mark.parametrize("T,dm,dff", [(1024, 512, 2048), (256, 1024, 4096), (100, 256, 768),
                                      (1, 64, 128), (300, 512, 1040)])
def test_mlp_per_channel_vs_oracle(capi_mlp, gpu, T, dm, dff):
    c, n = _mlp_case(T, dm, dff, seed=T + dm + dff, gpu=gpu)
    out, osc = capi.mlp_forward(c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"],
                                c["sW2"])
    torch.cuda.synchronize()
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out), _np(osc), ref, rsc, f"T{T} dm{dm} dff{dff}")


def test_mlp_bias_vs_oracle(ext, gpu):
    T, dm, dff = 384, 512, 2048
    c, n = _mlp_case(T, dm, dff, seed=42, gpu=gpu)
    bias = torch.randn(dff, generator=torch.Generator().manual_seed(1)) * 0.5
    out, osc = ext.int8_mlp_forward_per_channel_bias(c["x"], c["W1"], c["W2"], c["sx"],
                                                     c["sW1"], c["sW2"], bias.to(gpu))
    torch.cuda.synchronize()
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], bias1=bias.numpy(), gemm=oracle_c.gemm_i8_i32)
    assert tuple(out.shape) == (1, T, dm) and out.dtype == torch.int8
    _compare_mlp(_np(out).reshape(T, dm), _np(osc), ref, rsc, "bias")


# More than 512 rows, at most 128 tiles of 256 x 256 and no few-token path: both
# GEMMs run 128 x 128 tiles (gemm_i8_mid_kernel).  (2048, 1024, 4096): interior tiles;
# (1000, 528, 1040) and (777, 1040, 1552): ragged rows and columns, K not a multiple of
# 128 (the zero-filled operand path and the guarded epilogue).
@pytest.mark.parametrize("T,dm,dff", [(2048, 1024, 4096), (1000, 528, 1040), (777, 1040, 1552)])
def test_mlp_mid_tiles_vs_oracle(ext, gpu, T, dm, dff):
    c, n = _mlp_case(T, dm, dff, seed=T + 3 * dff, gpu=gpu)
    bias = torch.randn(dff, generator=torch.Generator().manual_seed(T)) * 0.5
    out, osc = ext.int8_mlp_forward_per_channel_bias(c["x"], c["W1"], c["W2"], c["sx"],
                                                     c["sW1"], c["sW2"], bias.to(gpu))
    torch.cuda.synchronize()
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], bias1=bias.numpy(), gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out).reshape(T, dm), _np(osc), ref, rsc, f"mid T{T} dm{dm} dff{dff}")
    # per-tensor output scale: the max over every 128-column partial
    out_t, osc_t = capi.mlp_forward(c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"],
                                    c["sW2"], flags=capi.MLP_OUT_PER_TENSOR)
    torch.cuda.synchronize()
    ref_t, rsc_t = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                                 n["sW2"], per_token_out=False, gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out_t), float(_np(osc_t).reshape(-1)[0]), ref_t, rsc_t,
                 f"mid per-tensor T{T}")


# Small GEMMs (M N K <= 2^31, K % 512 == 0) take the skinny path (32 x 32 tiles, K split
# over the waves of a block): 1, 33 (a partial row tile), 64, 128, 200, 256, 300 rows.
# K not a multiple of 512 takes split-K (128 x 128 tiles, K split over blocks, int32
# partials): GEMM2 of (96, 512, 1408), both GEMMs of (128, 640, 1408).
@pytest.mark.parametrize("T,dm,dff", [(128, 1024, 4096), (64, 512, 2048), (1, 512, 1024),
                                      (33, 512, 1024), (200, 1024, 4096), (256, 512, 2048),
                                      (300, 512, 1024), (96, 512, 1408), (128, 640, 1408)])
def test_mlp_few_tokens_split_k(capi_mlp, gpu, T, dm, dff):
    # decode-time token counts: fewer 256 x 256 tiles than CUs
    c, n = _mlp_case(T, dm, dff, seed=T + 5, gpu=gpu)
    out, osc = capi.mlp_forward(c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"],
                                c["sW2"])
    torch.cuda.synchronize()
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out), _np(osc), ref, rsc, f"split-K T{T}")
    # per-tensor output scale on the same path
    sx1 = c["sx"].reshape(-1)[:1].clone()
    sw1 = c["sW1"].reshape(-1)[:1].clone()
    sw2 = c["sW2"].reshape(-1)[:1].clone()
    out_t, osc_t = capi.mlp_forward(c["x"].reshape(T, dm), c["W1"], c["W2"], sx1, sw1, sw2,
                                    flags=capi.MLP_OUT_PER_TENSOR)
    torch.cuda.synchronize()
    ref_t, rsc_t = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], _np(sx1), _np(sw1),
                                 _np(sw2), per_token_out=False, gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out_t), _np(osc_t), ref_t, rsc_t, f"split-K per-tensor T{T}")


@pytest.mark.parametrize("T", [16, 128])
def test_mlp_few_tokens_bias(ext, gpu, T):
    # the bias on the skinny path (added before GELU)
    dm, dff = 512, 2048
    c, n = _mlp_case(T, dm, dff, seed=T + 77, gpu=gpu)
    bias = torch.randn(dff, generator=torch.Generator().manual_seed(T)) * 0.5
    out, osc = ext.int8_mlp_forward_per_channel_bias(c["x"], c["W1"], c["W2"], c["sx"],
                                                     c["sW1"], c["sW2"], bias.to(gpu))
    torch.cuda.synchronize()
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], bias1=bias.numpy(), gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out).reshape(T, dm), _np(osc), ref, rsc, f"bias T{T}")


def test_mlp_per_tensor_reference_config(ext, gpu):
    # tests/test_int8.py:130-154: batch 2, seq 512, 512 -> 2048, per-tensor scales
    g = torch.Generator().manual_seed(42)
    x = torch.randn(2, 512, 512, generator=g)
    W1 = torch.randn(512, 2048, generator=g) * 0.02
    W2 = torch.randn(2048, 512, generator=g) * 0.02
    xi, sx = O.quantize_per_tensor(x.numpy())
    w1i, s1 = O.quantize_per_tensor(W1.numpy())
    w2i, s2 = O.quantize_per_tensor(W2.numpy())
    out, osc = ext.int8_mlp_forward(torch.from_numpy(xi).to(gpu), torch.from_numpy(w1i).to(gpu),
                                    torch.from_numpy(w2i).to(gpu), float(sx), float(s1),
                                    float(s2))
    assert isinstance(osc, float) and tuple(out.shape) == (2, 512, 512)
    ref, rsc = O.mlp_forward(xi.reshape(1024, 512), w1i, w2i, sx, s1, s2, per_token_out=False,
                             gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out).reshape(1024, 512), osc, ref, rsc, "per-tensor")
    # and the dequantized result tracks the float MLP (common/baseline.py:25-37)
    deq = _np(out).reshape(1024, 512).astype(np.float64) * osc
    fref = O.mlp_dequant_reference(xi.reshape(1024, 512), w1i, w2i, sx, s1, s2)
    assert np.abs(deq - fref).max() < 0.1  # the reference's int8 atol (common/correctness.py:23)


def test_mlp_prepacked_matches_unpacked(ext, gpu):
    T, dm, dff = 512, 512, 2048
    c, _ = _mlp_case(T, dm, dff, seed=5, gpu=gpu)
    W1T, W2T = ext.transpose_int8_weights(c["W1"], c["W2"])
    assert torch.equal(W1T, c["W1"].t().contiguous()) and torch.equal(W2T, c["W2"].t().contiguous())
    a, sa = ext.int8_mlp_forward(c["x"], c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    b, sb = ext.int8_mlp_forward_prepacked(c["x"], W1T, W2T, c["sx"], c["sW1"], c["sW2"])
    assert torch.equal(a, b) and torch.equal(sa, sb)
    s = [float(v) for v in (0.01, 0.002, 0.003)]
    a, sa = ext.int8_mlp_forward(c["x"], c["W1"], c["W2"], *s)
    b, sb = ext.int8_mlp_forward_prepacked(c["x"], W1T, W2T, *s)
    assert torch.equal(a, b) and sa == sb


@pytest.mark.parametrize("dm,dff", [(512, 2048), (200, 300), (64, 129), (1000, 1040), (130, 4096),
                                    (33, 17)])
def test_transpose_int8_weights_shapes(gpu, dm, dff):
    # 128 x 128 tiles: interior tiles of 16-byte aligned matrices take the vector path,
    # edge tiles and other shapes the byte path; both give the exact transposes
    g = torch.Generator(device=gpu).manual_seed(dm * 7 + dff)
    W1 = torch.randint(-128, 128, (dm, dff), dtype=torch.int8, device=gpu, generator=g)
    W2 = torch.randint(-128, 128, (dff, dm), dtype=torch.int8, device=gpu, generator=g)
    W1T, W2T = capi.transpose_int8_weights(W1, W2)
    torch.cuda.synchronize()
    assert torch.equal(W1T, W1.t().contiguous()) and torch.equal(W2T, W2.t().contiguous())


def test_mlp_kats_zero_and_constant(ext, gpu):
    T, dm, dff = 256, 256, 512
    z = torch.zeros(1, T, dm, dtype=torch.int8, device=gpu)
    w1 = torch.zeros(dm, dff, dtype=torch.int8, device=gpu)
    w2 = torch.zeros(dff, dm, dtype=torch.int8, device=gpu)
    one = lambda n: torch.full((n,), 1e-8 / 127, device=gpu)  # noqa: E731
    out, osc = ext.int8_mlp_forward(z, w1, w2, one(T), one(dff), one(dm))
    assert int(out.abs().max()) == 0 and torch.isfinite(osc).all()
    # constant dataset: every code of the output is 127
    x = torch.full((1, T, dm), 127, dtype=torch.int8, device=gpu)
    w1 = torch.full((dm, dff), 127, dtype=torch.int8, device=gpu)
    w2 = torch.full((dff, dm), 127, dtype=torch.int8, device=gpu)
    out, osc = ext.int8_mlp_forward(x, w1, w2, torch.full((T,), 1 / 127, device=gpu),
                                    torch.full((dff,), 0.01 / 127, device=gpu),
                                    torch.full((dm,), 0.01 / 127, device=gpu))
    assert int(out.min()) == int(out.max()) == 127


def test_mlp_argument_errors(ext, gpu):
    x = torch.zeros(1, 4, 64, dtype=torch.int8, device=gpu)
    w1 = torch.zeros(64, 128, dtype=torch.int8, device=gpu)
    w2 = torch.zeros(128, 64, dtype=torch.int8, device=gpu)
    with pytest.raises(RuntimeError, match="W1 shape mismatch"):
        ext.int8_mlp_forward(x, w1[:32].contiguous(), w2, 1.0, 1.0, 1.0)
    with pytest.raises(RuntimeError, match="x must be 3-D"):
        ext.int8_mlp_forward(x[0], w1, w2, 1.0, 1.0, 1.0)
    with pytest.raises(RuntimeError, match="scale_x must have 4"):
        ext.int8_mlp_forward(x, w1, w2, torch.ones(3, device=gpu), torch.ones(128, device=gpu),
                             torch.ones(64, device=gpu))
    with pytest.raises(RuntimeError, match="multiples of 16"):
        ext.int8_mlp_forward(torch.zeros(1, 4, 60, dtype=torch.int8, device=gpu),
                             torch.zeros(60, 128, dtype=torch.int8, device=gpu),
                             torch.zeros(128, 60, dtype=torch.int8, device=gpu), 1.0, 1.0, 1.0)


@pytest.mark.parametrize("T,dm,dff,big_rows", [(1024, 1024, 4096, False),
                                                (700, 528, 1040, False),
                                                (1024, 1024, 4096, True)])
def test_mlp_gemm2_on_fp16_hidden_matches_requant_pass(capi_mlp, gpu, monkeypatch, T, dm, dff,
                                                        big_rows):
    # These shapes run GEMM2 as the 256 x 256 tiled kernel.  With
    # INT8K_MLP_GEMM2_FP16_HIDDEN=1 it reads the fp16 hidden and quantizes it per row
    # on load; by default a separate pass writes the int8 hidden.  The codes must be the
    # same, so the outputs are equal byte for byte.  big_rows: a few token rows scaled
    # so their hidden exceeds the fp16 range (infinite h, the clamping path).
    c, n = _mlp_case(T, dm, dff, seed=T + dff, gpu=gpu)
    if big_rows:
        c["sx"][::97] *= 2e5
        n["sx"] = _np(c["sx"])
    args = (c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    monkeypatch.delenv("INT8K_MLP_GEMM2_FP16_HIDDEN", raising=False)
    out_a, osc_a = capi.mlp_forward(*args)
    monkeypatch.setenv("INT8K_MLP_GEMM2_FP16_HIDDEN", "1")
    out_b, osc_b = capi.mlp_forward(*args)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.equal(osc_a, osc_b)
    ref, rsc = O.mlp_forward(n["x"].reshape(T, dm), n["W1"], n["W2"], n["sx"], n["sW1"],
                             n["sW2"], gemm=oracle_c.gemm_i8_i32)
    _compare_mlp(_np(out_b), _np(osc_b), ref, rsc, f"T{T} dm{dm} dff{dff} big={big_rows}")


def test_mlp_baseline_cfg4_full_size(ext, gpu):
    # T=4096, 4096 -> 16384 -> 4096, per-token / per-channel.  Every
    # row against the oracle (its exact int8 GEMMs in C), in blocks of 512 tokens (the
    # MLP is row-independent under per-token scales).
    T, dm, dff = 4096, 4096, 16384
    print("mlp cfg4 full size", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=77, device=gpu)
    W1T, W2T = ext.transpose_int8_weights(c["W1"], c["W2"])
    out, osc = ext.int8_mlp_forward_prepacked(c["x"], W1T, W2T, c["sx"], c["sW1"], c["sW2"])
    torch.cuda.synchronize()
    got, gsc = _np(out).reshape(T, dm), _np(osc)
    x, sx = _np(c["x"]).reshape(T, dm), _np(c["sx"])
    W1, W2, sW1, sW2 = _np(c["W1"]), _np(c["W2"]), _np(c["sW1"]), _np(c["sW2"])
    for r0 in range(0, T, 512):
        rows = slice(r0, r0 + 512)
        ref, rsc = O.mlp_forward(x[rows], W1, W2, sx[rows], sW1, sW2, gemm=oracle_c.gemm_i8_i32)
        _compare_mlp(got[rows], gsc[rows], ref, rsc, f"cfg4 rows {r0}..{r0 + 511}")
    assert (np.abs(got.astype(np.int32)).max(axis=-1) == 127).all()


@pytest.fixture
def capi_mlp(capi):
    return capi
