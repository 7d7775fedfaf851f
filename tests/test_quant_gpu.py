"""Quantizers and the INT8 KV cache against the CPU oracle (GPU tests).

The quantizers are bit-exact by construction (exact absmax, correctly rounded
fp32 division, round-half-even), so codes and scales must match the oracle
exactly; the cache-backed decode must equal the contiguous decode bit for bit.
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from oracle import int8_oracle as O

pytestmark = pytest.mark.gpu


# Row lengths for both kernels: one 16-byte chunk per lane with 1..64 lanes per row
# ((1000, 128), (3, 5, 64), (5, 256)), several chunks per lane ((33, 1024), (3, 3072),
# (64, 4096), (2, 8192)), and one element per lane ((1, 1), (7, 33); fp32 rows of 8192).
@pytest.mark.parametrize("shape", [(1, 1), (7, 33), (1000, 128), (3, 5, 64), (5, 256), (33, 1024),
                                   (3, 3072), (64, 4096), (2, 8192)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_quantize_per_token_bit_exact(ext, gpu, shape, dtype):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 3).to(dtype)
    q, s = ext.quantize_per_token(x.to(gpu))
    rq, rs = O.quantize_per_token(x.float().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    assert q.shape == x.shape and tuple(s.shape) == shape[:-1]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_quantize_per_token_unaligned_source(gpu, dtype):
    # a source that is not 16-byte aligned takes the one-element-per-lane kernel
    rows, cols = 9, 128
    base = (torch.randn(rows * cols + 1, generator=torch.Generator().manual_seed(5)) * 2).to(dtype)
    x = base.to(gpu)[1:].view(rows, cols)
    q, s = capi.quantize_per_token(x)
    torch.cuda.synchronize()
    rq, rs = O.quantize_per_token(x.float().cpu().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)


def test_quantize_per_token_kats(ext, gpu):
    x = torch.zeros(4, 64, device=gpu)
    x[1] = 2.0                                        # constant row -> code 127
    x[2, ::2], x[2, 1::2] = 0.5, -0.5
    x[3] = torch.linspace(-127, 127, 64, device=gpu)  # scale 1: codes are rint(x)
    q, s = ext.quantize_per_token(x)
    assert int(q[0].abs().max()) == 0 and float(s[0]) == np.float32(np.float32(1e-8) / 127)
    assert int(q[1].min()) == int(q[1].max()) == 127
    assert set(q[2].tolist()) == {127, -127}
    np.testing.assert_array_equal(q[3].cpu().numpy(), np.rint(x[3].cpu().numpy()).astype(np.int8))
    # boundary dataset (validation/generate_test_data.py:113-122): codes +-125..127
    g = torch.Generator().manual_seed(3)
    sign = torch.randint(0, 2, (32, 128), generator=g).float() * 2 - 1
    xb = sign * 4.0 * (0.985 + 0.015 * torch.rand(32, 128, generator=g))
    q, _ = ext.quantize_per_token(xb.to(gpu))
    assert set(q.abs().unique().tolist()) <= {125, 126, 127}


def test_quantize_per_token_matches_reference_formula_on_cpu(ext, gpu):
    # The reference quantizer's torch formula evaluated on the CPU (true fp32
    # division) is reproduced bit for bit.  (On the GPU torch turns the
    # division by the scalar 127 into a reciprocal multiply, so its scales may
    # differ from the formula in the last ulp.)
    x = torch.randn(512, 128, generator=torch.Generator().manual_seed(1))
    q, s = ext.quantize_per_token(x.to(gpu))
    rq, rs = workloads.quantize_per_token(x)
    assert torch.equal(q.cpu(), rq) and torch.equal(s.cpu(), rs)


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_quant_utils_per_tensor(ext, gpu, n):
    x = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 5).half()
    q, s = ext.quantize_fp16_to_int8(x.to(gpu))
    rq, rs = O.quantize_fp16_per_tensor(x.numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    assert float(s) == float(rs)
    y = ext.dequantize_int8_to_fp16(q, float(s))
    np.testing.assert_array_equal(y.cpu().numpy(), O.dequantize_int8_to_fp16(rq, rs))


def test_quant_utils_zero_input(ext, gpu):
    q, s = ext.quantize_fp16_to_int8(torch.zeros(4096, dtype=torch.float16, device=gpu))
    assert int(q.abs().max()) == 0                     # not -128 as the reference kernel gives
    assert float(s) == float(np.float32(np.float32(1e-8) / np.float32(127)))


@pytest.mark.parametrize("D,cap", [(128, 640), (64, 640), (64, 643)])
def test_kv_cache_append_and_decode(ext, gpu, D, cap):
    # cap 643: scale rows not 16-byte aligned, so the decode takes its per-row scale loads
    B, H = 2, 4
    g = torch.Generator().manual_seed(11)
    k_all = torch.randn(B, H, 300, D, generator=g).half().to(gpu)
    v_all = torch.randn(B, H, 300, D, generator=g).half().to(gpu)
    K = torch.zeros(B, H, cap, D, dtype=torch.int8, device=gpu)
    V = torch.zeros_like(K)
    sK = torch.zeros(B, H, cap, device=gpu)
    sV = torch.zeros_like(sK)
    ext.kv_cache_append(k_all[:, :, :257], v_all[:, :, :257], K, V, sK, sV, 0)  # prefill
    for p in range(257, 300):                                                   # decode steps
        ext.kv_cache_append(k_all[:, :, p:p + 1], v_all[:, :, p:p + 1], K, V, sK, sV, p)
    kq, ks = workloads.quantize_per_token(k_all.cpu())
    vq, vs = workloads.quantize_per_token(v_all.cpu())
    assert torch.equal(K[:, :, :300].cpu(), kq) and torch.equal(sK[:, :, :300].cpu(), ks)
    assert torch.equal(V[:, :, :300].cpu(), vq) and torch.equal(sV[:, :, :300].cpu(), vs)
    kq, ks, vq, vs = (t.to(gpu) for t in (kq, ks, vq, vs))
    assert int(K[:, :, 300:].abs().max()) == 0            # untouched past the append
    q, sq = workloads.quantize_per_token(torch.randn(B, H, D, generator=g).to(gpu))
    a = ext.int8_decode_attention_forward_cache(q, K, V, sq, sK, sV, 300)
    b = ext.int8_decode_attention_forward(q, kq.contiguous(), vq.contiguous(), sq, ks, vs)
    assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="capacity"):
        ext.kv_cache_append(k_all[:, :, :1], v_all[:, :, :1], K, V, sK, sV, cap)


def test_kv_cache_capi(gpu):
    B, H, D, cap = 1, 2, 64, 100
    k = torch.randn(B, H, 10, D, device=gpu)
    v = torch.randn(B, H, 10, D, device=gpu)
    K = torch.zeros(B, H, cap, D, dtype=torch.int8, device=gpu)
    V = torch.zeros_like(K)
    sK = torch.zeros(B, H, cap, device=gpu)
    sV = torch.zeros_like(sK)
    capi.kv_cache_append(k, v, K, V, sK, sV, 90)
    torch.cuda.synchronize()
    kq, ks = O.quantize_per_token(k.cpu().numpy())
    np.testing.assert_array_equal(K[:, :, 90:].cpu().numpy(), kq)
    np.testing.assert_array_equal(sK[:, :, 90:].cpu().numpy(), ks)


def test_quantize_per_token_beyond_2p32_work_items(ext, gpu):
    # 2^24 + 5 rows: one wave per row would need more than 2^32 work-items in one
    # launch; the row kernels stride over rows instead (regression test)
    rows, cols = (1 << 24) + 5, 4
    x = torch.randn(rows, cols, generator=torch.Generator(device=gpu).manual_seed(3), device=gpu)
    q, s = ext.quantize_per_token(x)
    torch.cuda.synchronize()
    idx = torch.tensor([0, 1, rows // 2, rows - 5, rows - 1], device=gpu)
    rq, rs = workloads.quantize_per_token(x[idx].cpu())
    assert torch.equal(q[idx].cpu(), rq) and torch.equal(s[idx].cpu(), rs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(3, 64), (129, 1024), (2, 5, 48), (7, 33)])
@pytest.mark.parametrize("residual", [False, True])
def test_dequantize_per_token_matches_torch(ext, gpu, dtype, shape, residual):
    # y = (q.float() * s[..., None]).to(dtype) (+ residual in its dtype), bit for bit;
    # (7, 33) and (2, 5, 48) also take the one-element-per-thread kernel
    g = torch.Generator().manual_seed(sum(shape) + residual)
    q = torch.randint(-128, 128, shape, generator=g, dtype=torch.int8).to(gpu)
    s = (torch.rand(shape[:-1], generator=g) * 0.05 + 1e-3).to(gpu)
    ref = (q.float() * s.unsqueeze(-1)).to(dtype)
    r = None
    if residual:
        r = (torch.randn(shape, generator=g) * 4).to(dtype).to(gpu)
        ref = r + ref
    y = ext.dequantize_per_token(q, s, residual=r, dtype=dtype)
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == q.shape
    assert torch.equal(y, ref)
    odt = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[dtype]
    want = O.dequantize_per_token_residual(q.cpu().numpy(), s.cpu().numpy(), odt,
                                           None if r is None else r.float().cpu().numpy())
    np.testing.assert_array_equal(y.float().cpu().numpy(), want)


def test_dequantize_per_token_capi_unaligned(gpu):
    # an output that is not 16-byte aligned takes the one-element-per-thread kernel
    rows, cols = 5, 64
    q = torch.randint(-128, 128, (rows, cols), dtype=torch.int8,
                      generator=torch.Generator().manual_seed(9)).to(gpu)
    s = torch.rand(rows, generator=torch.Generator().manual_seed(10)).to(gpu)
    base = torch.empty(rows * cols + 1, dtype=torch.float16, device=gpu)
    y = capi.dequantize_per_token(q, s)
    torch.cuda.synchronize()
    assert torch.equal(y, (q.float() * s[:, None]).half())
    out = base[1:].view(rows, cols)
    st = capi.load().int8k_dequantize_per_token(
        capi._ptr(q), capi._ptr(s), capi.DTYPE_F16, None, capi._ptr(out), rows, cols,
        capi._stream(q))
    assert st == capi.INT8K_OK
    torch.cuda.synchronize()
    assert torch.equal(out, (q.float() * s[:, None]).half())


def test_dequantize_per_token_dtype_must_match_residual(ext, gpu):
    # the residual sets the output dtype; a different explicit dtype is an error
    q = torch.zeros((4, 64), dtype=torch.int8, device=gpu)
    s = torch.ones(4, dtype=torch.float32, device=gpu)
    r = torch.zeros((4, 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="residual's dtype"):
        ext.dequantize_per_token(q, s, r, torch.float16)
    with pytest.raises(ValueError, match="residual's dtype"):
        capi.dequantize_per_token(q, s, residual=r, dtype=torch.float16)
    y = ext.dequantize_per_token(q, s, r, torch.bfloat16)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and torch.equal(y, r)


def _fp16_double_rounding_cases(rng, count):
    """(q, s) pairs with half(fp32(q * s)) != half(q * s): the fp32 product lands on
    an fp16 tie that the exact product does not.  The dequantizers must give the
    first (PyTorch's and the reference's rounding), not the fused single rounding."""
    qs, ss = [], []
    while len(qs) < count:
        q = rng.integers(-128, 128, 1 << 16).astype(np.int8)
        s = rng.uniform(1e-3, 0.05, 1 << 16).astype(np.float32)
        twice = (q.astype(np.float32) * s).astype(np.float16)
        once = (q.astype(np.float64) * s.astype(np.float64)).astype(np.float16)
        hit = np.nonzero(twice != once)[0]
        qs += list(q[hit]); ss += list(s[hit])
    return np.array(qs[:count], np.int8), np.array(ss[:count], np.float32)


@pytest.mark.parametrize("residual", [False, True])
def test_dequantize_fp16_rounds_through_fp32(ext, gpu, residual):
    # regression: hipcc folds half(float(q) * s) into one fused rounding unless the
    # fp32 product is pinned; 64 rows of 16 equal codes, one crafted (q, s) per row
    rng = np.random.default_rng(11)
    qv, sv = _fp16_double_rounding_cases(rng, 64)
    q = torch.from_numpy(np.repeat(qv[:, None], 16, axis=1)).to(gpu)
    s = torch.from_numpy(sv).to(gpu)
    ref = (q.float() * s[:, None]).half()
    r = None
    if residual:
        r = torch.zeros(64, 16, dtype=torch.float16, device=gpu)
        ref = r + ref
    y = ext.dequantize_per_token(q, s, residual=r, dtype=torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert not torch.equal(y.cpu(), torch.from_numpy(
        (qv.astype(np.float64) * sv.astype(np.float64)).astype(np.float16))[:, None].expand(64, 16))


def test_dequantize_int8_to_fp16_rounds_through_fp32(ext, gpu):
    # the per-tensor dequantizer, same regression: one scale whose products with some
    # of the 256 codes double-round differently from the fused rounding
    rng = np.random.default_rng(12)
    codes = np.arange(-128, 128, dtype=np.int8)
    while True:
        s = np.float32(rng.uniform(1e-3, 0.05))
        twice = (codes.astype(np.float32) * s).astype(np.float16)
        if (twice != (codes.astype(np.float64) * np.float64(s)).astype(np.float16)).any():
            break
    y = ext.dequantize_int8_to_fp16(torch.from_numpy(codes).to(gpu), float(s))
    np.testing.assert_array_equal(y.cpu().numpy(), O.dequantize_int8_to_fp16(codes, s))
    np.testing.assert_array_equal(y.cpu().numpy(), twice)


@pytest.mark.parametrize("cols", [128, 1024, 33])
def test_quantize_per_token_infinite_element(ext, gpu, cols):
    # a row with an infinite element has scale inf: its finite elements quantize to 0
    # (x / inf) and the infinite one to -128 (inf / inf is NaN, and the clamp
    # max(NaN, -128) gives -128), on the chunked kernels (128, 1024 columns) and the
    # one-element-per-lane kernel (33 columns); the other rows are unaffected
    x = torch.randn(4, cols, generator=torch.Generator().manual_seed(cols)).half()
    x[1, 5] = float("inf")
    x[2, 0] = float("-inf")
    q, s = ext.quantize_per_token(x.to(gpu))
    torch.cuda.synchronize()
    q, s = q.cpu(), s.cpu()
    for r, c in ((1, 5), (2, 0)):
        assert s[r] == float("inf")
        expect = torch.zeros(cols, dtype=torch.int8)
        expect[c] = -128
        assert torch.equal(q[r], expect)
    rq, rs = O.quantize_per_token(x[[0, 3]].float().numpy())
    np.testing.assert_array_equal(q[[0, 3]].numpy(), rq)
    np.testing.assert_array_equal(s[[0, 3]].numpy(), rs)
