"""Pins the CPU oracle (CPU-only tests).

Each check is chosen so a plausible slip in the oracle (wrong scale index,
dropped 1/sqrt(D), transposed operand, truncation instead of round-half-even,
clamp asymmetry, a missing GELU term) fails at least one of them: brute-force
loops on tiny inputs, closed forms and known-answer datasets of the reference
(validation/generate_test_data.py: zeros, constant, boundary), invariants, and
independent library routines (torch SDPA, torch GELU).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import int8_oracle as O
from oracle import oracle_c as C


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- quantizers

def test_quantize_per_token_kats():
    x = np.array([[0.0, 0.0, 0.0, 0.0],          # zeros -> scale 1e-8/127, codes 0
                  [2.0, 2.0, 2.0, 2.0],          # constant -> single code 127
                  [-4.0, 4.0, 1.0, -1.0],
                  [1.0, -0.5, 0.25, 127 * 0.5 / 127]], np.float32)
    q, s = O.quantize_per_token(x)
    assert q.dtype == np.int8 and s.dtype == np.float32
    np.testing.assert_array_equal(q[0], 0)
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127))
    np.testing.assert_array_equal(q[1], 127)
    assert s[1] == np.float32(2.0 / 127)
    np.testing.assert_array_equal(q[2], [-127, 127, 32, -32])   # 31.75 -> 32
    assert q[3, 0] == 127 and q[3, 1] == -64  # -63.5 -> -64 (half to even)


def test_quantize_round_half_even_and_clamp():
    # scale 1 exactly: amax 127 -> codes equal rint(x) with ties to even.
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49]], np.float32)
    q, s = O.quantize_per_token(x)
    assert s[0] == 1.0
    np.testing.assert_array_equal(q[0], [127, 0, 2, 2, 0, -2, -2, 3])


def test_quantize_boundary_dataset_codes():
    # validation/generate_test_data.py:113-122: |x| in amax*[0.985, 1] lands on +-126/127.
    g = rng(1)
    sign = g.integers(0, 2, (64, 128)) * 2 - 1
    mag = 4.0 * (0.985 + 0.015 * g.random((64, 128)))
    x = (sign * mag).astype(np.float32)
    q, s = O.quantize_per_token(x)
    assert set(np.unique(np.abs(q.astype(np.int32)))) <= {125, 126, 127}
    assert (np.abs(x - q.astype(np.float32) * s[:, None]) <= s[:, None] / 2 * (1 + 1e-6)).all()


def test_quantize_matches_torch_formula():
    # the reference quantizer written with torch ops (validation/check_decode.py:42-47)
    x = rng(2).standard_normal((33, 64)).astype(np.float32)
    t = torch.from_numpy(x)
    am = t.abs().amax(-1, keepdim=True).clamp(min=1e-8)
    sc = am / 127.0
    qt = (t / sc).round().clamp(-128, 127).to(torch.int8)
    q, s = O.quantize_per_token(x)
    np.testing.assert_array_equal(q, qt.numpy())
    np.testing.assert_array_equal(s, sc.squeeze(-1).numpy())


def test_quantize_per_channel_w_axis():
    w = np.zeros((4, 3), np.float32)
    w[:, 0] = [1, -2, 0.5, 0.0]
    w[:, 1] = [0.02, 0.01, -0.04, 0.0]
    q, s = O.quantize_per_channel_w(w)
    np.testing.assert_allclose(s, [2 / 127, 0.04 / 127, 1e-8 / 127], rtol=1e-7)
    np.testing.assert_array_equal(q[:, 0], [64, -127, 32, 0])  # 63.5 -> 64 (even)
    np.testing.assert_array_equal(q[:, 2], 0)


# ---------------------------------------------------------------- attention

def brute_decode(Q, K, V, sQ, sK, sV):
    BH, D = Q.shape
    S = K.shape[1]
    out = np.zeros((BH, D))
    for b in range(BH):
        sc = []
        for j in range(S):
            dot = sum(int(Q[b, d]) * int(K[b, j, d]) for d in range(D))
            sc.append(dot * float(sQ[b]) * float(sK[b, j]) / math.sqrt(D))
        m = max(sc)
        p = [math.exp(x - m) for x in sc]
        z = sum(p)
        for d in range(D):
            out[b, d] = sum(p[j] * float(V[b, j, d]) * float(sV[b, j]) for j in range(S)) / z
    return out


def rand_decode(BH, S, D, seed):
    g = rng(seed)
    Q, sQ = O.quantize_per_token(g.standard_normal((BH, D)).astype(np.float32))
    K, sK = O.quantize_per_token(g.standard_normal((BH, S, D)).astype(np.float32))
    V, sV = O.quantize_per_token(g.standard_normal((BH, S, D)).astype(np.float32))
    return Q, K, V, sQ, sK, sV


@pytest.mark.parametrize("BH,S,D", [(2, 5, 8), (1, 1, 4), (3, 7, 16)])
def test_decode_oracle_vs_brute_force(BH, S, D):
    args = rand_decode(BH, S, D, seed=BH * 100 + S)
    ref = brute_decode(*args)
    np.testing.assert_allclose(O.decode_attention(*args), ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(C.decode_attention(*args), ref, rtol=1e-12, atol=1e-12)


def test_decode_oracle_vs_torch_sdpa():
    # an independent library routine on the dequantized operands
    Q, K, V, sQ, sK, sV = rand_decode(6, 300, 64, seed=4)
    qd = torch.from_numpy(Q.astype(np.float64) * sQ[:, None])[:, None, None, :]
    kd = torch.from_numpy(K.astype(np.float64) * sK[..., None])[:, None]
    vd = torch.from_numpy(V.astype(np.float64) * sV[..., None])[:, None]
    ref = F.scaled_dot_product_attention(qd, kd, vd).reshape(6, 64).numpy()
    np.testing.assert_allclose(O.decode_attention(Q, K, V, sQ, sK, sV), ref, atol=1e-12)
    np.testing.assert_allclose(C.decode_attention(Q, K, V, sQ, sK, sV), ref, atol=1e-12)


def test_decode_oracle_closed_forms():
    Q, K, V, sQ, sK, sV = rand_decode(3, 1, 32, seed=5)
    out = C.decode_attention(Q, K, V, sQ, sK, sV)           # S=1 -> V row
    np.testing.assert_allclose(out, V[:, 0].astype(np.float64) * sV[:, :1], atol=1e-12)
    Q, K, V, sQ, sK, sV = rand_decode(3, 50, 32, seed=6)
    K[:] = K[:, :1]
    sK[:] = sK[:, :1]                                        # constant keys -> mean of V
    out = C.decode_attention(Q, K, V, sQ, sK, sV)
    np.testing.assert_allclose(out, (V.astype(np.float64) * sV[..., None]).mean(1), atol=1e-12)
    Q, K, V, sQ, sK, sV = rand_decode(2, 40, 16, seed=7)
    perm = rng(8).permutation(40)                            # permutation invariance
    a = C.decode_attention(Q, K, V, sQ, sK, sV)
    b = C.decode_attention(Q, K[:, perm], V[:, perm], sQ, sK[:, perm], sV[:, perm])
    np.testing.assert_allclose(a, b, atol=1e-12)


def brute_prefill(Q, K, V, sQ, sK, sV, causal):
    BH, S, D = Q.shape
    out = np.zeros((BH, S, D))
    for b in range(BH):
        for i in range(S):
            n = i + 1 if causal else S
            sc = [sum(int(Q[b, i, d]) * int(K[b, j, d]) for d in range(D)) * float(sQ[b, i])
                  * float(sK[b, j]) / math.sqrt(D) for j in range(n)]
            m = max(sc)
            p = [math.exp(x - m) for x in sc]
            z = sum(p)
            for d in range(D):
                out[b, i, d] = sum(p[j] * float(V[b, j, d]) * float(sV[b, j])
                                   for j in range(n)) / z
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_oracle_vs_brute_force(causal):
    g = rng(9)
    Q, sQ = O.quantize_per_token(g.standard_normal((2, 6, 8)).astype(np.float32))
    K, sK = O.quantize_per_token(g.standard_normal((2, 6, 8)).astype(np.float32))
    V, sV = O.quantize_per_token(g.standard_normal((2, 6, 8)).astype(np.float32))
    ref = brute_prefill(Q, K, V, sQ, sK, sV, causal)
    np.testing.assert_allclose(O.prefill_attention(Q, K, V, sQ, sK, sV, causal), ref, atol=1e-12)
    np.testing.assert_allclose(C.prefill_attention(Q, K, V, sQ, sK, sV, causal), ref, atol=1e-12)
    if causal:  # row 0 sees only key 0
        np.testing.assert_allclose(ref[:, 0], V[:, 0] * sV[:, :1], atol=1e-12)


def test_prefill_oracle_vs_torch_sdpa():
    g = rng(10)
    Q, sQ = O.quantize_per_token(g.standard_normal((3, 40, 32)).astype(np.float32))
    K, sK = O.quantize_per_token(g.standard_normal((3, 40, 32)).astype(np.float32))
    V, sV = O.quantize_per_token(g.standard_normal((3, 40, 32)).astype(np.float32))
    deq = lambda a, s: torch.from_numpy(a.astype(np.float64) * s[..., None].astype(np.float64))
    for causal in (False, True):
        ref = F.scaled_dot_product_attention(deq(Q, sQ), deq(K, sK), deq(V, sV),
                                             is_causal=causal).numpy()
        np.testing.assert_allclose(C.prefill_attention(Q, K, V, sQ, sK, sV, causal), ref,
                                   atol=1e-12)


# ---------------------------------------------------------------- GEMM / MLP

def test_gemm_vs_triple_loop_and_extremes():
    g = rng(11)
    A = g.integers(-128, 128, (5, 7)).astype(np.int8)
    B = g.integers(-128, 128, (7, 3)).astype(np.int8)
    ref = np.array([[sum(int(A[m, k]) * int(B[k, n]) for k in range(7)) for n in range(3)]
                    for m in range(5)])
    np.testing.assert_array_equal(O.gemm_i8_i32(A, B), ref)
    np.testing.assert_array_equal(C.gemm_i8_i32(A, B), ref)
    A = np.full((2, 16384), -128, np.int8)   # largest reduction of the MLP config
    B = np.full((16384, 2), -128, np.int8)
    np.testing.assert_array_equal(C.gemm_i8_i32(A, B), 16384 * 128 * 128)
    I = np.eye(8, dtype=np.int8)             # identity / transpose sanity
    X = g.integers(-128, 128, (8, 8)).astype(np.int8)
    np.testing.assert_array_equal(C.gemm_i8_i32(X, I), X)
    np.testing.assert_array_equal(C.gemm_i8_i32(I, X), X)
    with pytest.raises(OverflowError):
        C.gemm_i8_i32(np.full((1, 140000), -128, np.int8), np.full((140000, 1), -128, np.int8))


def test_gemm_c_matches_numpy_random():
    g = rng(12)
    A = g.integers(-128, 128, (64, 200)).astype(np.int8)
    B = g.integers(-128, 128, (200, 96)).astype(np.int8)
    np.testing.assert_array_equal(C.gemm_i8_i32(A, B), O.gemm_i8_i32(A, B))


def test_gelu_closed_form_and_torch():
    x = np.array([0.0, 1.0, -1.0, 3.0, -3.0, 10.0, -10.0], np.float32)
    y = O.gelu_tanh_f32(x)
    assert y[0] == 0.0 and abs(y[5] - 10.0) < 1e-6 and abs(y[6]) < 1e-6
    # closed form at 1: 0.5*(1+tanh(sqrt(2/pi)*(1+0.044715)))
    assert abs(y[1] - 0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * 1.044715))) < 1e-6
    xs = rng(13).standard_normal(10000).astype(np.float32) * 4
    ref = F.gelu(torch.from_numpy(xs), approximate="tanh").numpy()
    np.testing.assert_allclose(O.gelu_tanh_f32(xs), ref, rtol=2e-6, atol=2e-7)


def _mlp_inputs(T, dm, dff, seed):
    g = rng(seed)
    x, sx = O.quantize_per_token(g.standard_normal((T, dm)).astype(np.float32))
    W1, s1 = O.quantize_per_channel_w((g.standard_normal((dm, dff)) * 0.02).astype(np.float32))
    W2, s2 = O.quantize_per_channel_w((g.standard_normal((dff, dm)) * 0.02).astype(np.float32))
    return x, W1, W2, sx, s1, s2


def test_mlp_stages_restate_reference_order():
    x, W1, W2, sx, s1, s2 = _mlp_inputs(16, 64, 128, seed=14)
    out, osc, st = O.mlp_forward(x, W1, W2, sx, s1, s2, return_stages=True)
    # stage 1: exact accumulators, then ((acc*sx)*sW1) in fp32, GELU
    np.testing.assert_array_equal(st["acc1"], C.gemm_i8_i32(x, W1))
    v = O.gelu_tanh_f32((st["acc1"].astype(np.float32) * sx[:, None]) * s1[None, :])
    np.testing.assert_array_equal(st["v"], v)
    # the hidden row absmax is taken before fp16 rounding
    np.testing.assert_array_equal(st["h_amax"], np.abs(v).max(1))
    # requant: every code is within half a step of h16/sh (rounding), sh = amax/127
    np.testing.assert_allclose(st["sh"], st["h_amax"] / np.float32(127), rtol=1e-7)
    recon = st["hq"].astype(np.float64) * st["sh"][:, None]
    assert (np.abs(recon - st["h16"].astype(np.float64)) <= st["sh"][:, None] * 0.5001).all()
    assert np.abs(st["hq"]).max() == 127
    np.testing.assert_array_equal(st["acc2"], C.gemm_i8_i32(st["hq"], W2))
    # per-token output codes use the full range in every row
    assert (np.abs(out.astype(np.int32)).max(1) == 127).all()
    deq = out.astype(np.float64) * osc[:, None]
    ref = O.mlp_dequant_reference(x, W1, W2, sx, s1, s2)
    cos = (deq * ref).sum() / np.linalg.norm(deq) / np.linalg.norm(ref)
    assert cos > 0.999


def test_mlp_kats_zero_and_constant():
    T, dm, dff = 8, 32, 64
    z8 = np.zeros((T, dm), np.int8)
    out, osc = O.mlp_forward(z8, np.zeros((dm, dff), np.int8), np.zeros((dff, dm), np.int8),
                             np.full(T, 1e-8 / 127, np.float32), np.full(dff, 1e-8 / 127, np.float32),
                             np.full(dm, 1e-8 / 127, np.float32))
    np.testing.assert_array_equal(out, 0)
    # constant dataset (validation/generate_test_data.py:320-336): one code everywhere
    x, sx = O.quantize_per_token(np.ones((T, dm), np.float32))
    W1, s1 = O.quantize_per_channel_w(np.full((dm, dff), 0.01, np.float32))
    W2, s2 = O.quantize_per_channel_w(np.full((dff, dm), 0.01, np.float32))
    out, osc = O.mlp_forward(x, W1, W2, sx, s1, s2)
    np.testing.assert_array_equal(out, 127)


def test_mlp_per_tensor_output_path():
    x, W1, W2, _, _, _ = _mlp_inputs(16, 64, 128, seed=15)
    out, osc = O.mlp_forward(x, W1, W2, np.float32(0.01), np.float32(0.002),
                             np.float32(0.003), per_token_out=False)
    assert np.ndim(osc) == 0 and np.abs(out.astype(np.int32)).max() == 127


# ---------------------------------------------------------------- quant utils

def test_quant_utils_per_tensor():
    x = np.array([0.0, 1.0, -2.0, 0.5, 65504.0], np.float16)
    q, s = O.quantize_fp16_per_tensor(x)
    assert s == np.float32(np.float32(65504.0) / np.float32(127.0))
    assert q[4] == 127 and q[0] == 0
    q0, s0 = O.quantize_fp16_per_tensor(np.zeros(16, np.float16))
    np.testing.assert_array_equal(q0, 0)  # the 1e-8 guard (reference returns -128 here)
    d = O.dequantize_int8_to_fp16(np.array([-128, 0, 127], np.int8), np.float32(0.5))
    np.testing.assert_array_equal(d, np.array([-64.0, 0.0, 63.5], np.float16))


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("residual", [False, True])
def test_dequantize_per_token_residual_matches_torch(dtype, residual):
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    g = torch.Generator().manual_seed(7)
    q = torch.randint(-128, 128, (33, 256), generator=g, dtype=torch.int8)
    s = torch.rand(33, generator=g) * 0.05 + 1e-3
    ref = (q.float() * s.unsqueeze(-1)).to(tdt)
    r = None
    if residual:
        r = (torch.randn(33, 256, generator=g) * 4).to(tdt)
        ref = r + ref
    got = O.dequantize_per_token_residual(q.numpy(), s.numpy(), dtype,
                                          None if r is None else r.float().numpy())
    np.testing.assert_array_equal(got, ref.float().numpy())


def test_dequantize_per_token_residual_double_rounding():
    # (q, s) = (63, 0.04983569) etc.: pairs whose fp32 product sits on an fp16 tie that
    # the exact product misses; the oracle must round through fp32 as torch does
    rng = np.random.default_rng(11)
    q = rng.integers(-128, 128, 1 << 16).astype(np.int8)
    s = rng.uniform(1e-3, 0.05, 1 << 16).astype(np.float32)
    once = (q.astype(np.float64) * s.astype(np.float64)).astype(np.float16)
    hit = np.nonzero((q.astype(np.float32) * s).astype(np.float16) != once)[0]
    assert hit.size > 0
    got = O.dequantize_per_token_residual(q[hit, None], s[hit], "f16")[:, 0]
    want = (torch.from_numpy(q[hit]).float() * torch.from_numpy(s[hit])).half()
    np.testing.assert_array_equal(got, want.float().numpy())
    assert not np.array_equal(got, once[hit].astype(np.float32))


def _contiguous_as_pages(K, P):
    """[B, H, S, D] -> pages [B*npp, H, P, D] with sequence b in pages b*npp .. (b+1)*npp-1."""
    B, H, S = K.shape[:3]
    npp = -(-S // P)
    pad = np.zeros((B, H, npp * P) + K.shape[3:], K.dtype)
    pad[:, :, :S] = K
    pages = pad.reshape((B, H, npp, P) + K.shape[3:])
    pages = np.moveaxis(pages, 2, 1).reshape((B * npp, H, P) + K.shape[3:])
    tables = np.arange(B * npp, dtype=np.int32).reshape(B, npp)
    return pages, tables


def test_paged_decode_identity_tables_equal_contiguous():
    rng = np.random.default_rng(5)
    B, H, S, D, P = 2, 3, 50, 16, 16
    Q = rng.integers(-127, 128, (B, H, D), dtype=np.int8)
    K = rng.integers(-127, 128, (B, H, S, D), dtype=np.int8)
    V = rng.integers(-127, 128, (B, H, S, D), dtype=np.int8)
    sQ = rng.uniform(0.001, 0.02, (B, H)).astype(np.float32)
    sK = rng.uniform(0.001, 0.02, (B, H, S)).astype(np.float32)
    sV = rng.uniform(0.001, 0.02, (B, H, S)).astype(np.float32)
    Kp, tables = _contiguous_as_pages(K, P)
    Vp, _ = _contiguous_as_pages(V, P)
    sKp, _ = _contiguous_as_pages(sK, P)
    sVp, _ = _contiguous_as_pages(sV, P)
    lens = np.array([S, S], np.int32)
    got = O.decode_attention_paged(Q, Kp, Vp, sQ, sKp, sVp, tables, lens)
    ref = O.decode_attention(Q.reshape(B * H, D), K.reshape(B * H, S, D), V.reshape(B * H, S, D),
                             sQ.reshape(-1), sK.reshape(B * H, S), sV.reshape(B * H, S))
    np.testing.assert_allclose(got.reshape(B * H, D), ref, rtol=0, atol=1e-12)
    # a permuted physical order with the table permuted alike changes nothing
    perm = rng.permutation(Kp.shape[0])
    inv = np.argsort(perm)
    got2 = O.decode_attention_paged(Q, Kp[perm], Vp[perm], sQ, sKp[perm], sVp[perm],
                                    inv[tables].astype(np.int32), lens)
    np.testing.assert_array_equal(got2, got)
    # positions past a sequence's length never enter
    lens3 = np.array([17, 33], np.int32)
    a = O.decode_attention_paged(Q, Kp, Vp, sQ, sKp, sVp, tables, lens3)
    Kp2 = Kp.copy()
    Kp2[1, :, 1:] = 99          # sequence 0, positions 17.. (page 1, rows 1..)
    Kp2[tables[1][2], :, 1:] = -99  # sequence 1, positions 33..
    b_ = O.decode_attention_paged(Q, Kp2, Vp, sQ, sKp, sVp, tables, lens3)
    np.testing.assert_array_equal(a, b_)
    ref3 = O.decode_attention(Q[1], K[1, :, :33], V[1, :, :33], sQ[1], sK[1, :, :33], sV[1, :, :33])
    np.testing.assert_allclose(a[1], ref3, rtol=0, atol=1e-12)


@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_quantize_matches_torch_layer_norm(affine):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((33, 257)) * 3 + 1.5).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 257).astype(np.float32) if affine else None
    b = rng.uniform(-0.2, 0.2, 257).astype(np.float32) if affine else None
    q, s, y = O.layernorm_quantize_per_token(x, g, b, 1e-5, "f32")
    ref = torch.nn.functional.layer_norm(
        torch.from_numpy(x).double(), (257,),
        torch.from_numpy(g).double() if affine else None,
        torch.from_numpy(b).double() if affine else None, 1e-5).float().numpy()
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-6)
    rq, rs = O.quantize_per_token(ref)
    assert np.abs(q.astype(np.int32) - rq).max() <= 1
    np.testing.assert_allclose(s, rs, rtol=1e-6)
    # two-valued row: y = +-1 exactly -> codes +-127, scale 1/127
    q2, s2, y2 = O.layernorm_quantize_per_token(np.array([[3.0, 5.0] * 8]), None, None, 0.0, "f16")
    assert set(q2[0].tolist()) == {127, -127} and s2[0] == np.float32(np.float32(1.0) / 127)


def test_quantize_heads_matches_loop():
    rng = np.random.default_rng(8)
    B, S, P, H, Dh = 2, 3, 3, 2, 8
    x = rng.standard_normal((B, S, P * H * Dh)).astype(np.float32)
    outs = O.quantize_heads(x, H, P)
    for p in range(P):
        for b in range(B):
            for s in range(S):
                for h in range(H):
                    row = x[b, s, (p * H + h) * Dh:(p * H + h + 1) * Dh]
                    rq, rs = O.quantize_per_token(row[None])
                    np.testing.assert_array_equal(outs[p][0][b, h, s], rq[0])
                    assert outs[p][1][b, h, s] == rs[0]
