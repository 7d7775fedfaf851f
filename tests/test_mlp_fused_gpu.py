"""The MLP's fused requantization against the separate requant pass (GPU tests).

Where a GEMM runs on the 256 x 256 tiled kernel, its epilogue requantizes per
token itself: the tiles of a 256-row stripe exchange their row maxima and each
emits int8 codes from its live accumulators, so the fp16 hidden (and the fp16
output) never reach memory.  The codes are defined as those of the separate
pass (fp16 rows, then rint(clamp(h * 127 / amax))), so the fused and the
separate path (flag INT8K_MLP_SEPARATE_REQUANT) must agree byte for byte,
outputs and scales.  Sampled rows are also checked against the CPU oracle
(rows are independent under per-token scales).  Shapes: BASELINE config 4,
ragged rows, columns and K on both GEMMs, a GEMM1-only fusion (GEMM2 on the
128 x 128 kernel), bias with the per-tensor output, hidden rows beyond the
fp16 range, 128 column tiles per stripe (the widest stripe fused), and tall
inputs (16384 and 32768 tokens) whose GEMMs walk 4-8 groups of stripes.
After each case no tile's wait for its stripe may have given up.
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from oracle import int8_oracle as O
from oracle import oracle_c

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _check_rows_vs_oracle(c, out, osc, rows, T, dm, bias=None):
    x = _np(c["x"]).reshape(T, dm)[rows]
    ref, rsc = O.mlp_forward(x, _np(c["W1"]), _np(c["W2"]), _np(c["sx"])[rows], _np(c["sW1"]),
                             _np(c["sW2"]), bias1=bias, gemm=oracle_c.gemm_i8_i32)
    got = _np(out).reshape(T, dm)[rows].astype(np.int32)
    d = np.abs(got - ref.astype(np.int32))
    assert d.max() <= 1, d.max()
    assert (d > 0).mean() <= 0.02, (d > 0).mean()
    np.testing.assert_allclose(_np(osc)[rows], rsc, rtol=2e-3)


@pytest.mark.parametrize("T,dm,dff", [
    (4096, 4096, 16384),   # both GEMMs fused
    (4000, 4000, 16000),   # ragged rows, columns and K (4000 % 128 = 32) on both GEMMs
    (2048, 2048, 8192),    # GEMM1 fused, GEMM2 on the 128 x 128 kernel
    (768, 2048, 32768),    # 128 column tiles per stripe in GEMM1
    (16384, 1024, 4096),   # the block benchmark's longest prefill: GEMM1 in 4 dispatch rounds
    (32768, 1024, 2048),   # 128 stripes of 8 (GEMM1) and 4 (GEMM2) column tiles
])
def test_fused_requant_matches_separate_pass(gpu, T, dm, dff):
    print(f"fused requant T{T} dm{dm} dff{dff}", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=T + dff, device=gpu)
    args = (c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    before = capi.mlp_sync_timeouts()
    out_f, osc_f = capi.mlp_forward(*args)
    out_s, osc_s = capi.mlp_forward(*args, flags=capi.MLP_SEPARATE_REQUANT)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_s)
    assert torch.equal(osc_f, osc_s)
    assert capi.mlp_sync_timeouts() == before
    # the fused path's workspace holds no fp16 hidden
    assert capi.mlp_workspace_bytes(T, dm, dff) + T * dff < capi.mlp_workspace_bytes(
        T, dm, dff, capi.MLP_SEPARATE_REQUANT)
    rows = np.r_[0:64, T - 64:T]
    _check_rows_vs_oracle(c, out_f, osc_f, rows, T, dm)


def test_fused_requant_repeated_calls_agree(gpu):
    # the stripe counters and row maxima are cleared by every call: repeated calls on the
    # same workspace give the same bytes
    T, dm, dff = 4096, 4096, 16384
    print("fused requant repeated calls", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=9, device=gpu)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    flags = capi.MLP_WEIGHTS_PREPACKED
    ws = torch.empty(capi.mlp_workspace_bytes(T, dm, dff, flags), dtype=torch.uint8, device=gpu)
    args = (c["x"].reshape(T, dm), W1T, W2T, c["sx"], c["sW1"], c["sW2"])
    ref, rsc = capi.mlp_forward(*args, flags=flags, workspace=ws)
    for _ in range(4):
        out, osc = capi.mlp_forward(*args, flags=flags, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(osc, rsc)
    assert capi.mlp_sync_timeouts() == 0


def test_fused_requant_bias_per_tensor_output(gpu):
    # bias before GELU; per-tensor output (GEMM2 keeps the separate output pass)
    T, dm, dff = 2048, 2048, 8192
    print("fused requant bias + per-tensor output", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=31, device=gpu)
    bias = (torch.randn(dff, generator=torch.Generator().manual_seed(2)) * 0.5).to(gpu)
    args = (c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    for flags in (0, capi.MLP_OUT_PER_TENSOR):
        out_f, osc_f = capi.mlp_forward(*args, bias1=bias, flags=flags)
        out_s, osc_s = capi.mlp_forward(*args, bias1=bias,
                                        flags=flags | capi.MLP_SEPARATE_REQUANT)
        torch.cuda.synchronize()
        assert torch.equal(out_f, out_s) and torch.equal(osc_f, osc_s), flags
    rows = np.r_[0:48, 1000:1048]
    out_f, osc_f = capi.mlp_forward(*args, bias1=bias)
    torch.cuda.synchronize()
    _check_rows_vs_oracle(c, out_f, osc_f, rows, T, dm, bias=_np(bias))


def test_fused_requant_hidden_beyond_fp16_range(gpu):
    # a few token rows scaled so their hidden exceeds 65504: fp16(v) is infinite there and
    # the code clamps to +-127, as in the separate pass
    T, dm, dff = 2048, 2048, 8192
    print("fused requant fp16 overflow rows", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=5, device=gpu)
    c["sx"][::97] *= 2e5
    args = (c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    out_f, osc_f = capi.mlp_forward(*args)
    out_s, osc_s = capi.mlp_forward(*args, flags=capi.MLP_SEPARATE_REQUANT)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_s) and torch.equal(osc_f, osc_s)
    assert capi.mlp_sync_timeouts() == 0


def test_fused_requant_under_graph_capture(gpu):
    # the fused path is kernels only (the counters are cleared by a kernel, not a memset), so
    # a captured MLP replays; every replay, with eager work on the same workspace between
    # replays, equals the eager output byte for byte
    T, dm, dff = 4096, 4096, 16384
    print("fused requant graph capture", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=13, device=gpu)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    x = c["x"].reshape(T, dm)
    ws = torch.empty(capi.mlp_workspace_bytes(T, dm, dff, capi.MLP_WEIGHTS_PREPACKED),
                     dtype=torch.uint8, device=gpu)
    out = torch.empty(T, dm, dtype=torch.int8, device=gpu)
    osc = torch.empty(T, dtype=torch.float32, device=gpu)
    args = (x, W1T, W2T, c["sx"], c["sW1"], c["sW2"])
    kw = dict(flags=capi.MLP_WEIGHTS_PREPACKED, out=out, out_scale=osc, workspace=ws)
    capi.mlp_forward(*args, **kw)
    torch.cuda.synchronize()
    ref, rsc = out.clone(), osc.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.mlp_forward(*args, **kw)
    other = workloads.mlp_case(T, dm, dff, seed=14, device=gpu)
    for i in range(3):
        out.fill_(0)
        osc.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(osc, rsc), f"replay {i}"
        # eager work between replays leaves the workspace's counters and maxima dirty
        capi.mlp_forward(other["x"].reshape(T, dm), W1T, W2T, other["sx"], c["sW1"], c["sW2"],
                         flags=capi.MLP_WEIGHTS_PREPACKED, workspace=ws)
        torch.cuda.synchronize()
    assert capi.mlp_sync_timeouts() == 0


def test_fused_requant_dirty_workspace(gpu):
    # a workspace full of arbitrary bytes (as from the caching allocator) gives the same output
    T, dm, dff = 2048, 2048, 8192
    print("fused requant dirty workspace", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=21, device=gpu)
    args = (c["x"].reshape(T, dm), c["W1"], c["W2"], c["sx"], c["sW1"], c["sW2"])
    ref, rsc = capi.mlp_forward(*args)
    n = capi.mlp_workspace_bytes(T, dm, dff)
    for fill in (0xFF, 0x7F, 0xA5):
        ws = torch.full((n,), fill, dtype=torch.uint8, device=gpu)
        out, osc = capi.mlp_forward(*args, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(osc, rsc), hex(fill)
