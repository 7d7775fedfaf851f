"""The MLP on unpacked weights read as stored ([K][N]) against the prepacked path (GPU tests).

The reference's callers pass W1 [d_model, d_ff] and W2 [d_ff, d_model] to int8_mlp_forward
on every call (bench/bench_block.py:111, validation/validate_int8.py:248), and its forward
transposes both each time (kernels/int8_mlp.cu:1034-1049).  Here the 256 x 256 GEMM kernels
stage such a B tile as it arrives and form the K-contiguous MFMA fragments with transposing
LDS reads (ds_read_b64_tr_b8), so no transpose runs on those grids.  The int32 products are
the same sums, so the outputs must equal the prepacked path's byte for byte: with the fused
requantization and with the separate passes, per-token and per-tensor, with bias, and on
ragged shapes whose edge tiles zero-fill K rows and N columns.  Shapes on the other tilings
still transpose and are covered by tests/test_mlp_gpu.py.
"""
import pytest
import torch

import int8k_capi as capi
import workloads

pytestmark = pytest.mark.gpu

P = capi.MLP_WEIGHTS_PREPACKED


@pytest.mark.parametrize("T,dm,dff", [
    (4096, 4096, 16384),
    (4000, 4000, 16000),   # ragged rows, columns and K on both GEMMs
    (2048, 2048, 8192),    # GEMM1 on the tiled kernel, GEMM2 on the 128 x 128 kernel
    (1100, 1040, 8208),    # K % 128 != 0 and N % 256 != 0 on GEMM1
])
@pytest.mark.parametrize("extra", [0, capi.MLP_SEPARATE_REQUANT, capi.MLP_OUT_PER_TENSOR])
def test_unpacked_matches_prepacked(gpu, T, dm, dff, extra):
    print(f"unpacked T{T} dm{dm} dff{dff} flags {extra}", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=T + dm, device=gpu)
    x = c["x"].reshape(T, dm)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    scales = (c["sx"], c["sW1"], c["sW2"])
    out_u, sc_u = capi.mlp_forward(x, c["W1"], c["W2"], *scales, flags=extra)
    out_p, sc_p = capi.mlp_forward(x, W1T, W2T, *scales, flags=extra | P)
    torch.cuda.synchronize()
    assert torch.equal(out_u, out_p)
    assert torch.equal(sc_u, sc_p)
    assert capi.mlp_sync_timeouts() == 0


def test_unpacked_bias(gpu):
    T, dm, dff = 2048, 2048, 8192
    print("unpacked bias", flush=True)
    c = workloads.mlp_case(T, dm, dff, seed=3, device=gpu)
    bias = (torch.randn(dff, generator=torch.Generator().manual_seed(4)) * 0.5).to(gpu)
    x = c["x"].reshape(T, dm)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    scales = (c["sx"], c["sW1"], c["sW2"])
    out_u, sc_u = capi.mlp_forward(x, c["W1"], c["W2"], *scales, bias1=bias)
    out_p, sc_p = capi.mlp_forward(x, W1T, W2T, *scales, bias1=bias, flags=P)
    torch.cuda.synchronize()
    assert torch.equal(out_u, out_p) and torch.equal(sc_u, sc_p)

