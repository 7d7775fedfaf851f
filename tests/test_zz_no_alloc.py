"""int8k_decode_attention_forward_noalloc against int8k_decode_attention_forward.

The no-alloc entry point runs the same split and combine kernels with the
partials in the library's device scratch instead of a caller workspace, so its
output must equal the workspace entry point's byte for byte.  Two calls in a
row, the second smaller, check that the scratch left by the first call does
not leak into the second.  The size limit is checked on the CPU: a call that
needs more scratch than the library holds is rejected before any HIP call.
"""
import ctypes

import pytest

import workloads


def _flat(case):
    B, H, D = case["Qi"].shape
    S = case["Ki"].shape[2]
    BH = B * H
    return (case["Qi"].reshape(BH, D), case["Ki"].reshape(BH, S, D),
            case["Vi"].reshape(BH, S, D), case["sQ"].reshape(BH), case["sK"].reshape(BH * S),
            case["sV"].reshape(BH * S))


def test_noalloc_rejects_calls_above_the_scratch_size(capi):
    lib = capi.load()
    P = ctypes.c_void_p
    args = [P(0x10000 * (i + 1)) for i in range(7)]
    limit = 8 << 20
    # B128 H1 D64 S16384 with 256 splits: 32768 units of (64 + 2) floats = 8.6 MB of partials
    assert capi.decode_workspace_bytes(128, 16384, 64, 256) > limit
    st = lib.int8k_decode_attention_forward_noalloc(*args, 128, 16384, 64, 256, None)
    assert st == capi.INT8K_ERR_WORKSPACE
    assert b"8 MiB" in lib.int8k_last_error()
    assert lib.int8k_decode_attention_forward_noalloc(*args[:3], P(0), *args[4:], 4, 100, 128,
                                                      0, None) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_decode_attention_forward_noalloc(*args, 4, 100, 96, 0,
                                                      None) == capi.INT8K_ERR_UNSUPPORTED


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [
    ((8, 8, 128, 4096, 0), (2, 3, 128, 1000, 0)),   # automatic splits, then fewer units
    ((4, 16, 64, 8192, 0), (1, 5, 64, 777, 3)),     # D=64; a forced split count on the second
    ((32, 32, 128, 8192, 0), (4, 4, 128, 300, 2)),  # the headline shape: 8192 units of partials
])
def test_noalloc_matches_workspace_entry_point(capi, gpu, first, second):
    import torch

    for B, H, D, S, nsplit in (first, second):
        print(f"noalloc case B{B} H{H} D{D} S{S} nsplit={nsplit}", flush=True)
        case = workloads.decode_case(B, H, D, S, seed=B * 1000 + S, device=gpu,
                                     outlier_frac=0.01)
        args = _flat(case)
        ref = capi.decode_attention(*args, nsplit=nsplit)
        out = torch.full_like(ref, float("nan"))
        capi.decode_attention_noalloc(*args, out=out, nsplit=nsplit)
        torch.cuda.synchronize()
        assert capi.decode_num_splits(B * H, S, D, nsplit) >= 1
        assert torch.equal(out, ref), (B, H, D, S, nsplit)


@pytest.mark.gpu
def test_noalloc_repeated_calls_same_shape(capi, gpu):
    # the partials of one call are all rewritten by the next: repeated calls agree
    import torch

    case = workloads.decode_case(3, 5, 128, 2000, seed=3, device=gpu)
    args = _flat(case)
    ref = capi.decode_attention(*args)
    for _ in range(3):
        out = torch.empty_like(ref)
        capi.decode_attention_noalloc(*args, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
