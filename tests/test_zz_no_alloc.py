"""int8k_decode_attention_forward_noalloc against int8k_decode_attention_forward.

The no-alloc entry point runs the same kernels with the split partials in the
library's device scratch instead of a caller workspace, so its output must
equal the workspace entry point's byte for byte.  Only plans of more than 16
chunks per (b,h) run the split kernel and touch the scratch, so every pair
below forces such plans on both calls: the second call, smaller, must not see
the first call's partials.  Plans that merge their chunks on chip need no
scratch and are accepted at any size.  The size limit itself is checked on
the CPU: a call that needs more scratch than the library holds is rejected
before any HIP call.
"""
import ctypes

import pytest

import workloads

_SPLIT_KERNEL_MIN = 17  # plans above 16 chunks per (b,h) write split partials


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


def test_noalloc_on_chip_plans_need_no_scratch(capi):
    # 16384 heads of D=128 at a short context: one chunk per (b,h), merged on chip, so the
    # size check passes however many heads there are
    assert capi.decode_num_splits(16384, 256, 128) <= 16
    assert capi.decode_workspace_bytes(16384, 256, 128) == 0
    assert capi.decode_workspace_bytes(65536, 64, 64) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [
    ((2, 4, 128, 8192, 32), (1, 3, 128, 3000, 24)),   # D=128 through the scratch, twice
    ((4, 16, 64, 8192, 0), (1, 5, 64, 6000, 24)),     # D=64: automatic 32-chunk plan, then 24
    ((8, 8, 128, 4096, 24), (2, 2, 64, 6000, 32)),    # D=128 then D=64
])
def test_noalloc_matches_workspace_entry_point(capi, gpu, first, second):
    import torch

    for B, H, D, S, nsplit in (first, second):
        print(f"noalloc case B{B} H{H} D{D} S{S} nsplit={nsplit}", flush=True)
        assert capi.decode_num_splits(B * H, S, D, nsplit) >= _SPLIT_KERNEL_MIN
        assert capi.decode_workspace_bytes(B * H, S, D, nsplit) > 0
        case = workloads.decode_case(B, H, D, S, seed=B * 1000 + S, device=gpu,
                                     outlier_frac=0.01)
        args = _flat(case)
        ref = capi.decode_attention(*args, nsplit=nsplit)
        out = torch.full_like(ref, float("nan"))
        capi.decode_attention_noalloc(*args, out=out, nsplit=nsplit)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (B, H, D, S, nsplit)


@pytest.mark.gpu
def test_noalloc_repeated_calls_same_shape(capi, gpu):
    # every partial of one call is rewritten by the next: repeated calls agree
    import torch

    B, H, D, S, nsplit = 3, 5, 128, 6000, 32
    print(f"noalloc repeated B{B} H{H} D{D} S{S} nsplit={nsplit}", flush=True)
    assert capi.decode_num_splits(B * H, S, D, nsplit) >= _SPLIT_KERNEL_MIN
    case = workloads.decode_case(B, H, D, S, seed=3, device=gpu)
    args = _flat(case)
    ref = capi.decode_attention(*args, nsplit=nsplit)
    for _ in range(3):
        out = torch.empty_like(ref)
        capi.decode_attention_noalloc(*args, out=out, nsplit=nsplit)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


@pytest.mark.gpu
def test_noalloc_many_heads_short_context(capi, gpu):
    # 16384 (b,h) at D=128: the workspace size of a split plan would exceed the scratch, but
    # the automatic plan merges on chip and needs none
    import torch

    B, H, D, S = 128, 128, 128, 64
    print(f"noalloc many heads B{B} H{H} D{D} S{S}", flush=True)
    assert capi.decode_workspace_bytes(B * H, S, D) == 0
    case = workloads.decode_case(B, H, D, S, seed=11, device=gpu)
    args = _flat(case)
    ref = capi.decode_attention(*args)
    out = torch.full_like(ref, float("nan"))
    capi.decode_attention_noalloc(*args, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.gpu
def test_noalloc_under_graph_capture(capi, gpu):
    # one warm-up call (the device's scratch address is looked up on the first call), then
    # the call captured in a HIP graph; every replay, with eager work between replays,
    # equals the workspace entry point byte for byte
    import torch

    B, H, D, S, nsplit = 2, 4, 128, 8192, 32
    print(f"noalloc graph capture B{B} H{H} D{D} S{S} nsplit={nsplit}", flush=True)
    assert capi.decode_num_splits(B * H, S, D, nsplit) >= _SPLIT_KERNEL_MIN
    case = workloads.decode_case(B, H, D, S, seed=5, device=gpu)
    args = _flat(case)
    ref = capi.decode_attention(*args, nsplit=nsplit)
    out = torch.empty_like(ref)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        capi.decode_attention_noalloc(*args, out=out, nsplit=nsplit)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.decode_attention_noalloc(*args, out=out, nsplit=nsplit)
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        # eager work on the same scratch between replays: another shape's split plan
        other = capi.decode_attention_noalloc(*_flat(workloads.decode_case(
            1, 2, 128, 4000, seed=i, device=gpu)), out=torch.empty((2, 128), dtype=torch.float16,
                                                                   device=gpu), nsplit=24)
        torch.cuda.synchronize()
        assert torch.isfinite(other).all()
