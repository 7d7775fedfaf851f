"""C ABI checks that need no GPU: the library loads, exports every symbol
include/int8k.h declares, and rejects bad arguments before touching a device.
"""
import ctypes

import pytest


def test_library_exports_every_declared_symbol(capi):
    lib = capi.load()
    names = capi.declared_symbols()
    assert "int8k_decode_attention_forward" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes binding knows every one of them
    assert set(names) <= set(capi._SIGNATURES), set(names) - set(capi._SIGNATURES)


def test_status_strings_and_version(capi):
    lib = capi.load()
    assert lib.int8k_abi_version() == 1
    for code in range(6):
        assert lib.int8k_status_string(code)
    assert lib.int8k_status_string(99) == b"unknown status"


def _fake(addr):
    return ctypes.c_void_p(addr)


def _decode_call(lib, Q=0x10000, K=0x20000, V=0x30000, out=0x40000, sQ=0x50000, sK=0x60000,
                 sV=0x70000, BH=4, S=100, D=128, nsplit=0, ws=0x80000, ws_bytes=1 << 30):
    return lib.int8k_decode_attention_forward(
        _fake(Q), _fake(K), _fake(V), _fake(out), _fake(sQ), _fake(sK), _fake(sV), BH, S, D,
        nsplit, _fake(ws), ws_bytes, None)


def test_decode_argument_validation(capi):
    lib = capi.load()
    assert _decode_call(lib, Q=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert _decode_call(lib, sV=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert _decode_call(lib, BH=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert _decode_call(lib, S=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert _decode_call(lib, nsplit=-1) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert _decode_call(lib, D=96) == capi.INT8K_ERR_UNSUPPORTED
    assert _decode_call(lib, D=256) == capi.INT8K_ERR_UNSUPPORTED
    assert _decode_call(lib, K=0x20001) == capi.INT8K_ERR_MISALIGNED
    assert _decode_call(lib, sK=0x60002) == capi.INT8K_ERR_MISALIGNED
    # a forced 32-chunk plan runs the split kernel, whose partials need a workspace
    need = capi.decode_workspace_bytes(4, 8192, 128, 32)
    assert need > 0
    assert _decode_call(lib, S=8192, nsplit=32, ws_bytes=need - 1) == capi.INT8K_ERR_WORKSPACE
    assert _decode_call(lib, S=8192, nsplit=32, ws=0) == capi.INT8K_ERR_WORKSPACE
    assert _decode_call(lib, S=8192, nsplit=32, ws=0x80008) == capi.INT8K_ERR_MISALIGNED
    # plans merged on chip need none
    assert capi.decode_workspace_bytes(4, 100, 128) == 0


@pytest.mark.parametrize("BH,S,D", [(1, 1, 64), (12, 1024, 64), (1024, 8192, 128),
                                    (256, 32768, 64), (3, 1000, 128)])
def test_decode_split_plan(capi, BH, S, D):
    ns = capi.decode_num_splits(BH, S, D)
    assert 1 <= ns <= S
    ws = capi.decode_workspace_bytes(BH, S, D)
    if ns > 16:
        assert ws >= BH * ns * (D + 2) * 4
    else:
        assert ws == 0  # the one-launch kernel merges the chunks on chip
    # forced split counts are honoured up to what S allows
    assert capi.decode_num_splits(BH, S, D, 1) == 1
    assert capi.decode_num_splits(BH, S, D, 10 ** 6) <= S
    # the headline config fills 256 CUs many times over
    if (BH, S, D) == (1024, 8192, 128):
        assert BH * ns >= 4096


def test_decode_auto_plans_skip_9_to_16_chunks(capi):
    # automatic plans take at most 8 chunks per (b,h) on the one-launch kernel (the 8-wave
    # instance) or more than 16 on the split kernel; forced counts of 9..16 are honoured
    for D in (64, 128):
        for BH in (1, 2, 12, 32, 64, 128, 256, 384, 512, 1024, 4096):
            for S in (1, 63, 64, 100, 1024, 2048, 3000, 4096, 8192, 16384, 40000, 131072):
                ns = capi.decode_num_splits(BH, S, D)
                assert 1 <= ns <= 8 or ns > 16, (BH, S, D, ns)
        assert capi.decode_num_splits(12, 1024, D, 16) == 16
    assert capi.decode_num_splits(12, 1024, 64) == 8


@pytest.mark.parametrize("B,H,S,D", [(1, 1, 1, 64), (8, 32, 32768, 64), (32, 32, 8192, 128),
                                     (1, 2, 40000, 128)])
def test_decode_paged_split_plan(capi, B, H, S, D):
    ns = capi.decode_paged_num_splits(B, H, S, D)
    assert 1 <= ns <= S
    assert capi.decode_paged_workspace_bytes(B, H, S, D) >= B * H * ns * (D + 2) * 4
    assert capi.decode_paged_num_splits(B, H, S, D, 1) == 1
    assert capi.decode_paged_num_splits(B, H, S, D, 10 ** 6) <= S
    assert capi.decode_paged_num_splits(0, H, S, D) == 0
    assert capi.decode_paged_num_splits(B, H, S, 96) == 0
    # the BASELINE shapes plan 8 chunks per (b,h): the one-launch paged kernel
    if (B, H, S, D) in ((8, 32, 32768, 64), (32, 32, 8192, 128)):
        assert ns == 8


def test_prefill_argument_validation(capi):
    lib = capi.load()
    f = lambda **kw: lib.int8k_attention_forward(  # noqa: E731
        _fake(kw.get("Q", 0x10000)), _fake(0x20000), _fake(0x30000), _fake(kw.get("out", 0x40000)),
        _fake(0x50000), _fake(0x60000), _fake(0x70000), kw.get("B", 1), 2, kw.get("S", 64),
        kw.get("D", 128), 0, None)
    assert f(Q=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(S=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(B=-1) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(D=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(D=513) == capi.INT8K_ERR_UNSUPPORTED
    assert f(Q=0x10008) == capi.INT8K_ERR_MISALIGNED
    assert f(out=0x40002) == capi.INT8K_ERR_MISALIGNED
    # head dims off the MFMA kernel (generic kernel) need only element alignment
    assert f(D=96, Q=0x10008) == capi.INT8K_ERR_MISALIGNED  # 96: padded MFMA kernel
    assert f(D=72, out=0x40001) == capi.INT8K_ERR_MISALIGNED


def test_mlp_argument_validation(capi):
    lib = capi.load()

    def f(n_sx=4, dm=64, dff=128, flags=0, ws=0x90000, ws_bytes=1 << 30, x=0x10000):
        return lib.int8k_mlp_forward(_fake(x), _fake(0x20000), _fake(0x30000), _fake(0x40000),
                                     _fake(0x50000), n_sx, _fake(0x60000), 1, _fake(0x70000), 1,
                                     None, _fake(0x80000), 4, dm, dff, flags, _fake(ws),
                                     ws_bytes, None)
    assert f(x=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(n_sx=3) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(flags=8) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert f(dm=60) == capi.INT8K_ERR_UNSUPPORTED
    assert f(x=0x10004) == capi.INT8K_ERR_MISALIGNED
    need = capi.mlp_workspace_bytes(4, 64, 128, 0)
    assert f(ws_bytes=need - 1) == capi.INT8K_ERR_WORKSPACE
    assert capi.mlp_workspace_bytes(4, 64, 128, capi.MLP_WEIGHTS_PREPACKED) < need
    assert lib.int8k_gemm_i8_i32(_fake(0x10000), _fake(0x20000), _fake(0x30000), 4, 4, 40,
                                 None) == capi.INT8K_ERR_UNSUPPORTED


def test_operands_of_4gib_are_refused_before_launch(capi):
    # the 256 x 256 GEMMs address each operand with 32-bit buffer offsets: a call with an
    # operand of 4 GiB or more (here the T x d_ff hidden that GEMM2 reads) returns
    # UNSUPPORTED from its argument checks, with no GPU work enqueued (none exists here)
    lib = capi.load()
    T, dm, dff = 1 << 18, 4096, 16384
    flags = capi.MLP_WEIGHTS_PREPACKED
    ws_bytes = capi.mlp_workspace_bytes(T, dm, dff, flags)
    assert ws_bytes > T * dff
    st = lib.int8k_mlp_forward(_fake(0x10000), _fake(0x20000), _fake(0x30000), _fake(0x40000),
                               _fake(0x50000), 1, _fake(0x60000), 1, _fake(0x70000), 1, None,
                               _fake(0x80000), T, dm, dff, flags, _fake(0x100000), ws_bytes,
                               None)
    assert st == capi.INT8K_ERR_UNSUPPORTED
    assert b"4 GiB" in lib.int8k_last_error()
    assert lib.int8k_gemm_i8_i32(_fake(0x10000), _fake(0x20000), _fake(0x30000), 1 << 16, 256,
                                 1 << 16, None) == capi.INT8K_ERR_UNSUPPORTED


def test_quant_argument_validation(capi):
    lib = capi.load()
    # per-token dequant: unknown dtype, misaligned scales
    assert lib.int8k_dequantize_per_token(_fake(0x10000), _fake(0x20000), 5, None,
                                          _fake(0x30000), 4, 64,
                                          None) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_dequantize_per_token(_fake(0x10000), _fake(0x20002), 0, None,
                                          _fake(0x30000), 4, 64, None) == capi.INT8K_ERR_MISALIGNED
    assert lib.int8k_quantize_per_token(_fake(0x10000), 7, _fake(0x20000), _fake(0x30000), 4,
                                        64, None) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_quantize_per_token(_fake(0x10001), 0, _fake(0x20000), _fake(0x30000), 4,
                                        64, None) == capi.INT8K_ERR_MISALIGNED
    assert lib.int8k_quantize_fp16_to_int8(_fake(0x10000), _fake(0x20000), None, 16,
                                           None) == capi.INT8K_ERR_INVALID_ARGUMENT
    # append past the capacity
    assert lib.int8k_kv_cache_append(_fake(0x10000), _fake(0x20000), 0, _fake(0x30000),
                                     _fake(0x40000), _fake(0x50000), _fake(0x60000), 2, 5, 96,
                                     100, 64, None) == capi.INT8K_ERR_INVALID_ARGUMENT
    # decode over a cache shorter than the attended length
    assert lib.int8k_decode_attention_forward_cache(
        _fake(0x10000), _fake(0x20000), _fake(0x30000), _fake(0x40000), _fake(0x50000),
        _fake(0x60000), _fake(0x70000), 4, 200, 100, 128, 0, _fake(0x80000), 1 << 30,
        None) == capi.INT8K_ERR_INVALID_ARGUMENT


def test_quantized_attention_output_validation(capi):
    # the int8-output entry points: both outputs required, scale output 4-byte aligned,
    # the rest of the checks shared with the fp16 entry points
    lib = capi.load()
    F = _fake
    pre = lambda q=0x40000, s=0x48000, D=128: lib.int8k_attention_forward_quant(  # noqa: E731
        F(0x10000), F(0x20000), F(0x30000), F(q), F(s), F(0x50000), F(0x60000), F(0x70000),
        1, 2, 64, D, 1, None)
    assert pre(q=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert pre(s=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert pre(s=0x48002) == capi.INT8K_ERR_MISALIGNED
    assert pre(D=600) == capi.INT8K_ERR_UNSUPPORTED
    # flags: bit 0 causal, bit 1 [B,S,H,D] output; any other bit is refused
    fwd = lambda flags: lib.int8k_attention_forward(  # noqa: E731
        F(0x10000), F(0x20000), F(0x30000), F(0x40000), F(0x50000), F(0x60000), F(0x70000),
        1, 2, 64, 600, flags, None)
    assert capi.ATTN_CAUSAL == 1 and capi.ATTN_OUT_BSHD == 2
    for flags in (0, 1, 2, 3):  # valid flags reach the head_dim check
        assert fwd(flags) == capi.INT8K_ERR_UNSUPPORTED
    for flags in (4, 8, -1):
        assert fwd(flags) == capi.INT8K_ERR_INVALID_ARGUMENT
    # a forced 32-chunk plan: the split kernel, whose partials need a workspace
    dec = lambda q=0x40000, s=0x48000, ws_bytes=1 << 30: (  # noqa: E731
        lib.int8k_decode_attention_forward_quant(
            F(0x10000), F(0x20000), F(0x30000), F(q), F(s), F(0x50000), F(0x60000), F(0x70000),
            4, 8192, 128, 32, F(0x80000), ws_bytes, None))
    assert dec(q=0) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert dec(s=0x48001) == capi.INT8K_ERR_MISALIGNED
    assert dec(ws_bytes=capi.decode_workspace_bytes(4, 8192, 128, 32) - 1) == \
        capi.INT8K_ERR_WORKSPACE
    assert lib.int8k_decode_attention_forward_cache_quant(
        F(0x10000), F(0x20000), F(0x30000), F(0x40000), F(0), F(0x50000), F(0x60000),
        F(0x70000), 4, 100, 90, 128, 0, F(0x80000), 1 << 30, None) == \
        capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_decode_attention_forward_paged_quant(
        F(0x10000), F(0x20000), F(0x30000), F(0), F(0x48000), F(0x50000), F(0x60000),
        F(0x70000), F(0x80000), F(0x90000), 2, 4, 128, 8, 16, 4, 64, 0, F(0xa0000), 1 << 30,
        None) == capi.INT8K_ERR_INVALID_ARGUMENT


def test_paged_decode_argument_validation(capi):
    lib = capi.load()
    F = _fake

    def call(page=16, max_pages=4, max_context=64, D=128, K=0x20000, ws_bytes=1 << 30):
        return lib.int8k_decode_attention_forward_paged(
            F(0x10000), F(K), F(0x30000), F(0x40000), F(0x50000), F(0x60000), F(0x70000),
            F(0x80000), F(0x90000), 2, 4, D, 8, page, max_pages, max_context, 0, F(0xa0000),
            ws_bytes, None)

    assert call(page=24) == capi.INT8K_ERR_UNSUPPORTED      # not a power of two
    assert call(page=8) == capi.INT8K_ERR_UNSUPPORTED       # below 16
    assert call(page=2048) == capi.INT8K_ERR_UNSUPPORTED    # above 1024
    assert call(D=96) == capi.INT8K_ERR_UNSUPPORTED
    assert call(max_context=65) == capi.INT8K_ERR_INVALID_ARGUMENT  # > max_pages * page
    assert call(K=0x20008) == capi.INT8K_ERR_MISALIGNED
    need = lib.int8k_decode_attention_paged_workspace_bytes(2, 4, 64, 128, 0)
    assert need > 0
    assert call(ws_bytes=need - 1) == capi.INT8K_ERR_WORKSPACE


def test_producer_argument_validation(capi):
    lib = capi.load()
    F = _fake
    # LayerNorm + quantize: unknown dtype, negative eps
    assert lib.int8k_layernorm_quantize_per_token(F(0x10000), 9, None, None, 1e-5, F(0x20000),
                                                  F(0x30000), None, 4, 64,
                                                  None) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_layernorm_quantize_per_token(F(0x10000), 0, None, None, -1.0, F(0x20000),
                                                  F(0x30000), None, 4, 64,
                                                  None) == capi.INT8K_ERR_INVALID_ARGUMENT
    # zero rows is a no-op
    assert lib.int8k_layernorm_quantize_per_token(F(0x10000), 0, None, None, 1e-5, F(0x20000),
                                                  F(0x30000), None, 0, 64, None) == capi.INT8K_OK
    # split heads: parts out of range, a missing output of a requested part
    assert lib.int8k_quantize_heads(F(0x10000), 0, 4, F(1), F(2), F(3), F(4), F(5), F(6), 1, 2,
                                    2, 64, None) == capi.INT8K_ERR_INVALID_ARGUMENT
    assert lib.int8k_quantize_heads(F(0x10000), 0, 2, F(0x20000), F(0x30000), None, None, None,
                                    None, 1, 2, 2, 64, None) == capi.INT8K_ERR_INVALID_ARGUMENT


def test_bench_refuses_more_than_one_gpu():
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(repo, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_mlp_unpacked_workspace_holds_no_weight_copies(capi):
    # where both GEMMs run the 256 x 256 kernels, the unpacked weights are read as stored:
    # the workspace holds no transposed copies; the 128 x 128 GEMM2 of (2048, 2048, 8192)
    # still reads a transposed W2
    P = capi.MLP_WEIGHTS_PREPACKED
    assert capi.mlp_workspace_bytes(4096, 4096, 16384, 0) == capi.mlp_workspace_bytes(
        4096, 4096, 16384, P)
    assert capi.mlp_workspace_bytes(2048, 2048, 8192, 0) >= capi.mlp_workspace_bytes(
        2048, 2048, 8192, P) + 2048 * 8192
