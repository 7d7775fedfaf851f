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
    need = capi.decode_workspace_bytes(4, 100, 128)
    assert _decode_call(lib, ws_bytes=need - 1) == capi.INT8K_ERR_WORKSPACE
    assert _decode_call(lib, ws=0) == capi.INT8K_ERR_WORKSPACE


@pytest.mark.parametrize("BH,S,D", [(1, 1, 64), (12, 1024, 64), (1024, 8192, 128),
                                    (256, 32768, 64), (3, 1000, 128)])
def test_decode_split_plan(capi, BH, S, D):
    ns = capi.decode_num_splits(BH, S, D)
    assert 1 <= ns <= S
    ws = capi.decode_workspace_bytes(BH, S, D)
    assert ws >= BH * ns * (D + 2) * 4
    # forced split counts are honoured up to what S allows
    assert capi.decode_num_splits(BH, S, D, 1) == 1
    assert capi.decode_num_splits(BH, S, D, 10 ** 6) <= S
    # the headline config fills 256 CUs many times over
    if (BH, S, D) == (1024, 8192, 128):
        assert BH * ns >= 4096
