"""CPU checks of arithmetic identities the kernels rely on (no GPU).

The MLP's GEMM2 can quantize the fp16 hidden on its way to LDS
(gemm_i8_a16_kernel, mlp.hip): code = low byte of the fp32 bits of
fl(h * inv) + 1.5 * 2^23, which must equal the separate requantization pass's
rint(clamp(fl(h * inv), -128, 127)) (requant_rows_kernel; the reference's
quantize_rows, kernels/int8_mlp.cu:768-795) for every fp16 h the pass can
see, |h| <= fp16(amax).  Checked here exhaustively over all finite fp16
values and a spread of row maxima, in float32 arithmetic as the GPU does it.
"""
import numpy as np
import pytest

F32 = np.float32


def _magic_codes(h, inv):
    p = (h.astype(F32) * F32(inv)).astype(F32)  # fl(h * inv), one rounding
    t = (p + F32(12582912.0)).astype(F32)       # round half to even onto the integer grid
    return (t.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)


def _pass_codes(h, inv):
    p = (h.astype(F32) * F32(inv)).astype(F32)
    return np.rint(np.clip(p, F32(-128.0), F32(127.0))).astype(np.int8)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_magic_number_rounding_equals_requant_pass(seed):
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    allh = bits.view(np.float16)
    allh = allh[np.isfinite(allh)]
    rng = np.random.default_rng(seed)
    amaxes = np.concatenate([rng.uniform(1e-8, 1e-4, 8), rng.uniform(1e-4, 1.0, 8),
                             rng.uniform(1.0, 65504.0, 8), [1e-8, 0.5, 1.0, 127.0, 65504.0]])
    for amax in amaxes.astype(F32):
        amax = max(amax, F32(1e-8))
        inv = F32(F32(127.0) / amax)
        # the hidden the pass sees: fp16 of values |v| <= amax
        h = allh[np.abs(allh.astype(F32)) <= np.float16(amax).astype(F32)]
        np.testing.assert_array_equal(_magic_codes(h, inv), _pass_codes(h, inv))


def test_magic_number_rounding_ties_go_to_even():
    inv = F32(1.0)
    h = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5], dtype=np.float16)
    np.testing.assert_array_equal(_magic_codes(h, inv),
                                  np.array([0, 2, 2, 0, -2, -2, 126, -128], dtype=np.int8))
