"""Frozen small vectors (tests/golden/golden_small.npz, written by make_golden.py).

CPU: the oracle still reproduces them.  GPU: the kernels reproduce them to
the usual bars (attention 2e-2 / 0.9999, MLP +-1 LSB, quantizer bit-exact).
"""
import os

import numpy as np
import pytest
import torch

from helpers import assert_attn_close
from oracle import int8_oracle as O
from oracle import oracle_c

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_small.npz"))


def test_oracle_reproduces_golden():
    np.testing.assert_allclose(
        O.decode_attention(G["dec_q"], G["dec_k"], G["dec_v"], G["dec_sq"], G["dec_sk"],
                           G["dec_sv"]), G["dec_out"], atol=1e-12)
    np.testing.assert_allclose(
        oracle_c.decode_attention(G["dec_q"], G["dec_k"], G["dec_v"], G["dec_sq"], G["dec_sk"],
                                  G["dec_sv"]), G["dec_out"], atol=1e-12)
    for causal, key in ((False, "pre_out"), (True, "pre_out_causal")):
        np.testing.assert_allclose(
            oracle_c.prefill_attention(G["pre_q"], G["pre_k"], G["pre_v"], G["pre_sq"],
                                       G["pre_sk"], G["pre_sv"], causal=causal), G[key],
            atol=1e-12)
    out, osc = O.mlp_forward(G["mlp_x"], G["mlp_w1"], G["mlp_w2"], G["mlp_sx"], G["mlp_s1"],
                             G["mlp_s2"], bias1=G["mlp_b1"])
    np.testing.assert_array_equal(out, G["mlp_out"])
    np.testing.assert_array_equal(osc, G["mlp_out_scale"])
    q, s = O.quantize_per_token(G["qpt_x"])
    np.testing.assert_array_equal(q, G["qpt_q"])
    np.testing.assert_array_equal(s, G["qpt_s"])


@pytest.mark.gpu
def test_kernels_reproduce_golden(ext, gpu):
    t = lambda k: torch.from_numpy(np.ascontiguousarray(G[k])).to(gpu)  # noqa: E731
    BH = G["dec_q"].shape[0]
    out = ext.int8_decode_attention_forward(t("dec_q").reshape(1, BH, 64),
                                            t("dec_k").reshape(1, BH, 37, 64),
                                            t("dec_v").reshape(1, BH, 37, 64), t("dec_sq"),
                                            t("dec_sk"), t("dec_sv"))
    assert_attn_close(out.float().cpu().numpy().reshape(BH, 64), G["dec_out"], "golden decode")
    for causal, key in ((False, "pre_out"), (True, "pre_out_causal")):
        out = ext.int8_attention_forward(t("pre_q").reshape(1, 2, 20, 64),
                                         t("pre_k").reshape(1, 2, 20, 64),
                                         t("pre_v").reshape(1, 2, 20, 64), t("pre_sq"),
                                         t("pre_sk"), t("pre_sv"), causal)
        assert_attn_close(out.float().cpu().numpy().reshape(2, 20, 64), G[key], key)
    out, osc = ext.int8_mlp_forward_per_channel_bias(
        t("mlp_x").reshape(1, 16, 64), t("mlp_w1"), t("mlp_w2"), t("mlp_sx"), t("mlp_s1"),
        t("mlp_s2"), t("mlp_b1"))
    d = np.abs(out.cpu().numpy().reshape(16, 64).astype(np.int32) - G["mlp_out"].astype(np.int32))
    assert d.max() <= 1
    np.testing.assert_allclose(osc.cpu().numpy(), G["mlp_out_scale"], rtol=2e-3)
    q, s = ext.quantize_per_token(t("qpt_x"))
    np.testing.assert_array_equal(q.cpu().numpy(), G["qpt_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), G["qpt_s"])
