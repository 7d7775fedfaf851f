"""Writes tests/golden/golden_small.npz — small frozen input/output vectors.

Attention expectations come from pure-Python loops (independent of the oracle
code), the MLP and quantizer expectations from the oracle as of when the file
was made; tests/test_golden.py checks the oracle (CPU) and the kernels (GPU)
against them, so a later change to either shows up as a diff here.

    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import int8_oracle as O  # noqa: E402


def loops_attention(Q, K, V, sQ, sK, sV, causal):
    BH, Sq, D = Q.shape
    Sk = K.shape[1]
    out = np.zeros((BH, Sq, D))
    for b in range(BH):
        for i in range(Sq):
            n = i + 1 if causal else Sk
            sc = [sum(int(Q[b, i, d]) * int(K[b, j, d]) for d in range(D)) * float(sQ[b, i]) *
                  float(sK[b, j]) / math.sqrt(D) for j in range(n)]
            m = max(sc)
            p = [math.exp(x - m) for x in sc]
            z = sum(p)
            for d in range(D):
                out[b, i, d] = sum(p[j] * int(V[b, j, d]) * float(sV[b, j]) for j in range(n)) / z
    return out


def main():
    g = np.random.default_rng(20241201)
    f = {}
    # decode: BH=3, S=37, D=64 (one query per (b,h))
    q, sq = O.quantize_per_token(g.standard_normal((3, 1, 64)).astype(np.float32))
    k, sk = O.quantize_per_token(g.standard_normal((3, 37, 64)).astype(np.float32))
    v, sv = O.quantize_per_token(g.standard_normal((3, 37, 64)).astype(np.float32))
    f.update(dec_q=q[:, 0], dec_sq=sq[:, 0], dec_k=k, dec_sk=sk, dec_v=v, dec_sv=sv,
             dec_out=loops_attention(q, k, v, sq, sk, sv, False)[:, 0])
    # prefill: BH=2, S=20, D=64, causal and not
    q, sq = O.quantize_per_token(g.standard_normal((2, 20, 64)).astype(np.float32))
    k, sk = O.quantize_per_token(g.standard_normal((2, 20, 64)).astype(np.float32))
    v, sv = O.quantize_per_token(g.standard_normal((2, 20, 64)).astype(np.float32))
    f.update(pre_q=q, pre_sq=sq, pre_k=k, pre_sk=sk, pre_v=v, pre_sv=sv,
             pre_out=loops_attention(q, k, v, sq, sk, sv, False),
             pre_out_causal=loops_attention(q, k, v, sq, sk, sv, True))
    # MLP: T=16, 64 -> 128 -> 64, per token / per channel, with bias
    x, sx = O.quantize_per_token(g.standard_normal((16, 64)).astype(np.float32))
    w1, s1 = O.quantize_per_channel_w((g.standard_normal((64, 128)) * 0.02).astype(np.float32))
    w2, s2 = O.quantize_per_channel_w((g.standard_normal((128, 64)) * 0.02).astype(np.float32))
    b1 = (g.standard_normal(128) * 0.1).astype(np.float32)
    out, osc = O.mlp_forward(x, w1, w2, sx, s1, s2, bias1=b1)
    f.update(mlp_x=x, mlp_sx=sx, mlp_w1=w1, mlp_s1=s1, mlp_w2=w2, mlp_s2=s2, mlp_b1=b1,
             mlp_out=out, mlp_out_scale=osc)
    # per-token quantizer on a boundary-coded fp32 block
    xb = (np.sign(g.standard_normal((8, 96))) * 4 * (0.985 + 0.015 * g.random((8, 96))))
    xb = xb.astype(np.float32)
    qb, sb = O.quantize_per_token(xb)
    f.update(qpt_x=xb, qpt_q=qb, qpt_s=sb)
    np.savez_compressed(os.path.join(HERE, "golden_small.npz"), **f)
    print("wrote", os.path.join(HERE, "golden_small.npz"))


if __name__ == "__main__":
    main()
