"""Seeded synthetic inputs for the BASELINE configurations (bench and tests).

The recipes follow the benchmark definitions: fp16/fp32 N(0,1) activations,
per-token symmetric int8 quantization (s = max(|row|,1e-8)/127, round half to
even, clamp [-128,127] — validation/check_decode.py:42-47), optional outlier
channels scaled x8 before quantization, N(0,0.02) weights quantized per output
channel (validation/validate_int8.py:75-81).

Generation runs on `gen_device` with torch's seeded generator, in chunks over
the leading dimension so a 2 GiB int8 KV cache never needs its 8.6 GB fp32
source resident at once.  Inputs are returned on `device`.
"""
from __future__ import annotations

import torch


def quantize_per_token(x: torch.Tensor):
    """(int8 codes, fp32 scales) with one scale per last-dim row."""
    xf = x.float()
    s = xf.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / 127.0
    q = (xf / s).round().clamp(-128, 127).to(torch.int8)
    return q, s.squeeze(-1).contiguous()


def quantize_per_channel_w(w: torch.Tensor):
    """[in, out] weight -> (int8 [in,out], fp32 [out]); amax over the input dim."""
    wf = w.float()
    s = wf.abs().amax(dim=0).clamp(min=1e-8) / 127.0
    q = (wf / s).round().clamp(-128, 127).to(torch.int8)
    return q.contiguous(), s.contiguous()


def _outlier_channels(D: int, frac: float, gen: torch.Generator, device) -> torch.Tensor:
    n = max(1, round(frac * D))
    return torch.randperm(D, generator=gen, device=device)[:n]


def _normal(shape, gen, device):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)


def decode_case(B: int, H: int, D: int, S: int, seed: int, outlier_frac: float = 0.0,
                outlier_mult: float = 8.0, device="cuda", gen_device=None):
    """Single-query decode inputs: Q [B,H,D], K/V [B,H,S,D] int8 + per-token scales.

    With outlier_frac > 0, max(1, round(outlier_frac*D)) fixed channels of K and V
    (chosen by a seeded permutation) are multiplied by outlier_mult before
    quantization.
    """
    gen_device = gen_device or device
    g = torch.Generator(device=gen_device).manual_seed(seed)
    Qf = _normal((B, H, D), g, gen_device).half()
    Qi, sQ = quantize_per_token(Qf)
    ch = _outlier_channels(D, outlier_frac, g, gen_device) if outlier_frac > 0 else None
    Ki = torch.empty((B, H, S, D), dtype=torch.int8, device=device)
    Vi = torch.empty_like(Ki)
    sK = torch.empty((B, H, S), dtype=torch.float32, device=device)
    sV = torch.empty_like(sK)
    for b in range(B):
        for dst, sdst in ((Ki, sK), (Vi, sV)):
            x = _normal((H, S, D), g, gen_device)
            if ch is not None:
                x[..., ch] *= outlier_mult
            q, s = quantize_per_token(x)
            dst[b].copy_(q)
            sdst[b].copy_(s)
            del x, q, s
    return dict(Qi=Qi.to(device), Ki=Ki, Vi=Vi, sQ=sQ.to(device), sK=sK, sV=sV)


def prefill_case(B: int, H: int, S: int, D: int, seed: int, device="cuda", gen_device=None):
    """Q/K/V [B,H,S,D] int8 with per-token scales [B,H,S]."""
    gen_device = gen_device or device
    g = torch.Generator(device=gen_device).manual_seed(seed)
    out = {}
    for name in ("Q", "K", "V"):
        q = torch.empty((B, H, S, D), dtype=torch.int8, device=device)
        s = torch.empty((B, H, S), dtype=torch.float32, device=device)
        for b in range(B):
            qi, si = quantize_per_token(_normal((H, S, D), g, gen_device))
            q[b].copy_(qi)
            s[b].copy_(si)
        out[name + "i"] = q
        out["s" + name] = s
    return out


def mlp_case(T: int, d_model: int, d_ff: int, seed: int, device="cuda", gen_device=None,
             w_std: float = 0.02):
    """x [1,T,d_model] int8 per token; W1 [d_model,d_ff], W2 [d_ff,d_model] int8 per channel."""
    gen_device = gen_device or device
    g = torch.Generator(device=gen_device).manual_seed(seed)
    xi, sx = quantize_per_token(_normal((T, d_model), g, gen_device))
    W1i, sW1 = quantize_per_channel_w(_normal((d_model, d_ff), g, gen_device) * w_std)
    W2i, sW2 = quantize_per_channel_w(_normal((d_ff, d_model), g, gen_device) * w_std)
    return dict(x=xi.reshape(1, T, d_model).to(device), sx=sx.to(device), W1=W1i.to(device),
                sW1=sW1.to(device), W2=W2i.to(device), sW2=sW2.to(device))


def paged_case(B: int, H: int, D: int, page: int, lens, seed: int, spare_pages: int = 3,
               device="cuda", gen_device=None):
    """A paged INT8 KV cache holding B sequences of lengths `lens` (per-token quantized
    N(0,1) K/V), its pages in a seeded random physical order, plus spare pages filled with
    other data.  Returns Qi [B,H,D], sQ [B,H], K/V_pages [NP,H,page,D], sK/sV_pages
    [NP,H,page], block_tables [B, max_pages] int32 (unused entries point at spare pages),
    context_lens [B] int32."""
    gen_device = gen_device or device
    g = torch.Generator(device=gen_device).manual_seed(seed)
    lens = [int(n) for n in lens]
    max_pages = max(1, max((n + page - 1) // page for n in lens))
    n_used = sum((n + page - 1) // page for n in lens)
    NP = n_used + spare_pages
    Qi, sQ = quantize_per_token(_normal((B, H, D), g, gen_device).half())
    pages = {}
    for name in ("K", "V"):
        q, s = quantize_per_token(_normal((NP, H, page, D), g, gen_device))
        pages[name] = (q.to(device), s.to(device))
    perm = torch.randperm(NP, generator=torch.Generator().manual_seed(seed)).tolist()
    tables = torch.empty((B, max_pages), dtype=torch.int32)
    nxt = 0
    for b, n in enumerate(lens):
        need = (n + page - 1) // page
        for i in range(max_pages):
            if i < need:
                tables[b, i] = perm[nxt]
                nxt += 1
            else:
                tables[b, i] = perm[n_used + (i % max(spare_pages, 1))] if spare_pages else perm[0]
    return dict(Qi=Qi.to(device), sQ=sQ.to(device), K_pages=pages["K"][0], sK_pages=pages["K"][1],
                V_pages=pages["V"][0], sV_pages=pages["V"][1], block_tables=tables.to(device),
                context_lens=torch.tensor(lens, dtype=torch.int32, device=device),
                max_context=max(lens), page=page)
