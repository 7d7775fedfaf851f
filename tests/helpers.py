"""Shared comparison helpers for the parity tests."""
from __future__ import annotations

import numpy as np

# Tolerances for fp16 attention outputs against the float64 oracle on the
# same quantized inputs.
ATTN_MAX_ABS = 2e-2
ATTN_MIN_COS = 0.9999


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def attn_metrics(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    return dict(max_abs=float(np.abs(out - ref).max()), cos=cosine(out, ref),
                finite=bool(np.isfinite(out).all()))


def assert_attn_close(out, ref, label=""):
    m = attn_metrics(out, ref)
    assert m["finite"], f"{label}: non-finite output"
    assert m["max_abs"] <= ATTN_MAX_ABS, f"{label}: max_abs {m['max_abs']:.3e} > {ATTN_MAX_ABS}"
    assert m["cos"] >= ATTN_MIN_COS, f"{label}: cos {m['cos']:.6f} < {ATTN_MIN_COS}"
    return m
