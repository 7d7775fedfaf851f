"""ctypes binding of libint8k's C ABI (include/int8k.h).

This is the binding a Python caller that does not want the torch extension
would use; the tests drive the kernels through it so parity is checked at the
C boundary itself.  torch tensors are used only to hold device memory and to
name the current HIP stream.  Loading fails loudly if the library was not
built — there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libint8k.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "int8k.h")

INT8K_OK = 0
INT8K_ERR_INVALID_ARGUMENT = 1
INT8K_ERR_UNSUPPORTED = 2
INT8K_ERR_WORKSPACE = 3
INT8K_ERR_MISALIGNED = 4
INT8K_ERR_HIP = 5

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_LL = ctypes.c_longlong

# name -> (restype, argtypes)
_SIGNATURES = {
    "int8k_status_string": (ctypes.c_char_p, [_I]),
    "int8k_abi_version": (_I, []),
    "int8k_last_error": (ctypes.c_char_p, []),
    "int8k_decode_attention_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "int8k_decode_attention_num_splits": (_I, [_I, _I, _I, _I]),
    "int8k_decode_attention_forward": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P]),
    "int8k_mlp_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "int8k_mlp_forward": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _P, _I, _P, _P, _I, _I, _I, _I,
                               _P, _SZ, _P]),
    "int8k_transpose_int8_weights": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "int8k_gemm_i8_i32": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "int8k_attention_forward": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "int8k_decode_attention_forward_cache": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                                  _P, _SZ, _P]),
    "int8k_quantize_fp16_to_int8": (_I, [_P, _P, _P, _LL, _P]),
    "int8k_dequantize_int8_to_fp16": (_I, [_P, _P, _F, _LL, _P]),
    "int8k_quantize_per_token": (_I, [_P, _I, _P, _P, _LL, _I, _P]),
    "int8k_dequantize_per_token": (_I, [_P, _P, _I, _P, _P, _LL, _I, _P]),
    "int8k_kv_cache_append": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "int8k_decode_attention_paged_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "int8k_decode_attention_paged_num_splits": (_I, [_I, _I, _I, _I, _I]),
    "int8k_layernorm_quantize_per_token": (_I, [_P, _I, _P, _P, _F, _P, _P, _P, _LL, _I, _P]),
    "int8k_quantize_heads": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "int8k_decode_attention_forward_paged": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                                  _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "int8k_attention_forward_quant": (_I, [_P] * 8 + [_I] * 5 + [_P]),
    "int8k_decode_attention_forward_quant": (_I, [_P] * 8 + [_I] * 4 + [_P, _SZ, _P]),
    "int8k_decode_attention_forward_cache_quant": (_I, [_P] * 8 + [_I] * 5 + [_P, _SZ, _P]),
    "int8k_decode_attention_forward_paged_quant": (_I, [_P] * 10 + [_I] * 8 + [_P, _SZ, _P]),
    "int8k_decode_attention_forward_noalloc": (_I, [_P] * 7 + [_I] * 4 + [_P]),
    "int8k_mlp_sync_timeouts": (_I, [ctypes.POINTER(ctypes.c_uint)]),
    "int8k_decode_paged_bad_page_ids": (_I, [ctypes.POINTER(ctypes.c_uint)]),
}

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2

MLP_WEIGHTS_PREPACKED = 1
MLP_OUT_PER_TENSOR = 2
MLP_SEPARATE_REQUANT = 4

_lib = None


class Int8kError(RuntimeError):
    def __init__(self, op: str, status: int):
        lib = load()
        msg = lib.int8k_status_string(status).decode()
        detail = lib.int8k_last_error().decode()
        super().__init__(f"{op}: {msg}" + (f" — {detail}" if detail else ""))
        self.status = status


def declared_symbols() -> list[str]:
    """Every function name declared in include/int8k.h."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(int8k_[a-z0-9_]+)\s*\(", text)))


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with "
                f"`python {os.path.join(PKG_DIR, 'build.py')}` (no CPU fallback exists)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(t):
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def check(op: str, status: int) -> None:
    if status != INT8K_OK:
        raise Int8kError(op, status)


# --------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------


def decode_workspace_bytes(BH: int, S: int, D: int, nsplit: int = 0) -> int:
    return load().int8k_decode_attention_workspace_bytes(BH, S, D, nsplit)


def decode_num_splits(BH: int, S: int, D: int, nsplit: int = 0) -> int:
    return load().int8k_decode_attention_num_splits(BH, S, D, nsplit)


def decode_attention(Qi, Ki, Vi, sQ, sK, sV, nsplit: int = 0, out=None, workspace=None):
    """Qi [BH,D] int8, Ki/Vi [BH,S,D] int8, sQ [BH], sK/sV [BH*S] fp32 (device)."""
    import torch

    BH, D = Qi.shape[0], Qi.shape[-1]
    S = Ki.numel() // (BH * D)
    if out is None:
        out = torch.empty((BH, D), dtype=torch.float16, device=Qi.device)
    ws_bytes = decode_workspace_bytes(BH, S, D, nsplit)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=Qi.device)
    st = load().int8k_decode_attention_forward(
        _ptr(Qi), _ptr(Ki), _ptr(Vi), _ptr(out), _ptr(sQ), _ptr(sK), _ptr(sV),
        BH, S, D, nsplit, _ptr(workspace), workspace.numel(), _stream(Qi))
    check("int8k_decode_attention_forward", st)
    return out


def decode_attention_noalloc(Qi, Ki, Vi, sQ, sK, sV, out, nsplit: int = 0):
    """decode_attention into a caller-given `out` [BH,D] fp16, with the split partials in the
    library's own scratch (int8k_decode_attention_forward_noalloc): no device allocation."""
    BH, D = Qi.shape[0], Qi.shape[-1]
    S = Ki.numel() // (BH * D)
    st = load().int8k_decode_attention_forward_noalloc(
        _ptr(Qi), _ptr(Ki), _ptr(Vi), _ptr(out), _ptr(sQ), _ptr(sK), _ptr(sV),
        BH, S, D, nsplit, _stream(Qi))
    check("int8k_decode_attention_forward_noalloc", st)
    return out


def decode_attention_quant(Qi, Ki, Vi, sQ, sK, sV, nsplit: int = 0):
    """As decode_attention, emitting (int8 [BH,D], fp32 scales [BH])."""
    import torch

    BH, D = Qi.shape[0], Qi.shape[-1]
    S = Ki.numel() // (BH * D)
    q, s, _ = _quant_rows((BH, D), Qi.device)
    ws = torch.empty(max(decode_workspace_bytes(BH, S, D, nsplit), 1), dtype=torch.uint8,
                     device=Qi.device)
    st = load().int8k_decode_attention_forward_quant(
        _ptr(Qi), _ptr(Ki), _ptr(Vi), _ptr(q), _ptr(s), _ptr(sQ), _ptr(sK), _ptr(sV),
        BH, S, D, nsplit, _ptr(ws), ws.numel(), _stream(Qi))
    check("int8k_decode_attention_forward_quant", st)
    return q, s


# --------------------------------------------------------------------------
# MLP / GEMM
# --------------------------------------------------------------------------


def gemm_i8_i32(A, Bt, out=None):
    """C[M,N] = A[M,K] . Bt[N,K]^T, exact int32 (device tensors)."""
    import torch

    M, K = A.shape
    N = Bt.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=A.device)
    check("int8k_gemm_i8_i32",
          load().int8k_gemm_i8_i32(_ptr(A), _ptr(Bt), _ptr(out), M, N, K, _stream(A)))
    return out


def transpose_int8_weights(W1, W2):
    import torch

    dm, dff = W1.shape
    W1T = torch.empty((dff, dm), dtype=torch.int8, device=W1.device)
    W2T = torch.empty((dm, dff), dtype=torch.int8, device=W1.device)
    check("int8k_transpose_int8_weights",
          load().int8k_transpose_int8_weights(_ptr(W1), _ptr(W2), _ptr(W1T), _ptr(W2T), dm, dff,
                                              _stream(W1)))
    return W1T, W2T


def mlp_workspace_bytes(T, d_model, d_ff, flags=0):
    return load().int8k_mlp_workspace_bytes(T, d_model, d_ff, flags)


def mlp_sync_timeouts() -> int:
    """Tiles whose wait for their stripe's row maxima gave up (fused requantization), on the
    current device since the library was loaded; synchronises with the device."""
    n = ctypes.c_uint(0)
    check("int8k_mlp_sync_timeouts", load().int8k_mlp_sync_timeouts(ctypes.byref(n)))
    return int(n.value)


def mlp_forward(x, W1, W2, sx, sW1, sW2, bias1=None, flags=0, out=None, out_scale=None,
                workspace=None):
    """x [T, d_model] int8; W1/W2 int8 ([K][N], or [N][K] with MLP_WEIGHTS_PREPACKED);
    scales fp32 device tensors of length 1 or full.  Returns (out int8, out_scale fp32)."""
    import torch

    dm = x.shape[-1]
    T = x.numel() // dm
    prepacked = bool(flags & MLP_WEIGHTS_PREPACKED)
    dff = W1.shape[0] if prepacked else W1.shape[1]
    if out is None:
        out = torch.empty((T, dm), dtype=torch.int8, device=x.device)
    if out_scale is None:
        n = 1 if flags & MLP_OUT_PER_TENSOR else T
        out_scale = torch.empty(n, dtype=torch.float32, device=x.device)
    ws_bytes = mlp_workspace_bytes(T, dm, dff, flags)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    st = load().int8k_mlp_forward(
        _ptr(x), _ptr(W1), _ptr(W2), _ptr(out), _ptr(sx), sx.numel(), _ptr(sW1), sW1.numel(),
        _ptr(sW2), sW2.numel(), _ptr(bias1), _ptr(out_scale), T, dm, dff, flags,
        _ptr(workspace), workspace.numel(), _stream(x))
    check("int8k_mlp_forward", st)
    return out, out_scale


# --------------------------------------------------------------------------
# prefill attention
# --------------------------------------------------------------------------


ATTN_CAUSAL = 1    # INT8K_ATTN_CAUSAL
ATTN_OUT_BSHD = 2  # INT8K_ATTN_OUT_BSHD


def _attn_flags(causal, out_bshd):
    return (ATTN_CAUSAL if causal else 0) | (ATTN_OUT_BSHD if out_bshd else 0)


def attention_forward(Qi, Ki, Vi, sQ, sK, sV, causal=False, out=None, out_bshd=False):
    """Q/K/V int8 [B,H,S,D] (device), per-token fp32 scales (B*H*S) -> fp16 [B,H,S,D]
    ([B,S,H,D] with out_bshd)."""
    import torch

    B, H, S, D = Qi.shape
    if out is None:
        shape = (B, S, H, D) if out_bshd else (B, H, S, D)
        out = torch.empty(shape, dtype=torch.float16, device=Qi.device)
    st = load().int8k_attention_forward(_ptr(Qi), _ptr(Ki), _ptr(Vi), _ptr(out), _ptr(sQ),
                                        _ptr(sK), _ptr(sV), B, H, S, D,
                                        _attn_flags(causal, out_bshd), _stream(Qi))
    check("int8k_attention_forward", st)
    return out


def _quant_rows(shape, device):
    import torch

    n = 1
    for d in shape[:-1]:
        n *= d
    return (torch.empty(shape, dtype=torch.int8, device=device),
            torch.empty(shape[:-1], dtype=torch.float32, device=device), n)


def attention_forward_quant(Qi, Ki, Vi, sQ, sK, sV, causal=False, out_bshd=False):
    """As attention_forward, emitting the per-token int8 of the fp16 output:
    (int8 [B,H,S,D], fp32 scales [B,H,S]), or [B,S,H,D] / [B,S,H] with out_bshd."""
    B, H, S, D = Qi.shape
    q, s, _ = _quant_rows((B, S, H, D) if out_bshd else (B, H, S, D), Qi.device)
    st = load().int8k_attention_forward_quant(_ptr(Qi), _ptr(Ki), _ptr(Vi), _ptr(q), _ptr(s),
                                              _ptr(sQ), _ptr(sK), _ptr(sV), B, H, S, D,
                                              _attn_flags(causal, out_bshd), _stream(Qi))
    check("int8k_attention_forward_quant", st)
    return q, s


# --------------------------------------------------------------------------
# quantization and the KV cache
# --------------------------------------------------------------------------


def _dtype_code(t):
    import torch

    codes = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}
    if t.dtype not in codes:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return codes[t.dtype]


def quantize_fp16_to_int8(x):
    """Per-tensor: returns (int8 codes, fp32 device scale [1])."""
    import torch

    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    check("int8k_quantize_fp16_to_int8",
          load().int8k_quantize_fp16_to_int8(_ptr(x), _ptr(q), _ptr(s), x.numel(), _stream(x)))
    return q, s


def dequantize_int8_to_fp16(q, scale: float):
    import torch

    y = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    check("int8k_dequantize_int8_to_fp16",
          load().int8k_dequantize_int8_to_fp16(_ptr(q), _ptr(y), float(scale), q.numel(),
                                               _stream(q)))
    return y


def quantize_per_token(x):
    """Rows of the last dim: returns (int8 codes like x, fp32 scales x.shape[:-1])."""
    import torch

    cols = x.shape[-1]
    rows = x.numel() // cols
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    check("int8k_quantize_per_token",
          load().int8k_quantize_per_token(_ptr(x), _dtype_code(x), _ptr(q), _ptr(s), rows, cols,
                                          _stream(x)))
    return q, s


def dequantize_per_token(q, scales, residual=None, dtype=None):
    """y = (q.float() * scales[..., None]).to(dtype) [+ residual, in its dtype]."""
    import torch

    cols = q.shape[-1]
    rows = q.numel() // cols
    if residual is not None:
        if dtype is not None and dtype != residual.dtype:
            raise ValueError("dtype must match the residual's dtype, which sets the output dtype")
        dtype = residual.dtype
    elif dtype is None:
        dtype = torch.float16
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    check("int8k_dequantize_per_token",
          load().int8k_dequantize_per_token(_ptr(q), _ptr(scales), _dtype_code(y),
                                            _ptr(residual) if residual is not None else None,
                                            _ptr(y), rows, cols, _stream(q)))
    return y


def kv_cache_append(k_new, v_new, K_cache, V_cache, sK_cache, sV_cache, pos: int):
    """k_new/v_new [B,H,n,D]; caches [B,H,cap,D] int8 and [B,H,cap] fp32."""
    B, H, n, D = k_new.shape
    cap = K_cache.shape[2]
    check("int8k_kv_cache_append",
          load().int8k_kv_cache_append(_ptr(k_new), _ptr(v_new), _dtype_code(k_new),
                                       _ptr(K_cache), _ptr(V_cache), _ptr(sK_cache),
                                       _ptr(sV_cache), B * H, n, pos, cap, D, _stream(k_new)))


def decode_attention_cache(Qi, K_cache, V_cache, sQ, sK_cache, sV_cache, S, nsplit=0, out=None):
    """Decode over the first S positions of a [B,H,cap,D] cache."""
    import torch

    B, H, cap, D = K_cache.shape
    BH = B * H
    if out is None:
        out = torch.empty((BH, D), dtype=torch.float16, device=Qi.device)
    ws = torch.empty(max(decode_workspace_bytes(BH, S, D, nsplit), 1), dtype=torch.uint8,
                     device=Qi.device)
    st = load().int8k_decode_attention_forward_cache(
        _ptr(Qi), _ptr(K_cache), _ptr(V_cache), _ptr(out), _ptr(sQ), _ptr(sK_cache),
        _ptr(sV_cache), BH, S, cap, D, nsplit, _ptr(ws), ws.numel(), _stream(Qi))
    check("int8k_decode_attention_forward_cache", st)
    return out


def decode_attention_cache_quant(Qi, K_cache, V_cache, sQ, sK_cache, sV_cache, S, nsplit=0):
    """As decode_attention_cache, emitting (int8 [BH,D], fp32 scales [BH])."""
    import torch

    B, H, cap, D = K_cache.shape
    BH = B * H
    q, s, _ = _quant_rows((BH, D), Qi.device)
    ws = torch.empty(max(decode_workspace_bytes(BH, S, D, nsplit), 1), dtype=torch.uint8,
                     device=Qi.device)
    st = load().int8k_decode_attention_forward_cache_quant(
        _ptr(Qi), _ptr(K_cache), _ptr(V_cache), _ptr(q), _ptr(s), _ptr(sQ), _ptr(sK_cache),
        _ptr(sV_cache), BH, S, cap, D, nsplit, _ptr(ws), ws.numel(), _stream(Qi))
    check("int8k_decode_attention_forward_cache_quant", st)
    return q, s


def decode_paged_workspace_bytes(B, H, max_context, D, nsplit=0):
    return load().int8k_decode_attention_paged_workspace_bytes(B, H, max_context, D, nsplit)


def decode_paged_num_splits(B, H, max_context, D, nsplit=0):
    return load().int8k_decode_attention_paged_num_splits(B, H, max_context, D, nsplit)


def decode_paged_bad_page_ids() -> int:
    """Work units of paged decode calls that met a page id outside [0, num_pages) among the
    table entries they use, on the current device since the library was loaded;
    synchronises with the device."""
    n = ctypes.c_uint(0)
    check("int8k_decode_paged_bad_page_ids",
          load().int8k_decode_paged_bad_page_ids(ctypes.byref(n)))
    return int(n.value)


def decode_attention_paged(Qi, K_pages, V_pages, sQ, sK_pages, sV_pages, block_tables,
                           context_lens, max_context, nsplit=0, out=None):
    """Decode over a paged cache: K/V_pages [num_pages, H, page, D] int8, scales
    [num_pages, H, page] fp32, block_tables [B, max_pages] int32, context_lens [B] int32.
    Returns fp16 [B, H, D]."""
    import torch

    num_pages, H, page, D = K_pages.shape
    B, max_pages = block_tables.shape
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float16, device=Qi.device)
    ws = torch.empty(max(decode_paged_workspace_bytes(B, H, max_context, D, nsplit), 1),
                     dtype=torch.uint8, device=Qi.device)
    st = load().int8k_decode_attention_forward_paged(
        _ptr(Qi), _ptr(K_pages), _ptr(V_pages), _ptr(out), _ptr(sQ), _ptr(sK_pages),
        _ptr(sV_pages), _ptr(block_tables), _ptr(context_lens), B, H, D, num_pages, page,
        max_pages, max_context, nsplit, _ptr(ws), ws.numel(), _stream(Qi))
    check("int8k_decode_attention_forward_paged", st)
    return out


def decode_attention_paged_quant(Qi, K_pages, V_pages, sQ, sK_pages, sV_pages, block_tables,
                                 context_lens, max_context, nsplit=0):
    """As decode_attention_paged, emitting (int8 [B,H,D], fp32 scales [B,H])."""
    import torch

    num_pages, H, page, D = K_pages.shape
    B, max_pages = block_tables.shape
    q, s, _ = _quant_rows((B, H, D), Qi.device)
    ws = torch.empty(max(decode_paged_workspace_bytes(B, H, max_context, D, nsplit), 1),
                     dtype=torch.uint8, device=Qi.device)
    st = load().int8k_decode_attention_forward_paged_quant(
        _ptr(Qi), _ptr(K_pages), _ptr(V_pages), _ptr(q), _ptr(s), _ptr(sQ), _ptr(sK_pages),
        _ptr(sV_pages), _ptr(block_tables), _ptr(context_lens), B, H, D, num_pages, page,
        max_pages, max_context, nsplit, _ptr(ws), ws.numel(), _stream(Qi))
    check("int8k_decode_attention_forward_paged_quant", st)
    return q, s


def layernorm_quantize_per_token(x, gamma=None, beta=None, eps=1e-5, want_y=False):
    """LN over the last dim then per-token int8: returns (q, scales[, y])."""
    import torch

    x = x.contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    y = torch.empty_like(x) if want_y else None
    g = gamma.float().contiguous() if gamma is not None else None
    b = beta.float().contiguous() if beta is not None else None
    st = load().int8k_layernorm_quantize_per_token(
        _ptr(x), _dtype_code(x), _ptr(g) if g is not None else None,
        _ptr(b) if b is not None else None, eps, _ptr(q), _ptr(s),
        _ptr(y) if y is not None else None, rows, cols, _stream(x))
    check("int8k_layernorm_quantize_per_token", st)
    return (q, s, y) if want_y else (q, s)


def quantize_heads(x, heads, parts=3):
    """x [B, S, parts*heads*Dh] -> list of (q [B,H,S,Dh] int8, s [B,H,S] fp32) per part."""
    import torch

    x = x.contiguous()
    B, S, W = x.shape
    Dh = W // (parts * heads)
    outs = [(torch.empty((B, heads, S, Dh), dtype=torch.int8, device=x.device),
             torch.empty((B, heads, S), dtype=torch.float32, device=x.device))
            for _ in range(parts)]
    ptrs = []
    for p in range(3):
        ptrs += [_ptr(outs[p][0]), _ptr(outs[p][1])] if p < parts else [None, None]
    st = load().int8k_quantize_heads(_ptr(x), _dtype_code(x), parts, *ptrs, B, S, heads, Dh,
                                     _stream(x))
    check("int8k_quantize_heads", st)
    return outs
