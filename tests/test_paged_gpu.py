"""Decode over a paged INT8 KV cache (GPU tests).

Checked against the CPU oracle's gather-then-decode restatement at the attention
tolerances, against the contiguous decode kernel on the same data, and for the
documented edge behaviour: ragged lengths (1, page-1, page+1, non-multiples of the
64-row wave iteration), forced split counts, a zero-length sequence and out-of-range
page ids (any id outside [0, num_pages) reads the last page instead of memory outside
the cache, and is counted where the sequence uses it).
"""
import numpy as np
import pytest
import torch

import int8k_capi as capi
import workloads
from helpers import assert_attn_close
from oracle import int8_oracle as O

pytestmark = pytest.mark.gpu


def _oracle(c):
    return O.decode_attention_paged(*(c[k].cpu().numpy() for k in (
        "Qi", "K_pages", "V_pages", "sQ", "sK_pages", "sV_pages", "block_tables",
        "context_lens")))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("page", [16, 32, 64, 256, 1024])
def test_paged_decode_matches_oracle(gpu, D, page):
    lens = [1, page - 1, page + 1, 200, 777, 1024]
    c = workloads.paged_case(len(lens), 4, D, page, lens, seed=page + D, device=gpu)
    out = capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                      c["sK_pages"], c["sV_pages"], c["block_tables"],
                                      c["context_lens"], c["max_context"])
    torch.cuda.synchronize()
    assert_attn_close(out.float().cpu().numpy(), _oracle(c))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,H", [(4, 8), (16, 3)])
def test_paged_decode_head_pairs(gpu, D, B, H):
    # 16-token pages with 16 | B*H: the one-launch kernel runs heads 2k and 2k+1 side by
    # side on one XCD (they share each page's scale line); with H = 3 a pair spans two
    # sequences with different page tables and lengths
    rng = np.random.default_rng(B * H + D)
    lens = [int(v) for v in rng.integers(1, 3000, size=B)]
    c = workloads.paged_case(B, H, D, 16, lens, seed=B + H + D, device=gpu)
    out = capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                      c["sK_pages"], c["sV_pages"], c["block_tables"],
                                      c["context_lens"], c["max_context"], nsplit=8)
    torch.cuda.synchronize()
    assert capi.decode_paged_num_splits(B, H, c["max_context"], D, 8) <= 8  # one launch
    assert_attn_close(out.float().cpu().numpy(), _oracle(c))


def test_paged_decode_via_torch_op(ext, gpu):
    lens = [300, 5, 4096]
    c = workloads.paged_case(3, 8, 128, 16, lens, seed=9, device=gpu)
    out = ext.int8_decode_attention_forward_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                                  c["sK_pages"], c["sV_pages"],
                                                  c["block_tables"], c["context_lens"],
                                                  c["max_context"])
    torch.cuda.synchronize()
    assert out.shape == (3, 8, 128) and out.dtype == torch.float16
    assert_attn_close(out.float().cpu().numpy(), _oracle(c))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nsplit", [1, 2, 7, 64])
def test_paged_decode_forced_splits(gpu, D, nsplit):
    # up to 8 chunks: the one-launch kernel (paired rows at D=64, whose 8-row pair
    # blocks must stay inside one page); 64: the split kernel and the combine
    lens = [1000, 64, 513]
    c = workloads.paged_case(3, 2, D, 32, lens, seed=nsplit + D, device=gpu)
    out = capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                      c["sK_pages"], c["sV_pages"], c["block_tables"],
                                      c["context_lens"], c["max_context"], nsplit=nsplit)
    torch.cuda.synchronize()
    assert_attn_close(out.float().cpu().numpy(), _oracle(c))


@pytest.mark.parametrize("L", [190000, 196900])
def test_paged_decode_long_page_table(gpu, L):
    # up to 8 chunks per (b,h) run as one launch with the page ids staged in LDS
    # (11875 ids at L = 190000); a table past what LDS holds (12288 ids) runs the
    # split + combine pair instead (12307 ids at L = 196900)
    nsplit = 8
    lens = [L, 4000]
    c = workloads.paged_case(2, 1, 64, 16, lens, seed=11, device=gpu)
    out = capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                      c["sK_pages"], c["sV_pages"], c["block_tables"],
                                      c["context_lens"], c["max_context"], nsplit=nsplit)
    torch.cuda.synchronize()
    assert_attn_close(out.float().cpu().numpy(), _oracle(c))


def test_paged_equals_contiguous_kernel(gpu):
    # identity page tables over a contiguous cache: same positions, same math
    B, H, D, S, P = 2, 4, 128, 640, 64
    case = workloads.decode_case(B, H, D, S, seed=3, device=gpu)
    npp = S // P

    def pages(x):  # [B, H, S, ...] -> [B*npp, H, P, ...]
        x = x.reshape((B, H, npp, P) + tuple(x.shape[3:]))
        return x.movedim(2, 1).reshape((B * npp, H, P) + tuple(x.shape[4:])).contiguous()

    tables = torch.arange(B * npp, dtype=torch.int32, device=gpu).reshape(B, npp)
    lens = torch.full((B,), S, dtype=torch.int32, device=gpu)
    out = capi.decode_attention_paged(case["Qi"], pages(case["Ki"]), pages(case["Vi"]),
                                      case["sQ"], pages(case["sK"]), pages(case["sV"]), tables,
                                      lens, S)
    ref = capi.decode_attention(case["Qi"].reshape(B * H, D), case["Ki"].reshape(B * H, S, D),
                                case["Vi"].reshape(B * H, S, D), case["sQ"].reshape(-1),
                                case["sK"].reshape(-1), case["sV"].reshape(-1))
    torch.cuda.synchronize()
    d = (out.reshape(B * H, D).float() - ref.float()).abs().max().item()
    assert d <= 2e-3, d


def test_paged_decode_zero_length_and_clamped_pages(gpu):
    lens = [0, 100, 40]
    c = workloads.paged_case(3, 2, 64, 16, lens, seed=4, device=gpu)
    NP = c["K_pages"].shape[0]
    bt = c["block_tables"].clone()
    bt[2, 1] = NP + 5          # positions 16..31 of sequence 2 -> clamped to page NP-1
    bt[2, 2] = -3              # positions 32..39 -> also page NP-1 (any id outside [0, NP))
    out = capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                      c["sK_pages"], c["sV_pages"], bt, c["context_lens"],
                                      c["max_context"])
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.all(o[0] == 0)
    bt_ref = torch.where((bt < 0) | (bt >= NP), torch.full_like(bt, NP - 1), bt)
    ref = _oracle(dict(c, block_tables=bt_ref))
    assert_attn_close(o[1:], ref[1:])


@pytest.mark.parametrize("nsplit", [4, 64])
def test_paged_bad_page_ids_are_counted(gpu, nsplit):
    # an out-of-range id among the entries a sequence uses is counted (the one-launch kernel
    # at 4 chunks, the split kernel at 64); ids in entries past a sequence's length are never
    # read and never counted
    lens = [1000, 40]
    c = workloads.paged_case(2, 2, 64, 16, lens, seed=6, device=gpu)
    NP = c["K_pages"].shape[0]
    args = lambda bt: (c["Qi"], c["K_pages"], c["V_pages"], c["sQ"], c["sK_pages"],  # noqa: E731
                       c["sV_pages"], bt, c["context_lens"], c["max_context"])
    bt = c["block_tables"].clone()
    bt[1, 3:] = -1             # sequence 1 uses entries 0..2 (40 positions): padding past them
    assert (capi.decode_paged_num_splits(2, 2, c["max_context"], 64, nsplit) > 8) == (nsplit > 8)
    before = capi.decode_paged_bad_page_ids()
    capi.decode_attention_paged(*args(bt), nsplit=nsplit)
    torch.cuda.synchronize()
    assert capi.decode_paged_bad_page_ids() == before
    bt[0, 7] = NP + 1          # positions 112..127 of sequence 0
    capi.decode_attention_paged(*args(bt), nsplit=nsplit)
    torch.cuda.synchronize()
    assert capi.decode_paged_bad_page_ids() >= before + 2   # both heads of sequence 0


def test_paged_argument_validation(gpu):
    c = workloads.paged_case(1, 1, 64, 16, [20], seed=1, device=gpu)
    with pytest.raises(RuntimeError, match="unsupported"):
        capi.decode_attention_paged(c["Qi"], c["K_pages"][:, :, :12].contiguous(),
                                    c["V_pages"][:, :, :12].contiguous(), c["sQ"],
                                    c["sK_pages"][:, :, :12].contiguous(),
                                    c["sV_pages"][:, :, :12].contiguous(), c["block_tables"],
                                    c["context_lens"], 20)
    with pytest.raises(RuntimeError, match="invalid"):
        capi.decode_attention_paged(c["Qi"], c["K_pages"], c["V_pages"], c["sQ"],
                                    c["sK_pages"], c["sV_pages"], c["block_tables"],
                                    c["context_lens"], 10 ** 6)
