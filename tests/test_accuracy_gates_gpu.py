"""Accuracy gates of the reference's validation suite (validation/validate_int8.py,
validation/generate_test_data.py), restated for this build's kernels (GPU tests).

Each dataset is generated here from the reference's recipe (seeded; nothing is loaded
from the reference): normal, outlier, boundary, stress, short_seq, long_seq, zeros,
constant.  The INT8 path quantizes per token (Q, K, V, x) and per output channel (W1, W2)
and runs int8_attention_forward (non-causal, as the reference's validation does) and the
per-token/per-channel int8_mlp_forward.  The ground truth is the unquantized computation
in fp32 (the reference compares against fp16 PyTorch, common/baseline.py:7-37).

Gate 1 (validation/validate_int8.py:264-280) checks four things:
  * no NaN/Inf;
  * float64 cosine >= cos_min;
  * mean top-10 |value| index overlap per row >= top10_min (skipped for zeros and constant
    rows);
  * the share of elements off by more than max(atol, 10% relative) is <= outlier_ratio_max,
    with atol = max(0.1, 5% of the reference RMS).
Gate 4 (validation/validate_int8.py:315-327), edge datasets only: no NaN/Inf; zeros gives
|out| <= 1e-3, every other edge dataset cosine >= 0.99.

Thresholds and the expected failures are the reference's
(validation/generate_test_data.py:168-171, 180-336).  The attention kernel on outlier,
boundary and stress is an expected failure there: per-token scales, and near-tie argmax flips
under a peaky softmax.  Those cases are marked xfail (non-strict) here.  Gates 2 and 3 check
the reference's stage-by-stage Python simulations, not a kernel, so they have no counterpart.
"""
import math

import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu

SEED = 42
BATCH, HEADS, SEQ, HEAD_DIM = 2, 8, 512, 64
D_MODEL, D_FF = 512, 2048
LONG_SEQ, SHORT_SEQ = 4096, 4

DEFAULT = {"cos_min": 0.999, "top10_min": 0.8, "outlier_ratio_max": 0.01}
EDGE = {"cos_min": 0.99, "top10_min": 0.6, "outlier_ratio_max": 0.02, "edge_cos_min": 0.99}
THRESH = {
    "normal": DEFAULT,
    "outlier": {**DEFAULT, "cos_min": 0.995, "outlier_ratio_max": 0.02},
    "boundary": DEFAULT,
    "stress": {**DEFAULT, "cos_min": 0.995, "top10_min": 0.7, "outlier_ratio_max": 0.05},
    "short_seq": EDGE,
    "long_seq": EDGE,
    "zeros": {**EDGE, "zero_output": True},
    "constant": EDGE,
}
EDGE_SETS = ("short_seq", "long_seq", "zeros", "constant")
XFAIL = {("outlier", "attention"), ("boundary", "attention"), ("stress", "attention")}


# ----------------------------------------------------------------- datasets

def _randn(shape, g):
    return torch.randn(shape, generator=g)


def _student_t3(shape, g):
    # t(3) = N(0,1) / sqrt(chi2(3) / 3), clamped to +-30
    z = _randn(shape, g)
    chi2 = sum(_randn(shape, g) ** 2 for _ in range(3))
    return (z / torch.sqrt(chi2 / 3.0)).clamp(-30, 30)


def _outliers(t, g):
    # 1% fixed channels x 5% random tokens scaled by U(10, 100)
    t = t.clone().float()
    C = t.shape[-1]
    ch = torch.randperm(C, generator=g)[:max(1, int(C * 0.01))]
    flat = t.reshape(-1, C)
    tok = torch.randperm(flat.shape[0], generator=g)[:max(1, int(flat.shape[0] * 0.05))]
    mag = 10.0 + 90.0 * torch.rand(len(tok), len(ch), generator=g)
    flat[tok[:, None], ch[None, :]] *= mag
    return t.clamp(-65504, 65504).half()


def _boundary(shape, g, amax=4.0):
    sign = torch.randint(0, 2, shape, generator=g).float() * 2 - 1
    return (sign * amax * (0.985 + 0.015 * torch.rand(shape, generator=g))).half()


def _attn(seq, g, batch=BATCH):
    return [_randn((batch, HEADS, seq, HEAD_DIM), g).half() for _ in range(3)]


def _mlp(seq, g, batch=BATCH):
    return (_randn((batch, seq, D_MODEL), g).half(),
            (_randn((D_MODEL, D_FF), g) * 0.02).half(),
            (_randn((D_FF, D_MODEL), g) * 0.02).half())


def dataset(name):
    g = torch.Generator().manual_seed(SEED + sum(map(ord, name)))
    if name == "normal":
        return _attn(SEQ, g), _mlp(SEQ, g)
    if name == "outlier":
        q, k, v = _attn(SEQ, g)
        x, w1, w2 = _mlp(SEQ, g)
        return [q, _outliers(k, g), _outliers(v, g)], (_outliers(x, g), w1, w2)
    if name == "boundary":
        shape = (BATCH, HEADS, SEQ, HEAD_DIM)
        return ([_boundary(shape, g) for _ in range(3)],
                (_boundary((BATCH, SEQ, D_MODEL), g), _boundary((D_MODEL, D_FF), g, 0.05),
                 _boundary((D_FF, D_MODEL), g, 0.05)))
    if name == "stress":
        shape = (BATCH, HEADS, SEQ, HEAD_DIM)
        q = _student_t3(shape, g).half()
        k = (_student_t3(shape, g) * torch.logspace(-1, 1, HEAD_DIM)).clamp(-300, 300).half()
        v = _student_t3(shape, g).half()
        x = (_randn((BATCH, SEQ, D_MODEL), g) * torch.logspace(-2, 1, D_MODEL)).half()
        _, w1, w2 = _mlp(SEQ, g)
        return [q, k, v], (x, w1, w2)
    if name == "short_seq":
        return _attn(SHORT_SEQ, g), _mlp(SHORT_SEQ, g)
    if name == "long_seq":
        return _attn(LONG_SEQ, g, batch=1), _mlp(LONG_SEQ, g, batch=1)
    if name == "zeros":
        z = torch.zeros(BATCH, HEADS, SEQ, HEAD_DIM).half()
        return ([z, z, z], (torch.zeros(BATCH, SEQ, D_MODEL).half(),
                            torch.zeros(D_MODEL, D_FF).half(), torch.zeros(D_FF, D_MODEL).half()))
    if name == "constant":
        o = torch.ones(BATCH, HEADS, SEQ, HEAD_DIM).half()
        return ([o, o, o], (torch.ones(BATCH, SEQ, D_MODEL).half(),
                            torch.full((D_MODEL, D_FF), 0.01).half(),
                            torch.full((D_FF, D_MODEL), 0.01).half()))
    raise KeyError(name)


# ----------------------------------------------------------------- metrics

def cosine(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    na, nb = a.norm(), b.norm()
    if na < 1e-6 and nb < 1e-6:
        return 1.0
    if na < 1e-6 or nb < 1e-6:
        return 0.0
    return float(torch.dot(a / na, b / nb).clamp(max=1.0))


def top10_overlap(ref, act, max_rows=4096):
    r = ref.float().reshape(-1, ref.shape[-1])
    a = act.float().reshape(-1, act.shape[-1])
    if r.shape[0] > max_rows:
        idx = torch.linspace(0, r.shape[0] - 1, max_rows).long()
        r, a = r[idx], a[idx]
    if float(r.abs().std()) < 1e-6:
        return None  # constant rows: no ranking
    k = min(10, r.shape[-1])
    rt = r.abs().topk(k, dim=-1).indices
    at = a.abs().topk(k, dim=-1).indices
    return float((rt.unsqueeze(-1) == at.unsqueeze(-2)).any(-1).float().mean())


def outlier_ratio(ref, act):
    r, a = ref.float(), act.float()
    atol = max(0.1, 0.05 * float(r.square().mean().sqrt()))
    return float(((r - a).abs() > torch.clamp(0.10 * r.abs(), min=atol)).float().mean())


def gate_failures(name, ref, act):
    thr = THRESH[name]
    fails = []
    if not torch.isfinite(act).all():
        fails.append("NaN/Inf in the kernel output")
    c = cosine(ref, act)
    if c < thr["cos_min"]:
        fails.append(f"gate 1: cosine {c:.5f} < {thr['cos_min']}")
    ov = None if thr.get("zero_output") else top10_overlap(ref, act)
    if ov is not None and ov < thr["top10_min"]:
        fails.append(f"gate 1: top-10 overlap {ov:.3f} < {thr['top10_min']}")
    orr = outlier_ratio(ref, act)
    if orr > thr["outlier_ratio_max"]:
        fails.append(f"gate 1: outlier ratio {orr:.4f} > {thr['outlier_ratio_max']}")
    if name in EDGE_SETS:
        if thr.get("zero_output"):
            m = float(act.abs().max())
            if m > 1e-3:
                fails.append(f"gate 4: zeros dataset |out| max {m:.5f} > 1e-3")
        elif c < thr["edge_cos_min"]:
            fails.append(f"gate 4: edge cosine {c:.5f} < {thr['edge_cos_min']}")
    return fails, dict(cos=c, top10=ov, outlier_ratio=orr)


# ----------------------------------------------------------------- runners

def attention_ref(q, k, v):
    qf, kf, vf = (t.float() for t in (q, k, v))
    s = torch.matmul(qf, kf.transpose(-2, -1).contiguous()) * (q.shape[-1] ** -0.5)
    return torch.matmul(torch.softmax(s, dim=-1), vf)


def attention_int8(ext, q, k, v):
    (qi, sq), (ki, sk), (vi, sv) = (ext.quantize_per_token(t) for t in (q, k, v))
    return ext.int8_attention_forward(qi, ki, vi, sq, sk, sv).float()


def mlp_ref(x, w1, w2):
    h = torch.nn.functional.gelu(x.float() @ w1.float(), approximate="tanh")
    return h @ w2.float()


def mlp_int8(ext, x, w1, w2):
    B, S, dm = x.shape
    xi, sx = ext.quantize_per_token(x)
    w1i, s1 = workloads.quantize_per_channel_w(w1)
    w2i, s2 = workloads.quantize_per_channel_w(w2)
    out, osc = ext.int8_mlp_forward(xi.contiguous(), w1i, w2i, sx.reshape(-1).float(), s1, s2)
    return out.float() * osc.reshape(B, S, 1)


@pytest.mark.parametrize("kernel", ["attention", "mlp"])
@pytest.mark.parametrize("name", list(THRESH))
def test_accuracy_gates(ext, gpu, name, kernel):
    (q, k, v), (x, w1, w2) = dataset(name)
    if kernel == "attention":
        q, k, v = q.to(gpu), k.to(gpu), v.to(gpu)
        ref, act = attention_ref(q, k, v), attention_int8(ext, q, k, v)
    else:
        x, w1, w2 = x.to(gpu), w1.to(gpu), w2.to(gpu)
        ref, act = mlp_ref(x, w1, w2), mlp_int8(ext, x, w1, w2)
    torch.cuda.synchronize()
    fails, metrics = gate_failures(name, ref.cpu(), act.cpu())
    assert math.isfinite(metrics["cos"])
    if (name, kernel) in XFAIL:
        if fails:
            pytest.xfail(f"{name}/{kernel}: expected failure in the reference as well: "
                         + "; ".join(fails))
        return
    assert not fails, f"{name}/{kernel} {metrics}: " + "; ".join(fails)
