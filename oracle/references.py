"""Closed-form eager references (CPU torch).  Test infrastructure; see oracle/__init__.py.

reference / graph_reference / rel_tolerance / summation_tolerance restate the reference's
neptune_codegen/references.py:18-140 (same formulas, same clamp_min(1e-30), same declared-N
convention).  Structured references restate the canonical forms the reference verifies against:
  rms_norm_reference      README.md:121-127 and tests/test_neptune_opt.py:1852-1855 (_full_rms)
  segment_reference       torch.segment_reduce, as in tests/test_autotune.py:793-833
  l2_normalize_reference  F.normalize(x.float(), dim=-1, eps).to(dtype)  (no reference fn)
  attention_reference     softmax(scale * Q K^T + causal mask) V in fp32 (no reference fn)
Parity of these closed forms is pinned by the tests in tests/test_oracle_*.py.
"""
from __future__ import annotations

import sys
import pathlib

_PKG = pathlib.Path(__file__).resolve().parent.parent / "neptune-opt_amd"
if str(_PKG) not in sys.path:
    sys.path.insert(0, str(_PKG))


def _defaults(name):
    # the skeleton registry (pure spec, no device code) supplies declared defaults
    from neptune_codegen.skeleton import param_defaults

    return param_defaults(name)


def rel_tolerance(dtype, ulps: float = 4.0) -> float:
    import torch

    return ulps * float(torch.finfo(dtype).eps)


def summation_tolerance(dtype, n, ulps: float = 4.0) -> float:
    import torch

    n = max(int(n), 1)
    return ulps * float(torch.finfo(dtype).eps) + 2 * ulps * float(torch.finfo(torch.float32).eps) * n ** 0.5


def reference(name: str, x, **params):
    """Row-wise fp32 reference of a scalar skeleton over the last dimension of a 2-D view."""
    import torch

    p = {**_defaults(name), **params}
    t = x.reshape(x.shape[0], -1).float()
    if name == "logsumexp":
        return torch.logsumexp(t, dim=-1)
    if name == "lse_biased":
        return torch.logsumexp(t + p["alpha"], dim=-1)
    if name == "softcap_lse":
        return torch.logsumexp(torch.tanh(p["beta"] * t), dim=-1)
    if name == "lse_scaled":
        return torch.logsumexp(t / p["T"], dim=-1)
    if name == "rmsnorm_max":
        r = (t * t).mean(dim=-1, keepdim=True)
        return (t / torch.sqrt(r + p["eps"])).amax(dim=-1)
    if name == "variance":
        return t.var(dim=-1, unbiased=False)
    if name == "std":
        return t.std(dim=-1, unbiased=False)
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    if name == "stable_l2":
        return (m * torch.sqrt(((t / m) ** 2).sum(dim=-1, keepdim=True))).squeeze(-1)
    if name == "sumsq_div":
        return ((t * t) / m).sum(dim=-1)
    if name == "linear_attn":
        return (t / m).sum(dim=-1)
    if name == "decay_renorm":
        return (t / (m + p["N"])).sum(dim=-1)
    raise KeyError(name)


def graph_reference(name: str, x, **params):
    """The same skeleton in decomposed form (references.py:100-140): the producer reduction is
    a separate tensor, then the consumer's terms are summed (or maxed) against it and read out
    -- the graph Inductor would otherwise compile, with its materialised intermediate."""
    import torch

    p = {**_defaults(name), **params}
    t = x.reshape(x.shape[0], -1).float()
    n = t.shape[-1]
    lse_operand = {"logsumexp": lambda v: v, "lse_biased": lambda v: v + p["alpha"],
                   "softcap_lse": lambda v: torch.tanh(p["beta"] * v),
                   "lse_scaled": lambda v: v / p["T"]}
    if name in lse_operand:
        z = lse_operand[name](t)
        m = z.amax(dim=-1, keepdim=True)                       # producer: row max
        acc = torch.exp(z - m).sum(dim=-1, keepdim=True)       # consumer: sum of exp(phi - m)
        return (m + torch.log(acc)).squeeze(-1)
    if name == "rmsnorm_max":
        r = (t * t).sum(dim=-1, keepdim=True) / n              # producer: mean of squares
        return (t / torch.sqrt(r + p["eps"])).amax(dim=-1)    # consumer: max of the terms
    if name in ("variance", "std"):
        mu = t.sum(dim=-1, keepdim=True) / n                   # producer: mean (first pass)
        var = ((t - mu) ** 2).sum(dim=-1) / n                  # consumer: centred second pass
        return var if name == "variance" else torch.sqrt(var)
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)  # producer: floored max |x|
    terms = {"stable_l2": lambda: (t / m) ** 2, "sumsq_div": lambda: (t * t) / m,
             "linear_attn": lambda: t / m, "decay_renorm": lambda: t / (m + p["N"])}
    if name not in terms:
        raise KeyError(name)
    acc = terms[name]().sum(dim=-1, keepdim=True)
    out = m * torch.sqrt(acc) if name == "stable_l2" else acc
    return out.squeeze(-1)


def rms_norm_reference(x, gamma, eps=1e-6):
    """fp32 promote -> square/mean/eps/rsqrt/normalize -> round to dtype -> * gamma."""
    source = x.float()
    normalized = source * __import__("torch").rsqrt((source * source).mean(-1, keepdim=True) + eps)
    return normalized.to(x.dtype) * gamma


def l2_normalize_reference(x, eps=1e-6):
    import torch.nn.functional as F

    return F.normalize(x.float(), dim=-1, eps=eps).to(x.dtype)


def segment_reference(data, segments, reduce="sum", *, offsets=False, initial=None, unsafe=False):
    import torch

    key = "offsets" if offsets else "lengths"
    return torch.segment_reduce(data, reduce, axis=0, initial=initial, unsafe=unsafe, **{key: segments})


def attention_reference(q, k, v, *, scale=None, causal=True):
    """fp32 math: softmax(scale * Q K^T + causal mask) V, returned in q.dtype."""
    import math

    import torch

    qf, kf, vf = q.float(), k.float(), v.float()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    if causal:
        n, m = s.shape[-2], s.shape[-1]
        mask = torch.ones(n, m, dtype=torch.bool).tril(diagonal=0)  # torch is_causal: j <= i
        s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf).to(q.dtype)
