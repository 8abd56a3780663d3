"""numpy restatement of the scalar fold state machine.  Test infrastructure (oracle/__init__.py).

The reference's generated helpers (neptune_codegen/emitters.py:436-532) define, per skeleton:

  chunk        (emitters.py:459-488)  state (m, acc, seen, status) of one block of a row.
               Exponential folds: phi per element, status = any NaN * 1 | any +inf * 2, seen =
               any finite phi, m = max finite phi, acc = sum over finite of exp(phi - den) with
               den = m if seen else 0.  Other folds: seen = any element, m = producer
               reduction of the operand (0 if empty), den = m floored at 1e-30 when the
               coordinate needs a floor, acc = consumer reduction of term(v, den).
  merge_state  (emitters.py:491-517)  combined m = max or sum; both sides sanitised before the
               repair is evaluated; acc = combine(aA*rho(qA,qN) + beta, aB*rho(qB,qN) + beta);
               a side that was not seen passes the other through; seen/status OR.
  finalize     (emitters.py:522-532)  status&1 -> NaN, status&2 -> +inf, seen -> readout,
               else -inf (exponential folds); readout(m_eff, acc) otherwise.
  serial plan  (template.py:41-54)    left fold of chunk states over blocks of BLOCK columns.
  split plan   (template.py:137-165)  per-block partials merged by a reduction tree.
  two-pass     (template.py:62-103)   producer over the row, then the term at the final m.

Each skeleton's operand / term / repair / readout below restates its declaration
(neptune_codegen/library.py:19-177) together with the repair slope pinned by the reference's
golden table (tests/test_neptune_opt.py:344-353).  Arithmetic is fp32 (numpy float32 scalars),
as in the kernels.  Parity pins: tests/test_oracle_fold.py.
"""
from __future__ import annotations

import math

import numpy as np

F = np.float32
INF = F(np.inf)


def _f(x):
    return F(x)


# operand, term(v, den), rho(q, q2), readout(m, acc); p = parameters, n = row length
SPECS = {
    "logsumexp": dict(log=True, phi=lambda v, p, n: v),
    "lse_biased": dict(log=True, phi=lambda v, p, n: v + F(p["alpha"])),
    "softcap_lse": dict(log=True, phi=lambda v, p, n: np.tanh(F(p["beta"]) * v)),
    "lse_scaled": dict(log=True, phi=lambda v, p, n: v / F(p["T"])),
    "stable_l2": dict(log=False, prod="max", cons="sum", floor=True,
                      phi=lambda v, p, n: np.abs(v),
                      term=lambda v, d, p, n: (v / d) * (v / d),
                      rho=lambda q, q2, p: (q / q2) * (q / q2),
                      readout=lambda m, a, p, n: m * np.sqrt(a)),
    "linear_attn": dict(log=False, prod="max", cons="sum", floor=True,
                        phi=lambda v, p, n: np.abs(v),
                        term=lambda v, d, p, n: v / d,
                        rho=lambda q, q2, p: q / q2,
                        readout=lambda m, a, p, n: a),
    "decay_renorm": dict(log=False, prod="max", cons="sum", floor=False,
                         phi=lambda v, p, n: np.abs(v),
                         term=lambda v, d, p, n: v / (F(p["N"]) + d),
                         rho=lambda q, q2, p: (F(p["N"]) + q) / (F(p["N"]) + q2),
                         readout=lambda m, a, p, n: a),
    "sumsq_div": dict(log=False, prod="max", cons="sum", floor=True,
                      phi=lambda v, p, n: np.abs(v),
                      term=lambda v, d, p, n: v * v / d,
                      rho=lambda q, q2, p: q / q2,
                      readout=lambda m, a, p, n: a),
    "rmsnorm_max": dict(log=False, prod="sum", cons="max", floor=False,
                        phi=lambda v, p, n: v * v / F(n),
                        term=lambda v, d, p, n: v / np.sqrt(d + F(p["eps"])),
                        rho=lambda q, q2, p: np.sqrt(F(p["eps"]) + q) / np.sqrt(F(p["eps"]) + q2),
                        readout=lambda m, a, p, n: a),
    "variance": dict(two_pass=True, phi=lambda v, p, n: v / F(n),
                     term=lambda v, d, p, n: (v - d) * (v - d) / F(n),
                     readout=lambda m, a, p, n: a),
    "std": dict(two_pass=True, phi=lambda v, p, n: v / F(n),
                term=lambda v, d, p, n: (v - d) * (v - d) / F(n),
                readout=lambda m, a, p, n: np.sqrt(a)),
}
# declared defaults, and 1.0 for undeclared parameters (neptune_codegen/skeleton.py:255-267)
DEFAULTS = {"tiny": 0.0, "alpha": 1.0, "beta": 1.0, "T": 2.0, "N": 1.0, "eps": 1.0}


def params_for(name, **params):
    return {**DEFAULTS, **params}


def _eff(spec, m):
    return np.maximum(m, F(1e-30)) if spec.get("floor") else m


def empty_state(spec):
    cons_init = -INF if spec.get("cons") == "max" else F(0.0)
    return (F(0.0), cons_init, 0, 0)


def chunk(name, values, p, n):
    """State of one block (values: the block's elements, already masked to the row)."""
    spec = SPECS[name]
    v = np.asarray(values, dtype=F)
    with np.errstate(all="ignore"):
        if spec.get("log"):
            phi = spec["phi"](v, p, n).astype(F)
            status = (1 if np.isnan(phi).any() else 0) | (2 if (phi == INF).any() else 0)
            finite = np.isfinite(phi)
            seen = int(finite.any())
            m = phi[finite].max() if seen else -INF
            den = m if seen else F(0.0)
            acc = np.exp(phi[finite] - den).astype(F).sum(dtype=F) if seen else F(0.0)
            return (F(m), F(acc), seen, status)
        seen = int(v.size > 0)
        op = spec["phi"](v, p, n).astype(F)
        if spec["prod"] == "sum":
            m = op.sum(dtype=F)
        else:
            m = op.max() if seen else -INF
        m = F(m) if seen else F(0.0)
        den = _eff(spec, m)
        t = spec["term"](v, den, p, n).astype(F)
        if spec["cons"] == "max":
            acc = t.max() if seen else -INF
        else:
            acc = t.sum(dtype=F)
        return (F(m), F(acc), seen, 0)


def merge(name, A, B, p):
    """merge_state of two chunk states (emitters.py:491-517)."""
    spec = SPECS[name]
    mA, aA, vA, sA = A
    mB, aB, vB, sB = B
    both = bool(vA) and bool(vB)
    with np.errstate(all="ignore"):
        prod_sum = spec.get("prod") == "sum"
        cm = F(mA + mB) if prod_sum else F(max(mA, mB))
        oldA, oldB, fresh = (mA, mB, cm) if both else (F(1.0), F(1.0), F(1.0))
        qA, qB, qN = _eff(spec, F(oldA)), _eff(spec, F(oldB)), _eff(spec, F(fresh))
        safeA, safeB = (aA, aB) if both else (F(0.0), F(0.0))
        if spec.get("log"):
            tA, tB = F(safeA * np.exp(F(qA - qN))), F(safeB * np.exp(F(qB - qN)))
        else:
            tA, tB = F(safeA * spec["rho"](qA, qN, p)), F(safeB * spec["rho"](qB, qN, p))
        ca = F(max(tA, tB)) if spec.get("cons") == "max" else F(tA + tB)
    m = (cm if vB else mA) if vA else mB
    acc = (ca if vB else aA) if vA else aB
    return (F(m), F(acc), int(bool(vA) or bool(vB)), int(sA) | int(sB))


def finalize(name, state, p, n):
    spec = SPECS[name]
    m, acc, seen, status = state
    with np.errstate(all="ignore"):
        if spec.get("log"):
            if status & 1:
                return F(np.nan)
            if status & 2:
                return INF
            if not seen:
                return -INF
            return F(m + np.log(F(acc + F(p["tiny"]))))
        return F(spec["readout"](_eff(spec, m), acc, p, n))


def fold_row(name, row, *, block: int = 1024, plan: str = "serial", **params):
    """One row through the serial left fold, or split partials merged by a balanced tree."""
    spec = SPECS[name]
    p = params_for(name, **params)
    row = np.asarray(row, dtype=F)
    n = row.size
    if spec.get("two_pass"):
        with np.errstate(all="ignore"):
            m = spec["phi"](row, p, n).astype(F).sum(dtype=F)
            acc = spec["term"](row, m, p, n).astype(F).sum(dtype=F)
            return F(spec["readout"](m, acc, p, n))
    states = [chunk(name, row[i:i + block], p, n) for i in range(0, n, block)]
    if plan == "serial":
        s = empty_state(spec)
        for c in states:
            s = merge(name, s, c, p)
    else:
        while len(states) > 1:
            nxt = [merge(name, states[i], states[i + 1], p) for i in range(0, len(states) - 1, 2)]
            if len(states) % 2:
                nxt.append(states[-1])
            states = nxt
        s = states[0]
    return finalize(name, s, p, n)


def fold(name, x, **kw):
    x = np.asarray(x, dtype=F)
    x2 = x.reshape(-1, x.shape[-1])
    return np.array([fold_row(name, r, **kw) for r in x2], dtype=F).reshape(x.shape[:-1])


# ---------------------------------------------------------------- attention as a fold
def attention_fold(q, k, v, *, scale=None, causal=True, block=64):
    """Online-softmax attention over key tiles of `block` (float64): the logsumexp repair
    exp(m - m') applied to (m, l, O) per tile.  Pinned against the closed form."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    sq, d = q.shape[-2], q.shape[-1]
    sk = k.shape[-2]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    m = np.full(q.shape[:-1], -np.inf)
    l = np.zeros(q.shape[:-1])
    o = np.zeros(q.shape)
    qi = np.arange(sq)[:, None]
    for k0 in range(0, sk, block):
        s = scale * np.einsum("...qd,...kd->...qk", q, k[..., k0:k0 + block, :])
        if causal:
            kj = np.arange(k0, min(sk, k0 + block))[None, :]
            s = np.where(kj <= qi, s, -np.inf)
        m_new = np.maximum(m, s.max(-1))
        alpha = np.where(np.isfinite(m_new), np.exp(np.where(np.isfinite(m), m - m_new, -np.inf)), 1.0)
        pexp = np.exp(s - np.where(np.isfinite(m_new), m_new, 0.0)[..., None])
        l = l * alpha + pexp.sum(-1)
        o = o * alpha[..., None] + np.einsum("...qk,...kd->...qd", pexp, v[..., k0:k0 + block, :])
        m = m_new
    return o / l[..., None], m + np.log(l)
