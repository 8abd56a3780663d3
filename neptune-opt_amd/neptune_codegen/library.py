"""The registered scalar folds.

Each entry is a declaration of algebra; the repair, the consumer term and the HIP kernel all
follow from it.  The eleven operators and their algebra are those of the reference
(neptune_codegen/library.py:19-177): the same g, readout, producer mode, reducers, parameters
and defaults, because they define the operators a caller asks for by name.
"""
from __future__ import annotations

import sympy as sp

from neptune_codegen.skeleton import Skeleton, register
from neptune_codegen.symbols import *  # noqa: F401,F403

_c, _s = c_sym, s_sym
_LOG_READOUT = _FINAL_M + sp.log(_FINAL_ACC + _PARAM_TINY)
_TINY = (_PARAM_TINY, "tiny")


def _log_fold(name, g, params=(), defaults=(), doc=""):
    """An exponential fold: signed producer, m + log(acc + tiny) readout, tiny = 0 default."""
    return register(Skeleton(
        name=name, g=g, finalize=_LOG_READOUT, producer="signed", is_log=True,
        params=tuple(params) + (_TINY,), defaults=tuple(defaults) + ((_PARAM_TINY, 0.0),),
        doc=doc))


_log_fold("logsumexp", sp.exp(_c - _s),
          doc="softmax's max+sumexp fold, log-softmax, cross-entropy")
_log_fold("softcap_lse", sp.exp(sp.tanh(_PARAM_BETA * _c) - _s),
          params=((_PARAM_BETA, "beta"),),
          doc="Gemma-2 soft-capped attention: logsumexp(tanh(beta*x))")
_log_fold("lse_biased", sp.exp(_c + _PARAM_ALPHA - _s),
          params=((_PARAM_ALPHA, "alpha"),),
          doc="ALiBi-biased logsumexp: logsumexp(x + alpha)")
# T defaults to 2: T = 1 would make this the plain logsumexp.
_log_fold("lse_scaled", sp.exp(_c / _PARAM_T - _s),
          params=((_PARAM_T, "T"),), defaults=((_PARAM_T, 2.0),),
          doc="logsumexp(x / T): the softmax denominator for temperature-scaled logits")

register(Skeleton(
    name="stable_l2", g=(_c / _s) ** 2, finalize=_FINAL_M * sp.sqrt(_FINAL_ACC),
    producer="abs", doc="numerically stable L2 norm / RMS numerator (no torch equivalent)"))
register(Skeleton(
    name="linear_attn", g=_c / _s, finalize=_FINAL_ACC, producer="abs",
    doc="linear attention normaliser: sum(x)/max|x|"))
register(Skeleton(
    name="decay_renorm", g=_c / (_PARAM_N + _s), finalize=_FINAL_ACC, producer="abs",
    params=((_PARAM_N, "N"),), doc="duration/decay renormalisation: sum(x/(N+max|x|))"))
register(Skeleton(
    name="sumsq_div", g=_c ** 2 / _s, finalize=_FINAL_ACC, producer="abs",
    doc="sum(x^2)/max|x| -- a scale-normalised energy statistic"))
# producer: the running mean of squares (an additive reduction); consumer: a max.
register(Skeleton(
    name="rmsnorm_max", g=_c / sp.sqrt(_s + _PARAM_EPS), finalize=_FINAL_ACC, producer="abs",
    producer_expr=_c ** 2 / _PARAM_N, producer_reducer="sum", consumer_reducer="max",
    params=((_PARAM_EPS, "eps"),), intrinsic_params=((_PARAM_N, "ncols"),),
    doc="RMSNorm + row max: max_j x_j / sqrt(mean(x^2) + eps)"))
# Two-pass: the term needs the FINAL mean, so the row is read twice and nothing is repaired.
for _name, _readout, _doc in (
        ("variance", _FINAL_ACC, "torch.var(x, unbiased=False): mean((x - mean(x))^2)"),
        ("std", sp.sqrt(_FINAL_ACC), "torch.std(x, unbiased=False): sqrt(mean((x - mean(x))^2))")):
    register(Skeleton(
        name=_name, g=(_c - _s) ** 2 / _PARAM_N, finalize=_readout, producer="signed",
        producer_reducer="sum", two_pass=True, producer_expr=_c / _PARAM_N,
        intrinsic_params=((_PARAM_N, "ncols"),), doc=_doc))
