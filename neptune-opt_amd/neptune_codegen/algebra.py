"""Deriving and certifying the repair of a fold from its algebra.

For a skeleton with term producer g(s, c) the accumulator sum_j g(s, c_j) must be moved to a
new producer value s' when the producer changes.  The repair is affine,
acc' = a(s, s') * acc + b(s, s'); it exists when

  * the ratio g(s', c) / g(s, c) is free of c (multiplicative repair, b = 0), or
  * matching c-derivatives, a = g_c(s', c) / g_c(s, c) is free of c and so is
    b = g(s', c) - a g(s, c) (affine repair; b != 0 only distributes over a max consumer).

This is the derivation of the reference (neptune_codegen/algebra.py:70-174): the same two
separations in the same order, because the derived slopes are pinned by a golden table
(tests/test_neptune_opt.py:344-353).  The merge certificate (algebra.py:348-403) proves the
repair exactly -- condition (3), the cocycle a(q,r) a(p,q) = a(p,r), identity a(p,p) = 1, a
positive slope for max consumers, nonzero normalisers -- before a split plan may merge
partial states.  The structured certificate (algebra.py:417-500) proves identity,
associativity and integer closure of (sum, count) states.
"""
from __future__ import annotations

import dataclasses
import functools
import math
import random

import sympy as sp

from neptune_codegen.symbols import *  # noqa: F401,F403

# Residuals containing these may vanish on sympy's principal branch only.
_BRANCH_FUNCS = (sp.log, sp.atanh, sp.acosh, sp.atan, sp.acos, sp.asin)
_BRANCH_CUT = _BRANCH_FUNCS   # the reference package's name for the same tuple


class _Q(sp.Function):
    """Inert marker for a quotient power (a/b)**k, rendered as repeated (a/b) products.

    sympy normalises (a/b)**2 to a**2/b**2; in fp32 squaring before dividing loses precision
    (and overflows early), so the renderer needs the quotient form back.
    """

    nargs = 3


def _simplify(expr: sp.Expr) -> sp.Expr:
    """Simplify with hyperbolics rewritten through exp, so that exponentials can cancel."""
    try:
        expr = expr.rewrite(sp.exp)
    except (AttributeError, NotImplementedError):
        pass
    return sp.simplify(sp.simplify(expr))


def _numerically_zero(expr: sp.Expr, samples: int = 7, tol: float = 1e-9) -> bool:
    """Filter (not proof): does expr vanish at several fixed-seed positive rational points?"""
    free = sorted(expr.free_symbols, key=lambda z: z.name)
    if not free:
        return expr == 0
    rng = random.Random(20251012)
    for _ in range(samples):
        point = {z: sp.Rational(rng.randint(1, 40), rng.randint(1, 17)) for z in free}
        try:
            value = abs(complex(sp.N(expr.subs(point), 30)))
        except (TypeError, ValueError):
            return False
        if value > tol * max(1.0, value):
            return False
    return True


def vanishes(expr: sp.Expr, samples: int = 9, tol: float = 1e-9) -> bool:
    """Is expr identically zero?  Symbolic first; numeric fallback away from branch cuts."""
    if expr == 0 or sp.simplify(expr) == 0:
        return True
    if expr.has(sp.I) or any(expr.has(f) for f in _BRANCH_FUNCS):
        return False
    return _numerically_zero(expr, samples=samples, tol=tol)


def _check_slope_sign(sk, a: sp.Expr) -> None:
    """Condition (4) for a max consumer: the slope must not be provably negative."""
    if sk.consumer_reducer == "max" and a.is_negative is True:
        raise NotImplementedError(
            f"skeleton {sk.name!r}: repair factor {sp.simplify(a)} is negative, so it does "
            "not distribute over the max reducer (condition 4 fails)")


@functools.lru_cache(maxsize=None)
def repair_pair(sk, *, exact: bool = False) -> tuple[sp.Expr, sp.Expr]:
    """(a, b) with acc' = a(s, s') * acc + b(s, s'), or NotImplementedError."""
    for sym, what in ((s2_sym, "the FRESH producer value s'"), (u_sym, "the term value u")):
        if sk.g.has(sym):
            raise NotImplementedError(
                f"skeleton {sk.name!r}: g mentions {what}; a term may depend only on the "
                "stale producer s and the data c, so no (f, g, h) form exists")
    if not sk.g.has(s_sym):
        raise NotImplementedError(
            f"skeleton {sk.name!r}: g does not depend on the producer s at all, so the repair "
            "would be the identity and the accumulator unrelated to the reduction. This is not "
            "an (f, g, h) fold.")
    fresh = sk.g.xreplace({s_sym: s2_sym})
    ratio = fresh / sk.g
    a = _simplify(ratio)
    if not a.has(c_sym):
        same = _simplify(a - ratio) == 0 if exact else vanishes(a - ratio)
        if not same:
            raise NotImplementedError(
                f"skeleton {sk.name!r}: separating g changed its value; got {sp.simplify(a)}")
        _check_slope_sign(sk, a)
        return a, sp.Integer(0)
    d_fresh, d_stale = sp.diff(fresh, c_sym), sp.diff(sk.g, c_sym)
    slope = _simplify(d_fresh / d_stale) if (d_stale != 0 and d_fresh != 0) else a
    if slope.has(c_sym):
        raise NotImplementedError(
            f"skeleton {sk.name!r}: g does not separate, so no repair of the form "
            f"a(s,s')*t + b(s,s') exists; ratio {sp.simplify(a)}, slope {sp.simplify(slope)}")
    bias = _simplify(fresh - slope * sk.g)
    if bias.has(c_sym):
        raise NotImplementedError(
            f"skeleton {sk.name!r}: g does not separate; the affine remainder b = "
            f"{sp.simplify(bias)} still depends on the data")
    if bias != 0 and sk.consumer_reducer != "max":
        raise NotImplementedError(
            f"skeleton {sk.name!r}: the repair needs a bias b = {sp.simplify(bias)}, but an "
            f"additive {sk.consumer_reducer} reducer requires b = 0 (condition 4: "
            "a*(x+y)+b != (a*x+b)+(a*y+b) unless b = 0)")
    _check_slope_sign(sk, slope)
    return _simplify(slope), bias


def repair_factor(sk) -> sp.Expr:
    return repair_pair(sk)[0]


def repair_bias(sk) -> sp.Expr:
    return repair_pair(sk)[1]


@functools.lru_cache(maxsize=None)
def term_expr(sk) -> sp.Expr:
    """The consumer term g(s', c); plain simplify keeps tanh intact for rendering."""
    return sp.simplify(sk.g.xreplace({s_sym: s2_sym}))


def _as_quotient_power(expr: sp.Expr) -> sp.Expr:
    """num**k / den**k -> _Q(num, den, k) when both sides carry the same integer power."""
    num, den = sp.fraction(sp.together(expr))
    if num == 1 and den == 1:
        return expr
    nb, ne = num.as_base_exp()
    db, de = den.as_base_exp()
    if ne.is_Integer and ne == de and int(ne) > 0:
        return _Q(nb, db, int(ne))
    return expr


def _marked(expr: sp.Expr) -> sp.Expr:
    """Render-time form of a repair or term (never used for the algebraic checks)."""
    return _as_quotient_power(expr)


# ---------------------------------------------------------------- producer domain / floor
def reachable_producer_domain(sk, values: dict | None = None) -> str:
    """'nonnegative' when the raw producer operand is provably >= 0, else 'real'."""
    from neptune_codegen.emitters import derived_producer_expr

    if sk.producer_domain not in ("auto", "real", "nonnegative"):
        raise NotImplementedError(f"unknown producer domain {sk.producer_domain!r}")
    phi = derived_producer_expr(sk)
    if phi is None:
        phi = sp.Abs(c_sym) if sk.producer == "abs" else c_sym
    if phi.has(s_sym, s2_sym, u_sym, _FINAL_ACC, _FINAL_M):
        raise NotImplementedError("producer operand must be independent of state")
    widths = {}
    for sym, name in sk.intrinsic_params:
        if name != "ncols":
            raise NotImplementedError(f"merge cannot prove intrinsic domain for {name!r}")
        widths[sym] = sp.Symbol("merge_width", positive=True)
    phi = sp.simplify(phi.xreplace(_parameter_substitutions(sk, values)).xreplace(widths))
    nonnegative = phi.is_nonnegative is True
    if sk.producer_domain == "nonnegative" and not nonnegative:
        raise NotImplementedError("declared nonnegative producer domain is not proved")
    return "nonnegative" if nonnegative and sk.producer_domain != "real" else "real"


@functools.lru_cache(maxsize=None)
def coordinate_needs_floor(sk) -> bool:
    """Floor the coordinate at 1e-30 only for a nonnegative MAX producer that a term, slope
    or bias divides by at zero (an all-zero row would otherwise give 0/0)."""
    if sk.two_pass or sk.producer_reducer != "max":
        return False
    if reachable_producer_domain(sk) != "nonnegative":
        return False
    a, b = repair_pair(sk, exact=True)
    for expr in (term_expr(sk), a, b):
        den = sp.fraction(sp.together(expr))[1]
        if sp.simplify(den.subs(s2_sym, 0)) == 0:
            return True
    return False


# ---------------------------------------------------------------- merge certificate
@dataclasses.dataclass(frozen=True)
class MergeCertificate:
    """Exact real-algebra certificate of the merge; not an IEEE associativity claim."""

    factor: sp.Expr
    bias: sp.Expr
    producer_domain: str
    coordinate_floor: bool
    assumptions: tuple[str, ...]
    proof_kind: str = "exact-symbolic"
    requires_finite: bool = True


def _parameter_substitutions(sk, values: dict | None) -> dict:
    """Exact rationals for supplied parameter values, after checking declared signs."""
    out = {}
    if values is None:
        return out
    for sym, name in sk.params:
        if name not in values:
            raise KeyError(f"skeleton {sk.name!r}: missing parameter {name!r}")
        value = float(values[name])
        if not math.isfinite(value):
            raise NotImplementedError(f"parameter {name!r} must be finite")
        if sym.is_positive is True and value <= 0:
            raise NotImplementedError(f"parameter {name!r} must be positive")
        if sym.is_nonnegative is True and value < 0:
            raise NotImplementedError(f"parameter {name!r} must be nonnegative")
        out[sym] = sp.Rational(str(value))
    return out


_MERGE_CERTIFICATES: dict = {}


def derive_merge_certificate(sk, values: dict | None = None) -> MergeCertificate:
    """Prove the repair, its cocycle and identity exactly before partial states may merge.

    The proof is a pure function of the skeleton and its parameter values and takes about a
    millisecond of symbolic simplification, so a proved certificate is kept per (skeleton,
    values) -- values keyed by type and repr, so 1 and 1.0, 0.0 and -0.0 stay distinct -- and
    every split call after the first reuses it.  A refused pair is proved (and refused) again."""
    try:
        key = (sk, tuple(sorted((k, type(v).__name__, repr(v)) for k, v in (values or {}).items())))
        hash(key)
    except TypeError:
        return _prove_merge_certificate(sk, values)
    cert = _MERGE_CERTIFICATES.get(key)
    if cert is None:
        cert = _prove_merge_certificate(sk, values)
        _MERGE_CERTIFICATES[key] = cert
    return cert


def _prove_merge_certificate(sk, values: dict | None) -> MergeCertificate:
    if sk.two_pass:
        raise NotImplementedError("two_pass needs extended carried state; pair merge refused")
    if sk.producer_reducer not in ("max", "sum"):
        raise NotImplementedError("unknown producer reducer")
    if sk.consumer_reducer not in ("sum", "max"):
        raise NotImplementedError("unknown consumer reducer")
    if sk.producer not in ("signed", "abs"):
        raise NotImplementedError("unknown producer mode")
    domain = reachable_producer_domain(sk, values)
    floor = coordinate_needs_floor(sk)
    rho, beta = repair_pair(sk, exact=True)
    subs_params = _parameter_substitutions(sk, values)
    if floor:
        assumption = {"positive": True}
    elif domain == "nonnegative":
        assumption = {"nonnegative": True}
    else:
        assumption = {"real": True}
    p, q, r = (sp.Symbol(n, **assumption) for n in ("merge_p", "merge_q", "merge_r"))
    a = rho.xreplace({s_sym: p, s2_sym: q, **subs_params})
    b = beta.xreplace({s_sym: p, s2_sym: q, **subs_params})
    g = sk.g.xreplace(subs_params)
    # condition (3): a(p, q) g(p, c) + b(p, q) == g(q, c)
    if _simplify(a * g.xreplace({s_sym: p}) + b - g.xreplace({s_sym: q})) != 0:
        raise NotImplementedError("repair condition (3) lacks an exact symbolic proof")
    if sk.consumer_reducer == "sum":
        if _simplify(b) != 0:
            raise NotImplementedError("sum consumer requires zero affine bias")
    elif sp.simplify(a).is_positive is not True:
        raise NotImplementedError("max consumer slope is not proved strictly positive on reachable domain")

    def moved(expr, old, new):
        return expr.xreplace({p: old, q: new})

    # cocycle: transporting p -> q -> r equals p -> r; and p -> p is the identity
    obligations = (
        moved(a, q, r) * a - moved(a, p, r),
        moved(a, q, r) * b + moved(b, q, r) - moved(b, p, r),
        a.xreplace({q: p}) - 1,
        b.xreplace({q: p}),
    )
    if any(_simplify(e) != 0 for e in obligations):
        raise NotImplementedError("repair cocycle/identity lacks an exact symbolic proof")
    for expr in (g.xreplace({s_sym: p}), a, b):
        if sp.fraction(sp.together(expr))[1].is_nonzero is not True:
            raise NotImplementedError("normalizer is not proved nonzero on reachable producer domain")
    intrinsic = {sym for sym, _ in sk.intrinsic_params}
    if (rho.free_symbols | beta.free_symbols) & intrinsic:
        raise NotImplementedError("merge repair cannot depend on runtime shape intrinsics")
    assumptions = ["finite real inputs and finite reachable arithmetic", "ncols > 0"]
    assumptions.extend(f"{sym}: {sym.assumptions0}" for sym, _ in sk.params)
    if floor:
        assumptions.append("effective producer = max(raw producer, 1e-30) on BOTH repair endpoints")
    return MergeCertificate(rho, beta, domain, floor, tuple(assumptions))


# ---------------------------------------------------------------- structured certificate
@dataclasses.dataclass(frozen=True)
class StateCertificate:
    state_fields: tuple[str, ...]
    merge: tuple
    assumptions: tuple[str, ...]
    proof_kind: str = "exact-structured-real-algebra"
    ieee_associative: bool = False


@functools.lru_cache(maxsize=None)
def derive_state_certificate(spec) -> StateCertificate:
    """Prove identity, associativity and integer closure of a structured state exactly."""
    from neptune_codegen.skeleton import StateReduction

    if not isinstance(spec, StateReduction) or not spec.fields:
        raise NotImplementedError("structured state requires nonempty typed fields")
    names = tuple(f.name for f in spec.fields)
    symbols = tuple(f.symbol for f in spec.fields)
    if len(set(names)) != len(names) or len(set(symbols)) != len(symbols):
        raise NotImplementedError("structured state field names and symbols must be unique")
    for f in spec.fields:
        if f.dtype not in ("float32", "int64") or f.extent not in ("scalar", "channel"):
            raise NotImplementedError("unsupported structured field type or extent")
    if spec.domain not in ("row_last", "segments") or spec.output_kind not in ("map", "reduced"):
        raise NotImplementedError("unsupported structured access or output domain")
    bound_terms = set(spec.inputs) | {sym for sym, _ in spec.params}
    for f in spec.fields:
        if sp.sympify(f.term).free_symbols - bound_terms:
            raise NotImplementedError("state lift depends on unbound data or a previous state")
        if sp.sympify(f.identity).free_symbols:
            raise NotImplementedError("state identity must be a constant")
        if f.dtype == "int64":
            term, ident = sp.sympify(f.term), sp.sympify(f.identity)
            if term.is_integer is not True or ident.is_integer is not True:
                raise NotImplementedError("int64 state lift and identity require an integer domain proof")
            if f.symbol.is_integer is not True:
                raise NotImplementedError("int64 state symbol must declare the integer domain")
            if f.symbol.is_nonnegative is True and (term.is_nonnegative is not True
                                                    or ident.is_nonnegative is not True):
                raise NotImplementedError("nonnegative int64 state requires nonnegative lift/identity")
    readout_bound = set(symbols) | {sym for sym, _ in spec.params}
    if spec.output_kind == "map":
        readout_bound |= set(spec.inputs)
    if sp.sympify(spec.readout).free_symbols - readout_bound:
        raise NotImplementedError("structured readout has an unbound input")
    left, right = spec.left, spec.right
    merges = tuple(sp.sympify(e) for e in spec.merge_expressions)
    if len(merges) != len(spec.fields):
        raise NotImplementedError("state merge changes tuple arity")
    if any(e.free_symbols - set(left + right) for e in merges):
        raise NotImplementedError("state merge must be shape-free and data-free")
    typed = {}
    for lsym, rsym, f in zip(left, right, spec.fields):
        if f.dtype == "int64":
            kw = {"integer": True}
            if f.symbol.is_nonnegative is True:
                kw["nonnegative"] = True
            typed[lsym] = sp.Symbol("integer_left_" + f.name, **kw)
            typed[rsym] = sp.Symbol("integer_right_" + f.name, **kw)
    for e, f in zip(merges, spec.fields):
        if f.dtype == "int64":
            closed = e.xreplace(typed)
            if closed.is_integer is not True:
                raise NotImplementedError("int64 state merge lacks an integer closure proof")
            if f.symbol.is_nonnegative is True and closed.is_nonnegative is not True:
                raise NotImplementedError("int64 state merge lacks a nonnegative closure proof")
    identity = tuple(sp.sympify(f.identity) for f in spec.fields)
    xa, xb, xc = (tuple(sp.Symbol(f"state_{tag}_{n}", real=True) for n in names)
                  for tag in ("a", "b", "c"))

    def merge(lhs, rhs):
        bind = dict(zip(left + right, lhs + rhs))
        return tuple(e.xreplace(bind) for e in merges)

    obligations = [u - v for u, v in zip(merge(identity, xa), xa)]
    obligations += [u - v for u, v in zip(merge(xa, identity), xa)]
    obligations += [u - v for u, v in zip(merge(merge(xa, xb), xc), merge(xa, merge(xb, xc)))]
    if any(_simplify(e) != 0 for e in obligations):
        raise NotImplementedError("structured merge identity/associativity lacks exact proof")
    assumptions = (
        "finite real inputs and finite reachable arithmetic",
        "logical domain partitions contain every participating element exactly once",
        "identity represents an empty partition; initial applied once per output",
        "explicit dtype conversions and reduction order are not erased by real algebra",
        "reachable integer states fit their declared storage type; readout domain checked separately",
    )
    return StateCertificate(names, merges, assumptions)
