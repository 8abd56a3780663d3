"""Recovering a skeleton's scalar parameters from a graph expression.

`_solve_for(expr, sym)` finds the value of one parameter that makes `expr` vanish for every
value of the other symbols (the reference's params.py:1-92 has the same contract: symbolic
solve first, a checked numeric root second, and a declared-domain filter so that a degenerate
value -- N = 0 turning decay_renorm into linear_attn -- is never accepted).
"""
from __future__ import annotations

import sympy as sp


def _respects(sym, value) -> bool:
    """Does `value` lie in the symbol's declared domain (positive / nonnegative)?"""
    try:
        v = float(value)
    except (TypeError, ValueError):
        return False
    if sym.is_positive and not v > 0:
        return False
    if sym.is_nonnegative and not v >= 0:
        return False
    return True


def _sample_points(free, count, salt):
    """Deterministic positive rational points for the other free symbols (no RNG state)."""
    points = []
    for k in range(count):
        point = {}
        for i, f in enumerate(free):
            a = (7 * (k + salt) + 13 * i) % 29 + 1
            b = (5 * (k + salt) + 3 * i) % 10 + 1
            point[f] = sp.Rational(a, b)
        points.append(point)
    return points


def _infer_numerically(expr, sym, samples: int = 6):
    """A root of expr(sym) at fixed values of the other symbols, kept only if it also zeroes
    expr at five held-out points (a spurious root of one slice fails that)."""
    free = sorted((f for f in expr.free_symbols if f != sym), key=lambda z: z.name)
    if not free:
        return None
    held_out = _sample_points(free, 5, salt=101)
    for point in _sample_points(free, samples, salt=0):
        slice_ = expr.subs(point)
        for start in (1.0, 0.3, 2.0, 0.05):
            try:
                root = sp.nsolve(slice_, sym, start, tol=1e-13, maxsteps=80)
            except Exception:  # noqa: BLE001 -- a start that does not converge is skipped
                continue
            if not (root.is_number and root.is_real) or not _respects(sym, root):
                continue
            try:
                ok = all(abs(complex(sp.N(expr.subs({**held, sym: root}), 25))) <= 1e-9
                         for held in held_out)
            except (TypeError, ValueError):
                ok = False
            if ok:
                return sp.Float(root)
    return None


def _solve_for(expr, sym):
    """Value of `sym` with expr == 0: exact solve, else a verified numeric root, else None."""
    try:
        solutions = sp.solve(sp.Eq(expr, 0), sym, dict=True)
    except (NotImplementedError, ValueError, TypeError):
        solutions = []
    for sol in solutions:
        if len(sol) == 1:
            value = next(iter(sol.values()))
            if value.is_number and value.is_real and _respects(sym, value):
                return value
    return _infer_numerically(expr, sym)
