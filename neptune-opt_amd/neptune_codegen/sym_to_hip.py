"""sympy expression -> HIP C++ fp32 expression text.

Replaces the reference's Triton translator (neptune_codegen/sym_to_triton.py:105-245).  The
lowering rules that carry numerical meaning are kept:

  * exp is a true exponential, never clipped (a clipped exp breaks the repair cocycle);
    it lowers to nep::fast_exp, 2^(x log2 e) on the hardware exp2;
  * tanh(x) lowers to 2*sigmoid(2x) - 1 with the hardware reciprocal (v_rcp_f32, 1 ulp),
    saturating to +-1 instead of overflowing;
  * a marked quotient power _Q(a, b, k) lowers to k products of (a / b), never a**k / b**k;
  * with `shared` given, a quotient whose denominator does not mention that symbol (a fold
    term's divisor fixed per tile) lowers to nep::quot, a multiply by one shared reciprocal;
  * x**(1/2) is sqrtf(x), x**(-1/2) is 1.0f / sqrtf(x), integer powers are products;
  * with `fast` (repair slopes and biases, evaluated per tile and per merge, never per
    element), x**(1/2), x**(-1/2) and quotients use the hardware instructions instead
    (nep::fsqrt, nep::frsq, nep::fquot: 1 ulp each), the precision class of the reference's
    Triton lowering (tl.sqrt and fp32 division, neither correctly rounded);
  * other fractional powers are allowed only for a provably positive base (exp2(log2(b) p));
  * numeric literals are rounded to fp32 once and written as exact hex-float literals.
"""
from __future__ import annotations

import struct

import sympy as sp

from neptune_codegen.algebra import _Q


class TranslationError(NotImplementedError):
    """The expression uses a construct with no fp32 HIP lowering."""


def f32_literal(value: float) -> str:
    """Exact C++ literal of `value` rounded to fp32 (round to nearest even)."""
    value = float(value)
    if value != value:
        return "__builtin_nanf(\"\")"
    if value in (float("inf"), float("-inf")):
        return "nep::kInf" if value > 0 else "(-nep::kInf)"
    try:
        rounded = struct.unpack("f", struct.pack("f", value))[0]
    except OverflowError:
        return "nep::kInf" if value > 0 else "(-nep::kInf)"
    if rounded == 0.0:
        return "-0.0f" if str(rounded).startswith("-") else "0.0f"
    return f"{rounded.hex()}f".replace("0x", "0x", 1)


def _positive_base(base: sp.Expr) -> bool:
    return base.is_positive is True


def to_hip(expr: sp.Expr, names: dict, shared: sp.Symbol | None = None,
           fast: bool = False) -> str:
    """Render `expr` as an fp32 C++ expression; `names` maps symbols to source text.  With
    `shared` (the per-element symbol), divisors free of it become shared reciprocals; with
    `fast`, square roots and quotients use the 1-ulp hardware instructions."""
    expr = sp.sympify(expr)

    def divide(top: str, bottom: str, divisor: sp.Expr) -> str:
        if fast:
            return f"nep::fquot({top}, {bottom})"
        if shared is not None and not divisor.has(shared):
            return f"nep::quot({top}, {bottom})"
        return f"({top} / {bottom})"

    def rec(e: sp.Expr) -> str:
        if isinstance(e, _Q):
            num, den, k = e.args
            k = int(k)
            if k <= 0:
                raise TranslationError(f"quotient power needs a positive integer exponent: {e}")
            q = divide(rec(num), rec(den), den)
            return "(" + " * ".join([q] * k) + ")"
        if e.is_Symbol:
            if e not in names:
                raise TranslationError(f"no HIP binding for symbol {e}")
            return f"({names[e]})"
        if e.is_Number:
            if e is sp.nan:
                return "__builtin_nanf(\"\")"
            if e in (sp.oo, -sp.oo):
                return "nep::kInf" if e == sp.oo else "(-nep::kInf)"
            return f32_literal(float(e))
        if e.is_Add:
            return "(" + " + ".join(rec(a) for a in e.args) + ")"
        if e.is_Mul:
            coeff, rest = e.as_coeff_Mul()
            if coeff == -1:
                return f"(-{rec(rest)})"
            numer, denom, divisor = [], [], sp.Integer(1)
            for factor in e.args:
                base, ex = factor.as_base_exp()
                if fast and ex == sp.Rational(-1, 2):
                    numer.append(f"nep::frsq({rec(base)})")
                elif ex.is_Number and ex.is_negative:
                    denom.append(rec(base ** (-ex)))
                    divisor = divisor * base ** (-ex)
                else:
                    numer.append(rec(factor))
            top = " * ".join(numer) if numer else "1.0f"
            if not denom:
                return f"({top})"
            return divide(f"({top})", f"({' * '.join(denom)})", divisor)
        if e.is_Pow:
            base, ex = e.args
            if ex.is_Integer:
                k = int(ex)
                if k == 0:
                    return "1.0f"
                b = rec(base)
                prod = "(" + " * ".join([b] * abs(k)) + ")"
                return prod if k > 0 else divide("1.0f", prod, base)
            if ex == sp.Rational(1, 2):
                return f"nep::fsqrt({rec(base)})" if fast else f"sqrtf({rec(base)})"
            if ex == sp.Rational(-1, 2):
                return f"nep::frsq({rec(base)})" if fast else f"(1.0f / sqrtf({rec(base)}))"
            if _positive_base(base):
                return f"exp2f(log2f({rec(base)}) * {rec(ex)})"
            raise TranslationError(f"fractional power of a base not proved positive: {e}")
        if isinstance(e, sp.exp):
            return f"nep::fast_exp({rec(e.args[0])})"
        if isinstance(e, sp.log):
            if len(e.args) != 1:
                raise TranslationError(f"log with a base: {e}")
            return f"logf({rec(e.args[0])})"
        if isinstance(e, sp.tanh):
            x = rec(e.args[0])
            return f"(2.0f * __builtin_amdgcn_rcpf(1.0f + nep::fast_exp(-2.0f * {x})) - 1.0f)"
        if isinstance(e, sp.Abs):
            return f"fabsf({rec(e.args[0])})"
        if isinstance(e, (sp.Max, sp.Min)):
            fn = "fmaxf" if isinstance(e, sp.Max) else "fminf"
            out = rec(e.args[0])
            for a in e.args[1:]:
                out = f"{fn}({out}, {rec(a)})"
            return out
        raise TranslationError(f"no HIP lowering for {type(e).__name__}: {e}")

    return rec(expr)
