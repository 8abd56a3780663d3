"""Symbols the fold algebra is written over.

A skeleton describes its operator as sympy expressions over these names; the algebra module
derives the repair from them and the HIP emitter renders them as device code.  The names and
assumptions follow the reference's vocabulary (neptune_codegen/symbols.py:8-62) because the
skeleton declarations, the derived repair strings and recognition all speak in them.
"""
from __future__ import annotations

import sympy as sp

# u: an accumulated term value (only used to refuse skeletons that read it)
u_sym = sp.Symbol("u", positive=True)
# s: the producer value a term was computed against (stale); s2: the fresh producer value
s_sym = sp.Symbol("s", real=True)
s2_sym = sp.Symbol("s2", real=True)
# c: one element of the reduced row
c_sym = sp.Symbol("c", real=True)

# readout symbols of `finalize`
_FINAL_ACC = sp.Symbol("acc", real=True)
_FINAL_M = sp.Symbol("m", real=True)

# declared scalar parameters
_PARAM_TINY = sp.Symbol("tiny", nonnegative=True)   # additive constant of the log readout
_PARAM_N = sp.Symbol("N", positive=True)            # row length (bound to ncols at run time)
_PARAM_EPS = sp.Symbol("eps", positive=True)
_PARAM_ALPHA = sp.Symbol("alpha", real=True)
_PARAM_BETA = sp.Symbol("beta", positive=True)
_PARAM_T = sp.Symbol("T", positive=True)            # temperature

# Shape values a kernel has in scope; a parameter bound to one of these is not baked.
INTRINSICS = ("rows", "ncols", "stride_row")

__all__ = [
    "INTRINSICS",
    "u_sym", "s_sym", "s2_sym", "c_sym",
    "_FINAL_ACC", "_FINAL_M",
    "_PARAM_TINY", "_PARAM_N", "_PARAM_EPS", "_PARAM_ALPHA", "_PARAM_BETA", "_PARAM_T",
]
