"""Fold specifications: scalar repair skeletons and structured (sum, count) state reductions.

The spec is the input of the HIP emitter, exactly as it is the input of the reference's Triton
emitter.  Field names, defaults and the registry behaviour mirror neptune_codegen/skeleton.py
(Skeleton :21-105, register :110-115, supported :118-133, StateReduction :173-205, built-ins
:223-242, param_defaults :255-267) so that declarations and callers carry over unchanged.
"""
from __future__ import annotations

import dataclasses
from types import MappingProxyType

import sympy as sp

from neptune_codegen.symbols import *  # noqa: F401,F403

# Registered only to be refused: p >= 3 power folds lose small-sum precision.
NEGATIVE_CONTROLS = {"pnorm3"}


@dataclasses.dataclass(frozen=True)
class Skeleton:
    """One fusable row fold, declared as algebra.

    g                 term producer g(s, c); the repair and the consumer term derive from it
    finalize          readout over (acc, m)
    producer          "signed" (m = max v) or "abs" (m = max |v|)
    is_log            exponential fold (m + log(acc) readout, NaN/+inf status extension)
    params            ((sympy symbol, kernel argument name), ...) baked into the kernel
    producer_expr     explicit producer operand over c (derived for exponential folds)
    producer_reducer  "max" | "sum";  consumer_reducer "sum" | "max"
    defaults          ((symbol, value), ...) convenience values of declared params
    intrinsic_params  ((symbol, intrinsic name), ...) supplied by the kernel (e.g. ncols)
    two_pass          the term reads the FINAL producer: read the row twice, no repair
    producer_domain   "auto" | "real" | "nonnegative"
    """

    name: str
    g: sp.Expr
    finalize: sp.Expr
    producer: str = "abs"
    init: str = "0.0"
    doc: str = ""
    is_log: bool = False
    params: tuple = ()
    producer_expr: sp.Expr | None = None
    producer_reducer: str = "max"
    consumer_reducer: str = "sum"
    defaults: tuple = ()
    intrinsic_params: tuple = ()
    two_pass: bool = False
    producer_domain: str = "auto"


SKELETONS: dict[str, Skeleton] = {}


def register(sk: Skeleton) -> Skeleton:
    """Add a skeleton; re-registering a name with different algebra is refused."""
    existing = SKELETONS.get(sk.name)
    if existing is not None and existing != sk:
        raise ValueError(f"skeleton {sk.name!r} is already registered with different algebra; use a new name")
    SKELETONS[sk.name] = sk
    return sk


def supported() -> list[str]:
    """Registered skeletons the HIP emitter can lower (negative controls excluded)."""
    from neptune_codegen.emitters import check_supported

    names = []
    for name in sorted(SKELETONS):
        if name in NEGATIVE_CONTROLS:
            continue
        try:
            check_supported(SKELETONS[name])
        except NotImplementedError:
            continue
        names.append(name)
    return names


def all_registered() -> list[str]:
    return sorted(SKELETONS)


def unsupported_reason(name: str) -> str:
    """Why a registered skeleton cannot be emitted ("" when it can)."""
    from neptune_codegen.emitters import check_supported

    try:
        check_supported(SKELETONS[name])
    except NotImplementedError as exc:
        return str(exc)
    return ""


# ---------------------------------------------------------------- structured states
@dataclasses.dataclass(frozen=True)
class StateField:
    name: str
    symbol: sp.Symbol
    term: sp.Expr
    dtype: str = "float32"
    extent: str = "scalar"      # "scalar" or "channel" (one state per output channel)
    identity: sp.Expr = sp.Integer(0)


@dataclasses.dataclass(frozen=True)
class NumericalContract:
    accumulation_dtype: str
    reduction_order: str
    stages: tuple[str, ...]
    empty_policy: str
    nonfinite_policy: str = "source_ieee"
    bitwise_reassociation: bool = False


@dataclasses.dataclass(frozen=True)
class StateReduction:
    """A typed mergeable statistic plus a readout; `numeric` fixes rounding and empties."""

    name: str
    operation: str
    inputs: tuple[sp.Symbol, ...]
    fields: tuple[StateField, ...]
    readout: sp.Expr
    domain: str
    output_kind: str            # "map" reads the original element, "reduced" only the state
    params: tuple = ()
    numeric: NumericalContract = NumericalContract("float32", "tree", (), "reject")
    merge: tuple = ()           # empty: componentwise addition

    @property
    def left(self) -> tuple:
        return tuple(sp.Symbol("left_" + f.name, real=True) for f in self.fields)

    @property
    def right(self) -> tuple:
        return tuple(sp.Symbol("right_" + f.name, real=True) for f in self.fields)

    @property
    def merge_expressions(self) -> tuple:
        if self.merge:
            return self.merge
        return tuple(a + b for a, b in zip(self.left, self.right))


_STATE_TOTAL = sp.Symbol("state_total", real=True)
_STATE_COUNT = sp.Symbol("state_count", integer=True, nonnegative=True)
_STATE_DATA = sp.Symbol("state_data", real=True)
_STATE_GAMMA = sp.Symbol("state_gamma", real=True)
_STATE_INITIAL = sp.Symbol("state_initial", real=True)
_STATE_EPS = sp.Symbol("state_eps", positive=True)

_RMS_NUMERIC = NumericalContract(
    "float32", "tree_or_serial",
    ("promote_input_fp32", "square_fp32", "mean_fp32", "add_eps_fp32", "rsqrt_fp32",
     "normalize_fp32", "round_input_dtype", "multiply_gamma", "round_output_dtype"),
    "reject_empty_width")
# L2-normalize has no reference counterpart; its stages mirror the RMS contract with the
# torch.nn.functional.normalize readout x / max(||x||_2, eps).
_L2_NUMERIC = NumericalContract(
    "float32", "tree_or_serial",
    ("promote_input_fp32", "square_fp32", "sqrt_fp32", "clamp_min_eps_fp32", "divide_fp32",
     "round_output_dtype"),
    "reject_empty_width")
_SEGMENT_NUMERIC = NumericalContract(
    "input", "ordered",
    ("convert_initial_input_dtype", "ordered_add_round_input_dtype", "divide_count_input_dtype",
     "round_output_dtype"), "source_initial_or_nan")

_SUMSQ = StateField("total", _STATE_TOTAL, _STATE_DATA ** 2)
_COUNT = StateField("count", _STATE_COUNT, sp.Integer(1), "int64")
_CHANNEL_SUM = StateField("total", _STATE_TOTAL, _STATE_DATA, extent="channel")

_BUILTIN_STATE_REDUCTIONS = MappingProxyType({
    "rms_norm": StateReduction(
        "rms_norm", "rms_norm", (_STATE_DATA, _STATE_GAMMA), (_SUMSQ, _COUNT),
        _STATE_DATA * _STATE_GAMMA / sp.sqrt(_STATE_TOTAL / _STATE_COUNT + _STATE_EPS),
        "row_last", "map", ((_STATE_EPS, "eps"),), _RMS_NUMERIC),
    "l2_normalize": StateReduction(
        "l2_normalize", "l2_normalize", (_STATE_DATA,), (_SUMSQ, _COUNT),
        _STATE_DATA / sp.Max(sp.sqrt(_STATE_TOTAL), _STATE_EPS),
        "row_last", "map", ((_STATE_EPS, "eps"),), _L2_NUMERIC),
    "segment_sum": StateReduction(
        "segment_sum", "segment_pool", (_STATE_DATA,), (_CHANNEL_SUM, _COUNT),
        _STATE_TOTAL + _STATE_INITIAL, "segments", "reduced",
        ((_STATE_INITIAL, "initial"),), _SEGMENT_NUMERIC),
    "segment_mean": StateReduction(
        "segment_mean", "segment_pool", (_STATE_DATA,), (_CHANNEL_SUM, _COUNT),
        (_STATE_TOTAL + _STATE_INITIAL) / _STATE_COUNT, "segments", "reduced",
        ((_STATE_INITIAL, "initial"),), _SEGMENT_NUMERIC),
})
STATE_REDUCTIONS = _BUILTIN_STATE_REDUCTIONS


def state_reduction_spec(name: str) -> StateReduction:
    """The immutable built-in spec; a registry that was swapped or edited is refused."""
    spec = _BUILTIN_STATE_REDUCTIONS[name]
    if STATE_REDUCTIONS.get(name) != spec:
        raise NotImplementedError("structured registry differs from the immutable built-in specification")
    return spec


# ---------------------------------------------------------------- parameter defaults
def param_defaults(name: str) -> dict:
    """Declared default values of a skeleton's baked parameters (1.0 when undeclared).

    `run`, `as_triton_op` and the oracle all fill the same defaults, so a kernel and its
    reference never disagree on a constant nobody passed.
    """
    sk = SKELETONS[name]
    declared = {sym: float(value) for sym, value in sk.defaults}
    intrinsic = {sym for sym, _ in sk.intrinsic_params}
    return {arg: declared.get(sym, 1.0) for sym, arg in sk.params if sym not in intrinsic}
