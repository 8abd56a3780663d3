"""Symbolic reading of an ATen/FX graph as row algebra over one data symbol.

Every node downstream of a chosen tensor boundary (the *anchor*) is mapped to a sympy
expression in the row element `c`.  A reduction over the last dimension installs a fresh
symbol standing for its result, so a graph becomes a list of reductions whose operands are
expressions in `c` and in earlier reduction symbols.  A dependent pair -- a max- or sum-like
*producer* whose symbol appears in another reduction's operand (the *consumer*) -- is what the
fold algebra fuses.

Acceptance follows the reference's interpreter (neptune_recognize/interp.py:14-611): the same
pointwise and reduction vocabulary, the same guards read as identities (the 1e-30 floor of a
max-abs producer, torch.logsumexp's infinity guard), the same refusals (mutation, non-last-dim
reductions, unbiased variance, dtype-changing reductions, row-changing reshapes or broadcasts).
Those rules decide which graphs are rewritten, so they are the contract; the walk itself is
this module's own.
"""
from __future__ import annotations

import dataclasses
import math
import operator

import sympy as sp

from neptune_codegen import c_sym

# The producer result inside a matched consumer term.
S_RESULT = sp.Symbol("$producer", real=True)
# Row length and row count as graph symbols; a skeleton's intrinsic parameter binds to them.
NCOLS_SYM = sp.Symbol("$ncols", positive=True)
_INTRINSIC_SYMBOLS = {"ncols": NCOLS_SYM, "rows": sp.Symbol("$rows", positive=True)}

_BINARY = {
    "add": operator.add, "sub": operator.sub, "mul": operator.mul,
    "div": operator.truediv, "truediv": operator.truediv, "pow": operator.pow,
}
_UNARY = {
    "exp": sp.exp, "log": sp.log, "tanh": sp.tanh, "abs": sp.Abs, "sqrt": sp.sqrt,
    "rsqrt": lambda a: 1 / sp.sqrt(a), "neg": operator.neg, "reciprocal": lambda a: 1 / a,
}
_REDUCTIONS = ("amax", "sum", "max")
_MEANS = ("mean",)
_VAR_STD = ("var", "std")
_IGNORED = ("squeeze", "unsqueeze", "getitem", "detach", "alias")
# ops that carry no data path: allocations and export's tracing wrappers / metadata asserts
_NO_DATA = ("empty", "empty_like", "new_empty", "new_zeros", "new_ones",
            "wrap_with_set_grad_enabled", "_assert_tensor_metadata")
_CONST_FILL = ("full_like", "full", "scalar_tensor", "zeros_like", "ones_like")
FLOOR = 1e-30


class _Refusal(ValueError):
    """A semantic boundary of the interpreter (not an error of the caller)."""


@dataclasses.dataclass
class Candidate:
    """One dependent (producer, consumer) reduction pair of a graph."""

    phi: object                 # producer operand in c
    psi: object                 # consumer operand in c and S_RESULT
    prod_kind: str              # "max" | "sum"
    cons_kind: str
    producer_node: object
    consumer_node: object
    consumer_sym: object = None
    producer_sym: object = None
    producer_guarded: bool = False


# ---------------------------------------------------------------- node helpers
def _op(node) -> str:
    """Bare op name: aten schema name without namespace/overload, method name, or callable name."""
    if node.op == "call_method":
        return node.target if isinstance(node.target, str) else str(node.target)
    target = getattr(node, "target", None)
    schema = getattr(target, "_schema", None)
    if schema is not None:
        return schema.name.split("::")[-1]
    return getattr(target, "__name__", None) or str(target)


def _tensor_value(node):
    meta = getattr(node, "meta", None)
    if not meta:
        return None
    value = meta.get("val")
    return meta.get("example_value") if value is None else value


def _same_shape(a, b) -> bool:
    """Shape equality by printed form, so symbolic sizes are compared without guarding."""
    return len(a) == len(b) and all(str(x) == str(y) for x, y in zip(a, b))


def _rank_of(node):
    shape = getattr(_tensor_value(node), "shape", None)
    return None if shape is None else len(shape)


def _argument(node, name, default=None):
    """A call argument by schema name (positional or keyword)."""
    if name in node.kwargs:
        return node.kwargs[name]
    schema = getattr(node.target, "_schema", None)
    if schema is not None:
        for index, arg in enumerate(schema.arguments):
            if arg.name == name:
                return node.args[index] if index < len(node.args) else default
        return default
    fallback = {"dim": 1, "keepdim": 2, "min": 1, "max": 2}.get(name)
    return node.args[fallback] if fallback is not None and fallback < len(node.args) else default


def _last_dim_of(gm):
    """Concrete last dimension of the graph's first input, if known."""
    for node in gm.graph.nodes:
        if node.op != "placeholder":
            continue
        shape = getattr(_tensor_value(node), "shape", None)
        if not shape:
            return None
        try:
            return sp.Integer(int(shape[-1]))
        except (TypeError, ValueError):
            return None
    return None


def _scalar(value) -> sp.Expr:
    """Exact rational of a Python float literal (its shortest repr), else sympify."""
    if isinstance(value, float) and math.isfinite(value):
        return sp.Rational(repr(value))
    return sp.sympify(value)


def _as_expr(arg, env):
    """(expression, is_value) of one operand: a node's expression or a numeric literal."""
    if hasattr(arg, "op"):
        return env.get(arg), True
    if isinstance(arg, bool):
        return None, False
    if isinstance(arg, (int, float)):
        return _scalar(arg), True
    return None, False


def _flatten_nodes(arg, out: list) -> None:
    """Append to `out` the graph nodes inside a (possibly nested) FX argument, in order."""
    import torch.fx

    torch.fx.node.map_arg(arg, out.append)


def _operand(node, env, index=0) -> sp.Expr:
    if index >= len(node.args):
        raise _Refusal(f"a value operand is missing at {str(node.target)!r}")
    expr, is_value = _as_expr(node.args[index], env)
    if not is_value or expr is None:
        raise _Refusal(f"a value operand could not be interpreted at {str(node.target)!r}")
    return expr


def _is_const(arg, wanted: float) -> bool:
    """A literal or a scalar_tensor node holding exactly `wanted`."""
    if isinstance(arg, (int, float)) and not isinstance(arg, bool):
        return float(arg) == wanted
    if getattr(arg, "op", None) == "call_function" and _op(arg) == "scalar_tensor" and arg.args:
        return _is_const(arg.args[0], wanted)
    return False


def _reduced_dims(node):
    for arg in node.args[1:]:
        if isinstance(arg, bool):
            continue
        if isinstance(arg, int):
            return [arg]
        if isinstance(arg, (list, tuple)) and all(isinstance(d, int) for d in arg):
            return list(arg)
    dim = node.kwargs.get("dim")
    if isinstance(dim, int):
        return [dim]
    if isinstance(dim, (list, tuple)):
        return list(dim)
    return None


def _reduces_last_dim_only(node, rank) -> bool:
    dims = _reduced_dims(node)
    if not dims or len(dims) != 1:
        return False
    return dims[0] == -1 or (rank is not None and dims[0] == rank - 1)


def _var_is_biased(node) -> bool:
    """`correction=0` / `unbiased=False` only: torch's default is the /(N-1) operator."""
    if "correction" in node.kwargs:
        value = node.kwargs["correction"]
        return isinstance(value, (int, float)) and value == 0
    if "unbiased" in node.kwargs:
        return node.kwargs["unbiased"] is False
    return len(node.args) > 2 and node.args[2] is False


def _is_row_flatten(node, rank) -> bool:
    """`reshape(x, [rows, -1])` of a 2-D input with the same concrete row count is identity."""
    if rank != 2 or len(node.args) < 2 or not isinstance(node.args[1], (list, tuple)):
        return False
    if len(node.args[1]) != 2:
        return False
    first, second = node.args[1]
    shape = getattr(_tensor_value(node.args[0]), "shape", None)
    return (second == -1 and isinstance(first, int) and shape is not None and len(shape) == 2
            and isinstance(shape[0], int) and shape[0] == first)


# ---------------------------------------------------------------- the two guards
def _logsumexp_inf_guard(gm) -> dict:
    """torch.logsumexp's `where(abs(m) == inf, 0, m)` on an amax: {where: amax, cond/0: None}.

    For finite inputs the guard is the identity; its helper nodes are structure, not data."""
    table: dict = {}
    for node in gm.graph.nodes:
        if node.op != "call_function" or _op(node) != "where" or len(node.args) < 3:
            continue
        cond, low, high = node.args[:3]
        if not _is_const(low, 0.0) or getattr(cond, "op", None) != "call_function":
            continue
        if not str(cond.target).startswith("aten.eq") or len(cond.args) != 2:
            continue
        inner, bound = cond.args
        if not _is_const(bound, math.inf) or getattr(inner, "op", None) != "call_function":
            continue
        if not str(inner.target).startswith("aten.abs") or tuple(inner.args) != (high,):
            continue
        if getattr(high, "op", None) != "call_function" or _op(high) != "amax":
            continue
        table[node] = high
        for helper in (cond, low, inner, bound):
            if getattr(helper, "op", None) == "call_function":
                table[helper] = None
    return table


def _floor_guard(node, env) -> bool:
    """clamp_min(amax(abs(c)), 1e-30): the documented zero guard of a max-abs coordinate."""
    if _op(node) not in ("clamp", "clamp_min") or not node.args:
        return False
    low = _argument(node, "min")
    high = _argument(node, "max") if _op(node) == "clamp" else None
    if not isinstance(low, (int, float)) or low != FLOOR or high is not None:
        return False
    source = node.args[0]
    if getattr(source, "op", None) != "call_function" or _op(source) != "amax":
        return False
    if not getattr(env.get(source), "is_Symbol", False):
        return False
    return env.get(source.args[0] if source.args else None) == sp.Abs(c_sym)


# ---------------------------------------------------------------- the walk
class _RowWalk:
    """Interprets the nodes after one anchor; a refusal drops only that node's value."""

    def __init__(self, anchor, rank):
        self.anchor, self.rank = anchor, rank
        self.env: dict = {}
        self.reductions: list = []      # (kind, operand, symbol, node)
        self.guarded: dict = {}         # producer symbol -> Max(symbol, 1e-30)

    def _fresh(self):
        return sp.Symbol(f"$r{len(self.reductions)}", real=True)

    def _reduce(self, kind, operand, node):
        symbol = self._fresh()
        self.reductions.append((kind, operand, symbol, node))
        return symbol

    def _check_broadcast(self, node):
        """A reduction result may only broadcast along its own row ([..., 1] against data)."""
        operands = [(arg, self.env.get(arg)) for arg in node.args[:2] if hasattr(arg, "op")]
        data = [arg for arg, expr in operands if expr is not None and expr.has(c_sym)]
        if not data:
            return
        for arg, expr in operands:
            if expr is None or expr.has(c_sym) or not expr.free_symbols:
                continue
            dv, rv = _tensor_value(data[0]), _tensor_value(arg)
            if dv is None or rv is None:
                raise _Refusal("reduction broadcast metadata is unknown")
            row_vector = dv.shape[:-1] + (1,)
            scalar_row = len(dv.shape) == 1 and len(rv.shape) == 0
            if not scalar_row and not _same_shape(rv.shape, row_vector):
                raise _Refusal("a reduction is broadcast across columns instead of its own row")

    def _check_shape(self, node):
        expr = self.env.get(node)
        if expr is None or not expr.has(c_sym):
            return
        src, out = _tensor_value(self.anchor), _tensor_value(node)
        if src is not None and out is not None and hasattr(out, "shape"):
            if not _same_shape(out.shape, src.shape):
                raise _Refusal("pointwise broadcasting changes row shape; preserve it as a boundary")

    def node(self, node):
        name = _op(node)
        schema = getattr(node.target, "_schema", None)
        if schema is not None and (schema.is_mutable or not schema.name.startswith("aten::")):
            raise _Refusal(f"unsupported or mutable operation {node.target!s}")
        env = self.env
        if name in _NO_DATA:
            return
        if name in ("view", "reshape"):
            before, after = _tensor_value(node.args[0]) if node.args else None, _tensor_value(node)
            same = before is not None and after is not None and _same_shape(before.shape, after.shape)
            if not same and not _is_row_flatten(node, self.rank):
                raise _Refusal(f"a {name} changes the row structure")
            env[node] = _operand(node, env)
            return
        if name in _CONST_FILL:
            if name.startswith("zeros"):
                fill = 0.0
            elif name.startswith("ones"):
                fill = 1.0
            else:
                position = 0 if name == "scalar_tensor" else 1
                fill = node.args[position] if len(node.args) > position else None
            if not isinstance(fill, (int, float)) or isinstance(fill, bool):
                raise _Refusal("a fill value is not a scalar constant")
            env[node] = _scalar(fill)
            return
        if name in ("clamp", "clamp_min"):
            if not _floor_guard(node, env):
                raise _Refusal("a clamp is real computation, not the exact max-abs zero guard")
            value = _operand(node, env)
            self.guarded[value] = sp.Max(value, _scalar(FLOOR))
            env[node] = self.guarded[value]
            return
        if name in _IGNORED:
            if name == "getitem":
                src = node.args[0] if node.args else None
                if (len(node.args) != 2 or node.args[1] != 0
                        or getattr(src, "op", None) != "call_function" or _op(src) != "max"):
                    raise _Refusal("getitem may select data or reduction indices")
            value = _operand(node, env)
            if name in ("squeeze", "unsqueeze") and value.has(c_sym):
                before, after = _tensor_value(node.args[0]), _tensor_value(node)
                if before is None or after is None or not _same_shape(before.shape, after.shape):
                    raise _Refusal("a data reshape changes the row structure")
            env[node] = value
            return
        if name in (*_REDUCTIONS, *_MEANS, *_VAR_STD):
            value = _operand(node, env)
            source = node.args[0]
            source_rank = _rank_of(source)
            if not _reduces_last_dim_only(node, source_rank if source_rank is not None else self.rank):
                raise _Refusal("only a last-dimension row reduction is supported")
            dtype = _argument(node, "dtype")
            sv = _tensor_value(source)
            if dtype is not None and (sv is None or dtype != sv.dtype):
                raise _Refusal("a reduction changes dtype; preserve the conversion as a region boundary")
            if name in _VAR_STD:
                if not _var_is_biased(node):
                    raise _Refusal("unbiased variance/std requires a carried count")
                mean = self._reduce("sum", value / NCOLS_SYM, node)
                var = self._reduce("sum", (value - mean) ** 2 / NCOLS_SYM, node)
                env[node] = sp.sqrt(var) if name == "std" else var
                return
            kind = "max" if name in ("amax", "max") else "sum"
            env[node] = self._reduce(kind, value / NCOLS_SYM if name in _MEANS else value, node)
            return
        if name in _BINARY:
            left, right = _operand(node, env), _operand(node, env, 1)
            if name in ("add", "sub"):
                alpha = _argument(node, "alpha", 1)
                if not isinstance(alpha, (int, float)) or not math.isfinite(alpha):
                    raise _Refusal("alpha is not a finite scalar constant")
                right = right * _scalar(alpha)
            if name in ("div", "truediv") and _argument(node, "rounding_mode") is not None:
                raise _Refusal("rounded division is not real division")
            self._check_broadcast(node)
            env[node] = _BINARY[name](left, right)
            return
        if name in _UNARY:
            env[node] = _UNARY[name](_operand(node, env))
            return
        raise _Refusal(f"unfamiliar op {str(node.target)!r}; compound reductions may need "
                       "lowering/decomposition")


def _dependent_pairs(walk) -> list:
    """Producer/consumer pairs: the consumer operand uses exactly the producer's result and
    the producer operand uses no reduction result."""
    symbols = [r[2] for r in walk.reductions]
    pairs = []
    for pk, phi, producer, pnode in walk.reductions:
        if any(phi.has(s) for s in symbols):
            continue
        for ck, operand, consumer, cnode in walk.reductions:
            if consumer is producer or not operand.has(producer):
                continue
            if any(operand.has(s) for s in symbols if s is not producer):
                continue
            guard = walk.guarded.get(producer)
            uses_guard = guard is not None and operand.has(guard)
            coordinate = guard if uses_guard else producer
            psi = operand.subs({coordinate: S_RESULT})
            if psi.has(S_RESULT) and not psi.has(producer):
                pairs.append(Candidate(phi, psi, pk, ck, pnode, cnode, consumer, coordinate,
                                       uses_guard))
    return pairs


def interpret(gm, why: list | None = None, *, input_node=None, local=False):
    """(anchor, [Candidate], env) for the row data at `input_node` (default: first input).

    Strict mode (local=False) gives up at the first node it cannot read.  Local mode drops that
    node's value and continues, so unrelated operations (GEMMs, casts, masks) stay boundaries
    of other regions.  Returns None, with the reason appended to `why`, when no dependent
    pair exists."""
    def refuse(message):
        if why is not None:
            why.append(message)
        return None

    for node in gm.graph.nodes:
        schema = getattr(node.target, "_schema", None)
        if (schema is not None and schema.is_mutable) or (
                node.op == "call_method" and str(node.target).endswith("_")):
            return refuse("mutable graph must be functionalized before reduction fusion")
    anchor = input_node
    walk = _RowWalk(anchor, _rank_of(anchor) if anchor is not None else None)
    guards = _logsumexp_inf_guard(gm)
    for node in gm.graph.nodes:
        if node is walk.anchor:
            walk.env[node] = c_sym
            continue
        if node.op == "placeholder":
            if walk.anchor is None:
                walk.anchor, walk.rank = node, _rank_of(node)
                walk.env[node] = c_sym
            continue
        if node.op not in ("call_function", "call_method"):
            continue
        try:
            if node in guards:
                source = guards[node]
                if source is not None:
                    value, known = _as_expr(source, walk.env)
                    if not known or value is None:
                        raise _Refusal("infinity guard source is outside the region")
                    walk.env[node] = value
                continue
            walk.node(node)
            walk._check_shape(node)
        except _Refusal as error:
            walk.env.pop(node, None)
            if not local:
                return refuse(str(error))
    if walk.anchor is None:
        return refuse("no input placeholder found")
    if len(walk.reductions) < 2:
        return refuse(f"only {len(walk.reductions)} reduction(s) found; a dependent reduction "
                      "pair is required")
    pairs = _dependent_pairs(walk)
    if not pairs:
        return refuse(f"{len(walk.reductions)} reductions found, but none depends on another")
    return walk.anchor, pairs, walk.env


def region_inputs(gm):
    """Candidate anchors: floating tensors feeding a reduction through known pointwise ops
    (unknown producers -- GEMMs, casts, clamps -- end the walk and are anchors themselves)."""
    passthrough = set(_BINARY) | set(_UNARY) | {"view", "reshape", "detach", "alias"}
    anchors = set()
    for node in gm.graph.nodes:
        if node.op not in ("call_function", "call_method"):
            continue
        if _op(node) not in (*_REDUCTIONS, *_MEANS, *_VAR_STD):
            continue
        stack, seen = list(node.args[:1]), set()
        while stack:
            value = stack.pop()
            if not hasattr(value, "op") or value in seen:
                continue
            seen.add(value)
            meta = _tensor_value(value)
            if (meta is None or not hasattr(meta, "shape") or not meta.is_floating_point()
                    or len(meta.shape) < 1):
                continue
            anchors.add(value)
            if value.op in ("call_function", "call_method") and _op(value) in passthrough:
                stack.extend(value.all_input_nodes)
    return [node for node in gm.graph.nodes if node in anchors]
