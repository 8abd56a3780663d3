"""Targeted lowering of compound ATen ops into the decomposed form recognition reads.

Only `aten.logsumexp` and (opt-in, through neptune_opt) `aten.log_softmax` /
`aten._log_softmax` over the last dimension are expanded; nothing else is decomposed.  The
expansion is the reference's step list (neptune_recognize/lowering.py:64-111), because the
recognised region and the rewrite's readout fusion read exactly those nodes:

    [x = x.to(fp32)]                                     16-bit inputs accumulate in fp32
    m = amax(x, dim, keepdim)
    m_safe = where(|m| == inf, 0, m)                     torch.logsumexp's infinity guard
    lse = m_safe + log(sum(exp(x - m_safe), dim, keepdim))
    log_softmax:  where(lse == inf, nan, x - lse)        torch's NaN rows for +inf inputs
    logsumexp without keepdim: squeeze(lse, dim)
    [out = result.to(output dtype)]

Every emitted node carries `meta["neptune_lowering"] = <compound node name>`, so that a caller
can find the region grown from one compound node.  The table is data: one interpreter runs it
on Fake/meta tensors (the metadata of every step, computed by torch) and the same interpreter
emits it as graph nodes.  The structural gate certifies a complete fp32 LSE region, not
bitwise equality with torch's fused kernels.
"""
from __future__ import annotations

import copy
import dataclasses
from contextlib import nullcontext

# compound targets -> whether the op is a log_softmax (else logsumexp)
_COMPOUNDS = {"aten._log_softmax.default": True, "aten.log_softmax.int": True,
              "aten.log_softmax.default": True, "aten.logsumexp.default": False}
MARK = "neptune_lowering"


class _Ref(str):
    """In a step's argument template: the value named by an earlier step (or x / dim)."""


def _bind(template, env):
    if isinstance(template, _Ref):
        return env[template]
    if isinstance(template, (tuple, list)):
        return type(template)(_bind(item, env) for item in template)
    return template


_X, _DIM = _Ref("x"), _Ref("dim")
_LSE_STEPS = (
    ("amax.default", "m", (_X, [_DIM], True)),
    ("abs.default", "abs_m", (_Ref("m"),)),
    ("eq.Scalar", "infinite", (_Ref("abs_m"), float("inf"))),
    ("where.ScalarSelf", "m_safe", (_Ref("infinite"), 0.0, _Ref("m"))),
    ("sub.Tensor", "centred", (_X, _Ref("m_safe"))),
    ("exp.default", "e", (_Ref("centred"),)),
    ("sum.dim_IntList", "s", (_Ref("e"), [_DIM], True)),
    ("log.default", "lg", (_Ref("s"),)),
    ("add.Tensor", "lse", (_Ref("m_safe"), _Ref("lg"))),
)
_LOG_SOFTMAX_TAIL = (
    ("eq.Scalar", "posinf_row", (_Ref("lse"), float("inf"))),
    ("sub.Tensor", "readout", (_X, _Ref("lse"))),
    ("where.ScalarSelf", "log_out", (_Ref("posinf_row"), float("nan"), _Ref("readout"))),
)


def _program(dtype, output_dtype, *, log_softmax: bool, keepdim: bool):
    """[(aten overload path, value name, argument template, kwargs)] ending in the result."""
    import torch

    accumulate = torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
    steps = []
    if accumulate != dtype:
        steps.append(("_to_copy.default", "x", (_X,), {"dtype": accumulate}))
    steps += [(path, name, args, {}) for path, name, args in _LSE_STEPS]
    if log_softmax:
        steps += [(path, name, args, {}) for path, name, args in _LOG_SOFTMAX_TAIL]
    elif not keepdim:
        steps.append(("squeeze.dim", "squeezed", (_Ref("lse"), _DIM), {}))
    if output_dtype != accumulate:
        steps.append(("_to_copy.default", "out", (_Ref(steps[-1][1]),), {"dtype": output_dtype}))
    return steps


def _aten(path: str):
    import torch

    op = torch.ops.aten
    for part in path.split("."):
        op = getattr(op, part)
    return op


def _play(steps, env, apply):
    """Run `steps` over env (which holds x and dim); apply(op, args, kwargs, name) gives each
    step's value.  Returns env with every step's value under its name."""
    for path, name, template, kwargs in steps:
        env[name] = apply(_aten(path), _bind(template, env), kwargs, name)
    return env


def _value(node):
    meta = getattr(node, "meta", {})
    held = meta.get("val")
    return meta.get("example_value") if held is None else held


def _is_fake_or_meta(value) -> bool:
    return type(value).__name__ == "FakeTensor" or bool(getattr(value, "is_meta", False))


def _as_metadata(value):
    """value itself when it is Fake/meta; otherwise an empty meta tensor of its layout."""
    import torch

    if _is_fake_or_meta(value):
        return value
    return torch.empty_strided(value.shape, value.stride(), dtype=value.dtype, device="meta")


def _metadata_only(value) -> bool:
    """Lowering computes metadata with torch: it accepts Fake/meta values, and real values
    only as tiny CPU examples (never GPU work in this pass)."""
    if value is None:
        return False
    if _is_fake_or_meta(value):
        return True
    if getattr(getattr(value, "device", None), "type", None) != "cpu":
        return False
    numel = getattr(value, "numel", None)
    return callable(numel) and numel() <= 4096


@dataclasses.dataclass
class _Compound:
    """One lowerable call: what the expansion needs to know about it."""

    node: object
    x: object
    dim: int
    keepdim: bool
    log_softmax: bool
    cast_to: object          # log_softmax(x, dim, dtype): the dtype x converts to first
    source: object           # metadata of x
    output: object           # metadata of the call's result


def is_compound(node) -> bool:
    return node.op == "call_function" and str(node.target) in _COMPOUNDS


def is_log_softmax(node) -> bool:
    return is_compound(node) and _COMPOUNDS[str(node.target)]


def _schema_name(node) -> str:
    return str(node.target).split(".")[1]


def _argument(node, name, position, default=None):
    if name in node.kwargs:
        return node.kwargs[name]
    return node.args[position] if len(node.args) > position else default


def _describe(node):
    """The _Compound for node, or None when it is not one this pass lowers."""
    import torch

    if not is_compound(node):
        return None
    schema = _schema_name(node)
    if schema == "_log_softmax" and _argument(node, "half_to_float", 2, False) is not False:
        return None
    floats = (torch.float32, torch.float16, torch.bfloat16)
    x = _argument(node, "self", 0)
    source, output = _value(x), _value(node)
    if getattr(source, "dtype", None) not in floats or getattr(output, "dtype", None) not in floats:
        return None
    if not _metadata_only(source):
        return None
    rank = len(source.shape)
    dim = _argument(node, "dim", 1)
    if schema == "logsumexp" and isinstance(dim, (tuple, list)):
        dim = dim[0] if len(dim) == 1 else None
    if type(dim) is not int or rank < 1 or dim not in (-1, rank - 1):
        return None
    width = source.shape[-1]
    if type(width) is int and width <= 0:
        return None
    log_softmax = is_log_softmax(node)
    keepdim = True if log_softmax else _argument(node, "keepdim", 2, False)
    if type(keepdim) is not bool:
        return None
    cast_to = _argument(node, "dtype", 2) if schema == "log_softmax" else None
    if (cast_to or source.dtype) not in floats or output.dtype != (cast_to or source.dtype):
        return None
    return _Compound(node, x, dim, keepdim, log_softmax, cast_to, source, output)


def _expand(gm, node) -> bool:
    """Replace node by its expansion in gm's graph; False (and no edit) when it does not lower
    or the expansion's metadata would not reproduce the node's output shape."""
    call = _describe(node)
    if call is None:
        return False
    fake_x = call.source
    if call.cast_to is not None:
        with getattr(call.source, "fake_mode", None) or nullcontext():
            fake_x = _aten("_to_copy.default")(_as_metadata(call.source), dtype=call.cast_to)
    steps = _program(fake_x.dtype, call.output.dtype, log_softmax=call.log_softmax,
                     keepdim=call.keepdim)
    start = _as_metadata(fake_x)
    with getattr(start, "fake_mode", None) or nullcontext():
        fake = _play(steps, {"x": start, "dim": call.dim}, lambda op, args, kw, name: op(*args, **kw))
    result = steps[-1][1]
    if [str(size) for size in fake[result].shape] != [str(size) for size in call.output.shape]:
        return False
    graph = gm.graph

    def emit(op, args, kwargs, name):
        created = graph.call_function(op, args=args, kwargs=kwargs)
        created.meta.update({"val": fake[name], MARK: node.name})
        return created

    with graph.inserting_before(node):
        env = {"x": call.x, "dim": call.dim}
        if call.cast_to is not None:
            env["x"] = graph.call_function(_aten("_to_copy.default"), args=(call.x,),
                                           kwargs={"dtype": call.cast_to})
            env["x"].meta.update({"val": fake_x, MARK: node.name})
        _play(steps, env, emit)
    node.replace_all_uses_with(env[result])
    graph.erase_node(node)
    return True


def fork_graph(gm):
    """A GraphModule with a private copy of gm's graph; parameters and buffers are shared."""
    import torch.fx as fx

    return fx.GraphModule(gm, copy.deepcopy(gm.graph))


def install(gm, trial) -> None:
    """gm takes trial's (already compiled) graph.  Should gm's recompile fail, gm gets its
    previous graph (and code) back and the error propagates."""
    previous = gm.graph
    try:
        gm.graph = trial.graph
    except Exception:
        trial.graph.owning_module = trial
        gm.graph = previous
        raise


def _names(gm, nodes):
    if nodes is None:
        return {n.name for n in gm.graph.nodes if is_compound(n)}
    if isinstance(nodes, str) or hasattr(nodes, "op"):
        nodes = (nodes,)
    return {n if isinstance(n, str) else n.name for n in nodes}


def lower_compound(gm, nodes=None) -> int:
    """Expand every supported compound node of gm, or those given (nodes or names), in place.
    No benefit gate.  Returns how many were expanded; on any failure gm is untouched and 0 is
    returned."""
    wanted = _names(gm, nodes)
    if not wanted:
        return 0
    try:
        trial = fork_graph(gm)
        count = 0
        for node in list(trial.graph.nodes):
            if node.name in wanted and _expand(trial, node):
                count += 1
        if count:
            trial.graph.lint()
            trial.recompile()
            install(gm, trial)
        return count
    except Exception:  # noqa: BLE001 -- an unsupported trial never changes the caller's graph
        return 0


def grew_eligible_region(gm, name, values=None) -> bool:
    """True when gm (after lowering compound node `name`) holds an eligible region rooted in
    and built from that node's expansion, and `rewrite` would fuse a region of gm."""
    from neptune_recognize.match import recognize_regions
    from neptune_recognize.rewrite import region_contract, would_rewrite

    matches, _ = recognize_regions(gm, values)
    own = [m for m in matches if m.region_root.meta.get(MARK) == name
           and any(n.meta.get(MARK) == name for n in m.region_nodes)]
    return any(region_contract(m)[1] is None for m in own) and would_rewrite(gm, values)[0]


def lower_if_it_helps(gm, values=None) -> int:
    """Lower each compound node only when its own expansion becomes an eligible region (another
    region of the graph cannot vouch for it).  No kernel generation and no dead-code removal.
    Returns how many nodes were lowered."""
    lowered = 0
    for name in [n.name for n in gm.graph.nodes if is_compound(n)]:
        try:
            trial = fork_graph(gm)
            if lower_compound(trial, nodes=name) and grew_eligible_region(trial, name, values):
                install(gm, trial)
                lowered += 1
        except Exception:  # noqa: BLE001 -- each node is its own transaction
            continue
    return lowered
