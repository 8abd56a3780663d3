"""Targeted lowering of compound ATen ops into the decomposed form recognition reads.

`aten.logsumexp` and (opt-in) `aten.log_softmax` / `aten._log_softmax` over the last dimension
are expanded into explicit fp32 steps: an optional cast to fp32, the amax with torch's infinity
guard, exp/sum/log and the add that ends the LSE region; log_softmax adds the readout
x - LSE with NaN on rows whose LSE is +inf (torch's row classification), and the final cast.
Nothing else is decomposed.  The step list, the node metadata mark `neptune_lowering` and the
transactional commit follow the reference (neptune_recognize/lowering.py:1-282), because
apply() pairs each lowered node with the region recognised from it.
"""
from __future__ import annotations

import copy
from contextlib import nullcontext

_COMPOUND = ("aten._log_softmax.default", "aten.log_softmax.int", "aten.log_softmax.default",
             "aten.logsumexp.default")


def _name_of(target) -> str:
    text = str(target)
    return text[len("aten."):].split(".")[0] if text.startswith("aten.") else text.split(".")[0]


def _is_compound(node) -> bool:
    return node.op == "call_function" and str(node.target) in _COMPOUND


def _value(node):
    meta = getattr(node, "meta", {})
    value = meta.get("val")
    return meta.get("example_value") if value is None else value


def _arg(node, name, position, default=None):
    return node.kwargs.get(name, node.args[position] if len(node.args) > position else default)


def _aten(path: str):
    import torch

    op = torch.ops.aten
    for part in path.split("."):
        op = getattr(op, part)
    return op


def _steps(dtype, output_dtype, *, log_softmax: bool, keepdim: bool):
    """[(aten overload path, name, args(env), kwargs)], result name.  Accumulation is fp32 for
    16-bit inputs; casts stay explicit region boundaries."""
    import torch

    acc = torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
    steps = []
    if dtype != acc:
        steps.append(("_to_copy.default", "x", lambda e: (e["x"],), {"dtype": acc}))
    steps += [
        ("amax.default", "m", lambda e: (e["x"], [e["dim"]], True), {}),
        ("abs.default", "abs_m", lambda e: (e["m"],), {}),
        ("eq.Scalar", "infinite", lambda e: (e["abs_m"], float("inf")), {}),
        ("where.ScalarSelf", "m_safe", lambda e: (e["infinite"], 0.0, e["m"]), {}),
        ("sub.Tensor", "centred", lambda e: (e["x"], e["m_safe"]), {}),
        ("exp.default", "e", lambda e: (e["centred"],), {}),
        ("sum.dim_IntList", "s", lambda e: (e["e"], [e["dim"]], True), {}),
        ("log.default", "lg", lambda e: (e["s"],), {}),
        ("add.Tensor", "lse", lambda e: (e["m_safe"], e["lg"]), {}),
    ]
    result = "lse"
    if log_softmax:
        steps += [
            ("eq.Scalar", "posinf_row", lambda e: (e["lse"], float("inf")), {}),
            ("sub.Tensor", "readout", lambda e: (e["x"], e["lse"]), {}),
            ("where.ScalarSelf", "log_out", lambda e: (e["posinf_row"], float("nan"), e["readout"]), {}),
        ]
        result = "log_out"
    elif not keepdim:
        steps.append(("squeeze.dim", "squeezed", lambda e: (e["lse"], e["dim"]), {}))
        result = "squeezed"
    if output_dtype != acc:
        steps.append(("_to_copy.default", "out", lambda e, key=result: (e[key],), {"dtype": output_dtype}))
        result = "out"
    return steps, result


def _fake_run(value, dim, *, output_dtype, log_softmax, keepdim) -> dict:
    """Metadata of every step, computed by torch on Fake/meta tensors (no real arithmetic)."""
    import torch

    if type(value).__name__ != "FakeTensor" and not value.is_meta:
        value = torch.empty_strided(value.shape, value.stride(), dtype=value.dtype, device="meta")
    steps, result = _steps(value.dtype, output_dtype, log_softmax=log_softmax, keepdim=keepdim)
    env = {"x": value, "dim": dim}
    with getattr(value, "fake_mode", None) or nullcontext():
        for path, name, build, kwargs in steps:
            env[name] = _aten(path)(*build(env), **kwargs)
    env["out"] = env[result]
    return env


def _simulatable(value) -> bool:
    """Fake/meta metadata, or a tiny real CPU example; never GPU work."""
    if value is None:
        return False
    if type(value).__name__ == "FakeTensor" or getattr(value, "is_meta", False):
        return True
    if getattr(getattr(value, "device", None), "type", None) != "cpu":
        return False
    numel = getattr(value, "numel", None)
    return callable(numel) and numel() <= 4096


def _trial_graph(gm):
    import torch.fx as fx

    return fx.GraphModule(gm, copy.deepcopy(gm.graph))


def _commit(gm, trial):
    """Install trial's graph into gm; a failing recompile restores gm exactly."""
    saved = gm.__dict__.copy()
    cls = type(gm)
    generated = {key: cls.__dict__.get(key) for key in ("forward", "_wrapped_call")}
    try:
        gm.graph = trial.graph
    except Exception:
        gm.__dict__.clear()
        gm.__dict__.update(saved)
        gm.graph.owning_module = gm
        trial.graph.owning_module = trial
        for key, value in generated.items():
            if value is not None:
                setattr(cls, key, value)
            elif key in cls.__dict__:
                delattr(cls, key)
        raise


def _expand_node(gm, node) -> bool:
    import torch

    if not _is_compound(node):
        return False
    is_log = _name_of(node.target) in ("_log_softmax", "log_softmax")
    if _name_of(node.target) == "_log_softmax" and _arg(node, "half_to_float", 2, False) is not False:
        return False
    x = _arg(node, "self", 0)
    source, output = _value(x), _value(node)
    allowed = (torch.float32, torch.float16, torch.bfloat16)
    if (source is None or output is None or getattr(source, "dtype", None) not in allowed
            or getattr(output, "dtype", None) not in allowed or not _simulatable(source)):
        return False
    rank = len(source.shape)
    dim = _arg(node, "dim", 1)
    if _name_of(node.target) == "logsumexp" and isinstance(dim, (tuple, list)):
        dim = dim[0] if len(dim) == 1 else None
    if type(dim) is not int or rank < 1 or dim not in (-1, rank - 1):
        return False
    if type(source.shape[-1]) is int and source.shape[-1] <= 0:
        return False
    keepdim = True if is_log else _arg(node, "keepdim", 2, False)
    if type(keepdim) is not bool:
        return False
    # log_softmax(x, dim, dtype) converts before any arithmetic
    requested = _arg(node, "dtype", 2) if _name_of(node.target) == "log_softmax" else None
    effective = requested or source.dtype
    if effective not in allowed or output.dtype != effective:
        return False
    fake_source = source
    if requested is not None:
        with getattr(source, "fake_mode", None) or nullcontext():
            if type(source).__name__ != "FakeTensor" and not source.is_meta:
                fake_source = torch.empty_strided(source.shape, source.stride(), dtype=source.dtype,
                                                  device="meta")
            fake_source = _aten("_to_copy.default")(fake_source, dtype=requested)
    fake = _fake_run(fake_source, dim, output_dtype=output.dtype, log_softmax=is_log, keepdim=keepdim)
    if tuple(map(str, fake["out"].shape)) != tuple(map(str, output.shape)):
        return False
    steps, result = _steps(effective, output.dtype, log_softmax=is_log, keepdim=keepdim)
    graph = gm.graph
    with graph.inserting_before(node):
        env = {"x": x, "dim": dim}
        if requested is not None:
            cast = graph.call_function(_aten("_to_copy.default"), args=(x,), kwargs={"dtype": requested})
            cast.meta.update(val=fake_source, neptune_lowering=node.name)
            env["x"] = cast
        for path, name, build, kwargs in steps:
            call = graph.call_function(_aten(path), args=build(env), kwargs=kwargs)
            call.meta.update(val=fake[name], neptune_lowering=node.name)
            env[name] = call
    node.replace_all_uses_with(env[result])
    graph.erase_node(node)
    return True


def lower_compound(gm, nodes=None) -> int:
    """Expand the supported compound nodes (all, or the given nodes / names) in place.
    Returns how many were expanded; on any failure `gm` is left untouched and 0 returned."""
    if nodes is None:
        names = {n.name for n in gm.graph.nodes if _is_compound(n)}
    elif isinstance(nodes, str) or hasattr(nodes, "op"):
        names = {nodes if isinstance(nodes, str) else nodes.name}
    else:
        names = {n if isinstance(n, str) else n.name for n in nodes}
    if not names:
        return 0
    try:
        trial = _trial_graph(gm)
        count = sum(_expand_node(trial, n) for n in list(trial.graph.nodes) if n.name in names)
        if not count:
            return 0
        trial.graph.lint()
        trial.recompile()
        _commit(gm, trial)
        return count
    except Exception:  # noqa: BLE001 -- an unsupported trial never mutates the caller
        return 0


def lower_if_it_helps(gm, values=None) -> int:
    """Lower each compound node only when its own expansion becomes an eligible region."""
    from neptune_recognize.match import recognize_regions
    from neptune_recognize.rewrite import region_contract, would_rewrite

    lowered = 0
    for name in [n.name for n in gm.graph.nodes if _is_compound(n)]:
        try:
            trial = _trial_graph(gm)
            if not lower_compound(trial, nodes=name):
                continue
            matches, _ = recognize_regions(trial, values)
            eligible = any(
                m.region_root.meta.get("neptune_lowering") == name
                and any(n.meta.get("neptune_lowering") == name for n in m.region_nodes)
                and region_contract(m)[1] is None for m in matches)
            if not eligible or not would_rewrite(trial, values)[0]:
                continue
            _commit(gm, trial)
            lowered += 1
        except Exception:  # noqa: BLE001 -- each node is its own transaction
            continue
    return lowered
