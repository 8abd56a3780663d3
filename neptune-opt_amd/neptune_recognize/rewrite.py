"""Replacing a recognised region by one fused HIP op, without touching the dataflow around it.

The contract checks (dtype, exact output shape, structured ABI) and the rewrite semantics --
insert the op before the region root, redirect the root's users, erase only dead nodes of the
region, record root renames for the exported signature -- follow the reference's
neptune_recognize/rewrite.py:1-231, which callers and the transaction in neptune_opt rely on.
"""
from __future__ import annotations

import copy

import neptune_codegen as CG
from neptune_recognize.interp import _same_shape, _tensor_value
from neptune_recognize.match import recognize_regions


def _wants_keepdim(node, input_node=None):
    """False for [..., ] outputs, True for [..., 1], None when neither."""
    value = _tensor_value(node)
    if value is None or not hasattr(value, "shape"):
        return None
    if input_node is None:
        return len(value.shape) >= 2
    source = _tensor_value(input_node)
    if source is None or not hasattr(source, "shape"):
        return None
    if _same_shape(value.shape, source.shape[:-1]):
        return False
    if _same_shape(value.shape, source.shape[:-1] + (1,)):
        return True
    return None


def _launch_config(node):
    """(BLOCK, num_warps) from the MI355X launch table for the region input's shape."""
    value = _tensor_value(node)
    if value is None or not hasattr(value, "shape") or not value.shape:
        return None, None
    rows = 1
    for size in value.shape[:-1]:
        rows *= size
    return CG.autotune.best_config(rows, value.shape[-1], value.dtype, value.device)


def _canonical_metadata(value):
    """A fresh contiguous Fake tensor of value's shape/dtype/device (no real allocation)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

    if isinstance(value, FakeTensor) or value.device.type == "meta":
        return value.new_empty(value.shape)
    with FakeTensorMode():
        return torch.empty(value.shape, device=value.device, dtype=value.dtype)


def _structured_contract(match):
    """(False, None) when the structured op's ABI admits this region, else (None, reason)."""
    import math

    import torch

    if len(match.input_nodes) != 2 or match.input_node is not match.input_nodes[0]:
        return None, "structured operation requires two ordered input boundaries"
    held = getattr(match, "metadata", {}).get("boundary_values", ())
    inputs = []
    for i, node in enumerate(match.input_nodes):
        value = _tensor_value(node)
        if value is None and node.op == "get_attr" and i < len(held):
            value = held[i]
        inputs.append(value)
    values = [*inputs, _tensor_value(match.region_root)]
    if any(v is None or not hasattr(v, "shape") for v in values):
        return None, "structured input/output metadata is unknown"
    source, auxiliary, output = values
    if any(v.layout != torch.strided for v in values):
        return None, "structured operation requires strided tensor layout"
    if any(v.device != source.device for v in values):
        return None, "structured inputs and output must share a device"
    if source.device.type not in ("cpu", "cuda"):
        return None, "unsupported structured device"
    if source.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return None, f"unsupported structured dtype {source.dtype}"
    if output.dtype != source.dtype:
        return None, "structured output dtype differs from input"
    if len(source.shape) < 1:
        return None, "structured input must have rank >= 1"
    if not _same_shape(output.stride(), _canonical_metadata(output).stride()):
        return None, "structured output layout must be canonical contiguous"
    if match.operation == "rms_norm" and match.skeleton == "rms_norm":
        eps = match.params.get("eps")
        if type(eps) not in (float, int) or not math.isfinite(eps) or eps <= 0:
            return None, "RMSNorm requires finite positive eps"
        if type(source.shape[-1]) is int and source.shape[-1] <= 0:
            return None, "RMSNorm requires nonempty row width"
        if auxiliary.dtype != source.dtype or len(auxiliary.shape) != 1:
            return None, "RMSNorm gamma must be a same-dtype 1D vector"
        if not _same_shape(auxiliary.shape, source.shape[-1:]):
            return None, "RMSNorm gamma width differs from input"
        if not _same_shape(output.shape, source.shape):
            return None, "RMSNorm output shape must exactly equal input shape"
        return False, None
    if match.operation == "segment_pool" and match.skeleton in ("segment_sum", "segment_mean"):
        if auxiliary.dtype not in (torch.int32, torch.int64) or len(auxiliary.shape) != 1:
            return None, "segment lengths/offsets must be a 1D int32/int64 tensor"
        if type(match.params.get("offsets")) is not bool or type(match.params.get("unsafe")) is not bool:
            return None, "segment offsets/unsafe parameters must be explicit bools"
        initial = match.params.get("initial")
        if initial is not None and (type(initial) not in (int, float) or not math.isfinite(initial)):
            return None, "segment initial must be None or a finite scalar"
        count = auxiliary.shape[0] - int(match.params["offsets"])
        if type(count) is int and count < 0:
            return None, "segment offsets must contain at least one entry"
        if not _same_shape(output.shape, (count, *source.shape[1:])):
            return None, "segment output shape differs from axis-0 segment contour"
        return False, None
    return None, "unsupported structured operation/skeleton"


def region_contract(match):
    """(keepdim, None) when the region may become the fused op, else (None, reason)."""
    import torch

    if getattr(match, "kind", "scalar") == "structured":
        return _structured_contract(match)
    source, output = _tensor_value(match.input_node), _tensor_value(match.region_root)
    if source is None or not hasattr(source, "shape"):
        return None, "region input metadata is unknown"
    if output is None or not hasattr(output, "shape"):
        return None, "operator output rank is unknown"
    if source.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return None, f"unsupported region dtype {source.dtype}"
    if output.dtype != source.dtype:
        return None, "output dtype differs from the region input; preserve the cast boundary"
    # a hand-decomposed low-precision region rounds after every op; removing those roundings
    # needs the explicit fp32 lowering instead
    if source.dtype != torch.float32:
        return None, "low-precision intermediate rounding needs explicit fp32 lowering"
    if len(source.shape) < 1:
        return None, "row-reduction input must have rank >= 1"
    if type(source.shape[-1]) is int and source.shape[-1] <= 0:
        return None, "empty row width is unsupported"
    keepdim = _wants_keepdim(match.region_root, match.input_node)
    if keepdim is None:
        return None, "operator output shape is not the input's last-dimension reduction"
    return keepdim, None


def _locate(gm, values=None):
    matches, reason = recognize_regions(gm, values)
    for match in matches:
        keepdim, refusal = region_contract(match)
        if refusal is None:
            return match, match.region_root, keepdim, None
        reason = refusal
    return (matches[0] if matches else None), None, None, reason


def would_rewrite(gm, values=None):
    match, _, _, reason = _locate(gm, values)
    return (True, match.skeleton) if reason is None else (False, reason)


def _fused_op(gm, match, keepdim, lib, plan):
    """The op handle (and its graph inputs) for a match; ABI refusals raise here, before any
    graph mutation."""
    if getattr(match, "kind", "scalar") == "structured":
        from neptune_recognize.match import _structured_boundary_value

        inputs = match.input_nodes
        values = tuple(_structured_boundary_value(gm, node) for node in inputs)
        if match.operation == "rms_norm":
            from neptune_codegen.template import validate_rms_inputs

            validate_rms_inputs(*values, match.params, plan=plan, metadata=True)
        else:
            from neptune_codegen.torch_op import validate_segment_inputs

            validate_segment_inputs(*values, reduce=match.skeleton.removeprefix("segment_"),
                                    plan=plan, metadata=True, **match.params)
        return CG.state_op_handle(match.skeleton, params=match.params, plan=plan, lib=lib), inputs
    block, warps = _launch_config(match.input_node)
    if plan == "split":
        block, warps = 1024, 4
        CG.split_launch_shape(_tensor_value(match.input_node).shape[-1], block)
    params = {**CG.param_defaults(match.skeleton), **match.params}
    op = CG.op_handle(match.skeleton, params=params, lib=lib, keepdim=keepdim, block=block,
                      num_warps=warps, plan=plan)
    return op, (match.input_node,)


def rewrite_match(gm, match, *, lib="neptune", plan="serial"):
    """Replace one region in `gm` (a candidate graph; the caller owns the transaction).
    Returns (call node, None) or (None, reason)."""
    keepdim, reason = region_contract(match)
    if reason is not None:
        return None, reason
    op, inputs = _fused_op(gm, match, keepdim, lib, plan)
    graph, root = gm.graph, match.region_root
    with graph.inserting_before(root):
        call = graph.call_function(op, args=tuple(inputs))
    call.meta = copy.copy(root.meta)
    if getattr(match, "kind", "scalar") == "structured":
        value = _canonical_metadata(_tensor_value(root))
        call.meta["val"] = value
        if "example_value" in call.meta:
            call.meta["example_value"] = value
        if "tensor_meta" in call.meta:
            from torch.fx.passes.shape_prop import _extract_tensor_metadata

            call.meta["tensor_meta"] = _extract_tensor_metadata(value)
    renamed = copy.deepcopy(gm.meta.get("neptune_replaced_roots", {}))
    renamed[root.name] = call.name
    gm.meta["neptune_replaced_roots"] = renamed
    root.replace_all_uses_with(call)
    graph.erase_node(root)
    # only dead, pure nodes of this region go; shared values and side effects stay.  An
    # export-time metadata assert on a region-internal value is the one side effect dropped
    # with it: the value is no longer computed, so there is nothing left to check.
    for node in reversed(match.region_nodes):
        if node is root or node.op in ("placeholder", "output", "get_attr"):
            continue
        checks = [u for u in node.users if _is_metadata_assert(u)]
        if checks and len(checks) == len(node.users):
            for check in checks:
                graph.erase_node(check)
        if not node.users and not node.is_impure():
            graph.erase_node(node)
    if getattr(match, "kind", "scalar") != "structured":
        fused = _fuse_readout(gm, call, match, keepdim, lib, plan)
        call = fused if fused is not call else _absorb_casts(gm, call, match, keepdim, lib, plan)
    graph.lint()
    gm.recompile()
    return call, None


def _is_metadata_assert(node) -> bool:
    import torch

    return (node.op == "call_function" and not node.users
            and node.target is torch.ops.aten._assert_tensor_metadata.default)


def _dtype_cast(node, source=None):
    """The dtype of `node` when it is a pure dtype conversion of `source` (aten._to_copy with
    only dtype=, or aten.to.dtype with default non_blocking/copy/memory_format)."""
    import torch

    if node.op != "call_function":
        return None
    if node.target is torch.ops.aten._to_copy.default:
        if len(node.args) != 1 or set(node.kwargs) != {"dtype"}:
            return None
        dtype = node.kwargs["dtype"]
    elif node.target is torch.ops.aten.to.dtype:
        if len(node.args) != 2 or any(node.kwargs.get(k) not in (None, False)
                                      for k in ("non_blocking", "copy", "memory_format")):
            return None
        if set(node.kwargs) - {"non_blocking", "copy", "memory_format"}:
            return None
        dtype = node.args[1]
    else:
        return None
    if source is not None and node.args[0] is not source:
        return None
    return dtype


def _only_users(node, skip_checks: bool = True):
    return [u for u in node.users if not (skip_checks and _is_metadata_assert(u))]


def _fuse_readout(gm, call, match, keepdim, lib, plan):
    """lse = logsumexp fold (keepdim) read only as x - lse, optionally through
    where(lse == inf, nan, x - lse) -- the log_softmax readout of the compound lowering
    (lowering.py's readout steps) -- becomes one readout op writing the whole row
    (neptune_codegen.run_readout); a 16-bit input reached through its fp32 widening, with the
    result narrowed back, is read directly."""
    import math

    import torch

    if match.skeleton != "logsumexp" or not keepdim or plan != "serial":
        return call
    params = {**CG.param_defaults(match.skeleton), **match.params}
    if params.get("tiny", 0.0) != 0.0:
        return call
    aten = torch.ops.aten
    x = call.args[0]
    users = _only_users(call)
    sub = next((u for u in users if u.target is aten.sub.Tensor), None)
    if sub is None or sub.args != (x, call) or sub.kwargs:
        return call
    final, nan_rows, dropped = sub, False, [sub]
    if len(users) == 2:
        eq = next(u for u in users if u is not sub)
        if eq.target is not aten.eq.Scalar or eq.args != (call, math.inf) or eq.kwargs:
            return call
        where = list(sub.users)
        if (len(where) != 1 or list(eq.users) != where
                or where[0].target is not aten.where.ScalarSelf or where[0].kwargs):
            return call
        cond, fill, other = where[0].args
        if cond is not eq or other is not sub or not (isinstance(fill, float) and math.isnan(fill)):
            return call
        final, nan_rows, dropped = where[0], True, [where[0], sub, eq]
    elif len(users) != 1:
        return call
    source = x
    if _dtype_cast(x) is torch.float32:
        value = _tensor_value(x.args[0])
        narrow = list(final.users)
        if (value is not None and value.dtype in (torch.bfloat16, torch.float16)
                and len(narrow) == 1 and _dtype_cast(narrow[0], final) is value.dtype):
            source = x.args[0]
            dropped.insert(0, narrow[0])
            final = narrow[0]
    graph = gm.graph
    op = CG.readout_op_handle("logsumexp", params=params, nan_posinf_rows=nan_rows, lib=lib)
    with graph.inserting_before(final):
        fused = graph.call_function(op, args=(source,))
    fused.meta = copy.copy(final.meta)
    renamed = copy.deepcopy(gm.meta.get("neptune_replaced_roots", {}))
    for old, new in list(renamed.items()):
        if new == call.name:
            renamed[old] = fused.name
    renamed[final.name] = fused.name
    gm.meta["neptune_replaced_roots"] = renamed
    final.replace_all_uses_with(fused)
    for node in dropped:
        graph.erase_node(node)
    for check in [u for u in call.users if _is_metadata_assert(u)]:
        graph.erase_node(check)
    graph.erase_node(call)
    if source is not x and not x.users:
        graph.erase_node(x)
    return fused


def _absorb_casts(gm, call, match, keepdim, lib, plan):
    """fold(_to_copy(x, float32)) read only through _to_copy(., x.dtype), x 16-bit, becomes
    fold(x): the fold kernels widen 16-bit loads to fp32 exactly, accumulate in fp32 and round
    once to the input dtype on store -- the cast pair's arithmetic without the fp32 copy of x
    in HBM (compound lowering inserts that pair, lowering.py's accumulation casts)."""
    import torch

    widen = call.args[0]
    if _dtype_cast(widen) is not torch.float32:
        return call
    source = widen.args[0]
    value = _tensor_value(source)
    if value is None or value.dtype not in (torch.bfloat16, torch.float16):
        return call
    checks = [u for u in call.users if _is_metadata_assert(u)]
    users = [u for u in call.users if u not in checks]
    if len(users) != 1 or _dtype_cast(users[0], call) is not value.dtype:
        return call
    narrow = users[0]
    block, warps = _launch_config(source)
    if plan == "split":
        block, warps = 1024, 4
    params = {**CG.param_defaults(match.skeleton), **match.params}
    op = CG.op_handle(match.skeleton, params=params, lib=lib, keepdim=keepdim, block=block,
                      num_warps=warps, plan=plan)
    graph = gm.graph
    with graph.inserting_before(narrow):
        fused = graph.call_function(op, args=(source,))
    fused.meta = copy.copy(narrow.meta)
    renamed = copy.deepcopy(gm.meta.get("neptune_replaced_roots", {}))
    for old, new in list(renamed.items()):
        if new == call.name:
            renamed[old] = fused.name
    renamed[narrow.name] = fused.name
    gm.meta["neptune_replaced_roots"] = renamed
    narrow.replace_all_uses_with(fused)
    graph.erase_node(narrow)
    for check in checks:            # asserted the fp32 value, which is no longer computed
        graph.erase_node(check)
    graph.erase_node(call)
    if not widen.users:
        graph.erase_node(widen)
    return fused


def rewrite(gm, values=None, ops=None, lib="neptune", *, plan="serial"):
    """Rewrite the first eligible region of `gm`; on any refusal `gm` is returned unchanged.
    Returns (gm, skeleton | None, reason)."""
    trial = copy.deepcopy(gm)
    match, _, _, reason = _locate(trial, values)
    if reason is not None:
        return gm, None, reason
    call, reason = rewrite_match(trial, match, lib=lib, plan=plan)
    if call is None:
        return gm, None, reason
    gm.graph = trial.graph
    gm.recompile()
    return gm, match.skeleton, "rewritten"
