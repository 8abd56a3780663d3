"""Turning a recognised region into one fused HIP op call, leaving the dataflow around it as is.

Two stages:

* the region *contract* -- ordered checks over the metadata of the region's boundary values
  (dtypes, ranks, exact output shape, the structured ops' argument ABI).  The first failing
  check names the refusal; the refusal texts are the reference's
  (neptune_recognize/rewrite.py:52-146), since callers and reports match on them;
* the *splice* -- a new call node takes the region root's place, the root's users are
  redirected, the rename is written to the ledger (neptune_recognize/ledger.py), and only the
  region's own dead, pure nodes are erased.  Two follow-up edits fold more of the graph into
  the call: a log-softmax tail (x - lse, with NaN on +inf rows) becomes one readout op, and a
  widen/narrow cast pair around a fold on a 16-bit input becomes a fold reading that input.
"""
from __future__ import annotations

import copy
import math

import neptune_codegen as CG
from neptune_recognize import ledger
from neptune_recognize.interp import _same_shape, _tensor_value
from neptune_recognize.match import recognize_regions

_FLOATS = None


def _float_dtypes():
    global _FLOATS
    if _FLOATS is None:
        import torch

        _FLOATS = (torch.float32, torch.float16, torch.bfloat16)
    return _FLOATS


def _has_shape(value) -> bool:
    return value is not None and hasattr(value, "shape")


def _static_width_is_empty(value) -> bool:
    width = value.shape[-1]
    return type(width) is int and width <= 0


def _first_refusal(checks, *values):
    for check in checks:
        reason = check(*values)
        if reason:
            return reason
    return None


# ---------------------------------------------------------------- scalar fold regions
def _reduction_keepdim(source, output):
    """False when output is source reduced over its last dim, True when that dim is kept as
    size 1, None otherwise."""
    if not (_has_shape(source) and _has_shape(output)):
        return None
    rows = tuple(source.shape[:-1])
    for keep, shape in ((False, rows), (True, rows + (1,))):
        if _same_shape(output.shape, shape):
            return keep
    return None


def _wants_keepdim(node, input_node=None):
    """keepdim of a region root reading input_node (see _reduction_keepdim); without the input
    boundary, the older rank-only answer."""
    output = _tensor_value(node)
    if input_node is None:
        return len(output.shape) >= 2 if _has_shape(output) else None
    return _reduction_keepdim(_tensor_value(input_node), output)


def _fp32_only(source, output):
    # a hand-written 16-bit chain rounds after every op; dropping those roundings is not an
    # identity, so only the compound lowering (explicit fp32 steps) may fuse 16-bit inputs
    import torch

    if source.dtype != torch.float32:
        return "low-precision intermediate rounding needs explicit fp32 lowering"
    return None


_SCALAR_CHECKS = (
    lambda s, o: None if _has_shape(s) else "region input metadata is unknown",
    lambda s, o: None if _has_shape(o) else "operator output rank is unknown",
    lambda s, o: None if s.dtype in _float_dtypes() else f"unsupported region dtype {s.dtype}",
    lambda s, o: (None if o.dtype == s.dtype
                  else "output dtype differs from the region input; preserve the cast boundary"),
    _fp32_only,
    lambda s, o: None if len(s.shape) >= 1 else "row-reduction input must have rank >= 1",
    lambda s, o: "empty row width is unsupported" if _static_width_is_empty(s) else None,
    lambda s, o: (None if _reduction_keepdim(s, o) is not None
                  else "operator output shape is not the input's last-dimension reduction"),
)


# ---------------------------------------------------------------- structured regions
def _canonical_metadata(value):
    """Fresh contiguous Fake metadata of value's shape/dtype/device (nothing is allocated)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

    if isinstance(value, FakeTensor) or value.device.type == "meta":
        return value.new_empty(value.shape)
    with FakeTensorMode():
        return torch.empty(value.shape, device=value.device, dtype=value.dtype)


def _finite_number(value) -> bool:
    return type(value) in (int, float) and math.isfinite(value)


_STRUCTURED_COMMON = (
    lambda m, s, a, o: (None if all(v.layout == _strided() for v in (s, a, o))
                        else "structured operation requires strided tensor layout"),
    lambda m, s, a, o: (None if a.device == s.device and o.device == s.device
                        else "structured inputs and output must share a device"),
    lambda m, s, a, o: None if s.device.type in ("cpu", "cuda") else "unsupported structured device",
    lambda m, s, a, o: None if s.dtype in _float_dtypes() else f"unsupported structured dtype {s.dtype}",
    lambda m, s, a, o: None if o.dtype == s.dtype else "structured output dtype differs from input",
    lambda m, s, a, o: None if len(s.shape) >= 1 else "structured input must have rank >= 1",
    # the HIP ops return fresh contiguous outputs; a consumer that relied on another layout
    # would see different strides
    lambda m, s, a, o: (None if _same_shape(o.stride(), _canonical_metadata(o).stride())
                        else "structured output layout must be canonical contiguous"),
)

_RMS_CHECKS = (
    lambda m, s, a, o: (None if _finite_number(m.params.get("eps")) and m.params["eps"] > 0
                        else "RMSNorm requires finite positive eps"),
    lambda m, s, a, o: "RMSNorm requires nonempty row width" if _static_width_is_empty(s) else None,
    lambda m, s, a, o: (None if a.dtype == s.dtype and len(a.shape) == 1
                        else "RMSNorm gamma must be a same-dtype 1D vector"),
    lambda m, s, a, o: (None if _same_shape(a.shape, s.shape[-1:])
                        else "RMSNorm gamma width differs from input"),
    lambda m, s, a, o: (None if _same_shape(o.shape, s.shape)
                        else "RMSNorm output shape must exactly equal input shape"),
)


def _segment_count(m, a):
    return a.shape[0] - int(m.params["offsets"])


_SEGMENT_CHECKS = (
    lambda m, s, a, o: (None if a.dtype in _index_dtypes() and len(a.shape) == 1
                        else "segment lengths/offsets must be a 1D int32/int64 tensor"),
    lambda m, s, a, o: (None if type(m.params.get("offsets")) is bool and type(m.params.get("unsafe")) is bool
                        else "segment offsets/unsafe parameters must be explicit bools"),
    lambda m, s, a, o: (None if m.params.get("initial") is None or _finite_number(m.params["initial"])
                        else "segment initial must be None or a finite scalar"),
    lambda m, s, a, o: ("segment offsets must contain at least one entry"
                        if type(_segment_count(m, a)) is int and _segment_count(m, a) < 0 else None),
    lambda m, s, a, o: (None if _same_shape(o.shape, (_segment_count(m, a), *s.shape[1:]))
                        else "segment output shape differs from axis-0 segment contour"),
)

# (operation, accepted skeletons, checks)
_STRUCTURED_OPERATIONS = (
    ("rms_norm", ("rms_norm",), _RMS_CHECKS),
    ("segment_pool", ("segment_sum", "segment_mean"), _SEGMENT_CHECKS),
)


def _strided():
    import torch

    return torch.strided


def _index_dtypes():
    import torch

    return (torch.int32, torch.int64)


def _structured_values(match):
    """(source, auxiliary, output) metadata; a lifted get_attr input without metadata takes the
    value recognition resolved for it."""
    held = getattr(match, "metadata", {}).get("boundary_values", ())
    values = []
    for position, node in enumerate(match.input_nodes):
        value = _tensor_value(node)
        if value is None and node.op == "get_attr" and position < len(held):
            value = held[position]
        values.append(value)
    return (*values, _tensor_value(match.region_root))


def _structured_refusal(match):
    if len(match.input_nodes) != 2 or match.input_node is not match.input_nodes[0]:
        return "structured operation requires two ordered input boundaries"
    values = _structured_values(match)
    if not all(_has_shape(v) for v in values):
        return "structured input/output metadata is unknown"
    reason = _first_refusal(_STRUCTURED_COMMON, match, *values)
    if reason:
        return reason
    for operation, skeletons, checks in _STRUCTURED_OPERATIONS:
        if match.operation == operation and match.skeleton in skeletons:
            return _first_refusal(checks, match, *values)
    return "unsupported structured operation/skeleton"


def region_contract(match):
    """(keepdim, None) when the region may become a fused op, (None, reason) otherwise.  For a
    structured region keepdim is always False."""
    if getattr(match, "kind", "scalar") == "structured":
        reason = _structured_refusal(match)
        return (None, reason) if reason else (False, None)
    source, output = _tensor_value(match.input_node), _tensor_value(match.region_root)
    reason = _first_refusal(_SCALAR_CHECKS, source, output)
    if reason:
        return None, reason
    return _reduction_keepdim(source, output), None


def _first_eligible(gm, values=None):
    """(match, None) for the first region recognition finds eligible, else (first match or
    None, the last refusal or recognition's reason)."""
    matches, reason = recognize_regions(gm, values)
    for match in matches:
        refusal = region_contract(match)[1]
        if refusal is None:
            return match, None
        reason = refusal
    return (matches[0] if matches else None), reason


def would_rewrite(gm, values=None):
    """(True, skeleton) when `rewrite` would fuse a region of gm, else (False, reason)."""
    match, reason = _first_eligible(gm, values)
    return (False, reason) if reason is not None else (True, match.skeleton)


# ---------------------------------------------------------------- fused op selection
def _launch_config(node):
    """(BLOCK, num_warps) from the MI355X launch table for the region input's shape."""
    value = _tensor_value(node)
    if not _has_shape(value) or not value.shape:
        return None, None
    rows = math.prod(value.shape[:-1])
    return CG.autotune.best_config(rows, value.shape[-1], value.dtype, value.device)


def _fold_op(skeleton, params, source, keepdim, lib, plan):
    """The scalar fold op for `source` (a node), with the launch shape of its own dtype."""
    block, warps = _launch_config(source)
    if plan == "split":
        block, warps = 1024, 4
    return CG.op_handle(skeleton, params={**CG.param_defaults(skeleton), **params}, lib=lib,
                        keepdim=keepdim, block=block, num_warps=warps, plan=plan)


def _structured_op(gm, match, lib, plan):
    """The structured op for a match.  The real operator ABI is validated on metadata first,
    so a refusal raises here, before the graph is touched."""
    from neptune_recognize.match import _structured_boundary_value

    values = [_structured_boundary_value(gm, node) for node in match.input_nodes]
    if match.operation == "rms_norm":
        from neptune_codegen.template import validate_rms_inputs

        validate_rms_inputs(*values, match.params, plan=plan, metadata=True)
    else:
        from neptune_codegen.torch_op import validate_segment_inputs

        validate_segment_inputs(*values, reduce=match.skeleton.removeprefix("segment_"), plan=plan,
                                metadata=True, **match.params)
    return CG.state_op_handle(match.skeleton, params=match.params, plan=plan, lib=lib)


# ---------------------------------------------------------------- graph edits
def _is_metadata_assert(node) -> bool:
    import torch

    return (node.op == "call_function" and not node.users
            and node.target is torch.ops.aten._assert_tensor_metadata.default)


def _value_users(node):
    """Users of node other than export's metadata asserts."""
    return [u for u in node.users if not _is_metadata_assert(u)]


def _drop_asserts_on(graph, node):
    for check in [u for u in node.users if _is_metadata_assert(u)]:
        graph.erase_node(check)


class _Splice:
    """Edits of one graph: a new call takes over from an anchor node, renames go to the
    ledger, and replaced or dead nodes are erased."""

    def __init__(self, gm):
        self.gm, self.graph = gm, gm.graph

    def take_over(self, anchor, op, args, *, meta=None):
        with self.graph.inserting_before(anchor):
            node = self.graph.call_function(op, args=tuple(args))
        node.meta = copy.copy(anchor.meta if meta is None else meta)
        ledger.record(self.gm, anchor.name, node.name)
        anchor.replace_all_uses_with(node)
        self.graph.erase_node(anchor)
        return node

    def retire(self, old, new):
        """`old` (already without value users) is gone; `new` stands for it."""
        ledger.record(self.gm, old.name, new.name)
        _drop_asserts_on(self.graph, old)
        self.graph.erase_node(old)

    def erase(self, *nodes):
        for node in nodes:
            _drop_asserts_on(self.graph, node)
            self.graph.erase_node(node)

    def prune_region(self, nodes, root):
        """Erase the region's nodes that nothing reads any more, newest first.  Side effects
        and shared values stay; an export metadata assert whose only subject is such a node
        goes with it (the value it checked is no longer computed)."""
        for node in reversed(nodes):
            if node is root or node.op in ("placeholder", "output", "get_attr"):
                continue
            if node.users and not _value_users(node):
                _drop_asserts_on(self.graph, node)
            if not node.users and not node.is_impure():
                self.graph.erase_node(node)


def _set_structured_metadata(call, root):
    value = _canonical_metadata(_tensor_value(root))
    call.meta["val"] = value
    if "example_value" in call.meta:
        call.meta["example_value"] = value
    if "tensor_meta" in call.meta:
        from torch.fx.passes.shape_prop import _extract_tensor_metadata

        call.meta["tensor_meta"] = _extract_tensor_metadata(value)


def rewrite_match(gm, match, *, lib="neptune", plan="serial"):
    """Replace one region of gm by its fused op.  gm is a candidate graph: the caller owns the
    transaction.  Returns (call node, None), or (None, reason) when the contract refuses (an
    operator ABI refusal raises before any edit)."""
    keepdim, reason = region_contract(match)
    if reason is not None:
        return None, reason
    structured = getattr(match, "kind", "scalar") == "structured"
    if structured:
        op, args = _structured_op(gm, match, lib, plan), match.input_nodes
    else:
        if plan == "split":
            CG.split_launch_shape(_tensor_value(match.input_node).shape[-1], 1024)
        op = _fold_op(match.skeleton, match.params, match.input_node, keepdim, lib, plan)
        args = (match.input_node,)
    splice = _Splice(gm)
    root = match.region_root
    call = splice.take_over(root, op, args)
    if structured:
        _set_structured_metadata(call, root)
    splice.prune_region(match.region_nodes, root)
    if not structured:
        call = _fuse_log_softmax_tail(splice, call, match, keepdim, lib, plan) or \
            _absorb_cast_pair(splice, call, match, keepdim, lib, plan) or call
    gm.graph.lint()
    gm.recompile()
    return call, None


def _dtype_cast(node, source=None):
    """The target dtype when node is a pure dtype conversion (aten._to_copy with dtype= only,
    or aten.to.dtype with default flags) of `source` (any source when None), else None."""
    import torch

    if node.op != "call_function":
        return None
    if node.target is torch.ops.aten._to_copy.default:
        if len(node.args) != 1 or set(node.kwargs) != {"dtype"}:
            return None
        dtype = node.kwargs["dtype"]
    elif node.target is torch.ops.aten.to.dtype:
        flags = ("non_blocking", "copy", "memory_format")
        if len(node.args) != 2 or set(node.kwargs) - set(flags):
            return None
        if any(node.kwargs.get(flag) not in (None, False) for flag in flags):
            return None
        dtype = node.args[1]
    else:
        return None
    return dtype if source is None or node.args[0] is source else None


def _narrowed_source(widened, tail):
    """When `widened` is an fp32 widening of a 16-bit node x and `tail`'s only value user
    narrows it back to x's dtype: (x, that narrowing node); else None."""
    import torch

    if _dtype_cast(widened) is not torch.float32:
        return None
    source = widened.args[0]
    value = _tensor_value(source)
    if value is None or value.dtype not in (torch.bfloat16, torch.float16):
        return None
    users = _value_users(tail)
    if len(users) != 1 or _dtype_cast(users[0], tail) is not value.dtype:
        return None
    return source, users[0]


def _match_log_softmax_tail(call):
    """The nodes of `x - lse` or `where(lse == inf, nan, x - lse)` reading the fold `call`
    (the readout steps of the compound lowering), as (last node, nodes to remove, NaN rows);
    None when the fold has any other reader."""
    import torch

    aten = torch.ops.aten
    x = call.args[0]
    readers = _value_users(call)
    subs = [u for u in readers if u.target is aten.sub.Tensor and u.args == (x, call) and not u.kwargs]
    if len(subs) != 1:
        return None
    sub = subs[0]
    if len(readers) == 1:
        return sub, [sub], False
    if len(readers) != 2:
        return None
    eq = readers[0] if readers[1] is sub else readers[1]
    if eq.target is not aten.eq.Scalar or eq.args != (call, math.inf) or eq.kwargs:
        return None
    selects = list(sub.users)
    if len(selects) != 1 or list(eq.users) != selects:
        return None
    select = selects[0]
    if select.target is not aten.where.ScalarSelf or select.kwargs or len(select.args) != 3:
        return None
    cond, fill, other = select.args
    if cond is not eq or other is not sub or not (isinstance(fill, float) and math.isnan(fill)):
        return None
    return select, [select, sub, eq], True


def _fuse_log_softmax_tail(splice, call, match, keepdim, lib, plan):
    """A keepdim logsumexp fold read only by its log-softmax tail becomes one readout op over
    the row (neptune_codegen.run_readout); a 16-bit input reached through an fp32 widening,
    with the result narrowed back, is read directly.  Returns the readout node, or None."""
    params = {**CG.param_defaults(match.skeleton), **match.params}
    if match.skeleton != "logsumexp" or not keepdim or plan != "serial" or params.get("tiny", 0.0) != 0.0:
        return None
    tail = _match_log_softmax_tail(call)
    if tail is None:
        return None
    last, removed, nan_rows = tail
    x = call.args[0]
    source, anchor = x, last
    narrowing = _narrowed_source(x, last)
    if narrowing is not None:
        source, anchor = narrowing
    op = CG.readout_op_handle("logsumexp", params=params, nan_posinf_rows=nan_rows, lib=lib)
    readout = splice.take_over(anchor, op, (source,))
    if anchor is not last:
        splice.retire(last, readout)
    splice.erase(*removed[1:])          # removed[0] is `last`, gone with one of the two above
    splice.retire(call, readout)
    if source is not x and not x.users:
        splice.erase(x)
    return readout


def _absorb_cast_pair(splice, call, match, keepdim, lib, plan):
    """fold(widen(x)) read only through a narrowing back to x's 16-bit dtype becomes fold(x):
    the fold kernels widen 16-bit loads exactly, accumulate in fp32 and round once on store,
    which is the pair's arithmetic without an fp32 copy of x in HBM.  Returns the new fold
    node, or None."""
    widened = call.args[0]
    narrowing = _narrowed_source(widened, call)
    if narrowing is None:
        return None
    source, narrow = narrowing
    op = _fold_op(match.skeleton, match.params, source, keepdim, lib, plan)
    fold = splice.take_over(narrow, op, (source,))
    splice.retire(call, fold)
    if not widened.users:
        splice.erase(widened)
    return fold


def rewrite(gm, values=None, ops=None, lib="neptune", *, plan="serial"):
    """Fuse the first eligible region of gm.  The edit runs on a copy and gm takes the copy's
    graph only on success; otherwise gm is unchanged.  Returns (gm, skeleton | None, reason)."""
    trial = copy.deepcopy(gm)
    match, reason = _first_eligible(trial, values)
    if reason is None:
        call, reason = rewrite_match(trial, match, lib=lib, plan=plan)
        if call is not None:
            gm.graph = trial.graph
            gm.recompile()
            return gm, match.skeleton, "rewritten"
    return gm, None, reason
