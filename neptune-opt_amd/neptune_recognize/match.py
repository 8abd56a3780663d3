"""Which registered fold does a graph region implement?  Decided by comparing algebra.

A dependent pair (phi, psi) from the interpreter is compared with every registered skeleton's
producer operand and consumer term; scalar parameters the caller did not supply are solved
from the graph; the region's end is the node whose value equals the skeleton's readout.
Structured operators (RMSNorm's staged fp32 form, torch.segment_reduce) are recognised from
their exact ATen forms.  The accepted forms and the Match fields follow the reference
(neptune_recognize/match.py:1-680), since rewrite, the report and callers read them.
"""
from __future__ import annotations

import dataclasses
import functools
import math

import sympy as sp

import neptune_codegen as CG
from neptune_codegen import c_sym, vanishes
from neptune_recognize.interp import (_IGNORED, _INTRINSIC_SYMBOLS, S_RESULT, _flatten_nodes,
                                      _op, _same_shape, _tensor_value, interpret, region_inputs)
from neptune_recognize.params import _solve_for


@dataclasses.dataclass
class Match:
    """A recognised operator with the parameter values it implies and its region."""

    input_node: object
    skeleton: str
    params: dict
    inferred: tuple = ()
    consumer_node: object = None
    consumer_sym: object = None
    producer_sym: object = None
    region_root: object = None
    region_nodes: tuple = ()
    proof_kind: str = "legacy-symbolic-or-numeric-filter"
    domain_assumptions: tuple = ()
    input_nodes: tuple = ()
    kind: str = "scalar"
    operation: str = ""
    metadata: dict = dataclasses.field(default_factory=dict)

    def __repr__(self) -> str:
        extra = f" params={self.params}"
        if self.inferred:
            extra += f" (inferred: {', '.join(self.inferred)})"
        return f"<{self.skeleton}{extra}>"


# ---------------------------------------------------------------- scalar skeleton matching
def _intrinsic_substitution(sk) -> dict:
    """Intrinsic parameters (N = ncols) become the graph's own row-length symbol."""
    return {sym: _INTRINSIC_SYMBOLS[name] for sym, name in sk.intrinsic_params
            if name in _INTRINSIC_SYMBOLS}


def _producer_pattern(sk):
    derived = CG.derived_producer_expr(sk)
    if derived is not None:
        return derived
    return c_sym if sk.producer == "signed" else sp.Abs(c_sym)


def _exact_literal(value: float) -> sp.Rational:
    return sp.Rational(repr(float(value)))


def _solve_params(sk, target, expr, solved, supplied):
    """Extend `solved` so that target == expr, one unknown at a time; None if impossible."""
    unknowns = [sym for sym, arg in sk.params if arg not in (supplied or {}) and sym not in solved]
    local = dict(solved)
    difference = sp.simplify(target.subs(local) - expr)
    for sym in unknowns:
        if not difference.has(sym):
            continue
        value = _solve_for(difference, sym)
        if value is None:
            return None
        local[sym] = value
        difference = sp.simplify(difference.subs({sym: value}))
    return local


def _readout(sk, cand):
    return sk.finalize.xreplace({CG._FINAL_ACC: cand.consumer_sym, CG._FINAL_M: cand.producer_sym})


def _find_region_root(gm, env, sk, cand, solved, supplied, *, exact=False):
    """The LAST node (topological order) whose value is the skeleton's readout of this pair;
    `l2 * 2.0` therefore ends the region at the inner multiply, never swallowing the x2."""
    target = _readout(sk, cand).subs(_intrinsic_substitution(sk)).subs(solved)
    target = target.subs({sym: _exact_literal(supplied[arg]) for sym, arg in sk.params
                          if arg in (supplied or {})})
    zero = (lambda e: sp.simplify(e) == 0) if exact else vanishes
    # a node can only equal the readout if it mentions every reduction result the readout uses
    needed = [sym for sym in (cand.consumer_sym, cand.producer_sym) if target.has(sym)]
    best = (None, None)
    for node in gm.graph.nodes:
        expr = env.get(node)
        if expr is None or not all(expr.has(sym) for sym in needed):
            continue
        local = _solve_params(sk, target, expr, solved, supplied)
        if local is not None and zero(target.subs(local) - expr):
            best = (node, local)
    return best


@functools.lru_cache(maxsize=4096)
def _solve_unknowns_cached(patterns, graph_sides, unknown):
    solved, remaining = _solve_unknowns_uncached(patterns, graph_sides, unknown)
    return tuple(solved.items()), tuple(remaining)


def _solve_unknowns(sk, patterns, graph_sides, unknown):
    """Solve unknown parameters from (pattern - graph) of phi, then psi, one at a time.
    Returns (solved, remaining); memoised on the expressions, since apply rediscovers the
    remaining regions after every rewrite."""
    solved, remaining = _solve_unknowns_cached(tuple(patterns), tuple(graph_sides), tuple(unknown))
    return dict(solved), list(remaining)


def _solve_unknowns_uncached(patterns, graph_sides, unknown):
    solved: dict = {}
    remaining = list(unknown)
    for pattern, side in zip(patterns, graph_sides):
        difference = sp.simplify(pattern.subs(solved) - side)
        progress = True
        while remaining and progress:
            progress = False
            for sym in list(remaining):
                if not difference.has(sym):
                    continue
                value = _solve_for(difference, sym)
                if value is None:
                    continue
                solved[sym] = value
                remaining.remove(sym)
                difference = sp.simplify(difference.subs({sym: value}))
                progress = True
                break
    return solved, remaining


def _match_candidate(gm, input_node, cand, values, env, *, exact=False):
    """(Match, "matched") for the first fitting skeleton, or (None, reason)."""
    zero = (lambda e: sp.simplify(e) == 0) if exact else vanishes
    tried, fits = [], []
    order = sorted(CG.SKELETONS.items(), key=lambda item: (len(item[1].params), item[0]))
    for name, sk in order:
        if name in CG.NEGATIVE_CONTROLS:
            continue
        if (sk.producer_reducer, sk.consumer_reducer) != (cand.prod_kind, cand.cons_kind):
            tried.append(f"{name}(reducer {cand.prod_kind}/{cand.cons_kind})")
            continue
        supplied = (values or {}).get(name, {})
        intrinsic = _intrinsic_substitution(sk)
        known_args = {arg: float(supplied[arg]) for _, arg in sk.params if arg in supplied}
        known = {sym: _exact_literal(supplied[arg]) for sym, arg in sk.params if arg in supplied}
        phi_pat = _producer_pattern(sk).subs(intrinsic).subs(known)
        psi_pat = CG.term_expr(sk).xreplace({CG.s2_sym: S_RESULT}).subs(intrinsic).subs(known)
        unknown = [sym for sym, arg in sk.params if arg not in supplied and sym not in intrinsic]
        solved, remaining = _solve_unknowns(sk, (phi_pat, psi_pat), (cand.phi, cand.psi), unknown)
        if remaining:
            # a parameter of the readout only (tiny) is solved against the region root below
            relevant = [sym for sym in remaining
                        if sp.simplify(phi_pat.subs(solved) - cand.phi).has(sym)
                        or sp.simplify(psi_pat.subs(solved) - cand.psi).has(sym)]
            if relevant:
                tried.append(f"{name}(param-unsolved {relevant})")
                continue
        phi_pat, psi_pat = phi_pat.subs(solved), psi_pat.subs(solved)
        if not (zero(phi_pat - cand.phi) and zero(psi_pat - cand.psi)):
            continue
        if CG.coordinate_needs_floor(sk) != cand.producer_guarded:
            tried.append(f"{name}(producer-coordinate-contract-differs)")
            continue
        root, tail = _find_region_root(gm, env, sk, cand, solved, known_args, exact=exact)
        if root is None:
            tried.append(f"{name}(no-finalize)")
            continue
        everything = {**solved, **tail}
        merged = dict(known_args)
        merged.update({arg: float(everything[sym]) for sym, arg in sk.params if sym in everything})
        inferred = tuple(sorted(arg for sym, arg in sk.params if sym in everything))
        if exact:
            # certify the float literals the kernel will bake, not the solved exact roots
            bindings = {sym: _exact_literal(merged[arg]) for sym, arg in sk.params if arg in merged}
            if len(bindings) != len(sk.params):
                continue
            checks = (
                _producer_pattern(sk).subs(intrinsic).subs(bindings) - cand.phi,
                CG.term_expr(sk).xreplace({CG.s2_sym: S_RESULT}).subs(intrinsic).subs(bindings) - cand.psi,
                _readout(sk, cand).subs(intrinsic).subs(bindings) - env[root])
            if not all(zero(check) for check in checks):
                continue
            return Match(input_node, name, merged, inferred, cand.consumer_node, cand.consumer_sym,
                         cand.producer_sym, root), "matched"
        fits.append((len(unknown), name, merged, inferred, root))
    if fits:
        fits.sort(key=lambda fit: (fit[0], fit[1]))
        _, name, merged, inferred, root = fits[0]
        return Match(input_node, name, merged, inferred, cand.consumer_node, cand.consumer_sym,
                     cand.producer_sym, root), "matched"
    return None, "no registered skeleton matches (tried: " + ", ".join(tried) + ")"


def _region_nodes(root, anchor):
    """All nodes between the anchor and the root, or None when another tensor input (a
    placeholder or attribute) feeds the region."""
    region, stack = set(), [root]
    while stack:
        node = stack.pop()
        if node is anchor or node in region:
            continue
        if node.op in ("placeholder", "get_attr", "output"):
            return None
        region.add(node)
        stack.extend(node.all_input_nodes)
    return tuple(region)


def recognize_regions(gm, values=None):
    """([Match], reason): every certified single-boundary scalar region of the graph, largest
    per root, in graph order.  Unknown nodes are boundaries, never identities."""
    values = values or {}
    order = {node: i for i, node in enumerate(gm.graph.nodes)}
    by_root, reasons, pairs = {}, [], 0
    anchors = region_inputs(gm)
    for anchor in anchors:
        why: list = []
        info = interpret(gm, why=why, input_node=anchor, local=True)
        if info is None:
            reasons.extend(why)
            continue
        _, candidates, env = info
        pairs += len(candidates)
        for cand in candidates:
            if not cand.phi.has(c_sym) or not cand.psi.has(c_sym):
                continue
            match, reason = _match_candidate(gm, anchor, cand, values, env, exact=True)
            if match is None:
                reasons.append(reason)
                continue
            closure = _region_nodes(match.region_root, anchor)
            if closure is None:
                reasons.append("a matched region has more than one data boundary")
                continue
            if cand.producer_node not in closure or cand.consumer_node not in closure:
                continue
            source = _tensor_value(anchor)
            if source is not None and any(
                    v is not None and hasattr(v, "dtype") and v.is_floating_point()
                    and v.dtype != source.dtype for v in map(_tensor_value, closure)):
                reasons.append("mixed-dtype arithmetic remains a region boundary")
                continue
            sk = CG.SKELETONS[match.skeleton]
            try:
                if sk.two_pass:
                    assumptions = ("finite real inputs and finite reachable arithmetic", "ncols > 0")
                else:
                    params = {**CG.param_defaults(match.skeleton), **match.params}
                    assumptions = CG.derive_merge_certificate(sk, params).assumptions
            except (NotImplementedError, KeyError, ValueError) as error:
                reasons.append(str(error))
                continue
            match.region_nodes = tuple(sorted(closure, key=order.__getitem__))
            match.proof_kind = "exact-symbolic-real-algebra"
            match.domain_assumptions = tuple(assumptions)
            held = by_root.get(match.region_root)
            if held is None or len(match.region_nodes) > len(held.region_nodes):
                by_root[match.region_root] = match
    matches = sorted(by_root.values(), key=lambda m: order[m.region_root])
    if matches:
        return matches, f"matched {len(matches)} local reduction region(s)"
    detail = reasons[-1] if reasons else "no dependent reduction pair"
    compounds = sorted({str(n.target) for n in gm.graph.nodes if n.op == "call_function"
                        and str(n.target).startswith(("aten.logsumexp.", "aten.log_softmax.",
                                                      "aten._log_softmax."))})
    if compounds:
        detail += "; compound operations require targeted lowering: " + ", ".join(compounds)
    return [], (f"no certified local region: analyzed {len(anchors)} row-data boundaries, "
                f"{pairs} dependent pair(s); {detail}")


def recognize(gm, values=None):
    """(Match | None, reason) for a whole graph read from its first input (strict mode);
    parameters not given in `values` are inferred."""
    why: list = []
    info = interpret(gm, why=why)
    if info is None:
        return None, why[0] if why else "graph is not a producer/consumer reduction pair"
    anchor, candidates, env = info
    for cand in candidates:
        match, _ = _match_candidate(gm, anchor, cand, values or {}, env)
        if match is not None:
            return match, "matched"
    return None, f"no registered skeleton matches ({len(candidates)} candidate pair(s))"


def region_root(gm, match, env):
    """The node computing the operator's final value when it is the single graph output
    (walking the readout chain after the consumer); None otherwise."""
    if getattr(match, "region_root", None) is not None:
        return match.region_root
    allowed = {match.producer_sym, match.consumer_sym}
    region, stack = {match.consumer_node}, [match.consumer_node]
    while stack:
        node = stack.pop()
        for user in node.users:
            expr = env.get(user)
            if user in region or expr is None or not expr.free_symbols <= allowed:
                continue
            region.add(user)
            stack.append(user)
    out = next((n for n in reversed(list(gm.graph.nodes)) if n.op == "output"), None)
    if out is None or not out.args:
        return None
    leaves: list = []
    _flatten_nodes(out.args, leaves)
    if len(leaves) != 1:
        return None
    value = leaves[0]
    while (hasattr(value, "op") and value.op in ("call_function", "call_method")
           and _op(value) in _IGNORED):
        inputs = [a for a in value.args if hasattr(a, "op")]
        if len(inputs) != 1:
            break
        value = inputs[0]
    return value if value in region else None


# ---------------------------------------------------------------- structured operators
def _aten_arguments(node, target):
    """Bind a call of exactly `target` to its schema (defaults filled); None otherwise."""
    if getattr(node, "op", None) != "call_function" or node.target != target:
        return None
    arguments = target._schema.arguments
    if len(node.args) > len(arguments):
        return None
    bound = {arg.name: value for arg, value in zip(arguments, node.args)}
    names = {arg.name for arg in arguments}
    for key, value in node.kwargs.items():
        if key in bound or key not in names:
            return None
        bound[key] = value
    for arg in arguments:
        if arg.name not in bound:
            if not arg.has_default_value():
                return None
            bound[arg.name] = arg.default_value
    return bound


def _structured_cast(node, dtype):
    """The input node of `node` when node converts it to `dtype` and changes nothing else (same
    device, layout and shape; default pinning and memory format), else None."""
    import torch

    aten = torch.ops.aten
    bound = _aten_arguments(node, aten._to_copy.default) or _aten_arguments(node, aten.to.dtype)
    if bound is None or bound["dtype"] != dtype:
        return None
    source, result = _tensor_value(bound["self"]), _tensor_value(node)
    if source is None or result is None:
        return None
    # aten.to.dtype has no device / layout / pin_memory arguments: absent means unchanged
    requested = (bound.get("device"), bound.get("layout"), bound.get("pin_memory"), bound["memory_format"])
    unchanged = (source.device, source.layout, False, torch.preserve_format)
    if any(want is not None and want != keep for want, keep in zip(requested, unchanged)):
        return None
    if source.device != result.device or source.layout != result.layout:
        return None
    return bound["self"] if _same_shape(source.shape, result.shape) else None


def _square_of(node, z) -> bool:
    """square(z), pow(z, 2) or z * z."""
    import torch

    aten = torch.ops.aten
    unary = _aten_arguments(node, aten.square.default)
    if unary is not None and unary["self"] is z:
        return True
    power = _aten_arguments(node, aten.pow.Tensor_Scalar)
    if (power is not None and power["self"] is z and type(power["exponent"]) in (int, float)
            and power["exponent"] == 2):
        return True
    product = _aten_arguments(node, aten.mul.Tensor)
    return product is not None and product["self"] is z and product["other"] is z


def _rms_structured_candidate(root):
    """rms_norm from its staged form: cast(cast(x, f32) * rsqrt(mean(sq, -1, keepdim) + eps),
    dtype) * gamma, every stage fp32 on x's device (the cast is absent for fp32 x)."""
    import math

    import torch

    aten = torch.ops.aten
    final = _aten_arguments(root, aten.mul.Tensor)
    if final is None:
        return None
    for normalized, gamma in ((final["self"], final["other"]), (final["other"], final["self"])):
        out, weight = _tensor_value(root), _tensor_value(gamma)
        if out is None or weight is None or out.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            continue
        dtype = out.dtype
        product = _structured_cast(normalized, dtype)
        if product is None:
            if dtype != torch.float32:
                continue
            product = normalized
        multiply = _aten_arguments(product, aten.mul.Tensor)
        if multiply is None:
            continue
        for z, inverse in ((multiply["self"], multiply["other"]), (multiply["other"], multiply["self"])):
            rs = _aten_arguments(inverse, aten.rsqrt.default)
            add = _aten_arguments(rs["self"], aten.add.Tensor) if rs is not None else None
            if add is None or add["alpha"] != 1:
                continue
            mean, eps = add["self"], add["other"]
            if type(eps) not in (float, int) or not math.isfinite(eps) or eps <= 0:
                continue
            red = _aten_arguments(mean, aten.mean.dim)
            zv = _tensor_value(z)
            if red is None or red["keepdim"] is not True or zv is None or zv.dtype != torch.float32:
                continue
            dims = red["dim"]
            if (len(zv.shape) < 1 or not isinstance(dims, (tuple, list)) or len(dims) != 1
                    or dims[0] not in (-1, len(zv.shape) - 1) or red["dtype"] not in (None, torch.float32)):
                continue
            square = red["self"]
            if not _square_of(square, z):
                continue
            promoted = _structured_cast(z, torch.float32)
            if dtype == torch.float32:
                # an fp32 RMS over a promoted low-precision source would move gamma before
                # the input-dtype rounding: refused
                if promoted is not None and _tensor_value(promoted).dtype != torch.float32:
                    continue
                x = promoted if promoted is not None else z
            else:
                x = promoted
            xv = _tensor_value(x) if x is not None else None
            if xv is None or xv.dtype != dtype or not _same_shape(xv.shape, zv.shape):
                continue
            if (weight.dtype != dtype or weight.device != xv.device or len(weight.shape) != 1
                    or not _same_shape(weight.shape, xv.shape[-1:]) or not _same_shape(out.shape, xv.shape)):
                continue
            stages = (square, mean, rs["self"], inverse, product)
            if any(_tensor_value(s) is None or _tensor_value(s).dtype != torch.float32
                   or _tensor_value(s).device != xv.device for s in stages):
                continue
            row = xv.shape[:-1] + (1,)
            if (not _same_shape(_tensor_value(square).shape, xv.shape)
                    or not all(_same_shape(_tensor_value(s).shape, row) for s in (mean, rs["self"], inverse))
                    or not _same_shape(_tensor_value(product).shape, xv.shape)):
                continue
            owned = {root, product, inverse, rs["self"], mean, square, z, normalized} - {x, gamma}
            return Match(
                x, "rms_norm", {"eps": float(eps)}, ("eps",), consumer_node=mean, region_root=root,
                region_nodes=tuple(owned),
                proof_kind="exact-structured-real-algebra-with-explicit-rounding",
                domain_assumptions=("finite real inputs and finite reachable fp32 arithmetic",
                                    "finite positive eps and nonempty last dimension",
                                    "fp32 square/mean/add/rsqrt/product; input-dtype rounding before gamma multiplication",
                                    "gamma is a readonly same-device input-dtype vector"),
                input_nodes=(x, gamma), kind="structured", operation="rms_norm",
                metadata={"numerical_stages": "fp32_then_input_round_then_gamma"})
    return None


def _structured_boundary_value(gm, node):
    """Tensor metadata of a boundary; a lifted get_attr without metadata is resolved locally."""
    value = _tensor_value(node)
    if value is not None or getattr(node, "op", None) != "get_attr":
        return value
    import torch

    obj = gm
    try:
        for part in node.target.split("."):
            obj = getattr(obj, part)
    except AttributeError:
        return None
    return obj if isinstance(obj, torch.Tensor) else None


_SEGMENT_ASSUMPTIONS = (
    "finite real data and finite reachable accumulation",
    "readonly legal descriptors: nonnegative lengths with checked coverage unless unsafe, or monotone offsets within data bounds",
    "initial is None or a finite scalar; mean empty segment with initial=None returns NaN",
    "source unsafe is reused, not a proof of valid descriptors",
)


def _segment_structured_candidate(root):
    """A Match for torch.segment_reduce(data, 'sum' | 'mean', lengths= xor offsets=, axis=0)
    with an explicit bool `unsafe` and `initial` None or finite; None for anything else."""
    import torch

    bound = _aten_arguments(root, torch.ops.aten.segment_reduce.default)
    if bound is None:
        return None
    given = [key for key in ("lengths", "offsets") if bound[key] is not None]
    initial = bound["initial"]
    initial_ok = initial is None or (type(initial) in (int, float) and math.isfinite(initial))
    if (bound["reduce"] not in ("sum", "mean") or bound["axis"] != 0 or bound["indices"] is not None
            or len(given) != 1 or not initial_ok or type(bound["unsafe"]) is not bool):
        return None
    params = {"initial": None if initial is None else float(initial),
              "offsets": given[0] == "offsets", "unsafe": bound["unsafe"]}
    return Match(bound["data"], f"segment_{bound['reduce']}", params, region_root=root,
                 region_nodes=(root,),
                 proof_kind="exact-structured-real-algebra-with-explicit-rounding",
                 domain_assumptions=_SEGMENT_ASSUMPTIONS,
                 input_nodes=(bound["data"], bound[given[0]]), kind="structured",
                 operation="segment_pool", metadata={"numerical_stages": "input_round"})


def recognize_structured_regions(gm, capabilities=("rms_norm", "segment_pool")):
    """([Match], reason) for the opt-in structured operators, exact ATen forms only."""
    from neptune_codegen.skeleton import state_reduction_spec
    from neptune_recognize.rewrite import region_contract

    if isinstance(capabilities, str):
        capabilities = (capabilities,)
    capabilities = frozenset(capabilities)
    unknown = capabilities - {"rms_norm", "segment_pool"}
    if unknown:
        return [], "unsupported structured capabilities: " + ", ".join(sorted(unknown))
    if any(getattr(getattr(n.target, "_schema", None), "is_mutable", False) for n in gm.graph.nodes):
        return [], "structured recognition requires a functionalized graph"
    order = {node: i for i, node in enumerate(gm.graph.nodes)}
    matches, reasons = [], []
    for root in gm.graph.nodes:
        cand = _rms_structured_candidate(root) if "rms_norm" in capabilities else None
        if cand is None and "segment_pool" in capabilities:
            cand = _segment_structured_candidate(root)
        if cand is None:
            continue
        cand.metadata["boundary_values"] = tuple(_structured_boundary_value(gm, n)
                                                 for n in cand.input_nodes)
        _, refusal = region_contract(cand)
        if refusal is not None:
            reasons.append(refusal)
            continue
        spec = CG.STATE_REDUCTIONS.get(cand.skeleton)
        if (spec is None or spec != state_reduction_spec(cand.skeleton)
                or spec.operation != cand.operation):
            reasons.append("structured operation is not registered with the same access contract")
            continue
        try:
            certificate = CG.derive_state_certificate(spec)
        except (NotImplementedError, ValueError, TypeError) as error:
            reasons.append(str(error))
            continue
        cand.domain_assumptions += tuple(certificate.assumptions)
        cand.metadata["numeric_contract"] = spec.numeric.stages
        cand.metadata["state_fields"] = certificate.state_fields
        cand.region_nodes = tuple(sorted(cand.region_nodes, key=order.__getitem__))
        matches.append(cand)
    if matches:
        return matches, f"matched {len(matches)} structured region(s)"
    return [], "no certified structured region" + (": " + reasons[-1] if reasons else "")
