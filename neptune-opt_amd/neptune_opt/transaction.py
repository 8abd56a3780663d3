"""The graph transaction behind `apply`, `preview` and `backend`.

Nothing here edits the caller's graph.  Work happens on a *trial*: a GraphModule with a private
copy of the graph (parameters and buffers are shared, never copied) and a private rename ledger
(neptune_recognize/ledger.py).  The region pass fuses one region at a time and rediscovers
after every edit, since an edit can merge, remove or rename what the next region would read.
When nothing is eligible it may lower one compound op (logsumexp; log_softmax on request) and
fuse the region grown from it, as one step.  `program_with` then rebuilds an ExportedProgram
around the trial, renaming the signature through the ledger and refusing any other signature
change; `apply` verifies that program and only then publishes it into the caller's object.
"""
from __future__ import annotations

import copy
import dataclasses
import inspect

from neptune_opt.report import Fusion, Report
from neptune_recognize import ledger, recognize_regions
from neptune_recognize.lowering import MARK, install, is_compound, is_log_softmax, lower_compound
from neptune_recognize.rewrite import region_contract, rewrite_match


def fork(gm):
    """Trial copy of gm: own graph, own ledger, same tensors."""
    import torch

    trial = torch.fx.GraphModule(gm, copy.deepcopy(gm.graph))
    trial.meta = copy.copy(gm.meta)
    ledger.adopt(trial, gm)
    return trial


def _eligible(match) -> bool:
    return region_contract(match)[1] is None


def _is_structured(match) -> bool:
    return getattr(match, "kind", "scalar") == "structured"


def candidate_regions(gm, values, capabilities):
    """(matches, reason): eligible regions first -- structured before scalar, one per root
    (the largest), in graph order -- followed by every refused match."""
    if not capabilities:
        return recognize_regions(gm, values)
    from neptune_recognize import recognize_structured_regions

    structured, why_structured = recognize_structured_regions(gm, capabilities=capabilities)
    scalar, why_scalar = recognize_regions(gm, values)
    position = {node: i for i, node in enumerate(gm.graph.nodes)}
    ranked = sorted(structured + scalar, key=lambda m: (not _is_structured(m), -len(m.region_nodes),
                                                        position[m.region_root]))
    chosen, refused, roots = [], [], set()
    for match in ranked:
        if not _eligible(match):
            refused.append(match)
        elif match.region_root not in roots:
            roots.add(match.region_root)
            chosen.append(match)
    chosen.sort(key=lambda m: (not _is_structured(m), position[m.region_root]))
    return chosen + refused, why_structured or why_scalar


def lowered_regions(gm, values, experimental_log_softmax):
    """For each compound node of gm, in graph order, whose own expansion grows an eligible
    region: (node name, a trial of gm with that node lowered, the region's match).  Each trial
    is forked when it is reached, so it includes whatever the caller installed into gm from
    the earlier ones."""
    names = [n.name for n in gm.graph.nodes
             if is_compound(n) and (experimental_log_softmax or not is_log_softmax(n))]
    for name in names:
        trial = fork(gm)
        if not lower_compound(trial, nodes=name):
            continue
        found, _ = recognize_regions(trial, values)
        grown = [m for m in found if m.region_root.meta.get(MARK) == name and _eligible(m)]
        if grown:
            yield name, trial, grown[0]


def _expansion_result(trial, name):
    """The node that took over from lowered compound node `name`: its expansion's last step."""
    marked = [n for n in trial.graph.nodes if n.meta.get(MARK) == name]
    return marked[-1]


def _fuse(gm, match, plan, report):
    fusion = Fusion.from_match(match, plan)
    call, refusal = rewrite_match(gm, match, plan=plan)
    if call is None:
        raise RuntimeError(refusal)
    report.fusions.append(fusion)


def _fuse_first_lowering(gm, values, plan, experimental_log_softmax, report) -> bool:
    for name, trial, match in lowered_regions(gm, values, experimental_log_softmax):
        # the compound node's users read its expansion's result, which the fusion may replace
        ledger.record(trial, name, _expansion_result(trial, name).name)
        _fuse(trial, match, plan, report)
        install(gm, trial)
        ledger.adopt(gm, trial)
        return True
    return False


def fuse_regions(gm, values, *, plan="serial", max_regions=None, lower=False,
                 experimental_log_softmax=False, capabilities=()) -> Report:
    """Fuse regions of gm (a trial) one at a time, at most max_regions (default: one per
    node).  Refusals are noted once each; "no-fusion" is noted when nothing happened."""
    report = Report()
    budget = len(gm.graph.nodes) if max_regions is None else max_regions
    while budget > 0:
        budget -= 1
        matches, reason = candidate_regions(gm, values, capabilities)
        for match in matches:
            refusal = region_contract(match)[1]
            if refusal is not None and all(detail != refusal for _, detail in report.skipped):
                report.skipped.append(("refused", refusal))
        eligible = [m for m in matches if _eligible(m)]
        if eligible:
            _fuse(gm, eligible[0], plan, report)
            continue
        if lower and _fuse_first_lowering(gm, values, plan, experimental_log_softmax, report):
            continue
        if not report.fusions and not report.skipped:
            report.skipped.append(("no-fusion", reason))
        break
    report.graph_changed = bool(report.fusions)
    return report


# ---------------------------------------------------------------- signature rebuild
def _output_spec(spec, leaf, live, moved):
    """The output spec for a rewritten graph output leaf, or RuntimeError."""
    import torch
    from torch.export.graph_signature import ConstantArgument

    is_node = isinstance(leaf, torch.fx.Node)
    if isinstance(spec.arg, ConstantArgument):
        constant = spec.arg.value
        if is_node or type(leaf) is not type(constant) or leaf != constant:
            raise RuntimeError("rewrite changed a constant graph output")
        return spec
    if not hasattr(spec.arg, "name"):
        return spec
    if not is_node:
        raise RuntimeError("rewrite changed a graph output into a constant")
    old = spec.arg.name
    if old != leaf.name and (old in live or moved.get(old) != leaf.name):
        raise RuntimeError("rewrite changed output without a root replacement")
    return dataclasses.replace(spec, arg=dataclasses.replace(spec.arg, name=leaf.name))


def _renamed_arguments(arguments, resolve):
    from torch.export.graph_signature import ConstantArgument

    return [dataclasses.replace(a, name=resolve(a.name))
            if hasattr(a, "name") and not isinstance(a, ConstantArgument) else a for a in arguments]


def program_with(exported, trial):
    """An ExportedProgram around trial's graph.  Output names follow the ledger; graph inputs
    are never renamed and must all survive; module call signatures are resolved through the
    ledger (they may name internal values).  Anything else raises RuntimeError."""
    import torch
    from torch.utils._pytree import tree_flatten

    live = {n.name for n in trial.graph.nodes}
    renames = ledger.entries(trial)
    resolve = ledger.resolver(renames, live)
    moved = {old: resolve(old) for old in renames if old not in live}
    signature = copy.deepcopy(exported.graph_signature)
    output = next(n for n in trial.graph.nodes if n.op == "output")
    leaves = tree_flatten(output.args[0])[0]
    if len(leaves) != len(signature.output_specs):
        raise RuntimeError("rewrite changed exported output arity")
    signature.output_specs[:] = [_output_spec(spec, leaf, live, moved)
                                 for spec, leaf in zip(signature.output_specs, leaves)]
    if any(hasattr(spec.arg, "name") and spec.arg.name not in live for spec in signature.input_specs):
        raise RuntimeError("rewrite removed an exported graph input")
    calls = copy.deepcopy(exported.module_call_graph)
    for entry in calls:
        if entry.signature is not None:
            entry.signature.inputs = _renamed_arguments(entry.signature.inputs, resolve)
            entry.signature.outputs = _renamed_arguments(entry.signature.outputs, resolve)
    arguments = dict(root=trial, graph=trial.graph, graph_signature=signature,
                     state_dict=exported.state_dict,
                     range_constraints=copy.deepcopy(exported.range_constraints),
                     module_call_graph=calls, example_inputs=exported.example_inputs,
                     constants=exported.constants)
    accepted = inspect.signature(torch.export.ExportedProgram).parameters
    if "verifiers" in accepted:
        arguments["verifiers"] = list(exported.verifiers)
    elif "verifier" in accepted:
        arguments["verifier"] = exported.verifier
    return torch.export.ExportedProgram(**arguments)


def publish(exported, candidate) -> None:
    """Swap the candidate's graph, signature and call graph into the caller's program (object
    references only: nothing can fail half-way)."""
    exported._graph_module = candidate.graph_module
    exported._graph_signature = candidate.graph_signature
    exported._module_call_graph = candidate.module_call_graph
