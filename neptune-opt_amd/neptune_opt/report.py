"""What `apply` reports.  Field names, their order and the summary texts are the reference's
public contract (neptune_opt/__init__.py:30-71): callers read these fields and match on the
texts."""
from __future__ import annotations

import dataclasses

_VERIFIED = "  verified: fused output matches the supplied inputs"
_UNVERIFIED = "  unverified: real-algebra match; numerical verification not executed"
_STRUCTURED_SCOPE = ("  scope   : supplied-case values and read-only inputs/state; output aliasing "
                     "not proved")


def _shown(key, value) -> str:
    if value is None or isinstance(value, bool):
        return f"{key}={value!r}"
    return f"{key}={value:g}"


@dataclasses.dataclass
class Fusion:
    """One region that was (or, in a report of preview, would be) replaced by a fused op."""

    skeleton: str
    params: dict
    input_name: str = ""
    output_name: str = ""
    plan: str = "serial"
    proof_kind: str = ""
    domain_assumptions: tuple = ()
    input_names: tuple = ()
    kind: str = "scalar"
    operation: str = ""
    numeric_contract: tuple = ()

    @classmethod
    def from_match(cls, match, plan):
        meta = getattr(match, "metadata", {})
        stages = meta.get("numerical_stages")
        contract = meta.get("numeric_contract") or ((stages,) if stages else ())
        inputs = getattr(match, "input_nodes", ()) or (match.input_node,)
        return cls(skeleton=match.skeleton, params=dict(match.params),
                   input_name=match.input_node.name, output_name=match.region_root.name,
                   plan=plan, proof_kind=match.proof_kind,
                   domain_assumptions=match.domain_assumptions,
                   input_names=tuple(node.name for node in inputs),
                   kind=getattr(match, "kind", "scalar"), operation=getattr(match, "operation", ""),
                   numeric_contract=tuple(contract))

    def __str__(self) -> str:
        if not self.params:
            return self.skeleton
        return f"{self.skeleton}({', '.join(_shown(k, v) for k, v in sorted(self.params.items()))})"


@dataclasses.dataclass
class Report:
    """Fused regions, (reason, detail) refusals, and whether outputs were verified."""

    fusions: list = dataclasses.field(default_factory=list)
    skipped: list = dataclasses.field(default_factory=list)
    verified: bool = False
    graph_changed: bool = False
    verification_cases: int = 0

    def __bool__(self) -> bool:
        return bool(self.fusions)

    def summary(self) -> str:
        lines = [f"  fused   : {fusion}" for fusion in self.fusions]
        lines += [f"  skipped : {reason}: {detail}" for reason, detail in self.skipped]
        if self.fusions:
            lines.append(_VERIFIED if self.verified else _UNVERIFIED)
            if self.verified and any(f.kind == "structured" for f in self.fusions):
                lines.append(_STRUCTURED_SCOPE)
        return "\n".join(lines) if lines else "  (nothing to do)"
