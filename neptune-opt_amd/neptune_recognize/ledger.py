"""Rename ledger of a trial graph: which graph value took over from which.

Every edit in this package replaces a node by a new one: a fused call for a region root, a
readout op for a log-softmax tail, a 16-bit fold for a cast pair, the last step of a lowered
compound op for the compound node.  An ExportedProgram's signature and module call graph still
name the old values, so each replacement is written here and resolved when the signature is
rebuilt.  Entries may chain (compound -> its expansion's result -> fused call); resolution
follows a chain to the first name that is still a node of the graph.

The ledger lives in `GraphModule.meta` under KEY as a plain {old name: new name} dict.  FX
callers may shallow-copy `meta`, so writers replace the dict rather than mutate it.
"""
from __future__ import annotations

KEY = "neptune_renames"


def entries(gm) -> dict:
    """A private copy of gm's ledger."""
    return dict(gm.meta.get(KEY, {}))


def record(gm, old: str, new: str) -> None:
    """`new` now stands where `old` stood."""
    gm.meta[KEY] = {**gm.meta.get(KEY, {}), old: new}


def adopt(gm, source) -> None:
    """Give gm the ledger of `source` (a trial forked from gm whose graph gm just took)."""
    gm.meta[KEY] = entries(source)


def resolver(renames: dict, live):
    """name -> the live name it resolves to.  A live name resolves to itself.  A removed name
    with no entry, or a cycle, raises RuntimeError."""

    def resolve(name):
        seen = []
        while name not in live:
            if name in seen:
                raise RuntimeError("cyclic rewritten root mapping")
            seen.append(name)
            if name not in renames:
                raise RuntimeError(f"module signature references removed intermediate {name}")
            name = renames[name]
        return name

    return resolve
