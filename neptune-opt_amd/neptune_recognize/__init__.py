"""neptune_recognize -- which registered fold does an ATen graph implement, and where.

Recognition reads the same registry the HIP emitter generates from: a graph is interpreted as
row algebra over one data symbol (interp), its dependent reduction pairs are compared with
every registered skeleton (match), eligible regions are replaced by the fused HIP op
(rewrite), and compound ops are expanded only where that yields a region (lowering).  The
public names are those of the reference package (neptune_recognize/__init__.py:36-78).
"""
from __future__ import annotations

from neptune_recognize.interp import (_BINARY, _IGNORED, _MEANS, _REDUCTIONS, _UNARY, S_RESULT,
                                      Candidate, _as_expr, _flatten_nodes, _last_dim_of, _op,
                                      interpret)
from neptune_recognize.match import (Match, _find_region_root, _match_candidate,
                                     _producer_pattern, _solve_params, recognize,
                                     recognize_regions, region_root)
from neptune_recognize.params import _infer_numerically, _respects, _solve_for
from neptune_recognize.rewrite import (_wants_keepdim, region_contract, rewrite, rewrite_match,
                                       would_rewrite)


def recognize_structured_regions(gm, *, capabilities=()):
    from neptune_recognize.match import recognize_structured_regions as structured

    return structured(gm, capabilities=capabilities)


__all__ = [
    "Candidate", "Match", "S_RESULT", "_BINARY", "_IGNORED", "_MEANS", "_REDUCTIONS", "_UNARY",
    "_as_expr", "_find_region_root", "_flatten_nodes", "_infer_numerically", "_last_dim_of",
    "_match_candidate", "_op", "_producer_pattern", "_respects", "_solve_for", "_solve_params",
    "_wants_keepdim", "interpret", "recognize", "recognize_regions",
    "recognize_structured_regions", "region_contract", "rewrite_match", "region_root",
    "rewrite", "would_rewrite",
]
