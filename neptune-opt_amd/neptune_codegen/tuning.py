"""Measuring launch configurations on the GPU (the MI355X counterpart of the reference's
autotune.search / measure_shapes, neptune_codegen/autotune.py:445-544).

Each candidate `(BLOCK, num_warps)` is timed as the mean device time of back-to-back launches
replayed from a HIP graph (no host launch overhead), with the input rotated over copies larger
than the 256 MB Infinity Cache so every launch reads HBM.  Candidates are interleaved over
rounds and the minimum kept; `autotune.choose` then keeps the default unless a candidate beats
it by more than the noise margin.
"""
from __future__ import annotations

import math

COLD_BYTES = 768 << 20


def _graph_ms(launches, replays: int = 3) -> float:
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches[0]()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in launches:
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * len(launches))


def search(name: str, rows: int, ncols: int, dtype=None, candidates=None, params=None,
           plan: str = "serial", rounds: int = 3, launches: int = 16, seed: int = 0):
    """[((BLOCK, num_warps), ms), ...] fastest first, for one shape on the current GPU."""
    import torch

    from neptune_codegen.autotune import CANDIDATES
    from neptune_codegen.skeleton import param_defaults
    from neptune_codegen.template import run

    dtype = torch.float32 if dtype is None else dtype
    params = {**param_defaults(name), **(params or {})}
    candidates = CANDIDATES if candidates is None else candidates
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, ncols, generator=g).to(dtype).cuda()
    nbytes = x.numel() * x.element_size()
    copies = max(1, math.ceil(COLD_BYTES / nbytes))
    xs = [x] + [x.clone() for _ in range(copies - 1)]
    best = {}
    for _ in range(rounds):
        for cfg in candidates:
            block, warps = cfg
            try:
                fns = [lambda y=xs[i % copies]: run(name, y, block=block, num_warps=warps,
                                                    plan=plan, **params)
                       for i in range(max(launches, copies))]
                ms = _graph_ms(fns)
            except Exception as exc:  # noqa: BLE001 -- an unlaunchable candidate is skipped
                print(f"      {cfg}: cannot launch ({type(exc).__name__}: {str(exc)[:60]})")
                ms = float("inf")
            best[cfg] = min(best.get(cfg, float("inf")), ms)
    return sorted(best.items(), key=lambda kv: kv[1])
