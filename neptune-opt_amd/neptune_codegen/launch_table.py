"""Measured launch configurations per GPU (only deviations from the default are listed).

Keys inside `table` are (rows class, ncols bucket) -> (BLOCK, num_warps); see autotune.py for
the meaning of BLOCK on CDNA4.  A machine with no entry uses autotune.default_config.  Entries
come from neptune_codegen.tuning.search (graph-replayed, cold-cache launches) and are kept only
when they beat the default by more than the 5% noise margin.
"""
TABLES = {
    "gfx950": {
        "measured_on": "AMD Instinct MI355X (gfx950), torch 2.10.0+rocm7.0, hiprtc",
        "noise": 0.05,
        "table": {
            # 16384 x 4096 bf16 logsumexp: 22.8 us vs 24.2 us at the default (4096, 4)
            ("many", 4096): (2048, 2),
        },
    },
}
