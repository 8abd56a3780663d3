"""Measured launch configurations per GPU (only deviations from the default are listed).

Keys inside `table` are (rows class, ncols bucket) or (rows class, ncols bucket, dtype) ->
(BLOCK, num_warps); see autotune.py for the meaning of BLOCK on CDNA4.  A machine with no entry uses autotune.default_config.  Entries
come from neptune_codegen.tuning.search (graph-replayed, cold-cache launches) and are kept only
when they beat the default by more than the 5% noise margin.
"""
TABLES = {
    "gfx950": {
        "measured_on": "AMD Instinct MI355X (gfx950), torch 2.10.0+rocm7.0, hiprtc",
        "noise": 0.05,
        # No deviations: a sweep of every candidate at 16384 rows x {256 ... 16384} and 4096 x
        # 65536, bf16/fp16/fp32, found no shape where a candidate beats autotune.default_config
        # by more than the 5% noise margin (the 16-bit mid-width rule there came from it).
        "table": {},
    },
}
