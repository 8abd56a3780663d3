"""Measured launch configurations per GPU (only deviations from the default are listed).

Keys inside `table` are (rows class, ncols bucket) -> (BLOCK, num_warps); see autotune.py for
the meaning of BLOCK on CDNA4.  A machine with no entry uses autotune.default_config.
"""
TABLES = {
}
