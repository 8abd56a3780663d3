"""Launch configuration and operator identity.

A fold's launch configuration is `(BLOCK, num_warps)`, as in the reference
(neptune_codegen/autotune.py:41-53, 222-250), re-read for CDNA4:

  BLOCK      the row tile in elements that the lanes of one row cover per step; each lane
             covers UNROLL (=4) 16-byte slots of it, so lanes per row = BLOCK / (4 * VEC) with
             VEC = 16 bytes / element size (a whole wavefront per row for fp32 at BLOCK=1024).
             When that exceeds the workgroup's lanes, each lane takes more slots instead
             (up to MAX_UNROLL = 8) before the workgroup grows past 64 * num_warps lanes.
  num_warps  wave64s per workgroup (workgroup = 64 * num_warps lanes, at least one row)

Shapes with no measured entry use `default_config`, which sizes the tile to the row rather
than using one fixed block: short rows get a few lanes each (many rows per wavefront), long
rows a multi-wavefront workgroup.  Measured MI355X deviations live in launch_table.py, keyed
by (rows class, width bucket) as in the reference, or by (rows class, width bucket, dtype)
where the best tile differs between storage types (BLOCK counts elements, so the same BLOCK
is a different tile in bytes); a dtype key wins over the plain one.

Operator identity (`op_key`, `parameter_tag`, `parameter_identity`) is the reference's scheme
(autotune.py:392-432) unchanged: registered op names must stay stable across backends.
"""
from __future__ import annotations

import hashlib
import math

UNROLL = 4
MAX_UNROLL = 8
# 16-bit rows at least this wide take 8 slots per lane (BLOCK = 512 * VEC, 4 waves).  Measured
# on MI355X, bf16 logsumexp, cold cache: 32000 wide 157.9 vs 162.6 us, 65536 wide 159.0 vs
# 164.3 us, 262144 wide 161.2 vs 169.3 us; at 16384 wide 8 slots lose (174.6 vs 163.8 us).
WIDE_16BIT_ROW = 24576
# 16-bit rows from 2048 up to that width walk the row in two tiles of half its width on two
# waves.  Measured on MI355X, logsumexp, 16384 rows, cold cache, against the full-width tile on
# four waves: bf16 2048 wide 13.6 vs 14.1 us, 4096 22.9 vs 24.0, 8192 41.9 vs 46.7, 16384
# 79.4 vs 84.8; fp16 4096 23.2 vs 24.6, 8192 42.3 vs 47.7, 16384 79.7 vs 86.2.  fp32 keeps the
# full tile (within 2% of the best candidate at every width).
MID_16BIT_ROW = 2048
CANDIDATES: tuple = tuple((b, w) for b in (128, 256, 512, 1024, 2048, 4096, 8192, 16384)
                          for w in (1, 2, 4, 8))
DEFAULT: tuple = (1024, 4)
MIN_BUCKET = 128
MAX_BUCKET = 1 << 20
THIN_ROWS = 8
NOISE = 0.05
LEGACY_MACHINE = "legacy-flat-table"
MAX_TPR = 1024


def machine_key(device_name: str | None = None) -> str:
    """Normalised GPU name, e.g. 'AMD Instinct MI355X' -> 'amd-instinct-mi355x'."""
    name = device_name
    if name is None:
        try:  # pragma: no cover - needs a GPU
            import torch

            if not torch.cuda.is_available():
                return ""
            name = torch.cuda.get_device_name(torch.cuda.current_device())
        except Exception:  # noqa: BLE001
            return ""
    words = []
    for word in str(name).lower().replace("+", " ").split():
        if word in ("nvidia", "geforce", "tesla", "graphics", "corporation"):
            continue
        words.append("".join(ch if ch.isalnum() else "-" for ch in word).strip("-"))
    return "-".join(w for w in words if w)


def device_name_of(device) -> str | None:
    """GPU name of a torch device without importing torch (None when unresolvable)."""
    import sys

    if device is None or "torch" not in sys.modules:
        return None
    torch = sys.modules["torch"]
    try:
        device = torch.device(device)
        if device.type != "cuda":
            return None
        name = torch.cuda.get_device_name(device)
        # ROCm builds without the marketing-name table report a generic name; the ISA then
        # identifies the part (gfx950 = MI350X/MI355X) and keys its launch table.
        if not name or "Radeon Graphics" in name:
            name = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
        return name
    except Exception:  # noqa: BLE001
        return None


def ncols_bucket(ncols) -> int:
    if not isinstance(ncols, int):
        raise ValueError("a measured width bucket requires a static integer width")
    n = max(1, ncols)
    return max(MIN_BUCKET, min(MAX_BUCKET, 1 << (n - 1).bit_length()))


def rows_class(rows) -> str:
    if not isinstance(rows, int):
        return "many"
    if rows <= 1:
        return "single"
    return "few" if rows <= THIN_ROWS else "many"


def shape_key(rows, ncols) -> tuple:
    return rows_class(rows), ncols_bucket(ncols)


def dtype_name(dtype) -> str:
    """'float32' / 'bfloat16' / 'float16' (the optional third element of a table key)."""
    return str(dtype).replace("torch.", "")


def _valid(body) -> dict:
    return {tuple(k): tuple(v) for k, v in (body or {}).items() if tuple(v) in CANDIDATES}


def tables() -> dict:
    try:
        from neptune_codegen import launch_table
    except Exception:  # noqa: BLE001
        return {}
    raw = getattr(launch_table, "TABLES", None) or {}
    out = {}
    for machine, entry in raw.items():
        meta = {k: v for k, v in entry.items() if k != "table"}
        out[machine] = {**meta, "table": _valid(entry.get("table"))}
    return out


def machines() -> list:
    return sorted(tables())


def table(machine: str | None = None) -> dict:
    all_tables = tables()
    if machine is None:
        machine = machine_key()
    if machine in all_tables:
        return dict(all_tables[machine]["table"])
    return {}


def measured_on(machine: str | None = None) -> str:
    if machine is None:
        machine = machine_key()
    return tables().get(machine, {}).get("measured_on", "")


def vec_of(dtype) -> int:
    """Elements per 16-byte load."""
    size = getattr(dtype, "itemsize", None)
    if size is None:
        size = 4 if "32" in str(dtype) else 2
    return 16 // size


def default_config(rows, ncols, dtype=None) -> tuple:
    """MI355X default: tile the row so its lanes finish it in one to a few steps."""
    if not isinstance(rows, int) or not isinstance(ncols, int):
        return DEFAULT
    step = UNROLL * vec_of(dtype) if dtype is not None else 16
    if dtype is not None and vec_of(dtype) == 8 and ncols >= WIDE_16BIT_ROW:
        return step * 512, 4
    tile = 1 << max(0, (max(ncols, 1) - 1).bit_length())
    if dtype is not None and vec_of(dtype) == 8 and ncols >= MID_16BIT_ROW:
        return tile // 2, 2
    block = max(step * 4, min(tile, step * 256))
    return block, 4


_CHOICES: dict = {}
_CHOICES_MAX = 4096


def _table_token():
    try:
        from neptune_codegen import launch_table
    except Exception:  # noqa: BLE001
        return None
    return id(getattr(launch_table, "TABLES", None))


def best_config(rows, ncols, dtype=None, device=None, device_name=None,
                verbose: bool = False) -> tuple:
    """`(BLOCK, num_warps)` for a row length on this machine: measured entry, else default.

    The answer depends on the row class, the width, the dtype, the machine and the launch
    table, so it is memoised on exactly those (a replaced table is a new key)."""
    if not isinstance(rows, int) or not isinstance(ncols, int):
        return DEFAULT
    if not verbose:
        key = (rows_class(rows), ncols, str(dtype), str(device), device_name, _table_token())
        cfg = _CHOICES.get(key)
        if cfg is None:
            cfg = _best_config(rows, ncols, dtype, device, device_name, False)
            if len(_CHOICES) >= _CHOICES_MAX:
                _CHOICES.clear()
            _CHOICES[key] = cfg
        return cfg
    return _best_config(rows, ncols, dtype, device, device_name, verbose)


def _best_config(rows, ncols, dtype, device, device_name, verbose) -> tuple:
    if device is not None and str(device).split(":", 1)[0] != "cuda":
        return default_config(rows, ncols, dtype)
    if device_name is None:
        device_name = device_name_of(device)
    machine = machine_key(device_name) if device_name else ""
    entries = table(machine)
    key = shape_key(rows, ncols)
    cfg = entries.get(key + (dtype_name(dtype),)) if dtype is not None else None
    cfg = entries.get(key) if cfg is None else cfg
    source = "measured"
    if cfg is None:
        cfg, source = default_config(rows, ncols, dtype), "default"
    if verbose:
        print(f"    launch config rows={rows} ncols={ncols} on {machine or '<unknown gpu>'}: "
              f"BLOCK={cfg[0]} num_warps={cfg[1]} ({source})")
    return cfg


def lanes_per_row(block: int, vector_width: int) -> int:
    """Lanes per row for a tile of `block` elements (power of two in [1, MAX_TPR])."""
    tpr = max(1, block // (UNROLL * vector_width))
    tpr = 1 << (tpr - 1).bit_length() if tpr & (tpr - 1) else tpr
    return min(MAX_TPR, tpr)


# ---------------------------------------------------------------- choice rule (measurement)
def choose(results: list, default: tuple = DEFAULT, noise: float = NOISE) -> tuple:
    """Keep `default` unless the fastest measured config beats it by more than `noise`."""
    ok = [r for r in results if math.isfinite(r[1])]
    if not ok:
        raise RuntimeError("no candidate launch configuration could be measured")
    best = min(ok, key=lambda r: r[1])
    base = next((r for r in ok if tuple(r[0]) == tuple(default)), None)
    if base is None:
        return tuple(best[0]), float("nan"), "the default was not measurable"
    gain = base[1] / best[1]
    if gain <= 1.0 + noise:
        return tuple(default), gain, f"within noise ({gain:.2f}x): keeping the default"
    return tuple(best[0]), gain, f"{gain:.2f}x better than the default"


# ---------------------------------------------------------------- operator identity
def parameter_identity(params: dict | None) -> tuple:
    """Exact identity of the binary64 scalars baked into a kernel."""
    return tuple((key, float(value).hex()) for key, value in sorted((params or {}).items()))


def parameter_tag(params: dict | None) -> str:
    """Identifier-safe exact tag; short %g form only when it round-trips bit for bit."""
    identity = parameter_identity(params)
    tags = []
    for key, exact in identity:
        value = float.fromhex(exact)
        short = f"{value:g}"
        tag = short.replace(".", "p").replace("-", "m").replace("+", "a")
        if not math.isfinite(value) or float(short).hex() != exact:
            tag += "_h" + exact.replace("-", "m").replace("+", "a").replace(".", "p")
        tags.append("_" + key + tag)
    if len(identity) > 1 or any(not key.isalpha() for key, _ in identity):
        tags.append("_h" + hashlib.sha256(repr(identity).encode()).hexdigest()[:16])
    return "".join(tags)


def op_key(lib: str, name: str, params: dict | None, keepdim: bool,
           block: int | None = None, num_warps: int | None = None) -> str:
    """Registered op name: parameters, output rank and (when fixed) launch configuration."""
    tag = "_keep" if keepdim else ""
    tag += parameter_tag(params)
    if block is not None or num_warps is not None:
        tag += f"_b{block}w{num_warps}"
    return f"{lib}::{name}{tag}"
