"""Plans, validation, compilation caches and the launch ABI of the HIP backend.

Mirrors the reference's neptune_codegen/template.py: the same plan names and split capacity
(validate_plan :109-111, split_launch_shape :114-125), the same row-last contract and refusals
(_validate_row_last :338-352, _row_last_layout :355-365, validate_rms_inputs :267-291), the
same direct entry points (run :393-442, run_rms_norm :322-335) and the same ownership rule:
torch allocates every output and scratch buffer, kernels never allocate.  What differs is
below the launch: generated HIP units compiled by hiprtc and launched through
libneptune_hip on the caller's current stream.
"""
from __future__ import annotations

import math
import threading

from neptune_codegen import hip
from neptune_codegen.autotune import (MAX_TPR, MAX_UNROLL, UNROLL, WIDE_16BIT_ROW, best_config,
                                      lanes_per_row, parameter_identity, parameter_tag, vec_of)
from neptune_codegen.emitters import (BASE_OPTIONS, NO_CONTRACT, FoldVariant, RowVariant,
                                      check_supported, emit_kernel_source, emit_readout_source,
                                      emit_rms_state_source, fold_kernel_name,
                                      readout_kernel_name, readout_tile, rms_kernel_names)
from neptune_codegen.skeleton import SKELETONS, all_registered, param_defaults

MAX_SPLIT_PARTS = 4096
_CACHE: dict = {}
_STATE_CACHE: dict = {}
_STATE_SEEN: dict = {}
_cache_lock = threading.Lock()


def validate_plan(plan: str) -> None:
    if plan not in ("serial", "split"):
        raise ValueError(f"unknown reduction plan {plan!r}; expected 'serial' or 'split'")


def split_launch_shape(ncols, block: int) -> tuple[int, int]:
    """(nparts, merge width) of an explicit split; refuses symbolic width and over-capacity."""
    if type(ncols) is not int:
        raise NotImplementedError("explicit split requires a concrete width; use plan='serial' for dynamic width")
    if type(block) is not int or block <= 0 or block & (block - 1):
        raise ValueError("split BLOCK must be a positive power of two")
    if ncols <= 0:
        raise ValueError("split requires positive width")
    nparts = (ncols + block - 1) // block
    if nparts > MAX_SPLIT_PARTS:
        raise NotImplementedError(f"split needs {nparts} partials, exceeding capacity {MAX_SPLIT_PARTS}; use serial")
    return nparts, 1 << (nparts - 1).bit_length()


def _validate_row_last(x, *, metadata: bool = False):
    import torch

    if x.layout != torch.strided:
        raise TypeError("Neptune requires a strided tensor")
    if x.ndim < 1:
        raise ValueError("Neptune row-last reductions require rank >= 1")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported Neptune dtype {x.dtype}; expected float16/bfloat16/float32")
    if not metadata and x.device.type != "cuda":
        raise ValueError(f"unsupported Neptune device {x.device}; execution requires a ROCm (cuda) device")
    torch._check(x.shape[-1] > 0, lambda: "Neptune requires positive last-dimension width")


def _row_last_layout(x):
    """Flatten leading dimensions only; reshape copies exactly when no view exists."""
    rows = 1
    for size in x.shape[:-1]:
        rows = rows * size
    ncols = x.shape[-1]
    return x.reshape(rows, ncols), rows, ncols


# ---------------------------------------------------------------- compiled programs
class FoldProgram:
    """The generated kernels of one (skeleton, parameters, plan[, stage]); variants compile
    lazily, one hiprtc unit per launch shape."""

    def __init__(self, name: str, values: dict, plan: str, stage: str = ""):
        import sympy as sp

        from neptune_codegen.emitters import producer_operand_expr

        self.name, self.values, self.plan, self.stage = name, dict(values), plan, stage
        self.sk = SKELETONS[name]
        self.heavy_phi = self.sk.is_log and bool(
            producer_operand_expr(self.sk).atoms(sp.tanh, sp.exp, sp.log))
        self._programs: dict = {}

    def source(self, var: FoldVariant) -> str:
        return emit_kernel_source(self.sk, self.values, plan=self.plan, variants=(var,))

    def program(self, var: FoldVariant) -> hip.Program:
        prog = self._programs.get(var)
        if prog is None:
            prog = hip.Program(self.source(var), f"{self.name}_{self.plan}_{var.tag()}.hip",
                               BASE_OPTIONS)
            self._programs[var] = prog
        return prog

    def kernel(self, var: FoldVariant, stage: str, device: int) -> hip.Kernel:
        name = fold_kernel_name(self.sk, self.plan, stage, var)
        if stage == "partial":
            args = (hip.PTR,) * 5 + (hip.I64,) * 6
            block = var.wg
        elif stage == "merge":
            args = (hip.PTR,) * 5 + (hip.I64,) * 3
            block = 256
        else:
            args = (hip.PTR, hip.PTR) + (hip.I64,) * 4
            block = var.wg
        return self.program(var).kernel(name, args, block, device)


class ReadoutProgram:
    """The readout kernels phi(x) - r of one exponential fold (log-softmax for logsumexp)."""

    def __init__(self, name: str, values: dict, nan_posinf_rows: bool):
        self.name, self.values, self.nan_posinf_rows = name, dict(values), nan_posinf_rows
        self.sk = SKELETONS[name]
        self._programs: dict = {}

    def source(self, var: FoldVariant) -> str:
        return emit_readout_source(self.sk, self.values, variants=(var,),
                                   nan_posinf_rows=self.nan_posinf_rows)

    def program(self, var: FoldVariant) -> hip.Program:
        prog = self._programs.get(var)
        if prog is None:
            tag = "_nanrows" if self.nan_posinf_rows else ""
            prog = hip.Program(self.source(var), f"{self.name}_readout{tag}_{var.tag()}.hip",
                               BASE_OPTIONS)
            self._programs[var] = prog
        return prog

    def kernel(self, var: FoldVariant, device: int, resident: bool = False) -> hip.Kernel:
        """`resident` selects the kernel for rows of at most readout_tile(var) columns."""
        name = readout_kernel_name(self.sk, var, self.nan_posinf_rows, resident)
        return self.program(var).kernel(name, (hip.PTR, hip.PTR) + (hip.I64,) * 4, var.wg, device)


def compile_readout(name: str, values: dict | None = None, *, nan_posinf_rows: bool = True):
    """The readout program of an exponential fold; refusals surface here, before any launch."""
    values = {**param_defaults(name), **(values or {})} if name in SKELETONS else values
    key = ("readout", name, parameter_identity(values), bool(nan_posinf_rows))
    with _cache_lock:
        if key in _CACHE:
            return _CACHE[key]
    if name not in SKELETONS:
        raise KeyError(f"unknown skeleton {name!r}; have {all_registered()}")
    emit_readout_source(SKELETONS[name], values, variants=(), nan_posinf_rows=nan_posinf_rows)
    program = ReadoutProgram(name, values or {}, bool(nan_posinf_rows))
    with _cache_lock:
        _CACHE[key] = program
    return program


def launch_readout(program: ReadoutProgram, x2, out, rows, ncols, block, num_warps) -> None:
    """Launch a readout on the current stream: out [rows, ncols] contiguous."""
    import torch

    device = x2.device.index if x2.device.index is not None else torch.cuda.current_device()
    var = _fold_variant(x2, ncols, block, num_warps, resident=True)
    rpw = max(1, var.wg // var.tpr)
    program.kernel(var, device, resident=ncols <= readout_tile(var)).launch(
        (_grid_1d(rows, rpw),),
        (x2.data_ptr(), out.data_ptr(), rows, ncols, x2.stride(0), x2.stride(1)),
        hip.current_stream(x2.device))


def run_readout(name: str, x, *, nan_posinf_rows: bool = True, block: int | None = None,
                num_warps: int | None = None, **params):
    """phi(x) - r over the last dimension, r the row's exponential fold (fp32), rounded once to
    x.dtype: for logsumexp, log_softmax(x, -1).  With nan_posinf_rows a row containing +inf
    reads out NaN, as the reference's log_softmax lowering does (lowering.py:92-98).  Fresh
    contiguous output of x's shape and dtype; Fake/meta tensors return metadata only."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensor

    metadata = isinstance(x, FakeTensor) or x.device.type == "meta"
    _validate_row_last(x, metadata=metadata)
    program = compile_readout(name, params, nan_posinf_rows=nan_posinf_rows)
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    if metadata:
        return out
    x2, rows, ncols = _row_last_layout(x)
    if isinstance(rows, int) and rows == 0:
        return out
    if block is None or num_warps is None:
        cfg = best_config(rows, ncols, x.dtype, x.device)
        block = cfg[0] if block is None else block
        num_warps = cfg[1] if num_warps is None else num_warps
    launch_readout(program, x2, out, rows, ncols, block, num_warps)
    return out


def run_log_softmax(x, *, nan_posinf_rows: bool = True):
    """log_softmax over the last dimension through the logsumexp fold's readout."""
    return run_readout("logsumexp", x, nan_posinf_rows=nan_posinf_rows)


def compile_skeleton(name: str, values: dict | None = None, force: bool = False, *,
                     plan: str = "serial"):
    """Generate the fold for (name, values, plan): a FoldProgram, or (partial, merge) for split."""
    validate_plan(plan)
    key = (name, parameter_identity(values), plan)
    with _cache_lock:
        if not force and key in _CACHE:
            return _CACHE[key]
    if name not in SKELETONS:
        raise KeyError(f"unknown skeleton {name!r}; have {all_registered()}")
    sk = SKELETONS[name]
    check_supported(sk)
    # emit once now so that refusals (missing parameter, split of a two-pass fold, an
    # uncertified merge) surface at compile time, before any launch
    emit_kernel_source(sk, values, plan=plan)
    if plan == "serial":
        kernel = FoldProgram(name, values or {}, plan)
    else:
        shared = FoldProgram(name, values or {}, plan)
        kernel = (shared, shared)
    with _cache_lock:
        _CACHE[key] = kernel
    return kernel


def generated_path(name: str, values: dict | None = None, *, plan: str = "serial") -> str:
    """Identifier of one generated unit family (kept for API parity; units live in memory
    and in the code-object cache, keyed by their exact source)."""
    validate_plan(plan)
    suffix = "" if plan == "serial" else "_plan_split"
    return f"neptune_gen_{name}{parameter_tag(values)}{suffix}.hip"


# ---------------------------------------------------------------- scalar launch ABI
def _is_vector(x2, ncols: int, vec: int, extra_align: int = 0) -> bool:
    if x2.dim() != 2:
        return False
    col_ok = x2.stride(1) == 1 or ncols == 1
    return (col_ok and x2.stride(0) % vec == 0 and ncols % vec == 0
            and x2.data_ptr() % 16 == 0 and (extra_align == 0 or extra_align % vec == 0))


def _fold_variant(x2, ncols: int, block: int, num_warps: int, *, split_block: int = 0,
                  resident: bool = False, merge_heavy: bool = False,
                  heavy_phi: bool = False) -> FoldVariant:
    """Launch shape: 16-byte loads when the layout allows, lanes per row from BLOCK (a tile
    wider than the workgroup's lanes gives each lane up to MAX_UNROLL slots first), workgroup =
    max(64 * num_warps, lanes per row).  Three fold classes then adjust it (serial plan only):

    * `merge_heavy` -- single-pass folds without the exponential fast path, whose row combine
      evaluates the repair at every butterfly level -- and `heavy_phi` -- exponential folds
      whose producer operand is itself transcendental (softcap's tanh).  fp32 rows take
      MAX_UNROLL slots per lane on the same lanes and give lanes up while a tile would cover
      twice the row (fp32 16384 x 4096: rmsnorm_max 79.2 -> 47.2 us, softcap_lse 50.6 -> 40.8;
      softcap_lse 2096 x 32000: 53.8 -> 48.2).  16-bit `merge_heavy` rows take ~width/128 lanes
      (16 to 64) with 4 slots per lane (8 from 24576 wide) and walk several tiles: a butterfly
      level costs a repair, a lane's next tile only one (rmsnorm_max bf16 16384 x 4096: 31.1
      -> 26.9 us).  16-bit `heavy_phi` rows of more than 64 lanes trade half the lanes for
      twice the slots.
    * `resident` -- two-pass folds -- widens the tile until one tile holds the whole row where
      that fits (MAX_UNROLL slots of MAX_TPR lanes), so the second pass reads registers, not
      HBM: fp32 widens slots first, 16-bit rows lanes first, up to 512 (variance bf16
      16384 x 4096: 28.5 -> 23.5 us).
    * 16-bit `merge_heavy` and `resident` rows of exactly 64 lanes run one row per 64-lane
      workgroup (bf16 8192 wide: 54.0 -> 48.7 us).

    Every default is within ~5% of a full sweep of (BLOCK, num_warps) at widths 1000-32000
    (bf16 and fp32)."""
    vec = vec_of(x2.dtype)
    vector = _is_vector(x2, ncols, vec, split_block)
    if vector and split_block and split_block < vec:
        vector = False
    tpr = lanes_per_row(block, vec if vector else 1)
    waves = max(1, min(16, int(num_warps)))
    waves = 1 << (waves - 1).bit_length()
    unroll = UNROLL
    while tpr > 64 * waves and unroll < MAX_UNROLL and not split_block:
        tpr //= 2
        unroll *= 2
    per_slot = vec if vector else 1
    if merge_heavy and not split_block and per_slot == 8:
        # 16-bit rows: at most one wavefront per row, several short tiles per lane
        tpr = min(64, max(16, 1 << max(0, (max(1, ncols // 128) - 1).bit_length())))
        unroll = MAX_UNROLL if ncols >= WIDE_16BIT_ROW else UNROLL
    elif (merge_heavy or heavy_phi) and not split_block and per_slot == 4:
        # fp32 rows: 8 slots per lane on the same lanes, then lanes given up while a tile would
        # cover twice the row
        unroll = MAX_UNROLL
        while tpr > 16 and tpr * unroll * per_slot >= 2 * ncols:
            tpr //= 2
    elif (merge_heavy or heavy_phi) and not split_block:
        while tpr > 64 and unroll < MAX_UNROLL:
            tpr //= 2
            unroll *= 2
    if resident and not split_block:
        if per_slot == 8:      # 16-bit rows: lanes first (up to 512), then slots
            unroll = UNROLL
            tpr = min(512, 1 << max(0, (-(-ncols // (UNROLL * per_slot)) - 1).bit_length()))
        while tpr * unroll * per_slot < ncols and unroll < MAX_UNROLL:
            unroll *= 2
        while tpr * unroll * per_slot < ncols and tpr < MAX_TPR:
            tpr *= 2
    if per_slot == 8 and (merge_heavy or resident) and not split_block and tpr == 64:
        waves = 1              # one row per 64-lane workgroup (bf16 8192 wide: 54.0 -> 48.7 us)
    return FoldVariant(str(x2.dtype).replace("torch.", ""), vector, tpr, unroll, waves)


def _grid_1d(items: int, per_wg: int) -> int:
    return max(1, (items + per_wg - 1) // per_wg)


def launch_reduction(kernel, plan, x2, out, rows, ncols, block, num_warps, *, wrapper=None):
    """Launch a compiled fold on the current stream; scratch for split is torch-allocated."""
    import torch

    validate_plan(plan)
    device = x2.device.index if x2.device.index is not None else torch.cuda.current_device()
    stream = hip.current_stream(x2.device)
    if plan == "serial":
        sk = kernel.sk
        var = _fold_variant(x2, ncols, block, num_warps, resident=sk.two_pass,
                            merge_heavy=not sk.is_log and not sk.two_pass,
                            heavy_phi=kernel.heavy_phi)
        k = kernel.kernel(var, "", device)
        rpw = max(1, var.wg // var.tpr)
        grid = (_grid_1d(rows, rpw),)
        tail = (rows, ncols, x2.stride(0), x2.stride(1))
        k.launch(grid, (x2.data_ptr(), out.data_ptr()) + tail, stream)
        return k, grid, tail
    nparts, _merge = split_launch_shape(ncols, block)
    partial_m = hip.scratch(torch.empty((rows, nparts), device=x2.device, dtype=torch.float32))
    partial_a = hip.scratch(torch.empty((rows, nparts), device=x2.device, dtype=torch.float32))
    partial_v = hip.scratch(torch.empty((rows, nparts), device=x2.device, dtype=torch.int32))
    partial_s = hip.scratch(torch.empty((rows, nparts), device=x2.device, dtype=torch.int32))
    partial, merge = kernel
    var = _fold_variant(x2, ncols, block, num_warps, split_block=block)
    kp = partial.kernel(var, "partial", device)
    rpw = max(1, var.wg // var.tpr)
    grid_p, grid_m = (_grid_1d(rows * nparts, rpw),), (_grid_1d(rows, 4),)
    tail_p = (rows, ncols, x2.stride(0), x2.stride(1), nparts, block)
    tail_m = (rows, ncols, nparts)
    kp.launch(grid_p, (x2.data_ptr(), partial_m.data_ptr(), partial_a.data_ptr(),
                       partial_v.data_ptr(), partial_s.data_ptr()) + tail_p, stream)
    km = merge.kernel(var, "merge", device)
    km.launch(grid_m, (partial_m.data_ptr(), partial_a.data_ptr(), partial_v.data_ptr(),
                       partial_s.data_ptr(), out.data_ptr()) + tail_m, stream)
    return kp, grid_p, tail_p, km, grid_m, tail_m, rows * nparts


_RUN_SEEN: dict = {}
_RUN_SEEN_MAX = 4096


def run(name: str, x, block: int | None = None, num_warps: int | None = None,
        keepdim: bool = False, plan: str = "serial", **params):
    """Reduce the last dimension of `x` with the generated fold `name`.

    Rank >= 1 returns x.shape[:-1] (keepdim appends a 1).  Real execution needs a ROCm device
    and float16/bfloat16/float32; Fake/meta tensors return metadata only.  Declared parameter
    defaults are filled for anything not passed.

    A call on a plain device tensor whose (fold, plan, dtype, device, shape, strides, 16-byte
    alignment, launch options, parameter types and values) were seen before reuses that call's
    kernels and launch shapes: everything the validation and the launch choice read is in that
    key, so only the allocations and the launches remain (not while launches are recorded).
    """
    import torch
    from torch._subclasses.fake_tensor import FakeTensor

    from neptune_codegen.skeleton import param_defaults

    seen = None
    if type(x) is torch.Tensor and x.is_cuda and not hip.recording_active():
        try:
            seen = (name, plan, x.dtype, x.device, tuple(x.shape), tuple(x.stride()),
                    x.data_ptr() % 16, block, num_warps, keepdim,
                    tuple(sorted((k, type(v).__name__, repr(v)) for k, v in params.items())))
            entry = _RUN_SEEN.get(seen)
        except TypeError:
            seen, entry = None, None
        if entry is not None:
            out = torch.empty(entry[0], device=x.device, dtype=x.dtype)
            stream = hip.current_stream(x.device)
            if plan == "serial":
                _, kern, grid, tail = entry
                kern.launch(grid, (x.data_ptr(), out.data_ptr()) + tail, stream)
                return out
            _, kp, grid_p, tail_p, km, grid_m, tail_m, count = entry
            # one allocation holds the four partial arrays (m, acc: fp32; seen, status: int32)
            parts = torch.empty(4 * count, device=x.device, dtype=torch.float32)
            base = parts.data_ptr()
            ptrs = (base, base + 4 * count, base + 8 * count, base + 12 * count)
            kp.launch(grid_p, (x.data_ptr(),) + ptrs + tail_p, stream)
            km.launch(grid_m, ptrs + (out.data_ptr(),) + tail_m, stream)
            return out
    metadata = isinstance(x, FakeTensor) or x.device.type == "meta"
    _validate_row_last(x, metadata=metadata)
    params = {**param_defaults(name), **(params or {})}
    validate_plan(plan)
    if plan == "split":
        block = 1024 if block is None else block
        num_warps = 4 if num_warps is None else num_warps
        from neptune_codegen.algebra import derive_merge_certificate

        derive_merge_certificate(SKELETONS[name], params)
        split_launch_shape(x.shape[-1], block)
    shape = x.shape[:-1] + ((1,) if keepdim else ())
    out = torch.empty(shape, device=x.device, dtype=x.dtype)
    if metadata:
        return out
    x2, rows, ncols = _row_last_layout(x)
    if isinstance(rows, int) and rows == 0:
        return out
    kernel = compile_skeleton(name, params, plan=plan)
    if block is None or num_warps is None:
        cfg = best_config(rows, ncols, x.dtype, x.device)
        block = cfg[0] if block is None else block
        num_warps = cfg[1] if num_warps is None else num_warps
    launch = launch_reduction(kernel, plan, x2, out, rows, ncols, block, num_warps)
    if seen is not None and launch is not None and x2.data_ptr() == x.data_ptr():
        if len(_RUN_SEEN) >= _RUN_SEEN_MAX:
            _RUN_SEEN.clear()
        _RUN_SEEN[seen] = (tuple(out.shape),) + tuple(launch)
    return out


# ---------------------------------------------------------------- structured RMS / L2
class RowProgram:
    """Generated structured-state kernels of one (spec, eps, plan)."""

    def __init__(self, spec_name: str, params: dict, plan: str):
        self.spec_name, self.params, self.plan = spec_name, dict(params), plan
        self._programs: dict = {}

    def source(self, var: RowVariant) -> str:
        from neptune_codegen.skeleton import state_reduction_spec

        return emit_rms_state_source(state_reduction_spec(self.spec_name), self.params,
                                     plan=self.plan, variants=(var,))

    def program(self, var: RowVariant) -> hip.Program:
        prog = self._programs.get(var)
        if prog is None:
            prog = hip.Program(self.source(var), f"{self.spec_name}_{self.plan}_{var.tag()}.hip",
                               BASE_OPTIONS + NO_CONTRACT)
            self._programs[var] = prog
        return prog

    def kernels(self, var: RowVariant, device: int) -> tuple:
        names = rms_kernel_names(self.spec_name, self.plan, var)
        prog = self.program(var)
        if self.plan == "serial":
            return (prog.kernel(names[0], (hip.PTR,) * 3 + (hip.I64,) * 5, var.wg, device),)
        return (prog.kernel(names[0], (hip.PTR,) * 3 + (hip.I64,) * 6, var.wg, device),
                prog.kernel(names[1], (hip.PTR,) * 5 + (hip.I64,) * 7, var.wg, device))


def compile_state_reduction(name: str, params=None, *, plan: str = "serial"):
    """Compile a certified structured backend (RMSNorm, L2-normalize)."""
    from neptune_codegen.algebra import derive_state_certificate
    from neptune_codegen.skeleton import state_reduction_spec

    validate_plan(plan)
    if name not in ("rms_norm", "l2_normalize"):
        raise NotImplementedError("this structured compiler implements RMSNorm and L2-normalize; "
                                  "segments use the serial backend")
    params = dict(params or {})
    # parameters seen before, with the same types and values, were certified and validated by
    # an earlier call: skip the certificate lookup and the validating source emission (~20 us)
    try:
        seen = (name, plan, tuple(sorted((k, type(v).__name__, repr(v)) for k, v in params.items())))
        program = _STATE_SEEN.get(seen)
    except TypeError:
        seen, program = None, None
    if program is not None:
        return program
    spec = state_reduction_spec(name)
    derive_state_certificate(spec)
    emit_rms_state_source(spec, params, plan=plan)  # validates even on a cache hit
    key = (spec, parameter_identity(params), plan)
    with _cache_lock:
        if key not in _STATE_CACHE:
            _STATE_CACHE[key] = RowProgram(name, params, plan)
        if seen is not None:
            _STATE_SEEN[seen] = _STATE_CACHE[key]
        return _STATE_CACHE[key]


def _check_eps(params):
    eps = params.get("eps")
    if params.keys() != {"eps"} or type(eps) not in (int, float) or not math.isfinite(eps) or eps <= 0:
        raise ValueError("RMSNorm requires an explicit finite positive eps")


def validate_rms_inputs(x, gamma, params=None, *, plan="serial", metadata=False):
    """Full-vector RMSNorm contract (template.py:267-291); symbolic batch survives."""
    import torch

    validate_plan(plan)
    _validate_row_last(x, metadata=metadata)
    params = dict(params or {})
    _check_eps(params)
    if gamma.layout != torch.strided or gamma.ndim != 1:
        raise ValueError("RMSNorm gamma must be a strided 1D tensor")
    if gamma.dtype != x.dtype or gamma.device != x.device:
        raise ValueError("RMSNorm gamma dtype/device must match input")
    torch._check(gamma.shape[0] == x.shape[-1], lambda: "RMSNorm gamma width must match input")
    _check_static_width(x, plan)
    return x.shape


def validate_l2_inputs(x, params=None, *, plan="serial", metadata=False):
    """L2-normalize contract: the RMS row-last rules without gamma."""
    validate_plan(plan)
    _validate_row_last(x, metadata=metadata)
    _check_eps(dict(params or {}))
    _check_static_width(x, plan)
    return x.shape


def _check_static_width(x, plan):
    if type(x.shape[-1]) is not int:
        raise NotImplementedError("RMSNorm first backend requires a static feature width")
    if plan == "serial" and x.shape[-1] > 32768:
        raise NotImplementedError("resident RMSNorm width exceeds 32768; request split explicitly")
    if plan == "split":
        split_launch_shape(x.shape[-1], 1024)


def _row_variant(flat, gamma, width: int, *, tile: int | None = None) -> RowVariant:
    """Lanes per row and 16-byte slots per lane of the row-resident RMS / L2 kernels.  16-bit
    rows take 4 slots per lane from 256 to 1024 slots (2048-8192 elements), 2 from 128 (1024
    elements), and 8 otherwise.
    Measured on MI355X at 268 MB, one run per shape (noise ~1-2 us), RMSNorm / L2-normalize:
    width 1024: 2 slots 85.6 / 88.7 us, 4 slots 89.2 / 85.9, 8 slots 87.3 / 89.2;
    width 2048: 4 slots 87.3 / 86.8, 8 slots 88.4 / 92.1;
    width 4096: 4 slots 85.7 / 86.9, 2 slots 86.1 / 87.8, 8 slots 87.9 / 89.1 (a second run:
    4 slots 85.4-85.6 / 86.4-86.8, 8 slots 86.8-88.0 / 87.8-88.7);
    width 8192: 4 slots 87.4 / 88.6, 8 slots 89.0 / 90.5;
    width 16384: 8 slots 88.4 / 89.0, 4 slots 89.0 / 88.9."""
    vec = vec_of(flat.dtype)
    vector = _is_vector(flat, width, vec, tile or 0)
    if vector and gamma is not None:
        vector = gamma.stride(0) == 1 and gamma.data_ptr() % 16 == 0
    span = tile if tile is not None else width
    slots = (span + vec - 1) // vec if vector else span
    nv = 8 if vector else 16
    if vector and vec == 8 and 128 <= slots <= 1024:
        nv = 4 if slots >= 256 else 2
    if tile is not None:
        nv = 2 if vector else 8
    tpr = 1 << max(0, (max(1, -(-slots // nv)) - 1).bit_length())
    while tpr > 1024:
        nv *= 2
        tpr = 1 << max(0, (max(1, -(-slots // nv)) - 1).bit_length())
    nv = max(1, min(nv, -(-slots // tpr)))
    nv = 1 << (nv - 1).bit_length()
    return RowVariant(str(flat.dtype).replace("torch.", ""), vector, tpr, nv)


def _persistent_grid(items_per_wg: int, items: int, device) -> int:
    """Workgroups for the row-resident kernels: one per row block up to 64 per CU, beyond
    which workgroups loop.  Measured on MI355X at 32768 x 4096 bf16 (8192 row blocks): 8 per CU
    (looping) 107 us, 16 per CU 105 us, one per row block 89 us."""
    import torch

    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return max(1, min(_grid_1d(items, items_per_wg), cus * 64))


def launch_rms_norm(kernel, x, gamma, out, *, plan="serial", wrapper=None):
    """Shared launch of the structured RMS / L2 kernels; scratch is torch-allocated."""
    import torch

    flat, rows, width = _row_last_layout(x)
    if isinstance(rows, int) and rows == 0:
        return
    device = x.device.index if x.device.index is not None else torch.cuda.current_device()
    stream = hip.current_stream(x.device)
    g_ptr = gamma.data_ptr() if gamma is not None else 0
    g_stride = gamma.stride(0) if gamma is not None else 0
    if plan == "serial":
        var = _row_variant(flat, gamma, width)
        (k,) = kernel.kernels(var, device)
        rpw = max(1, var.wg // var.tpr)
        grid = (_persistent_grid(rpw, rows, x.device),)
        tail = (rows, width, flat.stride(0), flat.stride(1), g_stride)
        k.launch(grid, (flat.data_ptr(), g_ptr, out.data_ptr()) + tail, stream)
        return (k, grid, tail) if flat.data_ptr() == x.data_ptr() else None
    parts, _ = split_launch_shape(width, 1024)
    totals = hip.scratch(torch.empty((rows, parts), device=x.device, dtype=torch.float32))
    counts = hip.scratch(torch.empty((rows, parts), device=x.device, dtype=torch.int64))
    var = _row_variant(flat, gamma, width, tile=1024)
    kp, km = kernel.kernels(var, device)
    rpw = max(1, var.wg // var.tpr)
    grid = (_persistent_grid(rpw, rows * parts, x.device),)
    tail_p = (rows, width, flat.stride(0), flat.stride(1), parts, 1024)
    tail_m = (rows, width, flat.stride(0), flat.stride(1), g_stride, parts, 1024)
    kp.launch(grid, (flat.data_ptr(), totals.data_ptr(), counts.data_ptr()) + tail_p, stream)
    km.launch(grid, (flat.data_ptr(), g_ptr, totals.data_ptr(), counts.data_ptr(),
                     out.data_ptr()) + tail_m, stream)
    if flat.data_ptr() != x.data_ptr():
        return None
    return kp, km, grid, tail_p, tail_m, rows * parts


_ROW_SEEN: dict = {}


def _row_seen_key(name, x, gamma, eps, plan):
    """Key of an RMS / L2 call on plain device tensors: everything the validation and the
    launch choice read (plan, dtypes, devices, shapes, strides, 16-byte alignment, eps's type
    and value); None when the call takes the full path."""
    import torch

    if type(x) is not torch.Tensor or not x.is_cuda or hip.recording_active():
        return None
    if gamma is None:
        g = None
    elif type(gamma) is torch.Tensor:
        g = (gamma.dtype, gamma.device, gamma.layout, tuple(gamma.shape), tuple(gamma.stride()),
             gamma.data_ptr() % 16)
    else:
        return None
    try:
        key = (name, plan, x.dtype, x.device, tuple(x.shape), tuple(x.stride()),
               x.data_ptr() % 16, g, type(eps).__name__, repr(eps))
        hash(key)
    except TypeError:
        return None
    return key


def _row_run(name, x, gamma, eps, plan, validate):
    import torch
    from torch._subclasses.fake_tensor import FakeTensor

    key = _row_seen_key(name, x, gamma, eps, plan)
    entry = _ROW_SEEN.get(key) if key is not None else None
    if entry is not None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        g_ptr = gamma.data_ptr() if gamma is not None else 0
        stream = hip.current_stream(x.device)
        if plan == "serial":
            k, grid, tail = entry
            k.launch(grid, (x.data_ptr(), g_ptr, out.data_ptr()) + tail, stream)
            return out
        kp, km, grid, tail_p, tail_m, count = entry
        # one allocation: the int64 counts, then the fp32 totals
        scratch = torch.empty((3 * count + 1) // 2, device=x.device, dtype=torch.int64)
        counts, totals = scratch.data_ptr(), scratch.data_ptr() + 8 * count
        kp.launch(grid, (x.data_ptr(), totals, counts) + tail_p, stream)
        km.launch(grid, (x.data_ptr(), g_ptr, totals, counts, out.data_ptr()) + tail_m, stream)
        return out
    params = {"eps": eps}
    metadata = isinstance(x, FakeTensor) or x.device.type == "meta"
    shape = validate(params, metadata)
    out = torch.empty(shape, device=x.device, dtype=x.dtype)
    if metadata or x.numel() == 0:
        return out
    kernel = compile_state_reduction(name, params, plan=plan)
    launch = launch_rms_norm(kernel, x, gamma, out, plan=plan)
    if key is not None and launch is not None:
        if len(_ROW_SEEN) >= _RUN_SEEN_MAX:
            _ROW_SEEN.clear()
        _ROW_SEEN[key] = launch
    return out


def run_rms_norm(x, gamma, *, eps: float = 1e-6, plan="serial"):
    """Full-vector RMSNorm over the last dimension; fresh contiguous output in x.dtype.  A
    serial call whose tensors and eps match an earlier call's (dtypes, devices, shapes,
    strides, alignment, eps's type and value) reuses that call's kernel and launch shape."""
    return _row_run("rms_norm", x, gamma, eps, plan,
                    lambda params, metadata: validate_rms_inputs(x, gamma, params, plan=plan,
                                                                 metadata=metadata))


def run_l2_normalize(x, *, eps: float = 1e-6, plan="serial"):
    """x / max(||x||_2, eps) over the last dimension (fp32 statistics, dtype output); repeated
    serial calls reuse their launch as run_rms_norm's do."""
    return _row_run("l2_normalize", x, None, eps, plan,
                    lambda params, metadata: validate_l2_inputs(x, params, plan=plan,
                                                                metadata=metadata))
