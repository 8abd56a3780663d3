"""The HIP emitter: fold algebra -> hiprtc translation units for gfx950.

Replaces the reference's Triton text emitters (neptune_codegen/emitters.py, template.py:41-186,
torch_op.py:254-306).  Every operator-specific line of device code is derived here from the
skeleton's algebra and rendered by `to_hip`; the loops, cross-lane merges and memory mapping
are hand-written CDNA4 templates in csrc/kernels/*.h that the generated code instantiates.

A generated unit is: the kernel headers, one `Fold` policy struct (scalar folds) or a baked
constant block (structured states), and one extern "C" kernel per launch variant.
"""
from __future__ import annotations

import dataclasses
import functools
import pathlib
import struct

import sympy as sp

from neptune_codegen.algebra import (_marked, coordinate_needs_floor, derive_merge_certificate,
                                     repair_bias, repair_factor, term_expr)
from neptune_codegen.skeleton import Skeleton
from neptune_codegen.symbols import *  # noqa: F401,F403
from neptune_codegen.sym_to_hip import TranslationError, f32_literal, to_hip

KERNEL_DIR = pathlib.Path(__file__).resolve().parent.parent / "csrc" / "kernels"

# hiprtc options shared by every unit.  Packed fp32 ops are disabled for all HIP code.
BASE_OPTIONS = ("--offload-arch=gfx950", "-O3", "-std=c++17",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")
# Structured states are compiled without FMA contraction, the numerical contract of the
# reference (enable_fp_fusion=False at template.py:308 and torch_op.py:409).
NO_CONTRACT = ("-ffp-contract=off",)

DTYPE_TAGS = {"float32": ("f32", "nep::F32"), "bfloat16": ("bf16", "nep::BF16"),
              "float16": ("f16", "nep::F16")}


@functools.lru_cache(maxsize=None)
def kernel_header(*names: str) -> str:
    parts = []
    for name in names:
        text = (KERNEL_DIR / name).read_text()
        parts.append(f"// ---- {name}\n" + text.replace("#pragma once", ""))
    return "\n".join(parts)


def dtype_tag(dtype) -> tuple[str, str]:
    key = str(dtype).replace("torch.", "")
    if key not in DTYPE_TAGS:
        raise TypeError(f"unsupported Neptune dtype {dtype}; expected float16/bfloat16/float32")
    return DTYPE_TAGS[key]


# ---------------------------------------------------------------- skeleton analysis
@functools.lru_cache(maxsize=None)
def derived_producer_expr(sk: Skeleton) -> sp.Expr | None:
    """The expression whose row maximum is the producer.

    Declared explicitly, or -- for an exponential fold g = exp(phi(c) - s) -- derived as
    phi = log(g) + s.  Power folds keep their declared producer mode (None here).
    """
    if sk.producer_expr is not None:
        return sk.producer_expr
    if sk.is_log:
        phi = sp.simplify(sp.log(sk.g) + s_sym)
        if not phi.has(s_sym) and not phi.has(s2_sym) and not phi.has(u_sym):
            return phi
    return None


def producer_operand_expr(sk: Skeleton) -> sp.Expr:
    phi = derived_producer_expr(sk)
    if phi is not None:
        return phi
    return c_sym if sk.producer == "signed" else sp.Abs(c_sym)


def intrinsic_bindings(sk: Skeleton) -> dict:
    """Intrinsic parameters (the row length) bind to the kernel's fp32 `n`."""
    return {sym: "n" for sym, _name in sk.intrinsic_params}


def param_bindings(sk: Skeleton, values: dict | None = None) -> dict:
    """Bake each declared scalar as an fp32 literal; a missing value is an error."""
    values = values or {}
    out = dict(intrinsic_bindings(sk))
    for sym, arg in sk.params:
        if sym in out:
            continue
        if arg not in values:
            raise KeyError(f"skeleton {sk.name!r}: no value supplied for scalar parameter "
                           f"{arg!r}; pass it to compile_skeleton/emit_kernel_source")
        out[sym] = f32_literal(float(values[arg]))
    return out


def _names(sk: Skeleton) -> dict:
    names = {c_sym: "v", s_sym: "m", s2_sym: "den", u_sym: "acc", _FINAL_ACC: "acc",
             _FINAL_M: "m"}
    names.update({sym: name for sym, name in sk.params})
    names.update(intrinsic_bindings(sk))
    return names


def check_supported(sk: Skeleton) -> None:
    """Refuse a skeleton the HIP emitter cannot lower correctly (emitters.py:24-100)."""
    if sk.producer not in ("signed", "abs"):
        raise NotImplementedError(f"unknown producer mode {sk.producer!r}")
    if sk.producer_reducer not in ("max", "sum"):
        raise NotImplementedError(f"unknown producer reducer {sk.producer_reducer!r}")
    if sk.consumer_reducer not in ("sum", "max"):
        raise NotImplementedError(f"unknown consumer reducer {sk.consumer_reducer!r}")
    for _sym, intrinsic in sk.intrinsic_params:
        if intrinsic not in INTRINSICS:
            raise NotImplementedError(
                f"skeleton {sk.name!r}: unknown intrinsic {intrinsic!r}; have {INTRINSICS}")
    if sk.consumer_reducer == "max" and sk.is_log:
        raise NotImplementedError(
            f"skeleton {sk.name!r}: an exponential fold needs a SUM consumer (a max of "
            "exponentiated terms is a different operator)")
    if sk.producer_expr is not None:
        for bad, what in ((s2_sym, "the fresh producer value"), (u_sym, "u")):
            if sk.producer_expr.has(bad):
                raise NotImplementedError(f"skeleton {sk.name!r}: producer_expr mentions {what}")
        to_hip(sk.producer_expr, _names(sk))
    if sk.is_log and sk.producer != "signed":
        raise NotImplementedError(
            f"skeleton {sk.name!r}: an exponential fold requires producer='signed' "
            "(exp(v - m) <= 1); max|v| collapses rows whose values are all negative")
    if sk.two_pass:
        if sk.producer_expr is not None:
            to_hip(sk.producer_expr, _names(sk))
        if not term_expr(sk).has(s2_sym):
            raise NotImplementedError(
                f"skeleton {sk.name!r}: the term {term_expr(sk)} does not depend on the "
                "producer at all, so the first pass would be dead work. This is not a fold.")
        to_hip(term_expr(sk), _names(sk))
        return
    repair_factor(sk)
    repair_bias(sk)
    term_expr(sk)
    names = _names(sk)
    try:
        to_hip(_marked(term_expr(sk)), names)
        to_hip(sk.finalize, names)
        to_hip(producer_operand_expr(sk), names)
    except TranslationError as exc:
        raise NotImplementedError(f"skeleton {sk.name!r}: {exc}") from exc


# ---------------------------------------------------------------- scalar fold policy
def emit_fold_policy(sk: Skeleton, values: dict | None = None, *, struct_name: str = "Fold") -> str:
    """The C++ policy struct carrying one skeleton's algebra (see nep_fold.h)."""
    check_supported(sk)
    bind = param_bindings(sk, values)
    floor = (not sk.two_pass) and coordinate_needs_floor(sk)
    phi = to_hip(producer_operand_expr(sk), {**bind, c_sym: "v"}, shared=c_sym)
    if sk.two_pass:
        term = to_hip(term_expr(sk), {**bind, c_sym: "v", s2_sym: "den"}, shared=c_sym)
        rho, beta, has_bias = "1.0f", "0.0f", False
        fin_m = "m"
    else:
        if sk.is_log:
            term = f"nep::fast_exp({phi} - den)"
        else:
            term = to_hip(_marked(term_expr(sk)), {**bind, c_sym: "v", s2_sym: "den"},
                          shared=c_sym)
        a, b = repair_factor(sk), repair_bias(sk)
        rho = to_hip(_marked(a), {**bind, s_sym: "q", s2_sym: "q2"}, fast=True)
        has_bias = b != 0
        beta = (to_hip(_marked(b), {**bind, s_sym: "q", s2_sym: "q2"}, fast=True) if has_bias
                else "0.0f")
        fin_m = "nep::eff<Self>(m)" if floor else "m"
    finalize = to_hip(sk.finalize, {**bind, _FINAL_M: "m_", _FINAL_ACC: "acc"})
    return f"""struct {struct_name} {{
  typedef {struct_name} Self;
  static constexpr bool kLog = {str(bool(sk.is_log and not sk.two_pass)).lower()};
  static constexpr bool kProducerSum = {str(sk.producer_reducer == "sum").lower()};
  static constexpr bool kConsumerMax = {str(sk.consumer_reducer == "max").lower()};
  static constexpr bool kFloor = {str(bool(floor)).lower()};
  static constexpr bool kHasBias = {str(bool(has_bias)).lower()};
  static constexpr bool kPhiIdentity = {str(phi.replace("(", "").replace(")", "").strip() == "v").lower()};
  __device__ static __forceinline__ float phi(float v, float n) {{ return {phi}; }}
  __device__ static __forceinline__ float term(float v, float den, float n) {{ return {term}; }}
  __device__ static __forceinline__ float rho(float q, float q2) {{ return {rho}; }}
  __device__ static __forceinline__ float beta(float q, float q2) {{ return {beta}; }}
  __device__ static __forceinline__ float finalize(float m, float acc, float n) {{
    const float m_ = {fin_m};
    return {finalize};
  }}
}};
"""


@dataclasses.dataclass(frozen=True)
class FoldVariant:
    """One launch shape of a scalar fold kernel."""

    dtype: str          # "float32" | "bfloat16" | "float16"
    vector: bool        # 16-byte loads (unit column stride, aligned rows)
    tpr: int            # lanes per row (or per split partial)
    unroll: int = 4     # slots per lane per tile
    waves: int = 4      # wave64s per workgroup (at least one row)

    @property
    def wg(self) -> int:
        return max(64 * self.waves, self.tpr)

    def tag(self) -> str:
        return (f"{dtype_tag(self.dtype)[0]}_{'v' if self.vector else 's'}{self.tpr}"
                f"u{self.unroll}w{self.waves}")


_FOLD_ARGS_SERIAL = ("const void* x, void* out, long long rows, long long ncols, "
                     "long long stride_row, long long stride_col")


def _fold_kernel(sk: Skeleton, plan: str, part: str, var: FoldVariant) -> tuple[str, str]:
    """(kernel name, extern "C" definition) for one plan stage and variant."""
    _, st = dtype_tag(var.dtype)
    vec = "true" if var.vector else "false"
    tmpl = f"Fold, {st}, {var.tpr}, {var.unroll}, {vec}, {var.wg}"
    if plan == "serial":
        name = f"{sk.name}_serial_{var.tag()}"
        body = (f"nep::fold_serial<{tmpl}>((const {st}::T*)x, ({st}::T*)out, rows, ncols, "
                "stride_row, stride_col);")
        sig = _FOLD_ARGS_SERIAL
    elif plan == "two_pass":
        name = f"{sk.name}_two_pass_{var.tag()}"
        body = (f"nep::fold_two_pass<{tmpl}>((const {st}::T*)x, ({st}::T*)out, rows, ncols, "
                "stride_row, stride_col);")
        sig = _FOLD_ARGS_SERIAL
    elif part == "partial":
        name = f"{sk.name}_partial_{var.tag()}"
        sig = ("const void* x, float* pm, float* pa, int* pv, int* ps, long long rows, "
               "long long ncols, long long stride_row, long long stride_col, long long nparts, "
               "long long block")
        body = (f"nep::fold_split_partial<{tmpl}>((const {st}::T*)x, pm, pa, pv, ps, rows, "
                "ncols, stride_row, stride_col, nparts, block);")
    else:
        name = f"{sk.name}_merge_{dtype_tag(var.dtype)[0]}"
        sig = ("const float* pm, const float* pa, const int* pv, const int* ps, void* out, "
               "long long rows, long long ncols, long long nparts")
        body = f"nep::fold_split_merge<Fold, {st}>(pm, pa, pv, ps, ({st}::T*)out, rows, ncols, nparts);"
    wg = 256 if part == "merge" else var.wg
    marker = ""
    if part == "partial":
        # the (row, part) pairs one workgroup covers, as the size of a marker symbol: the C ABI
        # reads it with hipModuleGetGlobal (no copy) and checks the caller's launch numbers
        marker = (f'extern "C" __device__ __attribute__((used)) unsigned char '
                  f"{name}_parts_per_workgroup[{max(1, wg // var.tpr)}] = {{1}};\n")
    return name, (marker + f'extern "C" __global__ void __launch_bounds__({wg}) {name}({sig}) {{\n'
                  f"  {body}\n}}\n")


def emit_kernel_source(sk: Skeleton, values: dict | None = None, *, plan: str = "serial",
                       variants: tuple | None = None) -> str:
    """A complete hiprtc unit for `sk` under `plan` ("serial" | "split").

    `variants` selects the launch shapes instantiated; by default one generic (strided)
    variant per dtype, which is what source-level checks compile.
    """
    from neptune_codegen.template import validate_plan

    validate_plan(plan)
    check_supported(sk)
    if plan == "split" and sk.two_pass:
        raise NotImplementedError("two_pass needs extended carried state; split refused")
    if plan == "split":
        derive_merge_certificate(sk, values)
    if variants is None:
        variants = tuple(FoldVariant(d, False, 64) for d in DTYPE_TAGS)
    kind = "two_pass" if sk.two_pass else plan
    header = (f"// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
              f"// skeleton={sk.name!r}, plan={plan!r}, two_pass={sk.two_pass}\n"
              f"// doc={sk.doc!r}\n"
              "// exact real-algebra repair; not bitwise IEEE associativity.\n")
    parts = [header, kernel_header("nep_device.h", "nep_fold.h"),
             emit_fold_policy(sk, values)]
    seen = set()
    for var in variants:
        stages = ("partial", "merge") if plan == "split" else ("",)
        for stage in stages:
            name, text = _fold_kernel(sk, kind, stage, var)
            if name not in seen:
                seen.add(name)
                parts.append(text)
    return "\n".join(parts)


def readout_kernel_name(sk: Skeleton, var: FoldVariant, nan_posinf_rows: bool,
                        resident: bool = False) -> str:
    """`resident`: the kernel for rows that fit one tile (readout_tile), which keeps the row in
    registers; the other kernel takes any width and reads the row twice."""
    return (f"{sk.name}_readout{'_nanrows' if nan_posinf_rows else ''}_{var.tag()}"
            f"{'_resident' if resident else ''}")


def readout_tile(var: FoldVariant) -> int:
    """Columns of one tile of a readout launch shape (lanes x slots x elements per slot)."""
    per_slot = (4 if dtype_tag(var.dtype)[0] == "f32" else 8) if var.vector else 1
    return var.tpr * var.unroll * per_slot


def emit_readout_source(sk: Skeleton, values: dict | None = None, *, variants: tuple,
                        nan_posinf_rows: bool = True) -> str:
    """A hiprtc unit of the readout phi(x) - r of an exponential fold (log-softmax for
    logsumexp), one kernel per launch shape; see nep_fold.h fold_readout."""
    check_supported(sk)
    if not sk.is_log or sk.two_pass:
        raise NotImplementedError(f"skeleton {sk.name!r}: the readout needs an exponential fold")
    header = (f"// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
              f"// skeleton={sk.name!r}, readout phi(x) - r, nan_posinf_rows={nan_posinf_rows}\n")
    parts = [header, kernel_header("nep_device.h", "nep_fold.h"), emit_fold_policy(sk, values)]
    flag = "true" if nan_posinf_rows else "false"
    seen = set()
    for var in variants:
        _, st = dtype_tag(var.dtype)
        vec = "true" if var.vector else "false"
        for resident in (True, False):
            name = readout_kernel_name(sk, var, nan_posinf_rows, resident)
            if name in seen:
                continue
            seen.add(name)
            parts.append(
                f'extern "C" __global__ void __launch_bounds__({var.wg}) {name}({_FOLD_ARGS_SERIAL}) {{\n'
                f"  nep::fold_readout<Fold, {st}, {var.tpr}, {var.unroll}, {vec}, {var.wg}, {flag}, "
                f"{'true' if resident else 'false'}>("
                f"(const {st}::T*)x, ({st}::T*)out, rows, ncols, stride_row, stride_col);\n}}\n")
    return "\n".join(parts)


def fold_kernel_name(sk: Skeleton, plan: str, stage: str, var: FoldVariant) -> str:
    kind = "two_pass" if sk.two_pass else plan
    return _fold_kernel(sk, kind, stage, var)[0]


# ---------------------------------------------------------------- structured: RMS / L2
@dataclasses.dataclass(frozen=True)
class RowVariant:
    """One launch shape of a row-resident structured kernel."""

    dtype: str
    vector: bool
    tpr: int
    nv: int             # 16-byte slots (or elements) per lane

    @property
    def wg(self) -> int:
        return max(256, self.tpr)

    def tag(self) -> str:
        return f"{dtype_tag(self.dtype)[0]}_{'v' if self.vector else 's'}{self.tpr}n{self.nv}"


def _check_eps(params: dict) -> float:
    import math

    if params.keys() != {"eps"}:
        raise ValueError("RMSNorm requires only the explicit eps parameter")
    eps = params["eps"]
    if type(eps) not in (int, float) or not math.isfinite(eps) or eps <= 0:
        raise ValueError("RMSNorm eps must be finite and positive")
    return float(eps)


def emit_rms_state_source(spec, params=None, *, plan: str = "serial",
                          variants: tuple | None = None) -> str:
    """hiprtc unit for the structured RMSNorm / L2-normalize state (emitters.py:549-627).

    Validates the registered spec and the exact eps; bakes eps as an fp32 literal (the
    reference bakes repr(float(eps)) into its source).  Serial: one row-resident kernel;
    split: partial statistics + map kernel.
    """
    from neptune_codegen.algebra import derive_state_certificate
    from neptune_codegen.skeleton import state_reduction_spec

    if spec.name not in ("rms_norm", "l2_normalize") or spec != state_reduction_spec(spec.name):
        raise NotImplementedError("RMS backend requires the registered sum/count and rounding spec")
    if plan not in ("serial", "split"):
        raise ValueError("RMS plan must be serial or split")
    eps = _check_eps(dict(params or {}))
    derive_state_certificate(spec)
    l2 = "true" if spec.name == "l2_normalize" else "false"
    if variants is None:
        variants = tuple(RowVariant(d, False, 256, 4) for d in DTYPE_TAGS)
    parts = [f"// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
             f"// structured state {spec.name!r}: typed (sum, count); exact-real algebra, not IEEE "
             f"associativity.\n// plan={plan!r}; fp32 stages, input rounding before gamma, "
             "no FMA contraction; fresh output.\n",
             kernel_header("nep_device.h", "nep_rms.h"),
             f"constexpr float kEps = {f32_literal(eps)};  // eps={eps!r}\n"]
    for var in variants:
        _, st = dtype_tag(var.dtype)
        vec = "true" if var.vector else "false"
        if plan == "serial":
            name = f"{spec.name}_serial_{var.tag()}"
            parts.append(
                f'extern "C" __global__ void __launch_bounds__({var.wg}) {name}(const void* x, '
                "const void* gamma, void* out, long long rows, long long ncols, long long stride_row, "
                "long long stride_col, long long stride_gamma) {\n"
                f"  nep::rms_serial<{st}, {var.tpr}, {var.nv}, {vec}, {l2}, {var.wg}>((const {st}::T*)x, "
                f"(const {st}::T*)gamma, ({st}::T*)out, rows, ncols, stride_row, stride_col, "
                "stride_gamma, kEps);\n}\n")
        else:
            pname = f"{spec.name}_partial_{var.tag()}"
            mname = f"{spec.name}_map_{var.tag()}"
            parts.append(
                f'extern "C" __global__ void __launch_bounds__({var.wg}) {pname}(const void* x, '
                "float* totals, long long* counts, long long rows, long long ncols, "
                "long long stride_row, long long stride_col, long long nparts, long long block) {\n"
                f"  nep::rms_split_partial<{st}, {var.tpr}, {var.nv}, {vec}, {var.wg}>("
                f"(const {st}::T*)x, totals, counts, rows, ncols, stride_row, stride_col, nparts, "
                "block);\n}\n")
            parts.append(
                f'extern "C" __global__ void __launch_bounds__({var.wg}) {mname}(const void* x, '
                "const void* gamma, const float* totals, const long long* counts, void* out, "
                "long long rows, long long ncols, long long stride_row, long long stride_col, "
                "long long stride_gamma, long long nparts, long long block) {\n"
                f"  nep::rms_split_map<{st}, {var.tpr}, {var.nv}, {vec}, {l2}, {var.wg}>("
                f"(const {st}::T*)x, (const {st}::T*)gamma, totals, counts, ({st}::T*)out, rows, "
                "ncols, stride_row, stride_col, stride_gamma, nparts, block, kEps);\n}\n")
    return "\n".join(parts)


def rms_kernel_names(spec_name: str, plan: str, var: RowVariant) -> tuple[str, ...]:
    if plan == "serial":
        return (f"{spec_name}_serial_{var.tag()}",)
    return (f"{spec_name}_partial_{var.tag()}", f"{spec_name}_map_{var.tag()}")


# ---------------------------------------------------------------- structured: segments
@dataclasses.dataclass(frozen=True)
class SegmentVariant:
    dtype: str
    span_dtype: str     # "int32" | "int64"
    vector: bool
    lps: int            # lanes per segment (vector path); 64 for the generic path
    unroll: int = 8

    def tag(self) -> str:
        sd = "i32" if self.span_dtype == "int32" else "i64"
        return f"{dtype_tag(self.dtype)[0]}_{sd}_{'v' if self.vector else 's'}{self.lps}u{self.unroll}"


def initial_bits(initial: float | None) -> tuple[int, float]:
    """fp32 bit pattern of the initial value (0.0 when None); overflow saturates to inf."""
    value = 0.0 if initial is None else float(initial)
    try:
        value = struct.unpack("f", struct.pack("f", value))[0]
    except OverflowError:
        value = float("-inf") if value < 0 else float("inf")
    return struct.unpack("I", struct.pack("f", value))[0], value


def emit_segment_source(name: str, *, initial=None, offsets=False, plan="serial",
                        variants: tuple | None = None) -> str:
    """hiprtc unit for segment_sum / segment_mean with ordered storage-dtype rounding."""
    from neptune_codegen.algebra import derive_state_certificate
    from neptune_codegen.skeleton import state_reduction_spec
    from neptune_codegen.torch_op import _segment_params

    spec = state_reduction_spec(name)
    derive_state_certificate(spec)
    params = _segment_params(name, {"initial": initial, "offsets": offsets}, plan)
    bits, _value = initial_bits(params["initial"])
    mean = "true" if name == "segment_mean" else "false"
    none = "true" if params["initial"] is None else "false"
    if variants is None:
        variants = tuple(SegmentVariant(d, "int64", False, 64) for d in DTYPE_TAGS)
    parts = [f"// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
             f"// segment state=(sum,count); exact-real additive certificate only.\n"
             f"// Numeric contract: ordered per-token storage-dtype RTNE; no IEEE reassociation.\n"
             f"// name={name!r}, offsets={params['offsets']!r}, plan={plan!r}; no custom merges "
             "assumed.\n",
             kernel_header("nep_device.h", "nep_segment.h"),
             # the bit pattern keeps the sign of -0.0 and any exact value
             f"constexpr unsigned int kInitialBits = 0x{bits:08x}u;\n"]
    for var in variants:
        _, st = dtype_tag(var.dtype)
        span_t = "int" if var.span_dtype == "int32" else "long long"
        kname = f"{name}_{var.tag()}"
        if var.vector:
            body = (f"nep::segment_vector<{st}, {span_t}, {mean}, {none}, {var.lps}, {var.unroll}, 256>("
                    f"(const {st}::T*)data, (const {span_t}*)spans, ({st}::T*)out, nrows, channels, "
                    "nsegments, stride_row, stride_span, __builtin_bit_cast(float, kInitialBits), "
                    "status, cover);")
            wg = 256
        else:
            body = (f"nep::segment_generic<{st}, {span_t}, {mean}, {none}, {var.unroll}>("
                    f"(const {st}::T*)data, (const {span_t}*)spans, ({st}::T*)out, nrows, channels, "
                    "nsegments, stride_row, stride_channel, stride_span, "
                    "__builtin_bit_cast(float, kInitialBits), status, cover);")
            wg = 64
        parts.append(
            f'extern "C" __global__ void __launch_bounds__({wg}) {kname}(const void* data, '
            "const void* spans, void* out, long long nrows, long long channels, long long nsegments, "
            "long long stride_row, long long stride_channel, long long stride_span, int* status, "
            "long long cover) {\n"
            f"  {body}\n}}\n")
    return "\n".join(parts)


SPAN_BLOCK = 256 * 4           # lengths per workgroup of the spans kernels (nep_segment.h)


def emit_segment_spans_source() -> str:
    """hiprtc unit of the lengths -> spans prefix sum (int32 and int64 lengths)."""
    parts = ["// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
             "// segment lengths -> int64 spans [0, cumsum(lengths)]\n",
             kernel_header("nep_device.h", "nep_segment.h")]
    for tag, ctype in (("i32", "int"), ("i64", "long long")):
        parts.append(
            f'extern "C" __global__ void __launch_bounds__(256) segment_spans_sums_{tag}('
            "const void* lengths, long long n, long long* sums, int* status) {\n"
            f"  nep::spans_block_sums<{ctype}>((const {ctype}*)lengths, n, sums, status);\n}}\n")
        parts.append(
            f'extern "C" __global__ void __launch_bounds__(256) segment_spans_scan_{tag}('
            "const void* lengths, long long n, const long long* sums, long long* spans) {\n"
            f"  nep::spans_scan<{ctype}>((const {ctype}*)lengths, n, sums, spans);\n}}\n")
    return "\n".join(parts)


def segment_kernel_name(name: str, var: SegmentVariant) -> str:
    return f"{name}_{var.tag()}"


# ---------------------------------------------------------------- attention fold
# The attention fold's workgroup, one per CU: at head dim 64, 8 wave64s x 32 queries (two waves
# per SIMD, <= 256 VGPRs each); at head dim 128, 4 wave64s x 64 queries (one wave per SIMD,
# the instruction-scheduled loop of attention_asm.py); at head dim 256, 4 wave64s x 32 queries.
ATTN_HEAD_DIMS = (64, 128, 256)


def attention_w64(head_dim: int, w64: bool | None = None) -> bool:
    """Whether the fold at this head dim is the 64-queries-per-wave kernel (head dim 128;
    `w64=False` selects the compiler-scheduled 32-queries-per-wave kernel there instead)."""
    return head_dim == 128 if w64 is None else (w64 and head_dim == 128)


def attention_waves(head_dim: int, w64: bool | None = None) -> int:
    if attention_w64(head_dim, w64):
        return 4
    return 8 if head_dim <= 128 else 4


def attention_fold_threads(head_dim: int, w64: bool | None = None) -> int:
    return 64 * attention_waves(head_dim, w64)


def attention_block_m(head_dim: int, w64: bool | None = None) -> int:
    """Queries per fold workgroup."""
    per_wave = 64 if attention_w64(head_dim, w64) else 32
    return per_wave * attention_waves(head_dim, w64)


ATTN_DTYPES = {"bfloat16": ("bf16", "__bf16"), "float16": ("f16", "_Float16")}


def _attn_dtype(dtype) -> tuple[str, str]:
    key = str(dtype).replace("torch.", "")
    if key not in ATTN_DTYPES:
        raise TypeError(f"attention fold supports bfloat16 and float16 inputs, got {dtype}")
    return ATTN_DTYPES[key]


def emit_attention_source(head_dim: int, causal: bool, dtype="bfloat16",
                          waves_per_eu: int | None = None, w64: bool | None = None) -> str:
    """hiprtc unit of the online-softmax attention fold (no reference counterpart): the
    logsumexp repair exp(s - s2) applied per key tile to (m, l, O).  Holds two kernels: the
    V^T tile packer and the fold itself (with its exact fallback for out-of-range V)."""
    if head_dim not in ATTN_HEAD_DIMS:
        raise NotImplementedError("attention fold supports head_dim 64, 128 and 256")
    w64 = attention_w64(head_dim, w64)
    wpe = attention_waves(head_dim, w64) // 4 if waves_per_eu is None else waves_per_eu
    threads = attention_fold_threads(head_dim, w64)
    tag, ctype = _attn_dtype(dtype)
    name = attention_kernel_name(head_dim, causal, dtype, w64)
    pack = attention_pack_kernel_name(head_dim, dtype)
    cz = "true" if causal else "false"
    if w64:
        from neptune_codegen.attention_asm import asm_macro
        prefix = asm_macro(causal, tag) + "\n"
        call = f"  nep::attention_fwd_w64<{ctype}, {cz}>("
    else:
        prefix = ""
        call = f"  nep::attention_fwd<{ctype}, {head_dim}, {cz}>("
    return "\n".join([
        "// AUTO-GENERATED by neptune_codegen (HIP emitter) -- do not edit.\n"
        f"// online-softmax attention fold: head_dim={head_dim}, causal={causal}, {tag} inputs; "
        f"{tag} MFMA for Q K^T, fp16 MFMA for P V, fp32 running max/sum.\n",
        prefix + kernel_header("nep_device.h", "nep_attention.h"),
        f'extern "C" __global__ void __launch_bounds__(256) {pack}(const void* v, void* vt, int* exps, '
        "int heads, int sk, long long vsb, long long vsh, long long vss) {\n"
        f"  nep::attention_vt_pack<{ctype}, {head_dim}>((const {ctype}*)v, (nep::u16*)vt, exps, "
        "heads, sk, vsb, vsh, vss);\n}\n",
        f'extern "C" __global__ void __launch_bounds__({threads}, {wpe}) {name}(const void* q, const void* k, '
        "const void* vt, const int* exps, const void* v, void* o, float* lse, int heads, int sq, "
        "int sk, long long qsb, long long qsh, long long qss, long long ksb, long long ksh, "
        "long long kss, long long vsb, long long vsh, long long vss, int e_max, float scale_log2) {\n"
        + call + f"(const {ctype}*)q, "
        f"(const {ctype}*)k, (const nep::u16*)vt, exps, (const {ctype}*)v, ({ctype}*)o, lse, heads, "
        "sq, sk, qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss, e_max, scale_log2);\n}\n"])


def attention_kernel_name(head_dim: int, causal: bool, dtype="bfloat16", w64: bool = False) -> str:
    """The fold's symbol; the 64-queries-per-wave kernel carries a `_w64` suffix."""
    tag, _ = _attn_dtype(dtype)
    suffix = "_w64" if attention_w64(head_dim, w64) and w64 else ""
    return f"attention_fold_{tag}_d{head_dim}_{'causal' if causal else 'full'}{suffix}"


def attention_pack_kernel_name(head_dim: int, dtype="bfloat16") -> str:
    tag, _ = _attn_dtype(dtype)
    return f"attention_vt_pack_{tag}_d{head_dim}"
