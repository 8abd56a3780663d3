"""neptune_codegen -- MI355X (gfx950) HIP backend for neptune-opt's fused dependent-reduction folds.

The public surface mirrors the reference package's (neptune_codegen/__init__.py:63-174): fold
specs and the registry, the repair algebra and certificates, the emitter entry points, the
direct `run*` launches and the custom-op bridge.  Kernels are generated HIP compiled by hiprtc
and launched through the C-ABI library libneptune_hip.so; there is no other execution path.
The eager references the kernels are checked against live in the repository's `oracle/`
package (test infrastructure), not here.
"""
from __future__ import annotations

from neptune_codegen import hip, library  # noqa: F401  (library populates SKELETONS)
from neptune_codegen.algebra import (_BRANCH_CUT, MergeCertificate, StateCertificate, _Q,
                                     _as_quotient_power, _marked, _numerically_zero, _simplify,
                                     coordinate_needs_floor,
                                     derive_merge_certificate, derive_state_certificate,
                                     reachable_producer_domain, repair_bias, repair_factor,
                                     repair_pair, term_expr, vanishes)
from neptune_codegen.attention import (as_attention_op, attention_fold, exact_path_taken,
                                       launch_attention, run_attention)
from neptune_codegen.autotune import best_config, machine_key, op_key, parameter_tag
from neptune_codegen.emitters import (check_supported, derived_producer_expr, emit_fold_policy,
                                      emit_kernel_source, emit_rms_state_source,
                                      emit_segment_source, param_bindings)
from neptune_codegen.skeleton import (NEGATIVE_CONTROLS, SKELETONS, STATE_REDUCTIONS,
                                      NumericalContract, Skeleton, StateField, StateReduction,
                                      all_registered, param_defaults, register,
                                      state_reduction_spec, supported, unsupported_reason)
from neptune_codegen.sym_to_hip import TranslationError, to_hip
from neptune_codegen.symbols import *  # noqa: F401,F403
from neptune_codegen.template import (_CACHE, MAX_SPLIT_PARTS, compile_skeleton, compile_state_reduction,
                                      compile_readout, generated_path, launch_reduction,
                                      launch_rms_norm, run, run_l2_normalize, run_log_softmax,
                                      run_readout, run_rms_norm, split_launch_shape,
                                      validate_l2_inputs, validate_plan, validate_rms_inputs)
from neptune_codegen.torch_op import (_TRITON_OPS, as_hip_op, as_readout_op, as_segment_op, as_state_op,
                                      as_triton_op, compile_segment_reduction, op_handle,
                                      readout_op_handle, run_segment_pool,
                                      segment_op_handle, state_op_handle, triton_op_name,
                                      validate_segment_inputs)


def prebuilt_programs():
    """The hiprtc units behind the benchmark configurations (built ahead by build.py)."""
    from neptune_codegen.prebuilt import programs

    return programs()


__all__ = [
    "Skeleton", "SKELETONS", "register", "supported", "all_registered", "unsupported_reason",
    "param_defaults", "NEGATIVE_CONTROLS", "StateField", "StateReduction", "NumericalContract",
    "STATE_REDUCTIONS", "state_reduction_spec",
    "repair_pair", "repair_factor", "repair_bias", "term_expr", "vanishes", "_simplify",
    "_marked", "_as_quotient_power", "coordinate_needs_floor", "reachable_producer_domain",
    "derive_merge_certificate", "derive_state_certificate", "MergeCertificate",
    "StateCertificate",
    "to_hip", "TranslationError", "check_supported", "derived_producer_expr",
    "emit_fold_policy", "emit_kernel_source", "emit_rms_state_source", "emit_segment_source",
    "param_bindings",
    "MAX_SPLIT_PARTS", "validate_plan", "split_launch_shape", "compile_skeleton",
    "compile_state_reduction", "generated_path", "launch_reduction", "launch_rms_norm", "run",
    "run_rms_norm", "run_l2_normalize", "validate_rms_inputs", "validate_l2_inputs",
    "as_triton_op", "as_hip_op", "op_handle", "triton_op_name", "as_state_op",
    "state_op_handle", "as_segment_op", "segment_op_handle", "run_segment_pool",
    "compile_segment_reduction", "validate_segment_inputs",
    "run_attention", "attention_fold", "as_attention_op", "launch_attention", "exact_path_taken",
    "compile_readout", "run_readout", "run_log_softmax", "as_readout_op", "readout_op_handle",
    "best_config", "machine_key", "op_key", "parameter_tag", "prebuilt_programs",
    # internals the reference package also exports: the algebra's quotient-power marker and
    # numeric zero filter with its branch-cut list, the compiled-unit cache, the op registry
    # (HIP ops, under the reference's name) and the directory of generated artefacts (here
    # the code-object cache)
    "_Q", "_numerically_zero", "_BRANCH_CUT", "_CACHE", "_TRITON_OPS", "_GEN_DIR",
]
_GEN_DIR = str(hip.CACHE_DIR)
