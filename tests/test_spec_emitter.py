"""Spec, algebra and HIP emitter -- CPU only (hiprtc compiles for gfx950 without a GPU).

Mirrors the reference's algebra and source-shape tests (tests/test_neptune_opt.py:333-428,
787-853, 957-970; tests/test_autotune.py:374-421, 933-982) for the HIP emitter.
"""
import json
import math
import pathlib

import numpy as np
import pytest
import sympy as sp

import neptune_codegen as CG
from neptune_codegen import emitters as E
from neptune_codegen.symbols import c_sym, s2_sym, s_sym

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def test_repair_slope_golden_table():
    table = json.loads((GOLDEN / "repair_slopes.json").read_text())
    for name, want in table["slopes"].items():
        sk = CG.SKELETONS[name]
        assert str(CG.repair_factor(sk)) == want, name
        assert CG.repair_bias(sk) == table["bias"], name


def test_affine_repair_for_max_consumer_and_refusal_for_sum():
    sk = CG.Skeleton(name="affine_plus", g=c_sym + s_sym, finalize=CG._FINAL_ACC,
                     producer="signed", producer_reducer="max", consumer_reducer="max")
    a, b = CG.repair_pair(sk)
    assert a == 1 and CG._simplify(b - (s2_sym - s_sym)) == 0
    policy = CG.emit_fold_policy(sk, {})
    assert "kHasBias = true" in policy
    bad = CG.Skeleton(name="affine_plus_sum", g=c_sym + s_sym, finalize=CG._FINAL_ACC,
                      producer="signed", producer_reducer="max", consumer_reducer="sum")
    with pytest.raises(NotImplementedError, match="condition 4"):
        CG.repair_pair(bad)


def test_refusals():
    with pytest.raises(NotImplementedError, match="FRESH"):
        CG.repair_pair(CG.Skeleton(name="uses_fresh", g=c_sym * s2_sym, finalize=CG._FINAL_ACC))
    with pytest.raises(NotImplementedError, match="does not depend on the producer"):
        CG.repair_pair(CG.Skeleton(name="no_producer", g=sp.exp(c_sym - sp.Abs(c_sym)),
                                   finalize=CG._FINAL_ACC))
    with pytest.raises(NotImplementedError, match="nonzero"):
        CG.derive_merge_certificate(CG.Skeleton("signed_sum_ratio", c_sym / s_sym, CG._FINAL_ACC,
                                                producer="signed", producer_reducer="sum",
                                                producer_expr=c_sym))
    with pytest.raises(NotImplementedError, match="two_pass"):
        CG.derive_merge_certificate(CG.SKELETONS["variance"])
    with pytest.raises(NotImplementedError):
        CG.emit_kernel_source(CG.SKELETONS["variance"], {}, plan="split")
    with pytest.raises(NotImplementedError, match="SUM consumer"):
        CG.check_supported(CG.Skeleton("lse_max", sp.exp(c_sym - s_sym), CG._FINAL_ACC,
                                       producer="signed", is_log=True, consumer_reducer="max"))
    with pytest.raises(KeyError, match="no value supplied"):
        CG.emit_kernel_source(CG.SKELETONS["softcap_lse"], {"tiny": 0.0})


def test_floor_decisions_and_certificates():
    floors = {n: CG.coordinate_needs_floor(CG.SKELETONS[n]) for n in CG.SKELETONS
              if not CG.SKELETONS[n].two_pass}
    assert floors == {"logsumexp": False, "softcap_lse": False, "lse_biased": False,
                      "lse_scaled": False, "stable_l2": True, "linear_attn": True,
                      "decay_renorm": False, "sumsq_div": True, "rmsnorm_max": False}
    for name, sk in CG.SKELETONS.items():
        if sk.two_pass:
            continue
        params = {**CG.param_defaults(name), **({"eps": 1e-6} if name == "rmsnorm_max" else {})}
        cert = CG.derive_merge_certificate(sk, params)
        assert cert.coordinate_floor == floors[name]


def test_state_certificates():
    for name, spec in CG.STATE_REDUCTIONS.items():
        cert = CG.derive_state_certificate(spec)
        assert cert.state_fields == ("total", "count") and not cert.ieee_associative
    with pytest.raises(NotImplementedError, match="registered"):
        import dataclasses

        CG.emit_rms_state_source(dataclasses.replace(CG.STATE_REDUCTIONS["rms_norm"], name="other"),
                                 {"eps": 1e-6})


def test_translator_rules():
    x, y = sp.symbols("x y", real=True)
    names = {x: "x", y: "y"}
    assert CG.to_hip(sp.exp(x), names) == "nep::fast_exp((x))"          # true exp, no clipping
    assert "fminf" not in CG.to_hip(sp.exp(x), names) and "fmaxf" not in CG.to_hip(sp.exp(x), names)
    assert CG.to_hip(sp.tanh(x), names) == "(2.0f * __builtin_amdgcn_rcpf(1.0f + nep::fast_exp(-2.0f * (x))) - 1.0f)"
    assert CG.to_hip(sp.sqrt(x), names) == "sqrtf((x))"
    assert CG.to_hip(1 / sp.sqrt(x), names) == "(1.0f / sqrtf((x)))"
    assert CG.to_hip(CG._marked((x / y) ** 2), names) == "(((x) / (y)) * ((x) / (y)))"
    # repair slopes: hardware sqrt / rsq / reciprocal, no division left in the expression
    assert CG.to_hip(sp.sqrt(x), names, fast=True) == "nep::fsqrt((x))"
    assert CG.to_hip(1 / sp.sqrt(x), names, fast=True) == "nep::frsq((x))"
    assert CG.to_hip(sp.sqrt(x) / sp.sqrt(y), names, fast=True) == "(nep::fsqrt((x)) * nep::frsq((y)))"
    assert CG.to_hip(CG._marked((x / y) ** 2), names, fast=True) == \
        "(nep::fquot((x), (y)) * nep::fquot((x), (y)))"
    assert CG.to_hip(1 / x, names, fast=True) == "nep::fquot(1.0f, ((x)))"
    # literals are rounded to fp32 exactly once
    assert CG.to_hip(sp.Float(0.1), names) == f"{np.float32(0.1).item().hex()}f"
    with pytest.raises(CG.TranslationError):
        CG.to_hip(x ** sp.Rational(1, 3), names)  # base not provably positive


def test_emitted_units_compile_for_gfx950():
    """Every supported skeleton (serial, split where legal), RMS/L2 (both plans), both segment
    reductions and the attention fold compile with hiprtc for gfx950."""
    from neptune_codegen import hip

    names = []
    for name in CG.supported():
        sk = CG.SKELETONS[name]
        params = {**CG.param_defaults(name), **({"eps": 1e-6} if name == "rmsnorm_max" else {})}
        plans = ["serial"] if sk.two_pass else ["serial", "split"]
        for plan in plans:
            var = E.FoldVariant("bfloat16", True, 32, 4, 4)
            src = CG.emit_kernel_source(sk, params, plan=plan, variants=(var,))
            assert "fminf(fmaxf" not in src   # no clipped exponentials
            assert hip.compile_code_object(src, f"{name}_{plan}.hip", E.BASE_OPTIONS, write_cache=False) > 0
            names.append(E.fold_kernel_name(sk, plan, "partial" if plan == "split" else "", var))
    for spec in ("rms_norm", "l2_normalize"):
        for plan in ("serial", "split"):
            src = CG.emit_rms_state_source(CG.STATE_REDUCTIONS[spec], {"eps": 1e-6}, plan=plan)
            assert hip.compile_code_object(src, "rms.hip", E.BASE_OPTIONS + E.NO_CONTRACT, write_cache=False) > 0
    for name in ("segment_sum", "segment_mean"):
        src = CG.emit_segment_source(name, initial=-0.0)
        assert "0x80000000u" in src      # the sign of -0.0 survives as a bit pattern
        assert hip.compile_code_object(src, "seg.hip", E.BASE_OPTIONS + E.NO_CONTRACT, write_cache=False) > 0
    for w64 in (True, False):      # head dim 128: both fold kernels
        src = E.emit_attention_source(128, True, w64=w64)
        assert ("#define NEP_ATTN_W64_ASM" in src) == w64
        assert hip.compile_code_object(src, "attn.hip", E.BASE_OPTIONS, write_cache=False) > 0
    assert len(set(names)) == len(names)


def test_emitted_source_is_deterministic_and_parameter_exact():
    sk = CG.SKELETONS["softcap_lse"]
    a = CG.emit_kernel_source(sk, {"beta": 1.0000001, "tiny": 0.0})
    b = CG.emit_kernel_source(sk, {"tiny": 0.0, "beta": 1.0000001})
    c = CG.emit_kernel_source(sk, {"beta": 1.0000002, "tiny": 0.0})
    assert a == b and a != c
    rms = CG.emit_rms_state_source(CG.STATE_REDUCTIONS["rms_norm"], {"eps": 1e-6})
    assert f"kEps = {np.float32(1e-6).item().hex()}f" in rms
    assert "-ffp-contract=off" in E.NO_CONTRACT and "-packed-fp32-ops" in E.BASE_OPTIONS


def test_supported_and_registry():
    assert CG.supported() == ["decay_renorm", "linear_attn", "logsumexp", "lse_biased",
                              "lse_scaled", "rmsnorm_max", "softcap_lse", "stable_l2", "std",
                              "sumsq_div", "variance"]
    with pytest.raises(ValueError, match="already registered"):
        CG.register(CG.Skeleton(name="logsumexp", g=c_sym, finalize=CG._FINAL_ACC))
    assert CG.param_defaults("lse_scaled") == {"T": 2.0, "tiny": 0.0}
    assert CG.param_defaults("rmsnorm_max") == {"eps": 1.0}


def test_param_bindings_is_exported_and_bakes_fp32_literals():
    """The reference exports param_bindings from neptune_codegen (__init__.py:147-156): scalar
    parameters become source literals, intrinsic row lengths the kernel's n."""
    import neptune_codegen as CG

    bound = CG.param_bindings(CG.SKELETONS["lse_scaled"], {"T": 2.0, "tiny": 0.0})
    assert {str(k): v for k, v in bound.items()} == {"T": "0x1.0000000000000p+1f", "tiny": "0.0f"}
    assert {str(k): v for k, v in CG.param_bindings(CG.SKELETONS["variance"]).items()} == {"N": "n"}
    with pytest.raises(KeyError, match="beta"):
        CG.param_bindings(CG.SKELETONS["softcap_lse"], {"tiny": 0.0})


def test_readout_source_holds_a_resident_and_a_two_read_kernel_per_shape():
    """Each readout launch shape is emitted twice: the resident kernel (rows of at most
    readout_tile columns, held in registers) and the two-read kernel (any width)."""
    var = E.FoldVariant("bfloat16", True, 512, 8, 8)
    assert E.readout_tile(var) == 512 * 8 * 8
    assert E.readout_tile(E.FoldVariant("float32", True, 256, 4, 4)) == 256 * 4 * 4
    assert E.readout_tile(E.FoldVariant("float16", False, 64, 8, 1)) == 64 * 8
    sk = CG.SKELETONS["logsumexp"]
    src = E.emit_readout_source(sk, CG.param_defaults("logsumexp"), variants=(var,))
    resident = E.readout_kernel_name(sk, var, True, True)
    two_read = E.readout_kernel_name(sk, var, True, False)
    assert resident == two_read + "_resident"
    assert f"{resident}(" in src and f"{two_read}(" in src
    assert src.count("nep::fold_readout<") == 2


def test_row_variant_rule_for_16_bit_rows():
    """RMS / L2 launch shapes: 4 slots per lane for 16-bit rows of 2048-8192 elements, 2 at
    1024, 8 otherwise (fp32 rows keep 8)."""
    import torch

    from neptune_codegen import template as T

    want = {1000: (16, 8), 1024: (64, 2), 2048: (64, 4), 4096: (128, 4), 8192: (256, 4),
            16384: (256, 8), 32768: (512, 8)}
    for width, (tpr, nv) in want.items():
        x = torch.empty(4, width, dtype=torch.bfloat16, device="meta")
        var = T._row_variant(x, None, width)
        assert (var.tpr, var.nv, var.vector) == (tpr, nv, True), width
        assert var.tpr * var.nv * 8 >= width
    x = torch.empty(4, 4096, dtype=torch.float32, device="meta")
    assert T._row_variant(x, None, 4096).nv == 8
