"""Kernel units behind the benchmark configurations, enumerated without a GPU.

Launch-shape selection only reads shapes, strides, dtypes and pointer alignment, so meta
tensors (data pointer 0, always aligned) reproduce the variants a real launch picks.
"""
from __future__ import annotations


def _fold_programs():
    import torch

    from neptune_codegen.autotune import best_config
    from neptune_codegen.skeleton import param_defaults
    from neptune_codegen.template import _fold_variant, compile_skeleton

    out = []
    lse = param_defaults("logsumexp")
    shapes = [(8192, 1024, torch.float32)] + [(16384, w, torch.bfloat16) for w in (128, 1000, 4096, 32000)]
    for rows, ncols, dtype in shapes:
        x2 = torch.empty((rows, ncols), device="meta", dtype=dtype)
        block, warps = best_config(rows, ncols, dtype, None, device_name="gfx950")
        var = _fold_variant(x2, ncols, block, warps)
        out.append(compile_skeleton("logsumexp", lse).program(var))
    from neptune_codegen.skeleton import supported

    x2 = torch.empty((16384, 4096), device="meta", dtype=torch.float32)
    block, warps = best_config(16384, 4096, torch.float32, None, device_name="gfx950")
    for name in supported():
        params = {**param_defaults(name), **({"eps": 1e-6} if name == "rmsnorm_max" else {})}
        prog = compile_skeleton(name, params)
        sk = prog.sk
        out.append(prog.program(_fold_variant(x2, 4096, block, warps, resident=sk.two_pass,
                                              merge_heavy=not sk.is_log and not sk.two_pass,
                                              heavy_phi=prog.heavy_phi)))
    from neptune_codegen.template import compile_readout

    xw = torch.empty((16384, 32000), device="meta", dtype=torch.bfloat16)
    block, warps = best_config(16384, 32000, torch.bfloat16, None, device_name="gfx950")
    out.append(compile_readout("logsumexp").program(
        _fold_variant(xw, 32000, block, warps, resident=True)))
    x2 = torch.empty((64, 262144), device="meta", dtype=torch.bfloat16)
    partial, _merge = compile_skeleton("logsumexp", lse, plan="split")
    out.append(partial.program(_fold_variant(x2, 262144, 1024, 4, split_block=1024)))
    return out


def _row_programs():
    import torch

    from neptune_codegen.template import _row_variant, compile_state_reduction

    out = []
    x = torch.empty((32768, 4096), device="meta", dtype=torch.bfloat16)
    g = torch.empty((4096,), device="meta", dtype=torch.bfloat16)
    out.append(compile_state_reduction("rms_norm", {"eps": 1e-6}).program(_row_variant(x, g, 4096)))
    out.append(compile_state_reduction("l2_normalize", {"eps": 1e-6}).program(_row_variant(x, None, 4096)))
    return out


def _segment_programs():
    import torch

    from neptune_codegen.torch_op import _segment_variant, compile_segment_reduction

    out = []
    data = torch.empty((1310720, 128), device="meta", dtype=torch.float16)
    spans = torch.empty((65537,), device="meta", dtype=torch.int32)
    for name in ("segment_sum", "segment_mean"):
        prog = compile_segment_reduction(name, {"offsets": True})
        out.append(prog.program(_segment_variant(data, spans, 128)))
    return out


def _attention_programs():
    from neptune_codegen.attention import _program

    # head dim 128: both fold kernels (attention.use_w64 picks one by shape)
    return [_program(128, c, dt, w) for c in (True, False) for dt in ("bfloat16", "float16")
            for w in (True, False)] + [
        _program(64, True), _program(64, False), _program(64, False, "float16"),
        _program(256, True), _program(256, False), _program(256, True, "float16")]


def programs():
    return _fold_programs() + _row_programs() + _segment_programs() + _attention_programs()
