"""Writes the golden fixtures in this directory.

Inputs are the case tables of the reference's own tests (cited per fixture).  Expected values
come from closed forms evaluated in float64 (math / numpy) or, for segment pooling, from
torch.segment_reduce on the CPU -- the oracle the reference's own segment test uses
(tests/test_autotune.py:793-833).  No code of this repository computes an expected value here.

    python tests/golden/make_goldens.py
"""
from __future__ import annotations

import json
import math
import pathlib

HERE = pathlib.Path(__file__).resolve().parent


def enc(x: float):
    if math.isnan(x):
        return "nan"
    if math.isinf(x):
        return "inf" if x > 0 else "-inf"
    return x


def lse64(values):
    finite = [v for v in values if not math.isnan(v)]
    if any(math.isnan(v) for v in values):
        return float("nan")
    if any(v == math.inf for v in values):
        return math.inf
    finite = [v for v in values if v != -math.inf]
    if not finite:
        return -math.inf
    m = max(finite)
    return m + math.log(sum(math.exp(v - m) for v in finite))


def main():
    inf, nan = math.inf, math.nan
    # 1. repair slope golden table: tests/test_neptune_opt.py:344-353
    (HERE / "repair_slopes.json").write_text(json.dumps({
        "source": "reference tests/test_neptune_opt.py:344-353",
        "bias": 0,
        "slopes": {"decay_renorm": "(N + s)/(N + s2)", "linear_attn": "s/s2",
                   "logsumexp": "exp(s - s2)", "lse_biased": "exp(s - s2)",
                   "rmsnorm_max": "sqrt(eps + s)/sqrt(eps + s2)", "softcap_lse": "exp(s - s2)",
                   "stable_l2": "s**2/s2**2", "sumsq_div": "s/s2"}}, indent=1))
    # 2. exponential-fold chunk status / seen after merging two one-element chunks:
    #    tests/test_neptune_opt.py:938-955
    (HERE / "lse_chunk_status.json").write_text(json.dumps({
        "source": "reference tests/test_neptune_opt.py:938-955 (logsumexp, tiny=0, block 1)",
        "cases": [{"data": [enc(-inf), enc(-inf)], "status": 0, "seen": 0},
                  {"data": [enc(inf), 1.0], "status": 2, "seen": 1},
                  {"data": [enc(nan), enc(inf)], "status": 3, "seen": 0},
                  {"data": [enc(-inf), 1.0], "status": 0, "seen": 1}]}, indent=1))
    # 3. finalizer special values for every exponential fold: tests/test_neptune_opt.py:988-1015
    data_cases = [[nan, inf, 1.0], [inf, -inf, 1.0], [-inf, -inf, -inf], [0.0, -100.0, -200.0]]
    phis = {"logsumexp": lambda v: v, "lse_biased": lambda v: v + 1.0,
            "softcap_lse": lambda v: math.tanh(v) if not math.isnan(v) else nan,
            "lse_scaled": lambda v: v / 2.0}
    (HERE / "lse_finalizer_cases.json").write_text(json.dumps({
        "source": "reference tests/test_neptune_opt.py:988-1015; expected = float64 logsumexp of phi "
                  "(defaults: alpha=1, beta=1, T=2, tiny=0)",
        "cases": [{"skeleton": n, "data": [enc(v) for v in d], "expected": enc(lse64([phi(v) for v in d]))}
                  for n, phi in phis.items() for d in data_cases]}, indent=1))
    # 4. split capacity: tests/test_neptune_opt.py:957-970
    (HERE / "split_capacity.json").write_text(json.dumps({
        "source": "reference tests/test_neptune_opt.py:957-970",
        "ok": [[1025, 1024, 2, 2], [4096, 1, 4096, 4096], [262144, 1024, 256, 256]],
        "refused": [{"ncols": 4097, "block": 1, "error": "NotImplementedError", "match": "capacity"},
                    {"ncols": 32, "block": 3, "error": "ValueError", "match": "power of two"}]}, indent=1))
    # 5. operator identity: tests/test_autotune.py:106-112, 121-127, 279, 290
    (HERE / "op_keys.json").write_text(json.dumps({
        "source": "reference tests/test_autotune.py:106-112,121-127,279,290",
        "op_key": [[["neptune", "logsumexp", {}, True, 1024, 4], "neptune::logsumexp_keep_b1024w4"],
                   [["neptune", "logsumexp", {"tiny": 0.0}, True, 8192, 8], "neptune::logsumexp_keep_tiny0_b8192w8"],
                   [["neptune", "logsumexp", {"T": 2.0}, True, None, None], "neptune::logsumexp_keep_T2"]],
        "machine_key": [["NVIDIA GeForce RTX 5090 D v2", "rtx-5090-d-v2"], ["NVIDIA GeForce RTX 4090 D", "rtx-4090-d"],
                        ["Tesla V100-PCIE-32GB", "v100-pcie-32gb"], ["", ""]]}, indent=1))
    # 6. merge associativity inputs: tests/test_neptune_opt.py:907-936
    (HERE / "merge_invariants.json").write_text(json.dumps({
        "source": "reference tests/test_neptune_opt.py:907-936",
        "partition_data": [-3.0, 0.0, 2.0, 1.0, -1.0, 0.0, 5.0], "partition_block": 2, "rtol": 2e-6, "atol": 1e-6,
        "zero_floor_data": [0.0, 0.5e-30, 0.5e-30],
        "zero_floor_skeletons": ["stable_l2", "linear_attn", "sumsq_div"]}, indent=1))
    # 7. declared parameter defaults per skeleton, as the reference's registry states them
    #    (neptune_codegen/library.py:27-28 logsumexp, :55 decay_renorm, :67-68 softcap_lse,
    #    :87-88 rmsnorm_max, :109-110 lse_biased, :170-175 lse_scaled; no params for stable_l2,
    #    linear_attn, sumsq_div, variance, std) with param_defaults' 1.0 fallback for an
    #    undeclared scalar and intrinsic ncols left out (neptune_codegen/skeleton.py:255-267)
    (HERE / "param_defaults.json").write_text(json.dumps({
        "source": "reference neptune_codegen/library.py:19-177 declarations, "
                  "skeleton.py:255-267 fallback rule",
        "defaults": {"logsumexp": {"tiny": 0.0}, "stable_l2": {}, "linear_attn": {},
                     "decay_renorm": {"N": 1.0}, "softcap_lse": {"beta": 1.0, "tiny": 0.0},
                     "rmsnorm_max": {"eps": 1.0}, "sumsq_div": {},
                     "lse_biased": {"alpha": 1.0, "tiny": 0.0}, "variance": {}, "std": {},
                     "lse_scaled": {"T": 2.0, "tiny": 0.0}}}, indent=1))
    # 8. segment pooling: tests/test_autotune.py:793-833, expected from torch.segment_reduce (CPU)
    import torch

    cases = []
    for dtype in ("float16", "bfloat16", "float32"):
        dt = getattr(torch, dtype)
        base = torch.full((1027, 2, 6), 0.1, dtype=dt)
        base[1, 0, 0] = float("inf")
        base[2, 0, 0] = -float("inf")
        base[3, 1, 2] = float("nan")
        base[4, 1, 4] = -float("inf")
        data = base[:, :, ::2].contiguous().reshape(1027, 6)
        for initial in (None, 0.0, -2.125):
            for reduce in ("sum", "mean"):
                for lengths, offsets in (([0, 2, 1025, 0], False), ([1, 1, 3, 1026], True)):
                    seg = torch.tensor(lengths, dtype=torch.int64)
                    kw = {"offsets" if offsets else "lengths": seg}
                    out = torch.segment_reduce(data, reduce, axis=0, initial=initial, **kw)
                    view = torch.int16 if dt != torch.float32 else torch.int32
                    cases.append({"dtype": dtype, "initial": initial, "reduce": reduce,
                                  "segments": lengths, "offsets": offsets,
                                  "nan": torch.isnan(out).flatten().tolist(),
                                  "bits": out.masked_fill(torch.isnan(out), 0).view(view).flatten().tolist()})
        tiny = torch.tensor([[1e-40, -0.0], [1e-40, 0.0]], dtype=dt)
        for reduce in ("sum", "mean"):
            out = torch.segment_reduce(tiny, reduce, axis=0, lengths=torch.tensor([0, 2]), initial=-0.0)
            view = torch.int16 if dt != torch.float32 else torch.int32
            cases.append({"dtype": dtype, "initial": -0.0, "reduce": reduce, "segments": [0, 2],
                          "offsets": False, "data": "signed_zero_denormal",
                          "nan": torch.isnan(out).flatten().tolist(),
                          "bits": out.masked_fill(torch.isnan(out), 0).view(view).flatten().tolist()})
    (HERE / "segment_cases.json").write_text(json.dumps({
        "source": "reference tests/test_autotune.py:793-833 case table (data base[:, :, ::2] of a "
                  "(1027, 2, 6) tensor filled with 0.1 and inf/-inf/nan at [1,0,0],[2,0,0],[3,1,2],[4,1,4]); "
                  "expected bits from torch.segment_reduce on the CPU",
        "cases": cases}))
    print("goldens written to", HERE)


if __name__ == "__main__":
    main()
