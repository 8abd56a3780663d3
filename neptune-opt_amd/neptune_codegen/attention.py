"""Online-softmax attention fold: O = softmax(scale * Q K^T [+ causal mask]) V.

There is no reference function for this path (attention-chain fusion is a non-goal of the
reference, docs/roadmap.md:28-30); the fold is the logsumexp skeleton's repair
exp(s - s2) (tests/test_neptune_opt.py:347) applied per key tile to the running
(max, sum, output) state, with MFMA for Q K^T and P V.  The causal mask is torch's
`is_causal=True` (query i sees keys j <= i).  The oracle is the closed form in fp32.

Layout contract: q [B, H, Sq, D], k/v [B, H, Sk, D], D in {64, 128, 256}, one dtype (bf16 or
fp16), unit stride on D; other strides are honoured (rows must be 16-byte aligned, otherwise the input is made
contiguous).  Output is a fresh contiguous [B, H, Sq, D] tensor of the input dtype;
`return_lse` adds the fp32 [B, H, Sq] natural-log logsumexp of the scaled, masked scores.

Every input has a result; nothing is refused at run time and no device-side assert is used.
The MFMA path feeds V to the P.V product as fp16 images scaled per 64-key tile by a power of
two (exact for |v| < 2^28 in a tile, see V_EXPONENT_MAX).  A workgroup whose keys include a
tile beyond that (|v| >= 2^28, inf or NaN) recomputes its queries with the kernel's exact fp32
path: O = sum_j p_j v_j / sum_j p_j over the visible keys in IEEE fp32, so only rows that see
a non-finite V value become non-finite.
"""
from __future__ import annotations

import math
import threading

from neptune_codegen import hip
from neptune_codegen.emitters import (ATTN_HEAD_DIMS, BASE_OPTIONS, attention_block_m,
                                      attention_fold_threads, attention_kernel_name,
                                      attention_pack_kernel_name, attention_w64,
                                      emit_attention_source)

_PROGRAMS: dict = {}
_OPS: dict = {}
_lock = threading.Lock()
LOG2E = 1.4426950408889634
BLOCK_M = 256           # queries per fold workgroup up to head dim 128 (8 waves of 32)
BLOCK_N = 64            # keys per tile (one V^T image per tile)
K_ROW_STRIDE_MAX = 1 << 24   # K rows are addressed with 32-bit byte offsets within a tile
Q_ROW_STRIDE_MAX = 1 << 22   # head dim 128: Q rows, with 32-bit byte offsets within 256 rows
# V^T tiles are fp16 images of v * 2^-e, e the tile's exponent (0 below 2^15).  A tile value
# below 2^(e - 14) keeps only an absolute precision of 2^(e - 25), which bounds the error it
# adds to O; e <= 13 keeps that under 2^-12, a quarter of the bf16 absolute tolerance.  Blocks
# of queries that see a larger tile, or inf/NaN in V, take the exact fp32 path.  (fp32
# accumulation of O, |O acc| <= keys * 2^8 * 2^28, cannot overflow at this bound.)
V_EXPONENT_MAX = 13
# Head dim 128 has two fold kernels with bit-identical results: 8 waves x 32 queries
# (compiler-scheduled) and 4 waves x 64 queries (the instruction-scheduled loop of
# attention_asm.py).  The second is faster per key tile (one LDS fragment feeds two MFMAs, the
# softmax issues between them) but has the larger fixed cost per workgroup and idles a SIMD
# whenever one of its waves is past its causal diagonal.  Measured op-time ratios on MI355X
# (graph replays, the two kernels interleaved in one process, two boxes): non-causal 0.93-0.97
# from 512 keys (1.08 at 256); causal 0.957-0.990 from 3072 queries (B*H 32-128), 0.985 at
# 2048 and 1.03 at 1024, 1536 and 2560.
W64_MIN_SK = 512
W64_CAUSAL_MIN_SQ = 3072


def use_w64(head_dim: int, causal: bool, sq: int, sk: int) -> bool:
    """Whether a fold of this shape runs the 64-queries-per-wave kernel."""
    if head_dim != 128:
        return False
    return sq >= W64_CAUSAL_MIN_SQ if causal else sk >= W64_MIN_SK


def _program(head_dim: int, causal: bool, dtype="bfloat16", w64: bool | None = None) -> hip.Program:
    w64 = attention_w64(head_dim, w64)
    key = (head_dim, causal, str(dtype), w64)
    with _lock:
        prog = _PROGRAMS.get(key)
        if prog is None:
            prog = hip.Program(emit_attention_source(head_dim, causal, dtype, w64=w64),
                               f"{attention_kernel_name(head_dim, causal, dtype, w64)}.hip", BASE_OPTIONS)
            _PROGRAMS[key] = prog
        return prog


def validate_attention_inputs(q, k, v, *, metadata: bool = False):
    import torch

    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        if t.layout != torch.strided:
            raise TypeError(f"attention {nm} must be strided")
        if t.ndim != 4:
            raise ValueError(f"attention {nm} must be [batch, heads, seq, head_dim]")
        if t.dtype not in (torch.bfloat16, torch.float16):
            raise TypeError(f"attention fold supports bfloat16 and float16 inputs, got {t.dtype} for {nm}")
        if not metadata and t.device.type != "cuda":
            raise ValueError("attention execution requires a ROCm (cuda) device")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise ValueError(f"attention shapes do not match: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"attention q, k, v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.device != k.device or q.device != v.device:
        raise ValueError("attention tensors must be on the same device")
    if q.shape[3] not in ATTN_HEAD_DIMS:
        raise NotImplementedError("attention fold supports head_dim 64, 128 and 256")
    if k.shape[2] == 0:
        raise ValueError("attention needs at least one key")
    return tuple(q.shape)


def _kernel_ready(t):
    ok = (t.stride(3) == 1 and all(s % 8 == 0 for s in t.stride()[:3]) and t.data_ptr() % 16 == 0)
    return t if ok else t.contiguous()


def run_attention(q, k, v, *, scale: float | None = None, causal: bool = True,
                  return_lse: bool = False):
    """Attention fold on the current stream; see the module docstring for the contract."""
    out, lse, _ = launch_attention(q, k, v, scale=scale, causal=causal, return_lse=return_lse)
    return (out, lse) if return_lse else out


def launch_attention(q, k, v, *, scale: float | None = None, causal: bool = True,
                     return_lse: bool = False):
    """(out, lse or None, exps or None): the fold's two launches.  `exps` is the int32 tile
    exponent table [B*H*ceil(Sk/64)] the V^T pack wrote (None when nothing was launched);
    `exact_path_taken(exps)` tells whether some query block took the exact fp32 path."""
    return _launch(q, k, v, scale, causal, return_lse, V_EXPONENT_MAX)


def _launch(q, k, v, scale, causal, return_lse, e_max: int, w64: bool | None = None):
    """The launches with the exact path's threshold as a parameter: e_max = -1 sends every
    query block through the exact fp32 path (the tests compare the two paths with it).
    `w64=False` runs the compiler-scheduled 32-queries-per-wave kernel at head dim 128 instead
    of the instruction-scheduled one (the tests compare the two bit for bit)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensor

    metadata = isinstance(q, FakeTensor) or q.device.type == "meta"
    shape = validate_attention_inputs(q, k, v, metadata=metadata)
    B, H, Sq, D = shape
    out = torch.empty(shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device) if return_lse else None
    if metadata or out.numel() == 0:
        return out, lse, None
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("attention scale must be finite and positive")
    if w64 is None:
        w64 = use_w64(D, causal, Sq, k.shape[2])
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    if k.stride(2) >= K_ROW_STRIDE_MAX:
        k = k.contiguous()
    if q.stride(2) >= Q_ROW_STRIDE_MAX:
        q = q.contiguous()
    device = q.device.index if q.device.index is not None else torch.cuda.current_device()
    Sk = k.shape[2]
    ntiles = (Sk + BLOCK_N - 1) // BLOCK_N
    # V^T tile images (fp16, MFMA operand order) and one power-of-two exponent per tile
    vt = torch.empty((B * H * ntiles * D * BLOCK_N,), dtype=torch.float16, device=q.device)
    exps = torch.empty((B * H * ntiles,), dtype=torch.int32, device=q.device)
    prog = _program(D, causal, q.dtype, w64)
    pack = prog.kernel(attention_pack_kernel_name(D, q.dtype),
                       (hip.PTR,) * 3 + (hip.I32,) * 2 + (hip.I64,) * 3, 256, device)
    fold = prog.kernel(attention_kernel_name(D, causal, q.dtype, attention_w64(D, w64)),
                       (hip.PTR,) * 7 + (hip.I32,) * 3 + (hip.I64,) * 9 + (hip.I32, hip.F32),
                       attention_fold_threads(D, w64), device)
    stream = hip.current_stream(q.device)
    pack.launch((B * H * ntiles,),
                (v.data_ptr(), vt.data_ptr(), exps.data_ptr(), H, Sk,
                 v.stride(0), v.stride(1), v.stride(2)), stream)
    bm = attention_block_m(D, w64)
    nqb = (Sq + bm - 1) // bm
    fold.launch((nqb * B * H,),
                (q.data_ptr(), k.data_ptr(), vt.data_ptr(), exps.data_ptr(), v.data_ptr(),
                 out.data_ptr(), lse.data_ptr() if lse is not None else 0, H, Sq, Sk,
                 q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
                 v.stride(0), v.stride(1), v.stride(2), int(e_max), scale * LOG2E), stream)
    return out, lse, exps


def exact_path_taken(exps) -> bool:
    """Host check (synchronises): some V tile was beyond the MFMA path's range, so the query
    blocks that see it were computed by the exact fp32 path."""
    return bool((exps > V_EXPONENT_MAX).any().item())


attention_fold = run_attention


def as_attention_op(scale: float | None = None, causal: bool = True, lib: str = "neptune"):
    """Custom op `(Tensor q, Tensor k, Tensor v) -> Tensor` with scale and mask in its name."""
    import torch

    from neptune_codegen.autotune import parameter_tag

    params = {"scale": float(scale)} if scale is not None else {}
    key = (lib, tuple(sorted(params.items())), causal)
    with _lock:
        if key in _OPS:
            return _OPS[key]
    name = f"attention_fold{parameter_tag(params)}_{'causal' if causal else 'full'}"

    def _impl(q, k, v):
        return run_attention(q, k, v, scale=scale, causal=causal)

    def _fake(q, k, v):
        validate_attention_inputs(q, k, v, metadata=True)
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)

    op = torch.library.custom_op(f"{lib}::{name}", mutates_args=(),
                                 schema="(Tensor q, Tensor k, Tensor v) -> Tensor")(_impl)
    op.register_fake(_fake)
    with _lock:
        _OPS[key] = op
    return op
