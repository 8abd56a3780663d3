"""Test infrastructure: CPU restatements of the reference algorithms the HIP kernels must match.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and
only as the checker (or as the timed CPU baseline).  No product code path reaches it; the
neptune_codegen package fails loudly without its HIP library instead of falling back here.

Modules:
  references  closed-form eager references (torch on the CPU), restating
              neptune_codegen/references.py:18-97 of the reference plus the canonical RMSNorm
              (README.md:121-127), torch.segment_reduce, F.normalize and causal SDPA.
  fold        numpy replay of the fold state machine (chunk / merge_state / finalize) of
              neptune_codegen/emitters.py:436-532, used to pin the status/seen semantics.
  exact       ctypes bindings to the C restatement in oracle/csrc (bit-level: ordered
              segment rounding, correctly rounded rsqrt/div, RMS staging).

Parity status per function is stated in each module's header.
"""
