"""CPU checks of the generated head-dim-128 attention loop (neptune_codegen/attention_asm.py).

The GPU tests hold its results bit-identical to the compiler-scheduled kernel; these re-read the
emitted text with checkers written independently of the generator's own bookkeeping:
  * every branch target is defined once and every label is reached;
  * along execution paths through the loop (steady tiles, rescale and mask, a wave's first
    finite tile, its last tile, a wave past its last tile), the wait states the generator promises hold: 20 between an
    MFMA writing a register and a VALU touching it, 4 between a VALU write and an MFMA reading
    it, 2 after an exponential or a VCC write, 2 between an MFMA reading a fragment quad and
    the LDS read refilling it, 1 between an M0 write and the DMA (an instruction is one wait
    state, s_nop n is n + 1);
  * every MFMA reading a fragment quad waits (s_waitcnt lgkmcnt) for the LDS read that filled
    it, LDS reads retiring in order;
  * the DMA pipeline (vmcnt and barriers simulated): an LDS K / V^T buffer is read only after
    its DMA has landed in every wave and a barrier followed, a DMA overwrites a buffer only
    after a barrier that every wave reached with its reads of it retired, and no MFMA reads a
    Q^T register a buffer load is still filling;
  * per tile and wave: 64 MFMAs, 32 fragment reads, 64 exponentials;
  * the selection rule between the two kernels.
"""
import re

import pytest

from neptune_codegen import attention as A
from neptune_codegen import attention_asm as X

VARIANTS = [(c, op) for c in (True, False) for op in ("bf16", "f16")]
REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")


def _regs(text):
    out = []
    for m in REG.finditer(text):
        if m.group(1):
            out.append((m.group(1), int(m.group(2))))
        else:
            out += [(m.group(3), r) for r in range(int(m.group(4)), int(m.group(5)) + 1)]
    return out


@pytest.mark.parametrize("causal,op", VARIANTS)
def test_labels_are_defined_once_and_reached(causal, op):
    lines = X.generate_loop(causal, op).splitlines()
    defined = [l[:-1] for l in lines if l.endswith(":")]
    assert len(defined) == len(set(defined))
    targets = {l.split()[1] for l in lines if l.startswith("s_cbranch") or l.startswith("s_branch")}
    assert targets <= set(defined)
    assert set(defined) - targets == set(), set(defined) - targets


def _walk(lines, take, max_steps=60000):
    """Instructions along one execution path: conditional branches go to their label when
    take(label_name, visits) says so; the back edge to the loop label is taken twice."""
    where = {l[:-1]: i for i, l in enumerate(lines) if l.endswith(":")}
    visits = {}
    i, out = 0, []
    while i < len(lines) and len(out) < max_steps:
        line = lines[i]
        if line.endswith(":"):
            i += 1
            continue
        op = line.split()[0]
        if op == "s_branch":
            out.append(line)          # a branch is an instruction, taken or not
            i = where[line.split()[1]]
            continue
        if op.startswith("s_cbranch"):
            lab = line.split()[1]
            visits[lab] = visits.get(lab, 0) + 1
            if take(lab, visits[lab]):
                out.append(line)
                i = where[lab]
                continue
        out.append(line)
        i += 1
    return out


TRANS = ("v_exp_f32", "v_log_f32", "v_rcp_f32", "v_rsq_f32", "v_sqrt_f32")


def _check_hazards(trace):
    """The wait-state rules the generator promises, re-checked along a trace."""
    mfma_w, valu_w, trans_w, mfma_src, vcc_w, m0_w = {}, {}, {}, {}, -99, -99
    slot, n = 0, 0
    for line in trace:
        op, _, rest = line.partition(" ")
        if op == "s_nop":
            slot += int(rest) + 1
            continue
        if op.startswith("v_mfma"):
            parts = [p.strip() for p in rest.split(",")]
            dst, srcs = _regs(parts[0]), _regs(parts[1]) + _regs(parts[2]) + _regs(parts[3])
            for r in srcs + dst:
                for tab, w in ((valu_w, 4), (trans_w, 4)):
                    if r in tab:
                        assert slot - tab[r] - 1 >= w, line
            for r in dst:
                mfma_w[r] = slot
                valu_w.pop(r, None)
            for r in _regs(parts[1]) + _regs(parts[2]):
                mfma_src[r] = slot
        elif op.startswith("ds_read"):
            for r in _regs(rest.split(",")[0]):
                if r in mfma_src:
                    assert slot - mfma_src[r] - 1 >= 2, line
        elif op.startswith("buffer_load") and rest.endswith("lds"):
            assert slot - m0_w - 1 >= 1, line
        elif op.startswith("s_") and "m0" in rest.split(",")[0]:
            m0_w = slot
        elif op.startswith("v_"):
            regs = _regs(rest)
            dst = regs[:1] if not op.startswith("v_cmp") else []
            for r in regs:
                if r in mfma_w:
                    assert slot - mfma_w[r] - 1 >= 20, line
                    n += 1
            for r in regs[1:] if dst else regs:
                if r in trans_w:
                    assert slot - trans_w[r] - 1 >= 2, line
            if "vcc" in rest and not op.startswith("v_cmp"):
                assert slot - vcc_w - 1 >= 2, line
            if op.startswith("v_cmp") and "vcc" in rest:
                vcc_w = slot
            for r in dst:
                valu_w[r] = slot
                mfma_w.pop(r, None)
                if op in TRANS or op.startswith("v_exp"):
                    trans_w[r] = slot
                else:
                    trans_w.pop(r, None)
            if op == "v_permlane32_swap_b32":
                for r in regs:
                    valu_w[r] = slot
        slot += 1
    return n


POLICIES = {
    "steady": lambda lab, k: ("loop" in lab and k <= 2) or "_busy" in lab or "norescale" in lab
    or "nomask" in lab,
    "rescale and mask": lambda lab, k: ("loop" in lab and k <= 2) or "_busy" in lab
    or "domask" in lab,
    "last tile": lambda lab, k: ("loop" in lab and k <= 2) or "_busy" in lab or "_last" in lab,
    "first finite tile": lambda lab, k: ("loop" in lab and k <= 2) or "_busy" in lab
    or "firstrescale" in lab or "domask" in lab,
    "idle wave": lambda lab, k: ("loop" in lab and k <= 2) or "nomask" in lab,
}


@pytest.mark.parametrize("policy", sorted(POLICIES))
@pytest.mark.parametrize("causal,op", VARIANTS)
def test_wait_states_along_execution_paths(causal, op, policy):
    lines = X.generate_loop(causal, op).splitlines()
    trace = _walk(lines, POLICIES[policy])
    assert len(trace) > 1000
    checked = _check_hazards(trace)
    assert checked > (0 if policy == "idle wave" else 100)


def _check_lds_waits(trace):
    """Simulate lgkmcnt: LDS reads retire in order; s_waitcnt lgkmcnt(n) leaves the n newest
    outstanding (a scalar load in flight only makes a wait stricter, so it is not counted).
    No MFMA may read a register an outstanding read is still filling."""
    pending = []          # registers per outstanding LDS read, oldest first
    checked = 0
    for line in trace:
        op, _, rest = line.partition(" ")
        if op.startswith("ds_read"):
            pending.append(set(_regs(rest.split(",")[0])))
        elif op == "s_waitcnt" and "lgkmcnt" in rest:
            n = int(re.search(r"lgkmcnt\((\d+)\)", rest).group(1))
            pending = pending[len(pending) - n:] if n < len(pending) else pending
        elif op.startswith("v_mfma"):
            srcs = set()
            for part in [p.strip() for p in rest.split(",")][1:3]:
                srcs |= set(_regs(part))
            for regs in pending:
                assert not (regs & srcs), line
            checked += 1
    return checked


@pytest.mark.parametrize("policy", sorted(POLICIES))
@pytest.mark.parametrize("causal,op", VARIANTS)
def test_mfma_operands_wait_for_their_lds_reads(causal, op, policy):
    lines = X.generate_loop(causal, op).splitlines()
    trace = _walk(lines, POLICIES[policy])
    assert _check_lds_waits(trace) > (10 if policy == "idle wave" else 200)


def _lds_region(line):
    """(operand, buffer) an LDS fragment read addresses: K through v208-v215, V^T through
    v216-v219, 16 KB per buffer."""
    m = re.search(r", v(\d+)(?: offset:(\d+))?$", line)
    reg, off = int(m.group(1)), int(m.group(2) or 0)
    return ("K" if reg < X.VADDR else "V", off // 16384)


def _check_dma_pipeline(trace):
    """Simulate vmcnt (vector loads retire in order), lgkmcnt and barriers for one wave; every
    wave runs the same checks, so a condition that holds here at a barrier holds in all."""
    vm = []                   # outstanding vector loads: ("lds", region) or ("reg", registers)
    lgkm = []                 # outstanding LDS reads: region
    pending, state = {}, {}   # region -> DMA pieces in flight; "landed" / "visible"
    read_since_barrier = set()
    m0 = None
    reads = 0
    for line in trace:
        op, _, rest = line.partition(" ")
        if op == "s_add_i32" and rest.startswith("m0,"):
            _, base, off = [p.strip() for p in rest.split(",")]
            m0 = ("K" if base == "s90" else "V", int(off) // 16384)
        elif op.startswith("buffer_load"):
            if rest.endswith(" lds"):
                assert m0 not in read_since_barrier and m0 not in lgkm, line
                pending[m0] = pending.get(m0, 0) + 1
                state[m0] = "pending"
                vm.append(("lds", m0))
            else:
                vm.append(("reg", set(_regs(rest.split(",")[0]))))
        elif op == "s_waitcnt":
            n = re.search(r"vmcnt\((\d+)\)", rest)
            if n:
                keep = int(n.group(1))
                done, vm = (vm[:len(vm) - keep], vm[len(vm) - keep:]) if keep < len(vm) else ([], vm)
                for kind, what in done:
                    if kind == "lds":
                        pending[what] -= 1
                        if pending[what] == 0:
                            state[what] = "landed"
            n = re.search(r"lgkmcnt\((\d+)\)", rest)
            if n:
                keep = int(n.group(1))
                lgkm = lgkm[len(lgkm) - keep:] if keep < len(lgkm) else lgkm
        elif op == "s_barrier":
            assert not lgkm, "barrier with LDS reads in flight"
            for region, st in state.items():
                if st == "landed":
                    state[region] = "visible"
            read_since_barrier.clear()
        elif op.startswith("ds_read"):
            region = _lds_region(line)
            assert state.get(region) == "visible", line
            read_since_barrier.add(region)
            lgkm.append(region)
            reads += 1
        elif op.startswith("v_mfma"):
            srcs = set()
            for part in [p.strip() for p in rest.split(",")][1:3]:
                srcs |= set(_regs(part))
            for kind, what in vm:
                assert kind != "reg" or not (what & srcs), line
    return reads


@pytest.mark.parametrize("policy", sorted(POLICIES))
@pytest.mark.parametrize("causal,op", VARIANTS)
def test_dma_pipeline_buffers(causal, op, policy):
    lines = X.generate_loop(causal, op).splitlines()
    trace = _walk(lines, POLICIES[policy])
    assert _check_dma_pipeline(trace) >= 16


def _s_tile_macro_lines():
    """Instructions of the 32-query kernel's S-phase asm block (NEP_ATTN_S_TILE_D128)."""
    import pathlib

    text = (pathlib.Path(X.__file__).parents[1] / "csrc" / "kernels" / "nep_attention.h").read_text()
    start = text.index("#define NEP_ATTN_S_TILE_D128(OP)")
    body = text[start:text.index(": [s0]", start)]
    return [l.replace('" OP "', "bf16") for l in re.findall(r'"((?:[^"\\]|" OP ")*)\\n"', body)]


def test_s_tile_block_of_the_32_query_kernel():
    """Its K fragments: 16 reads into eight quads, each MFMA waits for its own read (lgkmcnt),
    each quad refilled at least 2 wait states after the MFMA that read it, and 20 wait states
    after the last MFMA before the compiler's code may read the scores."""
    lines = _s_tile_macro_lines()
    assert sum(l.startswith("ds_read_b128") for l in lines) == 16
    assert sum(l.startswith("v_mfma") for l in lines) == 16
    assert _check_lds_waits(lines) == 16
    _check_hazards(lines)
    last = max(i for i, l in enumerate(lines) if l.startswith("v_mfma"))
    tail = sum(int(l.split()[1]) + 1 if l.startswith("s_nop") else 1 for l in lines[last + 1:])
    assert tail >= X.W_MFMA_VALU


@pytest.mark.parametrize("causal", [True, False])
def test_tile_work_counts(causal):
    text = X.generate_loop(causal, "bf16")
    # the hot variant of one loop body: from a 'busy' label to the next 'last' label
    bodies = re.findall(r"L_w64_busyp0_%=:(.*?)L_w64_lastp0_%=:", text, re.S)
    assert len(bodies) == 1
    body = bodies[0]
    main = body.split("L_w64_norescalep0a_%=:")[1]
    assert main.count("v_mfma") == 64
    assert body.count("ds_read_b128") == 32
    assert main.count("v_exp_f32") == 64
    assert body.count("buffer_load_dwordx4") == 8


def test_macro_is_one_c_string():
    macro = X.asm_macro(True, "bf16")
    first = macro.splitlines()[0]
    assert first.startswith('#define NEP_ATTN_W64_ASM "') and first.endswith('\\n"')
    assert first.count('"') == 2
    assert f"#define NEP_ATTN_W64_NBUF {X.NBUF}" in macro


def test_w64_selection_rule():
    """Head dim 128 only: non-causal folds from W64_MIN_SK keys, causal ones from
    W64_CAUSAL_MIN_SQ queries."""
    assert A.use_w64(128, False, 1, A.W64_MIN_SK)
    assert not A.use_w64(128, False, 4096, A.W64_MIN_SK - 1)
    assert A.use_w64(128, True, A.W64_CAUSAL_MIN_SQ, 1)
    assert not A.use_w64(128, True, A.W64_CAUSAL_MIN_SQ - 1, 1 << 20)
    assert not A.use_w64(64, False, 8192, 8192) and not A.use_w64(256, False, 8192, 8192)
