"""Instruction-scheduled key-tile loop of the head-dim-128 attention fold (gfx950).

The fold kernel at head dim 128 runs one wave per SIMD with 64 queries per wave (two 32-query
blocks).  Each K or V^T fragment read from LDS then feeds two MFMAs (one per query block), and
the wave's own softmax VALU work is interleaved with its MFMAs instruction by instruction.
Measured on gfx950: one wave's independent VALU instructions issue while its own MFMAs run (8
MFMAs 268 cycles, 32 exponentials 334, both interleaved 360), while the compiler's ordering of
the same loop serialises the two phases (1956 ns per tile against 540 for the MFMAs alone),
hence this generator.  Per key tile the result is ~7% faster than the compiler-scheduled
kernel; attention.use_w64 says where that outweighs its larger fixed cost per workgroup.

The generated text is one `asm volatile` statement holding the whole key-tile loop: LDS DMA of
the next K and V^T tiles, the barrier, the lazy-rescale check and rescale, the softmax of tile
t interleaved with S(t+1) = K(t+1) Q^T, the causal / ragged mask of tile t+1, and
O^T += V^T(t) P^T(t) interleaved with the row sums of tile t and the row max of tile t+1.
Arithmetic is the same, operation for operation, as the compiler-scheduled kernel
(`attention_fwd` in nep_attention.h); the tests compare the two bit for bit.

Register map (fixed; the statement's operands pin its inputs and outputs to these):
  v16-v79, v80-v143   score buffers SA / SB: [query block][key block] x 16 accumulators
  v144-v175           P^T operands (fp16 pairs): [query block] x 16
  v176-v207           eight LDS fragment quads (K, then V^T)
  v208-v215           K fragment LDS addresses (k-steps 0-7, key block 0 of buffer 0)
  v216-v219           V^T fragment LDS addresses (key steps 0-3, dim block 0 of buffer 0)
  v220-v221 m_ref, v222-v225 row sums (even/odd chains per block), v226-v227 tile max,
  v228-v229 shift, v230-v238 temporaries, v239 -inf, v240-v243 K DMA offsets per piece,
  v244-v245 mask limits per block, v246 V^T DMA offset, v247-v255 temporaries (v254-v255
  hold the two query blocks' Q row offsets on entry)
  a0-a127  O^T accumulators [query block][dim block];  a128-a191  Q^T operands [block][k-step]
  s48-s63 and s97-s99 inputs (bound in nep_attention.h), s64-s96 loop state, m0 for the DMA.

Hazards: the generator counts wait states along every path (an instruction is one, s_nop n is
n+1) and inserts s_nop where gfx950 needs them: 20 between an XDL MFMA writing a register and
a VALU touching it, 4 between a VALU write and an MFMA reading it, 2 after a transcendental or
a VALU mask write before a VALU reads it, 2 before and 4 after a permlane swap, 2 between an
MFMA reading a fragment quad and the LDS read refilling it, 1 between an M0 write and the DMA.
Each loop iteration ends with every window expired, so the back edge carries no hazard.
"""
from __future__ import annotations

# wait states required, by rule
W_MFMA_VALU = 20       # XDL MFMA result -> any VALU access of that register
W_VALU_MFMA = 4        # VALU write -> MFMA source read
W_TRANS_USE = 2        # transcendental result -> VALU read
W_MASK_USE = 2         # VALU write of VCC / SGPR pair -> VALU mask read
W_PERM_IN = 2          # VALU write -> permlane swap read
W_PERM_OUT = 4         # permlane swap result -> VALU read
W_MFMA_SRC_WAR = 2     # MFMA source read -> LDS read overwriting it
W_M0_DMA = 1           # M0 write -> LDS DMA

SA, SB = 16, 80
P0 = 144
WIN = 176
KADDR, VADDR = 208, 216
MREF, LSUM, TMAX, SHIFT = 220, 222, 226, 228
T0 = 230
NEGINF = 239
KOFF, LB, VOFF = 240, 244, 246
U0 = 247
QOFF = 254          # Q row offsets of the two query blocks (inputs; temporaries afterwards)
OACC, QREG = 256, 256 + 128     # AGPRs are numbered 256 + i


def _rname(r: int) -> str:
    return f"a{r - 256}" if r >= 256 else f"v{r}"


def _range(r: int, n: int) -> str:
    p = "a" if r >= 256 else "v"
    b = r - 256 if r >= 256 else r
    return f"{p}[{b}:{b + n - 1}]"


def s_reg(buf: int, qb: int, kb: int) -> int:
    return buf + (qb * 2 + kb) * 16


def o_reg(qb: int, a: int) -> int:
    return OACC + (qb * 4 + a) * 16


def q_reg(qb: int, s: int) -> int:
    return QREG + qb * 32 + 4 * s


def p_reg(qb: int, cs: int) -> int:
    return P0 + qb * 16 + 4 * cs


class _State:
    """Slots of the last writes / reads that hazards are measured from."""

    def __init__(self):
        self.mfma_w: dict = {}
        self.mfma_r: dict = {}
        self.valu_w: dict = {}
        self.trans_w: dict = {}
        self.perm_w: dict = {}
        self.mask_w: dict = {}     # 'vcc' or SGPR pair name -> slot
        self.m0_w = -1000

    def copy(self):
        s = _State()
        for k in ("mfma_w", "mfma_r", "valu_w", "trans_w", "perm_w", "mask_w"):
            setattr(s, k, dict(getattr(self, k)))
        s.m0_w = self.m0_w
        return s

    def shifted(self, d: int):
        s = _State()
        for k in ("mfma_w", "mfma_r", "valu_w", "trans_w", "perm_w", "mask_w"):
            setattr(s, k, {r: v + d for r, v in getattr(self, k).items()})
        s.m0_w = self.m0_w + d
        return s

    def merge(self, o):
        for k in ("mfma_w", "mfma_r", "valu_w", "trans_w", "perm_w", "mask_w"):
            a, b = getattr(self, k), getattr(o, k)
            for r, v in b.items():
                if v > a.get(r, -1000):
                    a[r] = v
        self.m0_w = max(self.m0_w, o.m0_w)


class Emitter:
    def __init__(self, uid: str):
        self.lines: list = []
        self.n = 0                  # slot of the next instruction
        self.st = _State()
        self.saved: dict = {}       # label -> [(state, slot after the branch)]
        self.dead = False
        self.uid = uid

    # ------------------------------------------------------------------ plumbing
    def lab(self, name: str) -> str:
        return f"L_{self.uid}_{name}_%="

    def _raw(self, text: str, slots: int = 1):
        self.lines.append(text)
        self.n += slots

    def _pad_to(self, slot: int):
        while self.n < slot:
            k = min(8, slot - self.n)
            self._raw(f"s_nop {k - 1}", k)

    def nop(self, k: int):
        while k > 0:
            j = min(8, k)
            self._raw(f"s_nop {j - 1}", j)
            k -= j

    def quiesce(self):
        """Pad until no hazard window is open."""
        st, need = self.st, self.n
        for v in st.mfma_w.values():
            need = max(need, v + W_MFMA_VALU + 1)
        for v in st.valu_w.values():
            need = max(need, v + W_VALU_MFMA + 1)
        for v in st.trans_w.values():
            need = max(need, v + W_TRANS_USE + 1)
        for v in st.perm_w.values():
            need = max(need, v + W_PERM_OUT + 1)
        for v in st.mask_w.values():
            need = max(need, v + W_MASK_USE + 1)
        for v in st.mfma_r.values():
            need = max(need, v + W_MFMA_SRC_WAR + 1)
        need = max(need, st.m0_w + W_M0_DMA + 1)
        self._pad_to(need)

    def branch(self, op: str, label: str):
        self._raw(f"{op} {self.lab(label)}")
        self.saved.setdefault(label, []).append((self.st.copy(), self.n))
        if op == "s_branch":
            self.dead = True

    def label(self, label: str):
        incoming = [] if self.dead else [(self.st, self.n)]
        incoming += self.saved.pop(label, [])
        assert incoming, f"label {label} is unreachable"
        merged = _State()
        for st, at in incoming:
            merged.merge(st.shifted(self.n - at))
        self.st = merged
        self.dead = False
        self.lines.append(f"{self.lab(label)}:")

    # ------------------------------------------------------------------ instructions
    def salu(self, text: str):
        self._raw(text)

    def m0(self, text: str):
        self._raw(text)
        self.st.m0_w = self.n - 1

    def dma(self, text: str):
        self._pad_to(self.st.m0_w + W_M0_DMA + 1)
        self._raw(text)

    def valu(self, text: str, reads=(), writes=(), trans=False, perm=False, mask_in=None,
             mask_out=None):
        st, need = self.st, self.n
        for r in list(reads) + list(writes):
            if r in st.mfma_w:
                need = max(need, st.mfma_w[r] + W_MFMA_VALU + 1)
        for r in reads:
            if r in st.trans_w:
                need = max(need, st.trans_w[r] + W_TRANS_USE + 1)
            if r in st.perm_w:
                need = max(need, st.perm_w[r] + W_PERM_OUT + 1)
            if perm and r in st.valu_w:
                need = max(need, st.valu_w[r] + W_PERM_IN + 1)
        if mask_in is not None and mask_in in st.mask_w:
            need = max(need, st.mask_w[mask_in] + W_MASK_USE + 1)
        self._pad_to(need)
        self._raw(text)
        slot = self.n - 1
        for r in writes:
            st.valu_w[r] = slot
            st.mfma_w.pop(r, None)
            if trans:
                st.trans_w[r] = slot
            else:
                st.trans_w.pop(r, None)
            if perm:
                st.perm_w[r] = slot
            else:
                st.perm_w.pop(r, None)
        if mask_out is not None:
            st.mask_w[mask_out] = slot

    def mfma(self, op: str, dst: int, a: int, b: int, c):
        st, need = self.st, self.n
        srcs = list(range(a, a + 4)) + list(range(b, b + 4))
        accs = list(range(dst, dst + 16))
        for r in srcs + (accs if c is not None else []):
            for tab in (st.valu_w, st.trans_w):
                if r in tab:
                    need = max(need, tab[r] + W_VALU_MFMA + 1)
        self._pad_to(need)
        ctext = _range(dst, 16) if c is not None else "0"
        self._raw(f"v_mfma_f32_32x32x16_{op} {_range(dst, 16)}, {_range(a, 4)}, {_range(b, 4)}, {ctext}")
        slot = self.n - 1
        for r in accs:
            st.mfma_w[r] = slot
            st.valu_w.pop(r, None)
        for r in srcs:
            st.mfma_r[r] = slot

    def ds_read(self, dst: int, addr: int, offset: int):
        st, need = self.st, self.n
        for r in range(dst, dst + 4):
            if r in st.mfma_r:
                need = max(need, st.mfma_r[r] + W_MFMA_SRC_WAR + 1)
        self._pad_to(need)
        off = f" offset:{offset}" if offset else ""
        self._raw(f"ds_read_b128 {_range(dst, 4)}, v{addr}{off}")
        for r in range(dst, dst + 4):
            st.valu_w.pop(r, None)
            st.mfma_r.pop(r, None)

    def text(self) -> str:
        return "\n".join(self.lines)


# ---------------------------------------------------------------------- VALU op lists
# An op is (text, reads, writes, kind) with kind "" / "trans" / "perm"; ops run in list order.

def softmax_ops(ybuf: int):
    """p = exp2(s * scale - shift) in place and the fp16 pairs of P^T, for both query blocks
    (key block 0 first, which the first P V MFMAs need); within a group the FMAs lead the
    exponentials by 4 and the packs trail them by 4, so every share mixes the three."""
    ops = []
    for kb in (0, 1):
        for qb in (0, 1):
            base = s_reg(ybuf, qb, kb)
            sh = SHIFT + qb
            for step in range(24):
                if step < 16:
                    r = base + step
                    ops.append((f"v_fma_f32 v{r}, v{r}, s58, -v{sh}", (r, sh), (r,), ""))
                e = step - 4
                if 0 <= e < 16:
                    ops.append((f"v_exp_f32 v{base + e}, v{base + e}", (base + e,), (base + e,), "trans"))
                c = step - 8
                if 0 <= c < 16 and c % 2 == 1:
                    pr = P0 + qb * 16 + kb * 8 + c // 2
                    ops.append((f"v_cvt_pk_f16_f32 v{pr}, v{base + c - 1}, v{base + c}",
                                (base + c - 1, base + c), (pr,), ""))
    return ops


def rowsum_ops(ybuf: int):
    """l_even += p_r * wl, l_odd += p_(r+1) * wl per query block, each chain in the
    compiler-scheduled kernel's order; the four chains alternate."""
    chains = []
    for qb in (0, 1):
        le, lo = LSUM + 2 * qb, LSUM + 2 * qb + 1
        ce, co = [], []
        for kb in (0, 1):
            base = s_reg(ybuf, qb, kb)
            for r in range(0, 16, 2):
                ce.append((f"v_fmac_f32 v{le}, s77, v{base + r}", (le, base + r), (le,), ""))
                co.append((f"v_fmac_f32 v{lo}, s77, v{base + r + 1}", (lo, base + r + 1), (lo,), ""))
        chains += [ce, co]
    return [op for grp in zip(*chains) for op in grp]


def rowmax_ops(xbuf: int):
    """Raw (unscaled) max of each query's 64 scores of the tile (both 32-lane halves through a
    permlane32 swap); the two query blocks' chains alternate."""
    chains = []
    for qb in (0, 1):
        b0, b1 = s_reg(xbuf, qb, 0), s_reg(xbuf, qb, 1)
        regs = [b0 + r for r in range(16)] + [b1 + r for r in range(16)]
        acc = T0 + qb
        ops = [(f"v_max3_f32 v{acc}, v{regs[0]}, s86, v{regs[1]}", (regs[0], regs[1]), (acc,), "")]
        for i in range(2, 32, 2):
            ops.append((f"v_max3_f32 v{acc}, v{acc}, v{regs[i]}, v{regs[i + 1]}",
                        (acc, regs[i], regs[i + 1]), (acc,), ""))
        x, y = U0 + 2 * qb, U0 + 2 * qb + 1
        ops.append((f"v_mov_b32 v{x}, v{acc}", (acc,), (x,), ""))
        ops.append((f"v_mov_b32 v{y}, v{acc}", (acc,), (y,), ""))
        ops.append((f"v_permlane32_swap_b32 v{x}, v{y}", (x, y), (x, y), "perm"))
        ops.append((f"v_max_f32 v{TMAX + qb}, v{x}, v{y}", (x, y), (TMAX + qb,), ""))
        chains.append(ops)
    return [op for pair in zip(*chains) for op in pair]


def emit_op(em: Emitter, op):
    text, reads, writes, kind = op
    em.valu(text, reads, writes, trans=(kind == "trans"), perm=(kind == "perm"))


# ---------------------------------------------------------------------- interleaved phase
class Pipe:
    """MFMAs issued in order with their LDS fragments: reads go into an 8-quad window (read j
    reuses the quad of read j-8 once every MFMA naming read j-8 has issued) and each MFMA waits
    only for its own fragment (LDS reads retire in order, so lgkmcnt counts down).

    reads: list of (addr_vgpr, offset); mfmas: list of (kind, dst, read_index, b, c) with kind
    "s" (the Q K^T MFMA type) or "pv" (f16)."""

    def __init__(self, em: Emitter, op: str, reads, mfmas):
        self.em, self.op, self.reads, self.mfmas = em, op, reads, mfmas
        last = [-1] * len(reads)
        for i, m in enumerate(mfmas):
            last[m[2]] = max(last[m[2]], i)
        self.last_user = last
        self.issued = 0     # reads issued
        self.done = -1      # highest read index known complete
        self.emitted = 0    # MFMAs emitted

    def _can_issue(self, j):
        if j >= len(self.reads):
            return False
        return j < 8 or self.last_user[j - 8] < self.emitted

    def issue(self, limit=8):
        k = 0
        while k < limit and self._can_issue(self.issued):
            addr, off = self.reads[self.issued]
            self.em.ds_read(WIN + 4 * (self.issued % 8), addr, off)
            self.issued += 1
            k += 1

    def run(self, hi: int, valu_ops, after=None):
        """Emit MFMAs up to index `hi`, each followed by its share of `valu_ops`, by the
        callables `after[i]` (other instructions placed behind MFMA i) and by the fragment
        reads its issue frees; the first MFMA of the pipe is preceded by one share, which covers
        the first fragment's LDS latency."""
        em = self.em
        after = after or {}
        vi = 0
        lo = self.emitted
        n = hi - lo

        def share(i):
            nonlocal vi
            rem = len(valu_ops) - vi
            q = -(-rem // (hi - i)) if rem > 0 else 0
            for _ in range(q):
                emit_op(em, valu_ops[vi])
                vi += 1

        if lo == 0 and n > 0:
            share(lo)
        for i in range(lo, hi):
            kind, dst, rj, b, c = self.mfmas[i]
            if rj > self.done:
                cnt = min(self.issued - (rj + 1), 15)
                em.salu(f"s_waitcnt lgkmcnt({cnt})")
                self.done = self.issued - cnt - 1
            em.mfma(self.op if kind == "s" else "f16", dst, WIN + 4 * (rj % 8), b, c)
            self.emitted = i + 1
            for f in after.get(i, ()):
                f()
            share(i + 1) if i + 1 < hi else None
            self.issue(2)
        while vi < len(valu_ops):
            emit_op(em, valu_ops[vi])
            vi += 1


def s_phase_parts(kbuf: int, xbuf: int):
    """Fragment reads and MFMAs of S(tile) = K(tile) Q^T from K buffer `kbuf` into `xbuf`:
    k-step major, so the four accumulator chains (query block x key block) interleave and each
    MFMA's predecessor in its chain issued three MFMAs earlier."""
    reads = [(KADDR + s, kbuf * 16384 + kb * 8192) for s in range(8) for kb in (0, 1)]
    mfmas = []
    for s in range(8):
        for kb in (0, 1):
            for qb in (0, 1):
                d = s_reg(xbuf, qb, kb)
                mfmas.append(("s", d, s * 2 + kb, q_reg(qb, s), None if s == 0 else d))
    return reads, mfmas


def pv_phase_parts(vbuf: int, read_base: int):
    reads = [(VADDR + cs, vbuf * 16384 + a * 4096) for cs in range(4) for a in range(4)]
    mfmas = []
    for cs in range(4):
        for a in range(4):
            for qb in (0, 1):
                mfmas.append(("pv", o_reg(qb, a), read_base + cs * 4 + a, p_reg(qb, cs), True))
    return reads, mfmas


NBUF = 4            # K and V^T tile buffers: tile j lives in buffer j % NBUF (128 KB of LDS)


# ---------------------------------------------------------------------- blocks
def dma_k(em: Emitter, tile_sreg: str, kbuf: int, want_sreg: str | None = None):
    """K rows of the tile whose index is in `tile_sreg` -> LDS K buffer `kbuf` (4 pieces),
    issued at once."""
    for piece in dma_k_pieces(em, tile_sreg, kbuf, want_sreg):
        piece()


def dma_v(em: Emitter, tile_sreg: str, vbuf: int, want_sreg: str | None = None):
    for piece in dma_v_pieces(em, tile_sreg, vbuf, want_sreg):
        piece()


def dma_k_pieces(em: Emitter, tile_sreg: str, kbuf: int, want_sreg: str | None = None):
    """Sets up the K tile's buffer descriptor in s[64:67] now and returns the four loads as
    callables, to be issued later (each sets M0 first).  With `want_sreg` (the unclamped tile
    index) past the last tile, the descriptor's range is 0: the loads return without touching
    memory and only keep the per-iteration load count constant."""
    em.salu(f"s_lshl_b32 s84, {tile_sreg}, 6")            # first key of the tile
    em.salu("s_mul_i32 s88, s84, s54")
    em.salu("s_mul_hi_u32 s89, s84, s54")
    em.salu("s_add_u32 s64, s48, s88")
    em.salu("s_addc_u32 s65, s49, s89")
    em.salu("s_and_b32 s65, s65, 0xffff")
    em.salu("s_sub_i32 s85, s55, s84")
    em.salu("s_min_i32 s85, s85, 64")                     # rows of the tile
    em.salu("s_add_i32 s85, s85, -1")
    em.salu("s_mul_i32 s85, s85, s54")
    em.salu("s_add_i32 s66, s85, 0x100")                  # (rows - 1) * row bytes + 256
    em.salu("s_mov_b32 s67, 0x20000")
    if want_sreg is not None:
        em.salu(f"s_cmp_gt_i32 {want_sreg}, s62")
        em.salu("s_cselect_b32 s66, 0, s66")

    def piece(i):
        def f():
            em.m0(f"s_add_i32 m0, s90, {kbuf * 16384 + i * 4096}")
            em.dma(f"buffer_load_dwordx4 v{KOFF + i}, s[64:67], 0 offen lds")
        return f
    return [piece(i) for i in range(4)]


def dma_v_pieces(em: Emitter, tile_sreg: str, vbuf: int, want_sreg: str | None = None):
    """As dma_k_pieces for the V^T image of the tile (descriptor in s[68:71])."""
    em.salu(f"s_lshl_b32 s84, {tile_sreg}, 14")
    em.salu("s_add_u32 s68, s50, s84")
    em.salu("s_addc_u32 s69, s51, 0")
    em.salu("s_and_b32 s69, s69, 0xffff")
    em.salu("s_mov_b32 s70, 0x4000")
    em.salu("s_mov_b32 s71, 0x20000")
    if want_sreg is not None:
        em.salu(f"s_cmp_gt_i32 {want_sreg}, s62")
        em.salu("s_cselect_b32 s70, 0, s70")

    def piece(i):
        def f():
            em.m0(f"s_add_i32 m0, s91, {vbuf * 16384 + i * 4096}")
            em.dma(f"buffer_load_dwordx4 v{VOFF}, s[68:71], s{92 + i} offen lds")
        return f
    return [piece(i) for i in range(4)]


def mask_block(em: Emitter, xbuf: int, tile_sreg: str, causal: bool, tag: str):
    """-inf for keys past the query (causal) or past sk, on the tile in `tile_sreg`."""
    em.salu(f"s_lshl_b32 s84, {tile_sreg}, 6")
    em.salu("s_add_i32 s85, s84, 64")
    em.salu("s_cmp_gt_i32 s85, s55")
    em.branch("s_cbranch_scc1", f"domask{tag}")
    if causal:
        em.salu("s_add_i32 s85, s85, -1")
        em.salu("s_cmp_gt_i32 s85, s60")
        em.branch("s_cbranch_scc1", f"domask{tag}")
    em.branch("s_branch", f"nomask{tag}")
    em.label(f"domask{tag}")
    for qb in (0, 1):
        em.valu(f"v_subrev_u32 v{T0 + 2 + qb}, s84, v{LB + qb}", (LB + qb,), (T0 + 2 + qb,))
    for qb in (0, 1):
        lim = T0 + 2 + qb
        for kb in (0, 1):
            base = s_reg(xbuf, qb, kb)
            for r in range(16):
                c = kb * 32 + 8 * (r >> 2) + (r & 3)
                em.valu(f"v_cmp_gt_i32 vcc, {c}, v{lim}", (lim,), (), mask_out="vcc")
                em.valu(f"v_cndmask_b32 v{base + r}, v{base + r}, v{NEGINF}, vcc",
                        (base + r, NEGINF), (base + r,), mask_in="vcc")
    em.label(f"nomask{tag}")


def rescale_block(em: Emitter, tag: str):
    """Lazy rescale check of tile t (tile max in TMAX) and, when a lane's max moved, the
    rescale of (m_ref, l, O) for both query blocks.  While every lane's m_ref is still -inf
    (a wave's first tile with a finite score), the factor is 0 and l and O hold only zeros
    (or NaN from 0 * inf/NaN in V), which multiplying by 0 leaves as they are: only m_ref
    moves then."""
    lift = T0
    em.valu("v_cvt_f32_u32 v230, s76", (), (lift,))
    for qb in (0, 1):
        em.valu(f"v_fma_f32 v{T0 + 1 + qb}, v{TMAX + qb}, s58, v230", (TMAX + qb, lift), (T0 + 1 + qb,))
        em.valu(f"v_add_f32 v{T0 + 3 + qb}, 0x41000000, v{MREF + qb}", (MREF + qb,), (T0 + 3 + qb,))
    em.valu("v_cmp_gt_f32_e64 s[80:81], v231, v233", (T0 + 1, T0 + 3), (), mask_out="s80")
    em.valu("v_cmp_gt_f32_e64 s[82:83], v232, v234", (T0 + 2, T0 + 4), (), mask_out="s82")
    em.nop(4)
    em.salu("s_or_b64 s[88:89], s[80:81], s[82:83]")
    em.branch("s_cbranch_scc0", f"norescale{tag}")
    em.valu(f"v_cmp_neq_f32 vcc, s86, v{MREF}", (MREF,), (), mask_out="vcc")
    em.valu(f"v_cmp_neq_f32_e64 s[84:85], s86, v{MREF + 1}", (MREF + 1,), (), mask_out="s84")
    em.nop(4)
    em.salu("s_or_b64 s[84:85], vcc, s[84:85]")
    em.branch("s_cbranch_scc0", f"firstrescale{tag}")
    for qb in (0, 1):
        tl, mr, pair = T0 + 1 + qb, MREF + qb, f"s[{80 + 2 * qb}:{81 + 2 * qb}]"
        mn, al = T0 + 5, T0 + 6
        em.valu(f"v_cndmask_b32_e64 v{mn}, v{mr}, v{tl}, {pair}", (mr, tl), (mn,), mask_in=f"s{80 + 2 * qb}")
        em.valu(f"v_sub_f32 v{al}, v{mr}, v{mn}", (mr, mn), (al,))
        em.valu(f"v_exp_f32 v{al}, v{al}", (al,), (al,), trans=True)
        em.valu(f"v_cmp_neq_f32 vcc, s86, v{mr}", (mr,), (), mask_out="vcc")
        em.valu(f"v_cndmask_b32 v{al}, 0, v{al}, vcc", (al,), (al,), mask_in="vcc")
        em.valu(f"v_mul_f32 v{LSUM + 2 * qb}, v{LSUM + 2 * qb}, v{al}", (LSUM + 2 * qb, al), (LSUM + 2 * qb,))
        em.valu(f"v_mul_f32 v{LSUM + 2 * qb + 1}, v{LSUM + 2 * qb + 1}, v{al}",
                (LSUM + 2 * qb + 1, al), (LSUM + 2 * qb + 1,))
        for a in range(4):
            base = o_reg(qb, a)
            for g in range(0, 16, 8):
                tmp = [U0 + i for i in range(8)]
                for i in range(8):
                    em.valu(f"v_accvgpr_read_b32 v{tmp[i]}, {_rname(base + g + i)}", (base + g + i,), (tmp[i],))
                for i in range(8):
                    em.valu(f"v_mul_f32 v{tmp[i]}, v{tmp[i]}, v{al}", (tmp[i], al), (tmp[i],))
                for i in range(8):
                    em.valu(f"v_accvgpr_write_b32 {_rname(base + g + i)}, v{tmp[i]}", (tmp[i],), (base + g + i,))
        em.valu(f"v_mov_b32 v{mr}, v{mn}", (mn,), (mr,))
    em.branch("s_branch", f"norescale{tag}")
    em.label(f"firstrescale{tag}")
    for qb in (0, 1):
        tl, mr = T0 + 1 + qb, MREF + qb
        em.valu(f"v_cndmask_b32_e64 v{mr}, v{mr}, v{tl}, s[{80 + 2 * qb}:{81 + 2 * qb}]", (mr, tl),
                (mr,), mask_in=f"s{80 + 2 * qb}")
    em.label(f"norescale{tag}")


def shift_block(em: Emitter):
    em.valu("v_cvt_f32_i32 v235, s75", (), (T0 + 5,))
    for qb in (0, 1):
        mr = MREF + qb
        em.valu(f"v_cmp_neq_f32 vcc, s86, v{mr}", (mr,), (), mask_out="vcc")
        em.valu(f"v_cndmask_b32 v{T0 + 6}, 0, v{mr}, vcc", (mr,), (T0 + 6,), mask_in="vcc")
        em.valu(f"v_sub_f32 v{SHIFT + qb}, v236, v235", (T0 + 6, T0 + 5), (SHIFT + qb,))


def generate_loop(causal: bool, op: str = "bf16", nbuf: int = NBUF) -> str:
    """The asm text of the whole key-tile loop (see the module docstring).

    Tile j's K rows and V^T image live in buffers j % nbuf.  At the top of iteration t the K
    of t+1 and the V^T of t are in LDS and the following nbuf-2 tiles are in flight; the
    iteration issues the K of t+nbuf and the V^T of t+nbuf-1 and ends waiting for all but the
    loads of its last nbuf-2 iterations, then the barrier.  Every iteration issues eight loads:
    those for tiles past the last have an empty range and return without a memory access."""
    assert nbuf >= 3
    em = Emitter("w64")
    ahead = 8 * (nbuf - 2)                         # loads left in flight at a barrier
    # ---- prologue
    em.salu("s_mov_b32 s86, 0xff800000")
    em.valu(f"v_mov_b32 v{NEGINF}, s86", (), (NEGINF,))
    for qb in (0, 1):
        em.valu(f"v_mov_b32 v{MREF + qb}, s86", (), (MREF + qb,))
        em.valu(f"v_mov_b32 v{LSUM + 2 * qb}, 0", (), (LSUM + 2 * qb,))
        em.valu(f"v_mov_b32 v{LSUM + 2 * qb + 1}, 0", (), (LSUM + 2 * qb + 1,))
    em.salu("s_mov_b32 s74, 0")                    # exact-path flag
    em.salu("s_mov_b32 s72, 0")                    # tile
    em.salu("s_add_i32 s62, s56, -1")              # last tile of the workgroup
    em.salu("s_min_i32 s96, s62, 1")
    em.salu("s_lshl_b32 s96, s96, 2")
    em.salu("s_lshl_b32 s92, s63, 10")             # wave * 1 KB
    em.salu("s_add_i32 s90, s61, s92")             # K DMA base of this wave
    em.salu(f"s_add_i32 s91, s90, {nbuf * 16384}")  # V^T DMA base of this wave
    em.salu("s_add_i32 s93, s92, 0x1000")
    em.salu("s_add_i32 s94, s92, 0x2000")
    em.salu("s_add_i32 s95, s92, 0x3000")
    em.salu("s_load_dword s73, s[52:53], 0x0")     # exponent of tile 0
    em.salu("s_load_dword s87, s[52:53], s96")     # exponent of tile 1 (s96 = min(1, last) * 4)
    dma_k(em, "s72", 0)
    dma_v(em, "s72", 0)
    # Q^T operands straight into a128-a191 behind the first tile's DMA: rows past sq are out
    # of the descriptor's range (s97 bytes from the workgroup's first query row) and read 0
    em.salu("s_mov_b32 s68, s98")
    em.salu("s_and_b32 s69, s99, 0xffff")
    em.salu("s_mov_b32 s70, s97")
    em.salu("s_mov_b32 s71, 0x20000")
    for qb in (0, 1):
        for st in range(8):
            r = q_reg(qb, st)
            em.salu(f"buffer_load_dwordx4 {_range(r, 4)}, v{QOFF + qb}, s[68:71], 0 offen offset:{32 * st}")
    em.salu("s_mov_b32 s78, 1")
    em.salu("s_min_i32 s79, s62, 1")
    dma_k(em, "s79", 1, "s78")
    for i in range(128):                           # O^T = 0 while the loads are in flight
        em.valu(f"v_accvgpr_write_b32 a{i}, 0", (), (OACC + i,))
    em.salu("s_waitcnt vmcnt(4) lgkmcnt(0)")
    em.salu("s_barrier")
    reads, mfmas = s_phase_parts(0, SA)
    pipe = Pipe(em, op, reads, mfmas)
    pipe.issue()
    pipe.run(len(mfmas), [])
    mask_block(em, SA, "s72", causal, "pro")
    for o in rowmax_ops(SA):
        emit_op(em, o)
    for j in range(2, nbuf):
        em.salu(f"s_mov_b32 s78, {j}")
        em.salu(f"s_min_i32 s79, s62, {j}")
        dma_k(em, "s79", j, "s78")
        em.salu(f"s_mov_b32 s78, {j - 1}")
        em.salu(f"s_min_i32 s79, s62, {j - 1}")
        dma_v(em, "s79", j - 1, "s78")
    em.quiesce()
    em.salu(f"s_waitcnt vmcnt({ahead})")
    em.salu("s_barrier")
    # ---- the loop, unrolled over the period of (t % 2, t % nbuf)
    period = 2 * nbuf // (2 if nbuf % 2 == 0 else 1)
    em.label("loop")
    for p in range(period):
        ybuf, xbuf = (SA, SB) if p % 2 == 0 else (SB, SA)
        kcur, vcur = (p + 1) % nbuf, p % nbuf
        t = f"p{p}"
        em.salu("s_cmp_gt_i32 s73, s59")
        em.salu("s_cselect_b32 s79, 1, 0")
        em.salu("s_or_b32 s74, s74, s79")          # exact |= e(t) > e_max
        em.salu("s_min_i32 s75, s73, 24")          # e
        em.salu("s_max_i32 s76, s75, 7")
        em.salu("s_add_i32 s76, s76, -7")          # lift = max(0, e - 7)
        em.salu("s_lshl_b32 s77, s75, 23")
        em.salu("s_sub_i32 s77, 0x3f800000, s77")  # wl = 2^-e
        # K(t+nbuf) -> the buffer of K(t), V(t+nbuf-1) -> the buffer of V(t-1): descriptors
        # now, the eight loads spread between MFMAs (a wave stalled issuing them idles its SIMD)
        em.salu(f"s_add_i32 s78, s72, {nbuf}")
        em.salu("s_min_i32 s79, s78, s62")
        pieces = dma_k_pieces(em, "s79", p % nbuf, "s78")
        em.salu(f"s_add_i32 s78, s72, {nbuf - 1}")
        em.salu("s_min_i32 s79, s78, s62")
        pieces += dma_v_pieces(em, "s79", (p + nbuf - 1) % nbuf, "s78")
        em.salu("s_cmp_le_i32 s72, s57")
        em.branch("s_cbranch_scc1", f"busy{t}")
        for f in pieces:                           # past this wave's last tile
            f()
        em.branch("s_branch", f"tail{t}")
        em.label(f"busy{t}")
        em.salu("s_add_i32 s79, s72, 1")
        em.salu("s_cmp_gt_i32 s79, s57")
        em.branch("s_cbranch_scc1", f"last{t}")
        # tile t+1 is this wave's: S(t+1) under softmax(t); mask(t+1); P V(t) under the row
        # sums of t and the row max of t+1
        kr, km = s_phase_parts(kcur, xbuf)
        vr, vm = pv_phase_parts(vcur, len(kr))
        pipe = Pipe(em, op, kr + vr, km + vm)
        pipe.issue()
        rescale_block(em, t + "a")
        shift_block(em)
        pipe.run(len(km), softmax_ops(ybuf), {4 * i + 3: [f] for i, f in enumerate(pieces)})
        mask_block(em, xbuf, "s79", causal, t)
        pipe.run(len(km) + len(vm), rowsum_ops(ybuf) + rowmax_ops(xbuf))
        assert pipe.issued == len(kr) + len(vr)
        em.branch("s_branch", f"tail{t}")
        # tile t is this wave's last: softmax(t), then P V(t) under the row sums of t
        em.label(f"last{t}")
        vr, vm = pv_phase_parts(vcur, 0)
        pipe = Pipe(em, op, vr, vm)
        pipe.issue()
        rescale_block(em, t + "b")
        shift_block(em)
        for o in softmax_ops(ybuf):
            emit_op(em, o)
        pipe.run(len(vm), rowsum_ops(ybuf), {4 * i + 3: [f] for i, f in enumerate(pieces)})
        em.label(f"tail{t}")
        # exponents run two tiles ahead: e(t+1), loaded an iteration ago, moves to s73 and
        # e(t+2) is loaded into s87 (clamped to the last tile).  The load stays outstanding
        # across the next iteration's LDS reads; their lgkmcnt waits then only get stricter.
        em.salu("s_waitcnt lgkmcnt(0)")
        em.salu("s_mov_b32 s73, s87")
        em.salu("s_add_i32 s79, s72, 2")
        em.salu("s_min_i32 s79, s79, s62")
        em.salu("s_lshl_b32 s84, s79, 2")
        em.salu("s_load_dword s87, s[52:53], s84")
        em.quiesce()
        em.salu(f"s_waitcnt vmcnt({ahead})")
        em.salu("s_barrier")
        em.salu("s_add_i32 s72, s72, 1")
        em.salu("s_cmp_lt_i32 s72, s56")
        if p < period - 1:
            em.branch("s_cbranch_scc0", "end")
        else:
            em.salu(f"s_cbranch_scc1 {em.lab('loop')}")   # back edge: quiesced above
    em.label("end")
    em.salu("s_waitcnt vmcnt(0) lgkmcnt(0)")
    em.quiesce()
    return em.text()


# SGPR and VGPR operands of the statement, in the order nep_attention.h binds them
CLOBBER_VGPRS = [r for r in range(16, 256)
                 if not (KADDR <= r < VADDR + 4 or MREF <= r < MREF + 8 or KOFF <= r <= VOFF
                         or r >= QOFF)]
CLOBBER_AGPRS = list(range(128, 192))
CLOBBER_SGPRS = [62] + list(range(64, 97))   # s62: last tile index; s97-s99 are inputs


def asm_macro(causal: bool, op: str, nbuf: int = NBUF) -> str:
    """`#define NEP_ATTN_W64_ASM "..."`: the loop text as one C string literal, plus the
    tile-buffer count and the clobber list macro the statement in nep_attention.h uses."""
    body = generate_loop(causal, op, nbuf)
    lit = "\\n".join(body.splitlines())
    lines = [f'#define NEP_ATTN_W64_ASM "{lit}\\n"', f"#define NEP_ATTN_W64_NBUF {nbuf}"]
    clob = ([f'"v{r}"' for r in CLOBBER_VGPRS] + [f'"a{r}"' for r in CLOBBER_AGPRS]
            + [f'"s{r}"' for r in CLOBBER_SGPRS])
    lines.append("#define NEP_ATTN_W64_CLOBBERS " + ", ".join(clob) + ', "m0", "vcc", "memory"')
    return "\n".join(lines)
