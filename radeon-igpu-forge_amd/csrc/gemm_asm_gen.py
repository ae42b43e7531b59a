"""Generate gemm_asm.h: the hand-scheduled K loops of the whole-tile GEMM kernels (linear.hip).

    python radeon-igpu-forge_amd/csrc/gemm_asm_gen.py          # rewrite gemm_asm.h
    python radeon-igpu-forge_amd/csrc/gemm_asm_gen.py --check  # verify only (used by the tests)

Three products of a linear layer, each a workgroup of 4 waves on a 256 x (64 NJ) tile of C,
each wave 128 x (32 NJ) as 4 x NJ blocks of `v_mfma_f32_32x32x16_bf16` whose fp32
accumulators stay in AGPRs for the whole K loop (one inline-asm statement):

  fwd    C = X W^T      X (M x K), W (N x K): K runs along the rows of both ("row" operands)
  dgrad  C = dY W       dY (M x K) a row operand, W (K x N) with K down its rows ("col")
  wgrad  C = dY^T X     dY (K x M), X (K x N): both col operands (K = tokens)

K advances in steps of 32 held in 4 LDS stages.  A stage holds the M-side operand's tile,
then the N-side's.  The loops with a row operand (fwd, dgrad) keep the stages in two
buffers of two steps and load a buffer every other step: a row's segments of both steps are
then one 128-byte run (a whole cache line: loaded one 64-byte step at a time, every line was
requested twice, and from HBM those requests, not the bytes, set the pace: 1-8 % faster
when the operands come from HBM).  The weight gradient keeps four one-step buffers.
  row operand: one LDS row per tile row, 144 bytes in a two-step buffer (2 x 32 bf16 and
    16 of padding), 80 in a one-step one (the 32 rows of a read fall in distinct banks); an
    operand block is one `ds_read_b128`, lane l taking row l%32 and K 8 (l/32) + 0..7;
  col operand: one LDS row per K (32 rows per step), the tile's columns + 32 bf16 of
    padding (the 4 rows of a transposed read fall in disjoint banks); an operand block is two
    `ds_read_b64_tr_b16` (4 K each).  With a row operand on the other side (dgrad) the two
    reads take K 8 g + 0..3 and 8 g + 4..7 (g = l/32), the row operand's order; in wgrad both
    sides take 4 g + 0..3 and 8 + 4 g + 0..3 (fx_mfma.h's lds_op_t, the general kernel's
    order, so the two kernels agree bit for bit).
The operand sets are fixed VGPRs at the top of the file (declared clobbered): transposed
reads write 2-register halves of the 4-register MFMA operands, which inline-asm operands
cannot name.

Per step: the first half runs 4 NJ MFMAs on chunk 0 while the reads of chunk 1 follow the
first MFMAs; `s_waitcnt vmcnt` for the next stage's loads, `lgkmcnt(0)` and `s_barrier`
(every wave is then done reading this stage); the second half runs chunk 1's MFMAs with the
reads of the next step's chunk 0 and, spread evenly over its MFMAs, the loads of the buffer
every wave has just finished reading (`global_load_lds_dwordx4`, L per wave; instruction
q = wave + 4 t of a buffer covers 64 16-byte slots, the M-side's, then the N-side's, then a
never-read pad that rounds the count to a multiple of 4), each pointer then advanced by its
stride (one SGPR pair per t: the region of instruction q may differ between waves).
One-step buffers: each step loads step j + 4, three steps ahead; at the barrier of step j
only the loads of steps j + 2 and j + 3 may be outstanding (`vmcnt(2 L)`), fewer in the last
three steps.  Two-step buffers: odd steps load steps j + 3 and j + 4 into the buffer of j - 1
and j; the barrier before a buffer's first step is read waits for it (`vmcnt(0)`, nothing was
issued after it), the other barriers need no wait (the second step came with the first).
The operands rotate through 4 register sets (one per half step, refilled three halves after
the MFMAs that read it).

Any number of steps >= 4: the loop body is 4 steps (stages rotate with period 4, operand sets
with period 2) and the last 4 steps are a tail without loads, so a product of n steps enters
the body at step p = (4 - n % 4) % 4 (`phase`), its prologue having loaded steps 0..3 into
stages p, p + 1, p + 2, p + 3 (mod 4).  Two-step buffers take an even n: an odd K / 32 gets a
leading step of zeros (loop_steps), which the prologue loads from the zero line and which adds
exact zeros to the accumulators.

Operands of each loop (FX_<KIND>_OUTS / _INS / _CLOBBERS): acc[4 j + i] ("+a"; i: M-side
block, j: N-side block), the L load pointers P[t] ("+v", 64-bit), the loop iterations
("+s"), the saved M0 ("=&s"); the stages' M-side and N-side read addresses vM[s], vN[s]
("v"), the wave's LDS load base sbase, phase, and the L pointer strides S[t] in bytes ("s").
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gemm_asm.h")
STAGES = 4          # LDS stages
SETS = 4            # operand register sets


class Kind:
    """Layout and operand numbering of one loop."""

    def __init__(self, name, m_mode, n_mode, nj, order):
        self.name, self.m_mode, self.n_mode, self.nj, self.order = name, m_mode, n_mode, nj, order
        self.set_size = 4 + nj                        # operand blocks per set
        self.fb = 256 - 4 * SETS * self.set_size      # first VGPR of the operand sets
        self.n_acc = 4 * nj
        # Two-step buffers when an operand has K along its rows: a row operand's 64-byte
        # segment of one step is half of a 128-byte line, and loading each row's segments of
        # two steps together (one 128-byte run per row) halves the cache-line requests; so
        # the four stages are two buffers of two steps, loaded every other step.
        self.pair = "row" in (m_mode, n_mode)
        self.ksteps = 2 if self.pair else 1           # K steps of 32 per buffer
        self.bufs = STAGES // self.ksteps             # LDS buffers
        self.row_stride = 144 if self.pair else 80    # LDS bytes per row of a row operand
        self.region = []                              # (mode, bytes, wave-instructions) per buffer side
        for mode, rows in ((m_mode, 256), (n_mode, 64 * nj)):
            if mode == "row":
                self.region.append(("row", rows * self.row_stride, rows * self.row_stride // 1024))
            else:
                row_bytes = (rows + 32) * 2
                nb = 32 * self.ksteps * row_bytes
                self.region.append(("col", nb, nb // 1024))
        self.col_row = {side: ((64 * (nj if side else 4) + 32) * 2 if self.region[side][0] == "col" else None)
                        for side in (0, 1)}
        n_ins = self.region[0][2] + self.region[1][2]
        self.loads = -(-n_ins // 4)                   # L
        self.pad_ins = 4 * self.loads - n_ins
        self.stage = 1024 * 4 * self.loads            # bytes of one buffer
        self.n_off = self.region[0][1]                # N-side region offset in a buffer
        # operand numbers
        self.acc0 = 0
        self.ptr0 = self.n_acc
        self.iters = self.ptr0 + self.loads
        self.m0s = self.iters + 1
        self.vm0 = self.m0s + 1
        self.vn0 = self.vm0 + STAGES
        self.sbase = self.vn0 + STAGES
        self.phase = self.sbase + 1
        self.stride0 = self.phase + 1

    def freg(self, b, x):
        """first VGPR of operand set b, block x (x < 4: M-side block x, else N-side x - 4)"""
        return self.fb + 4 * (self.set_size * b + x)

    def ins_region(self, q):
        """side of wave-instruction q of a stage: 0 (M), 1 (N) or 2 (pad)"""
        if q < self.region[0][2]:
            return 0
        return 1 if q < self.region[0][2] + self.region[1][2] else 2

    def hi_off(self, side):
        """offset of a col block's second transposed read (4 K rows on, or 8 in lds_op_t's order)"""
        return (8 if self.order == "lds_op_t" else 4) * self.col_row[side]


KINDS = [Kind("FWD_NJ4", "row", "row", 4, "natural"), Kind("FWD_NJ3", "row", "row", 3, "natural"),
         Kind("DGRAD_NJ4", "row", "col", 4, "natural"), Kind("DGRAD_NJ3", "row", "col", 3, "natural"),
         Kind("WGRAD", "col", "col", 4, "lds_op_t"), Kind("WGRAD_NJ3", "col", "col", 3, "lds_op_t")]


def block_reads(kd, b, x, stage, ch):
    """the read instructions that fill operand set b, block x with chunk ch of a stage"""
    side = 0 if x < 4 else 1
    blk = x if x < 4 else x - 4
    base = (kd.vm0 if side == 0 else kd.vn0) + stage
    r = kd.freg(b, x)
    if kd.region[side][0] == "row":
        return [f"ds_read_b128 v[{r}:{r + 3}], %{base} offset:{32 * ch + 32 * kd.row_stride * blk}"]
    lo = ch * 16 * kd.col_row[side] + 64 * blk
    return [f"ds_read_b64_tr_b16 v[{r}:{r + 1}], %{base} offset:{lo}",
            f"ds_read_b64_tr_b16 v[{r + 2}:{r + 3}], %{base} offset:{lo + kd.hi_off(side)}"]


def generate(kd):
    out = []
    e = out.append
    n_mfma = kd.n_acc

    def reads(b, stage, ch):
        return [block_reads(kd, b, x, stage, ch) for x in range(kd.set_size)]

    def loads(stage):
        # spread evenly over the half step's MFMAs: issued in bursts (the last 8 MFMAs) the
        # loads of the four waves queued up in the address unit and delayed MFMA issue
        groups = [[] for _ in range(n_mfma)]
        for t in range(kd.loads):
            groups[(t * n_mfma) // kd.loads] += [
                f"s_add_u32 m0, %{kd.sbase}, {stage * kd.stage + 4096 * t}", "s_nop 0",
                f"global_load_lds_dwordx4 %{kd.ptr0 + t}, off", "s_nop 0"]
        for t in range(kd.loads):
            groups[n_mfma - 1].append(f"v_lshl_add_u64 %{kd.ptr0 + t}, %{kd.ptr0 + t}, 0, %{kd.stride0 + t}")
        return groups

    def loads_buf(buf):
        # a two-step buffer's loads, spread evenly over the half step's MFMAs
        groups = [[] for _ in range(n_mfma)]
        for t in range(kd.loads):
            groups[(t * n_mfma) // kd.loads] += [
                f"s_add_u32 m0, %{kd.sbase}, {buf * kd.stage + 4096 * t}", "s_nop 0",
                f"global_load_lds_dwordx4 %{kd.ptr0 + t}, off", "s_nop 0"]
        for t in range(kd.loads):
            groups[n_mfma - 1].append(f"v_lshl_add_u64 %{kd.ptr0 + t}, %{kd.ptr0 + t}, 0, %{kd.stride0 + t}")
        return groups

    def mfma(k, cur):
        j, i = k // 4, k % 4
        m_reg, n_reg = kd.freg(cur, i), kd.freg(cur, 4 + j)
        a, b_ = (n_reg, m_reg) if not kd.name.startswith("WGRAD") else (m_reg, n_reg)
        e(f"v_mfma_f32_32x32x16_bf16 %{kd.acc0 + k}, v[{a}:{a + 3}], v[{b_}:{b_ + 3}], %{kd.acc0 + k}")

    def half(cur, rd, extra):
        e("s_waitcnt lgkmcnt(0)")
        for k in range(n_mfma):
            mfma(k, cur)
            if rd and k < len(rd):
                for x in rd[k]:
                    e(x)
            if extra:
                for x in extra[k]:
                    e(x)

    def step(u, vm, do_load, next_reads):
        c0, c1, c2 = (2 * u) % SETS, (2 * u + 1) % SETS, (2 * u + 2) % SETS
        half(c0, reads(c1, u % STAGES, 1), None)
        if vm is not None:
            e(f"s_waitcnt vmcnt({vm})")
        e("s_waitcnt lgkmcnt(0)")
        e("s_barrier")
        if not do_load:
            ld = None
        elif kd.pair:   # both steps of buffer u // 2 are read by now (odd u)
            ld = loads_buf(u // 2) if u % 2 else None
        else:
            ld = loads(u % STAGES)
        half(c1, reads(c2, (u + 1) % STAGES, 0) if next_reads else None, ld)

    L = kd.loads
    if kd.pair:
        # at the barrier of step k the loads of step k + 1 must have landed: at an even stage
        # k + 1 shares step k's buffer (landed already), at an odd one its buffer is the last
        # issued (vmcnt(0)); the prologue loaded two buffers, the first of which the entry
        # step reads
        body_vm, tail_vm, entry_vm = [None, 0, None, 0], [None, 0, None, None], L
    else:
        body_vm = [(STAGES - 2) * L] * STAGES
        tail_vm = [max(0, STAGES - 2 - u) * L for u in range(STAGES)]
        entry_vm = (STAGES - 1) * L
    e(f"s_mov_b32 %{kd.m0s}, m0")
    e(f"s_waitcnt vmcnt({entry_vm})")
    e("s_barrier")
    entries = range(0, STAGES, kd.ksteps)   # two-step buffers: even step counts, even phases
    for p in entries[1:]:
        e(f"s_cmp_eq_u32 %{kd.phase}, {p}")
        e(f"s_cbranch_scc1 .Lp{p}%=")
    for p in entries:
        if p:
            e(f".Lp{p}%=:")
        for blk in reads((2 * p) % SETS, p, 0):
            for x in blk:
                e(x)
        if p == 0:
            e(f"s_cmp_eq_u32 %{kd.iters}, 0")
            e("s_cbranch_scc1 .Ltail%=")
        e(f"s_branch .Lu{p}%=")
    for u in range(STAGES):
        e(f".Lu{u}%=:")
        step(u, body_vm[u], True, True)
    e(f"s_sub_u32 %{kd.iters}, %{kd.iters}, 1")
    e(f"s_cmp_lg_u32 %{kd.iters}, 0")
    e("s_cbranch_scc1 .Lu0%=")
    e(".Ltail%=:")
    for u in range(STAGES):   # the last STAGES steps: no loads; the next step's were issued
        step(u, tail_vm[u], False, u < STAGES - 1)
    for _ in range(8):  # the last MFMAs' results before the compiler reads the AGPRs
        e("s_nop 7")
    e(f"s_mov_b32 m0, %{kd.m0s}")
    return out


def loop_steps(kd, nsteps):
    """K steps the loop runs for a product of nsteps: two-step buffers take an even count, a
    leading step of zeros (loaded from the zero line by the prologue) making up an odd one"""
    return nsteps + (nsteps % 2 if kd.pair else 0)


def schedule(nsteps):
    """(phase, iterations) for a loop of nsteps K steps"""
    p = (STAGES - nsteps % STAGES) % STAGES
    return p, (nsteps - STAGES + p) // STAGES


def decode_read(kd, ins):
    """(register, half, side, stage, chunk, block) of a read instruction"""
    if m := re.match(r"ds_read_b128 v\[(\d+):(\d+)\], %(\d+) offset:(\d+)$", ins):
        reg, op, off = int(m[1]), int(m[3]), int(m[4])
        assert int(m[2]) == reg + 3
        side = 0 if kd.vm0 <= op < kd.vm0 + STAGES else 1
        assert kd.region[side][0] == "row", ("b128 read of a col operand", ins)
        blk, r = divmod(off, 32 * kd.row_stride)
        ch, r = divmod(r, 32)
        assert r == 0 and ch in (0, 1) and blk < 4
        return reg, None, side, op - (kd.vm0 if side == 0 else kd.vn0), ch, blk
    m = re.match(r"ds_read_b64_tr_b16 v\[(\d+):(\d+)\], %(\d+) offset:(\d+)$", ins)
    assert m, ins
    reg, op, off = int(m[1]), int(m[3]), int(m[4])
    assert int(m[2]) == reg + 1
    side = 0 if kd.vm0 <= op < kd.vm0 + STAGES else 1
    assert kd.region[side][0] == "col", ("transposed read of a row operand", ins)
    rowb = kd.col_row[side]
    ch, r = divmod(off, 16 * rowb)
    hi, r = divmod(r, kd.hi_off(side))
    blk, r2 = divmod(r, 64)
    assert r2 == 0 and ch in (0, 1) and hi in (0, 1) and blk < 4
    return reg, hi, side, op - (kd.vm0 if side == 0 else kd.vn0), ch, blk


def check(kd, nsteps):
    """Interpret one wave's instruction stream (control flow included) for nsteps K steps and
    verify the data flow: every MFMA multiplies operand blocks that all hold the same
    (step, chunk), the blocks its accumulator index names (M-side block i, N-side block j, on
    the A/B inputs the kind's C layout needs), and each accumulator sees (0, 0), (0, 1),
    (1, 0), ... in order; every read of a stage sees the step the reader expects, loaded
    completely (this wave's vmcnt wait, then a barrier: the other waves' waits precede their
    arrival) and writes the register its block and half belong to; a stage is reloaded only
    after a barrier that follows this wave's lgkmcnt(0) after its last read of it; loads go to
    their pointer's slots at the stage of their step, and each pointer advances by its own
    stride after its load; an operand set is refilled only 4 MFMAs or more after its last use."""
    assert nsteps >= STAGES
    prog = generate(kd)
    labels = {l[:-1]: n for n, l in enumerate(prog) if l.endswith(":")}
    phase, iters = schedule(nsteps)
    sreg = {kd.iters: iters, kd.phase: phase}
    stage_of = lambda j: (j + phase) % STAGES  # noqa: E731
    L = kd.loads
    kst = kd.ksteps
    # each load instruction fills its slots of one buffer: kst consecutive steps, one stage each
    vmq = [[(stage_of(j0 + i), j0 + i) for i in range(kst)] for j0 in range(0, STAGES, kst) for _ in range(L)]
    stage_data = {stage_of(j): [j, L, None] for j in range(STAGES)}
    ptr_step = {kd.ptr0 + t: STAGES for t in range(L)}
    loaded = {}
    reg_holds, pending = {}, []
    last_read = {s_: -1 for s_ in range(STAGES)}
    last_wait = {s_: -1 for s_ in range(STAGES)}
    last_barrier = -1
    set_last_use = {}
    acc_seq = {k: [] for k in range(kd.n_acc)}
    mfmas = halves = cur_step = 0
    m0 = None
    scc = False
    pc = pos = 0
    per_half = kd.n_acc
    while pc < len(prog):
        ins = prog[pc]
        pos += 1
        assert pos < 10 ** 7
        nxt = pc + 1
        if ins.endswith(":"):
            pass
        elif m := re.match(r"s_cmp_(eq|lg)_u32 %(\d+), (\d+)$", ins):
            v = sreg[int(m[2])]
            scc = (v == int(m[3])) if m[1] == "eq" else (v != int(m[3]))
        elif m := re.match(r"s_cbranch_scc1 (\S+)$", ins):
            nxt = labels[m[1]] if scc else nxt
        elif m := re.match(r"s_branch (\S+)$", ins):
            nxt = labels[m[1]]
        elif m := re.match(r"s_sub_u32 %(\d+), %(\d+), 1$", ins):
            assert m[1] == m[2]
            sreg[int(m[1])] -= 1
        elif m := re.match(r"s_waitcnt vmcnt\((\d+)\)$", ins):
            while len(vmq) > int(m[1]):
                for st, j in vmq.pop(0):
                    d = stage_data[st]
                    assert d[0] == j
                    d[1] -= 1
                    if d[1] == 0:
                        d[2] = pos
        elif ins == "s_waitcnt lgkmcnt(0)":
            for reg, val, st in pending:
                reg_holds[reg] = val
                last_wait[st] = pos
            pending = []
        elif ins == "s_barrier":
            last_barrier = pos
        elif ins.startswith("ds_read"):
            reg, hi, side, st, ch, blk = decode_read(kd, ins)
            b, q = divmod(reg - kd.fb, 4 * kd.set_size)
            x, h = divmod(q, 4)
            want_x = blk if side == 0 else 4 + blk
            assert x == want_x and h == (0 if hi is None else 2 * hi), ("read into the wrong register", ins)
            d = stage_data[st]
            want = cur_step if ch == 1 else (cur_step + 1 if halves % 2 else cur_step)
            assert d[0] == want, ("stage holds the wrong step", kd.name, nsteps, ins, d, want)
            assert d[1] == 0 and d[2] is not None and last_barrier > d[2], ("read before the loads landed", ins)
            assert mfmas - set_last_use.get(b, -100) >= 4, ("operand set refilled too early", ins)
            regs = [reg, reg + 1, reg + 2, reg + 3] if hi is None else [reg, reg + 1]
            for r_ in regs:
                reg_holds.pop(r_, None)
                pending.append((r_, (want, ch), st))
            last_read[st] = pos
        elif m := re.match(r"v_mfma_f32_32x32x16_bf16 %(\d+), v\[(\d+):(\d+)\], v\[(\d+):(\d+)\], %(\d+)$", ins):
            k = int(m[1]) - kd.acc0
            assert int(m[6]) == int(m[1]) and int(m[3]) == int(m[2]) + 3 and int(m[5]) == int(m[4]) + 3
            ra, rb = int(m[2]), int(m[4])
            m_reg, n_reg = (rb, ra) if not kd.name.startswith("WGRAD") else (ra, rb)
            bm, qm = divmod(m_reg - kd.fb, 4 * kd.set_size)
            bn, qn = divmod(n_reg - kd.fb, 4 * kd.set_size)
            assert bm == bn and qm == 4 * (k % 4) and qn == 4 * (4 + k // 4), ("wrong operand blocks", ins)
            vals = {reg_holds.get(r_) for r_ in list(range(ra, ra + 4)) + list(range(rb, rb + 4))}
            assert len(vals) == 1 and None not in vals, ("operands incomplete or mixed", ins, vals)
            acc_seq[k].append(vals.pop())
            set_last_use[bm] = mfmas
            mfmas += 1
            if mfmas % per_half == 0:
                halves += 1
                if halves % 2 == 0:
                    cur_step += 1
        elif m := re.match(r"s_add_u32 m0, %(\d+), (\d+)$", ins):
            assert int(m[1]) == kd.sbase
            m0 = int(m[2])
        elif m := re.match(r"global_load_lds_dwordx4 %(\d+), off$", ins):
            p = int(m[1])
            j0 = ptr_step[p]
            buf, rel = divmod(m0, kd.stage)
            t = p - kd.ptr0
            assert rel == 4096 * t, ("load to another pointer's slots", ins)
            item = []
            for i in range(kst):
                j, st = j0 + i, buf * kst + i
                assert j < nsteps and st == stage_of(j), ("load of the wrong step or stage", ins, j, st)
                assert last_read[st] < last_wait[st] < last_barrier, ("reload before the reads ended", ins)
                d = stage_data[st]
                if d[0] != j:
                    assert d[1] == 0 and d[0] == j - STAGES
                    stage_data[st] = d = [j, 0, None]
                d[1] += 1
                loaded.setdefault(j, []).append(t)
                item.append((st, j))
            vmq.append(item)
            m0 = None
        elif m := re.match(r"v_lshl_add_u64 %(\d+), %(\d+), 0, %(\d+)$", ins):
            p = int(m[1])
            assert int(m[2]) == p and int(m[3]) == kd.stride0 + (p - kd.ptr0), ("wrong stride", ins)
            assert loaded.get(ptr_step[p], []).count(p - kd.ptr0) == 1, ("advance before the load", ins)
            ptr_step[p] += kst
        elif ins.startswith("s_nop") or ins.startswith("s_mov_b32"):
            pass
        else:
            raise AssertionError(f"unknown instruction {ins}")
        pc = nxt
    assert not pending and cur_step == nsteps, (cur_step, nsteps)
    assert all(v == nsteps for v in ptr_step.values()), ptr_step
    for j in range(STAGES, nsteps):
        assert sorted(loaded[j]) == list(range(L)), (j, loaded[j])
    want = [(j, c) for j in range(nsteps) for c in (0, 1)]
    for k in range(kd.n_acc):
        assert acc_seq[k] == want, ("accumulation order", kd.name, k)
    return phase, iters


def header_text():
    parts = ["// Generated by gemm_asm_gen.py (do not edit): the K loops of the whole-tile GEMM kernels.",
             "#pragma once", ""]
    for kd in KINDS:
        out = generate(kd)
        outs = [f'"+a"(acc[{k}])' for k in range(kd.n_acc)] + [f'"+v"(P[{t}])' for t in range(kd.loads)]
        outs += ['"+s"(iters)', '"=&s"(m0save)']
        ins = [f'"v"(vM[{s}])' for s in range(STAGES)] + [f'"v"(vN[{s}])' for s in range(STAGES)]
        ins += ['"s"(sbase)', '"s"(phase)'] + [f'"s"(S[{t}])' for t in range(kd.loads)]
        clob = ['"memory"', '"scc"'] + [f'"v{r}"' for r in range(kd.fb, 256)]
        body = " \\\n    ".join('"' + x + '\\n\\t"' for x in out)
        n = kd.name
        parts += [f"// {n}: M side {kd.region[0][0]}, N side {kd.region[1][0]}, NJ = {kd.nj}; "
                  f"{len(out)} instructions",
                  f"#define FX_{n}_STAGE {kd.stage}",
                  f"#define FX_{n}_STAGES {STAGES}",
                  f"#define FX_{n}_BUFS {kd.bufs}",
                  f"#define FX_{n}_KSTEPS {kd.ksteps}",
                  f"#define FX_{n}_ROW {kd.row_stride}",
                  f"#define FX_{n}_LOADS {kd.loads}",
                  f"#define FX_{n}_N_OFF {kd.n_off}",
                  f"#define FX_{n}_M_INS {kd.region[0][2]}",
                  f"#define FX_{n}_N_INS {kd.region[1][2]}",
                  f"#define FX_{n}_KLOOP \\\n    {body}",
                  f"#define FX_{n}_OUTS \\\n    " + ", \\\n    ".join(outs),
                  f"#define FX_{n}_INS \\\n    " + ", \\\n    ".join(ins),
                  f"#define FX_{n}_CLOBBERS \\\n    " + ", \\\n    ".join(clob), ""]
    return "\n".join(parts)


STEP_COUNTS = (4, 5, 6, 7, 8, 9, 24, 72, 73, 74, 75, 96)


def main(argv):
    for kd in KINDS:
        for n in STEP_COUNTS:
            check(kd, loop_steps(kd, n))
    text = header_text()
    if "--check" in argv:
        with open(OUT) as f:
            assert f.read() == text, "gemm_asm.h differs from the generator's output"
        print("gemm_asm.h matches the generator; schedule checks passed")
        return
    with open(OUT, "w") as f:
        f.write(text)
    print(f"wrote {OUT}; schedule checks passed")


if __name__ == "__main__":
    main(sys.argv[1:])
