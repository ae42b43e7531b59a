"""Generate gemm_wgrad_kloop.h: the hand-scheduled K loop of gemm_wgrad_fast_kernel (linear.hip).

    python radeon-igpu-forge_amd/csrc/gemm_wgrad_gen.py          # rewrite gemm_wgrad_kloop.h
    python radeon-igpu-forge_amd/csrc/gemm_wgrad_gen.py --check  # verify only (used by the tests)

The weight gradient C (M x N) = A^T B contracts over token rows: A = dY (T x M) and B = X
(T x N) are row-major with the tokens down the rows.  A workgroup of 4 waves owns a 256 x 256
tile of C and a range of the tokens (a split-K slice); each wave accumulates 128 x 128 of it
in 16 blocks of `v_mfma_f32_32x32x16_bf16` whose fp32 accumulators stay in AGPRs for the
whole loop (one inline-asm statement).

K advances in steps of 32 tokens held in 3 LDS stages.  A stage holds the step's 32 rows of
the A tile, then of the B tile, 576 bytes a row (256 bf16 and 32 bytes of padding, so that
the four rows a transposed read touches fall in disjoint banks).  The MFMA operands take 8
consecutive tokens per lane for one column, so they are read with `ds_read_b64_tr_b16`
(two per 32 x 16 operand block: tokens k0 + 4 (g' / 2) + 0..3 and k0 + 8 + the same, g' the
16-lane group, the K permutation of fx_mfma.h's lds_op_t; both operands see the same
permutation, so each MFMA is the plain contraction).  The operand register sets are fixed
VGPRs (v160..v255, declared clobbered): the transposed reads write 2-register halves of
the 4-register MFMA operands, which inline-asm operands cannot name.

Per step: the first half runs 16 MFMAs on chunk 0's operand set while the reads of chunk 1
follow the first 8; `s_waitcnt vmcnt` for the next stage's loads, `lgkmcnt(0)` and
`s_barrier` (every wave is then done reading this stage); the second half runs chunk 1's
MFMAs with the reads of the next step's chunk 0 and the loads of step j + 3 into this stage
(`global_load_lds_dwordx4`, 9 per wave: the 36 wave-instructions of 64 16-byte slots that
cover 2 x 32 rows x 36 slots) after its last 8 MFMAs, each pointer then advanced by 32 rows.
Loads run two steps ahead: at the barrier of step j only the loads of step j + 2 may be
outstanding (`vmcnt(9)`), none in the last two steps.

Any number of steps >= 3: the loop body is 3 steps (stages and register sets both rotate
with period 3) and the last 3 steps are a tail without loads, so a slice of n steps enters
the body at step p = (3 - n % 3) % 3 (`phase`), the prologue having loaded steps 0..2 into
stages p, p + 1, p + 2 (mod 3).

Operands (FX_WGRAD_KLOOP_OUTS / _INS): %0..%15 acc[4 j + i] ("+a"; i: A column block,
j: B column block); %16..%24 the 9 load pointers ("+v", 64-bit); %25 loop iterations
("+s"); %26 saved M0 ("=&s"); %27..%29 the stages' A read addresses and %30..%32 B read
addresses ("v"); %33 the wave's LDS load base, %34 phase, %35..%37 the pointer strides for
32 rows of A, of the 5th load (A for waves 0 and 1, B for 2 and 3) and of B ("s").
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gemm_wgrad_kloop.h")

ROW = 576                      # LDS bytes per token row of an operand tile
OP_BYTES = 32 * ROW            # one operand's 32 rows
STAGE = 2 * OP_BYTES           # A then B
LOADS = 9                      # per wave and stage
FB = 160                       # first VGPR of the operand sets
ACC, PTR, ITERS, M0S = 0, 16, 25, 26
VA, VB, SBASE, PHASE, STRIDE = 27, 30, 33, 34, 35   # STRIDE + 0: A, + 1: 5th load, + 2: B


def freg(b, x):
    """first VGPR of operand set b, block x (x < 4: A column block x, else B block x - 4)"""
    return FB + 32 * b + 4 * x


def stride_of(t):
    return STRIDE + (0 if t < 4 else 1 if t == 4 else 2)


def generate():
    out = []
    e = out.append

    def reads(b, stage, ch):
        """the 16 transposed reads that fill operand set b with chunk ch of a stage"""
        rs = []
        for x in range(8):
            base = VA + stage if x < 4 else VB + stage
            lo = ch * 16 * ROW + 64 * (x % 4)
            r = freg(b, x)
            rs.append(f"ds_read_b64_tr_b16 v[{r}:{r + 1}], %{base} offset:{lo}")
            rs.append(f"ds_read_b64_tr_b16 v[{r + 2}:{r + 3}], %{base} offset:{lo + 8 * ROW}")
        return rs

    def loads(stage):
        groups = [[] for _ in range(8)]
        slot = [0, 0, 1, 2, 3, 4, 5, 6, 7]
        for t in range(LOADS):
            groups[slot[t]] += [f"s_add_u32 m0, %{SBASE}, {stage * STAGE + 4096 * t}", "s_nop 0",
                                f"global_load_lds_dwordx4 %{PTR + t}, off", "s_nop 0"]
        for t in range(LOADS):
            groups[7].append(f"v_lshl_add_u64 %{PTR + t}, %{PTR + t}, 0, %{stride_of(t)}")
        return groups

    def half(cur, rd, extra):
        e("s_waitcnt lgkmcnt(0)")
        for k in range(16):
            j, i = k // 4, k % 4
            e(f"v_mfma_f32_32x32x16_bf16 %{ACC + k}, v[{freg(cur, i)}:{freg(cur, i) + 3}], "
              f"v[{freg(cur, 4 + j)}:{freg(cur, 4 + j) + 3}], %{ACC + k}")
            if rd and k < 8:
                e(rd[2 * k])
                e(rd[2 * k + 1])
            if extra and k >= 8:
                for x in extra[k - 8]:
                    e(x)

    def step(u, vm, do_load, next_reads):
        c0, c1, c2 = (2 * u) % 3, (2 * u + 1) % 3, (2 * u + 2) % 3
        half(c0, reads(c1, u, 1), None)
        e(f"s_waitcnt vmcnt({vm})")
        e("s_waitcnt lgkmcnt(0)")
        e("s_barrier")
        half(c1, reads(c2, (u + 1) % 3, 0) if next_reads else None, loads(u) if do_load else None)

    e(f"s_mov_b32 %{M0S}, m0")
    e(f"s_waitcnt vmcnt({2 * LOADS})")
    e("s_barrier")
    e(f"s_cmp_eq_u32 %{PHASE}, 1")
    e("s_cbranch_scc1 .Lp1%=")
    e(f"s_cmp_eq_u32 %{PHASE}, 2")
    e("s_cbranch_scc1 .Lp2%=")
    for r in reads(0, 0, 0):
        e(r)
    e(f"s_cmp_eq_u32 %{ITERS}, 0")
    e("s_cbranch_scc1 .Ltail%=")
    e("s_branch .Lu0%=")
    e(".Lp1%=:")
    for r in reads(2, 1, 0):
        e(r)
    e("s_branch .Lu1%=")
    e(".Lp2%=:")
    for r in reads(1, 2, 0):
        e(r)
    e("s_branch .Lu2%=")
    for u in range(3):
        e(f".Lu{u}%=:")
        step(u, LOADS, True, True)
    e(f"s_sub_u32 %{ITERS}, %{ITERS}, 1")
    e(f"s_cmp_lg_u32 %{ITERS}, 0")
    e("s_cbranch_scc1 .Lu0%=")
    e(".Ltail%=:")
    step(0, LOADS, False, True)
    step(1, 0, False, True)
    step(2, 0, False, False)
    for _ in range(8):  # the last MFMAs' results before the compiler reads the AGPRs
        e("s_nop 7")
    e(f"s_mov_b32 m0, %{M0S}")
    return out


def schedule(nsteps):
    """(phase, iterations) for a slice of nsteps K steps"""
    p = (3 - nsteps % 3) % 3
    return p, (nsteps - 3 + p) // 3


def check(nsteps):
    """Interpret one wave's instruction stream (control flow included) for a slice of nsteps
    steps and verify the data flow: every MFMA multiplies operand blocks that all hold the
    same (step, chunk), each accumulator sees (0, 0), (0, 1), (1, 0), ... in order, and the
    A and B blocks are the ones its index names; every read of a stage sees the step the
    reader expects, loaded completely (this wave's vmcnt wait, then a barrier: the other
    waves' waits precede their arrival); a stage is reloaded only after a barrier that
    follows this wave's lgkmcnt(0) after its last read of the stage; loads go to the slots of
    their pointer at the stage of their step, and pointers advance by their own stride after
    their load; an operand register is refilled only 4 MFMAs or more after its last use."""
    assert nsteps >= 3
    prog = generate()
    labels = {l[:-1]: n for n, l in enumerate(prog) if l.endswith(":")}
    phase, iters = schedule(nsteps)
    sreg = {ITERS: iters, PHASE: phase}
    stage_of = lambda j: (j + phase) % 3  # noqa: E731
    # prologue (C++): steps 0, 1, 2 into their stages, 9 loads each, pointers then at step 3
    vmq = [(stage_of(j), j) for j in range(3) for _ in range(LOADS)]
    stage_data = {}        # stage -> [step, loads outstanding, position of completion]
    for j in range(3):
        stage_data[stage_of(j)] = [j, LOADS, None]
    ptr_step = {PTR + t: 3 for t in range(LOADS)}
    loaded_slots = {}
    reg_holds = {}         # VGPR pair -> (step, chunk, stage-read position) once complete
    pending = []           # reads issued since the last lgkmcnt(0): (pair, value, stage)
    last_read = {0: -1, 1: -1, 2: -1}
    last_wait_after_read = {0: -1, 1: -1, 2: -1}
    last_barrier = -1
    set_last_use = {}
    acc_seq = {k: [] for k in range(16)}
    mfmas = 0
    cur_step = 0           # the step whose MFMAs run next
    halves_done = 0
    m0 = None
    scc = False
    pc, pos = 0, 0
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
            if scc:
                nxt = labels[m[1]]
        elif m := re.match(r"s_branch (\S+)$", ins):
            nxt = labels[m[1]]
        elif m := re.match(r"s_sub_u32 %(\d+), %(\d+), 1$", ins):
            assert m[1] == m[2]
            sreg[int(m[1])] -= 1
        elif m := re.match(r"s_waitcnt vmcnt\((\d+)\)$", ins):
            while len(vmq) > int(m[1]):
                st, j = vmq.pop(0)
                d = stage_data[st]
                assert d[0] == j
                d[1] -= 1
                if d[1] == 0:
                    d[2] = pos
        elif ins == "s_waitcnt lgkmcnt(0)":
            for pair, val, st in pending:
                reg_holds[pair] = val
                last_wait_after_read[st] = pos
            pending = []
        elif ins == "s_barrier":
            last_barrier = pos
        elif m := re.match(r"ds_read_b64_tr_b16 v\[(\d+):(\d+)\], %(\d+) offset:(\d+)$", ins):
            lo_reg, op, off = int(m[1]), int(m[3]), int(m[4])
            assert int(m[2]) == lo_reg + 1
            is_a = VA <= op < VA + 3
            st = op - (VA if is_a else VB)
            ch, rem = divmod(off, 16 * ROW)
            hi, rem = divmod(rem, 8 * ROW)
            blk, r = divmod(rem, 64)
            assert r == 0 and hi in (0, 1) and ch in (0, 1) and blk < 4
            b, q = divmod(lo_reg - FB, 32)
            x, h = divmod(q, 4)
            assert h == 2 * hi and (x < 4) == is_a and x % 4 == blk, ("read into the wrong register", ins)
            d = stage_data[st]
            # chunk 1 is read during step cur_step, chunk 0 during the step before it runs
            want = cur_step if ch == 1 else (cur_step + 1 if halves_done % 2 else cur_step)
            assert d[0] == want, ("stage holds the wrong step", nsteps, ins, d, want)
            assert d[1] == 0 and d[2] is not None and last_barrier > d[2], ("read before the loads landed", ins)
            assert mfmas - set_last_use.get(b, -100) >= 4, ("operand register refilled too early", ins)
            reg_holds.pop(lo_reg, None)
            pending.append((lo_reg, (want, ch, st), st))
            last_read[st] = pos
        elif m := re.match(r"v_mfma_f32_32x32x16_bf16 %(\d+), v\[(\d+):(\d+)\], v\[(\d+):(\d+)\], %(\d+)$", ins):
            k = int(m[1])
            assert int(m[6]) == k and int(m[3]) == int(m[2]) + 3 and int(m[5]) == int(m[4]) + 3
            ra, rb = int(m[2]), int(m[4])
            ba, xa = divmod(ra - FB, 32)
            bb, xb = divmod(rb - FB, 32)
            assert ba == bb and xa == 4 * (k % 4) and xb == 4 * (4 + k // 4), ("wrong operand blocks", ins)
            vals = {reg_holds.get(r) for r in (ra, ra + 2, rb, rb + 2)}
            assert len(vals) == 1 and None not in vals, ("operands incomplete or mixed", ins, vals)
            (step_, ch_, _), = vals
            acc_seq[k].append((step_, ch_))
            set_last_use[ba] = mfmas
            mfmas += 1
            if mfmas % 16 == 0:
                halves_done += 1
                if halves_done % 2 == 0:
                    cur_step += 1
        elif m := re.match(r"s_add_u32 m0, %(\d+), (\d+)$", ins):
            assert int(m[1]) == SBASE
            m0 = int(m[2])
        elif m := re.match(r"global_load_lds_dwordx4 %(\d+), off$", ins):
            p = int(m[1])
            j = ptr_step[p]
            st, rel = divmod(m0, STAGE)
            t = p - PTR
            assert j < nsteps and st == stage_of(j), ("load of the wrong step or stage", ins, j, st)
            assert rel == 4096 * t, ("load to another pointer's slots", ins)
            assert last_read[st] < last_wait_after_read[st] < last_barrier, ("reload before the reads ended", ins)
            d = stage_data[st]
            if d[0] != j:
                assert d[1] == 0 and d[0] == j - 3
                stage_data[st] = d = [j, 0, None]
            d[1] += 1
            loaded_slots.setdefault(j, []).append(t)
            vmq.append((st, j))
            m0 = None
        elif m := re.match(r"v_lshl_add_u64 %(\d+), %(\d+), 0, %(\d+)$", ins):
            p = int(m[1])
            assert int(m[2]) == p and int(m[3]) == stride_of(p - PTR), ("wrong stride", ins)
            assert loaded_slots.get(ptr_step[p], []).count(p - PTR) == 1, ("advance before the load", ins)
            ptr_step[p] += 1
        elif ins.startswith("s_nop") or ins.startswith("s_mov_b32"):
            pass
        else:
            raise AssertionError(f"unknown instruction {ins}")
        pc = nxt
    assert not pending and cur_step == nsteps, (cur_step, nsteps)
    assert all(v == nsteps for v in ptr_step.values()), ptr_step
    for j in range(3, nsteps):
        assert sorted(loaded_slots[j]) == list(range(LOADS)), (j, loaded_slots[j])
    want = [(j, c) for j in range(nsteps) for c in (0, 1)]
    for k in range(16):
        assert acc_seq[k] == want, ("accumulation order", k)
    return phase, iters


def header_text():
    out = generate()
    outs = [f'"+a"(acc[{k}])' for k in range(16)] + [f'"+v"(P[{t}])' for t in range(LOADS)]
    outs += ['"+s"(iters)', '"=&s"(m0save)']
    ins = [f'"v"(vA[{s}])' for s in range(3)] + [f'"v"(vB[{s}])' for s in range(3)]
    ins += ['"s"(sbase)', '"s"(phase)', '"s"(stride_a)', '"s"(stride_4)', '"s"(stride_b)']
    clob = ['"memory"', '"scc"'] + [f'"v{r}"' for r in range(FB, FB + 96)]
    body = " \\\n    ".join('"' + x + '\\n\\t"' for x in out)
    return "\n".join([
        "// Generated by gemm_wgrad_gen.py (do not edit): the K loop of gemm_wgrad_fast_kernel.",
        "#pragma once", "",
        f"// {len(out)} instructions; stage {STAGE} bytes, {LOADS} loads per wave and stage",
        f"#define FX_WGRAD_STAGE_BYTES {STAGE}",
        f"#define FX_WGRAD_ROW_BYTES {ROW}",
        f"#define FX_WGRAD_LOADS {LOADS}",
        f"#define FX_WGRAD_KLOOP \\\n    {body}",
        "#define FX_WGRAD_KLOOP_OUTS \\\n    " + ", \\\n    ".join(outs),
        "#define FX_WGRAD_KLOOP_INS \\\n    " + ", \\\n    ".join(ins),
        "#define FX_WGRAD_KLOOP_CLOBBERS \\\n    " + ", \\\n    ".join(clob), ""])


def main(argv):
    for n in (3, 4, 5, 6, 7, 8, 11, 72, 73, 74, 512):
        check(n)
    text = header_text()
    if "--check" in argv:
        with open(OUT) as f:
            assert f.read() == text, "gemm_wgrad_kloop.h differs from the generator's output"
        print("gemm_wgrad_kloop.h matches the generator; schedule checks passed")
        return
    with open(OUT, "w") as f:
        f.write(text)
    print(f"wrote {OUT}; schedule checks passed")


if __name__ == "__main__":
    main(sys.argv[1:])
