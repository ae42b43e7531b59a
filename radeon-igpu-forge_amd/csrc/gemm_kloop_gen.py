"""Generate gemm_kloop.h: the hand-scheduled K loop of gemm_fast_kernel (linear.hip).

    python radeon-igpu-forge_amd/csrc/gemm_kloop_gen.py          # rewrite gemm_kloop.h
    python radeon-igpu-forge_amd/csrc/gemm_kloop_gen.py --check  # verify only (used by the tests)

The loop is one inline-asm statement so that a wave's fp32 accumulators stay in AGPRs for its
whole length (asm statements in a C++ loop make the compiler carry them in VGPRs between
statements: 760 spilled registers).  A workgroup of 4 waves computes a 256 x (64 NJ) tile of
C = X W^T, each wave 128 x (32 NJ) as 4 x NJ blocks of `v_mfma_f32_32x32x16_bf16` (NJ = 4:
256 x 256 tiles, 256 AGPRs; NJ = 3: 256 x 192 tiles, 192 AGPRs).  K advances in steps of 32
held in 3 LDS stages: X rows then W rows, 80 bytes a row (32 bf16 and 16 bytes of padding,
so the 32 rows one read instruction touches fall in distinct banks).

* A K step is two halves of 4 NJ MFMAs, one per 16-deep chunk.  The 4 + NJ operand reads of
  the next chunk (`ds_read_b128`: 4 X blocks, then NJ W blocks) follow the first MFMAs of a
  half, so they land while the rest run.  Operands rotate through 3 register sets: a set is
  refilled one half after the MFMAs that read it.
* Between the halves: `s_waitcnt vmcnt` for the loads of the next stage (counts below),
  `lgkmcnt(0)`, `s_barrier`.  Every wave has then finished reading this step's stage, so the
  loads of step j + 3 into it (`global_load_lds_dwordx4`, L per wave) go out during the
  last 8 MFMAs of the second half; each load pointer then advances by 64 bytes.
* Loads run two steps ahead.  At the barrier of step j, the loads of step j + 1 must be done,
  and only the L loads of step j + 2 were issued after them: `vmcnt(L)`, or `vmcnt(0)` in
  the last two steps, which issue no loads.

Per wave and stage: 5 loads of X (20 wave-instructions of 64 16-byte slots cover the 256
rows x 5 slots) and 5 (NJ = 4) or 4 (NJ = 3: 15 instructions cover 192 rows; the 16th
fills a 1 KiB pad after the W rows that is never read) loads of W, so L = 10 or 9.

Operand numbering of the asm statement (FX_GEMM_KLOOP_OUTS_NJ<n> and _INS_NJ<n> list them in this order):
accumulators acc[4 j + i] ("+a"), operand sets F[b][x], b = 0..2, x = X0..3 then W0..NJ-1
("=&v"), the 5 X and 5 or 4 W load pointers ("+v", 64-bit), the number of 3-step loop
iterations ("+s"), the saved M0 ("=&s"); inputs: the 3 stages' X read addresses and W read
addresses ("v"), the wave's LDS load base ("s").
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gemm_kloop.h")
ROW_BYTES, BLOCK_BYTES, X_BYTES = 80, 32 * 80, 256 * 80


class Layout:
    """Operand numbers and LDS offsets for NJ 32-column blocks per wave."""

    def __init__(self, nj):
        assert nj in (3, 4)
        self.nj = nj
        self.set_size = 4 + nj
        self.n_acc = 4 * nj
        self.pw = 5 if nj == 4 else 4                     # W loads per wave and stage
        self.loads = 5 + self.pw                          # L
        self.w_bytes = 64 * nj * ROW_BYTES + (1024 if nj == 3 else 0)
        self.stage_bytes = X_BYTES + self.w_bytes
        f0 = self.n_acc
        p0 = f0 + 3 * self.set_size
        self.iters = p0 + 5 + self.pw
        self.m0s = self.iters + 1
        self.va0 = self.m0s + 1
        self.vb0 = self.va0 + 3
        self.sbase = self.vb0 + 3
        self.f0, self.p0 = f0, p0

    def F(self, b, x):
        return self.f0 + self.set_size * b + x

    def PA(self, t):
        return self.p0 + t

    def PB(self, t):
        return self.p0 + 5 + t

    def VA(self, s):
        return self.va0 + s

    def VB(self, s):
        return self.vb0 + s


def generate(nj):
    """(instructions, events): the asm lines and, per line, a tuple describing it for check()."""
    L = Layout(nj)
    out, ev = [], []
    n_mfma = L.n_acc
    dma_from = n_mfma - 8                                 # loads go out after MFMAs dma_from..

    def e(s, what=None):
        out.append(s)
        ev.append(what)

    def read(b, x, stage, chunk):
        base = L.VA(stage) if x < 4 else L.VB(stage)
        e(f"ds_read_b128 %{L.F(b, x)}, %{base} offset:{32 * chunk + (x % 4) * BLOCK_BYTES}", ("read", stage, b))

    def half(cur, nxt, stage, chunk, extra=None):
        e("s_waitcnt lgkmcnt(0)", ("lgkm0",))
        for k in range(n_mfma):
            j, i = k // 4, k % 4
            e(f"v_mfma_f32_32x32x16_bf16 %{k}, %{L.F(cur, 4 + j)}, %{L.F(cur, i)}, %{k}", ("mfma", cur))
            if nxt is not None and k < L.set_size:
                read(nxt, k, stage, chunk)
            if extra is not None and k >= dma_from:
                for x, w in extra[k - dma_from]:
                    e(x, w)

    def dma_groups(stage):
        ins = []   # X and W loads alternating: (pointer, LDS offset)
        for t in range(5):
            ins.append((L.PA(t), stage * L.stage_bytes + t * 4096))
            if t < L.pw:
                ins.append((L.PB(t), stage * L.stage_bytes + X_BYTES + t * 4096))
        slot = [0, 0, 1, 1, 2, 3, 4, 5, 6, 7][:L.loads]   # MFMA slot after which each goes out
        groups = [[] for _ in range(8)]
        for n, (p, m0) in enumerate(ins):
            groups[slot[n]].extend([(f"s_add_u32 m0, %{L.sbase}, {m0}", None), ("s_nop 0", None),
                                    (f"global_load_lds_dwordx4 %{p}, off", ("load", stage, p, m0)),
                                    ("s_nop 0", None)])
        for p, _ in ins:
            groups[7].append((f"v_lshl_add_u64 %{p}, %{p}, 0, 64", ("advance", p)))
        return groups

    def step(u, vm, do_load, next_reads):
        c0, c1, c2 = (2 * u) % 3, (2 * u + 1) % 3, (2 * u + 2) % 3
        half(c0, c1, u, 1)
        e(f"s_waitcnt vmcnt({vm})", ("vm", vm))
        e("s_waitcnt lgkmcnt(0)", ("lgkm0",))
        e("s_barrier", ("barrier",))
        extra = dma_groups(u) if do_load else None
        half(c1, c2 if next_reads else None, (u + 1) % 3, 0, extra)

    e(f"s_mov_b32 %{L.m0s}, m0")
    e(f"s_waitcnt vmcnt({2 * L.loads})", ("vm", 2 * L.loads))
    e("s_barrier", ("barrier",))
    for x in range(L.set_size):
        read(0, x, 0, 0)
    e(f"s_cmp_eq_u32 %{L.iters}, 0")
    e("s_cbranch_scc1 .Ltail%=", ("to_tail",))
    e(".Lloop%=:", ("loop",))
    for u in range(3):
        step(u, L.loads, True, True)
    e(f"s_sub_u32 %{L.iters}, %{L.iters}, 1")
    e(f"s_cmp_lg_u32 %{L.iters}, 0")
    e("s_cbranch_scc1 .Lloop%=", ("back",))
    e(".Ltail%=:", ("tail",))
    step(0, L.loads, False, True)
    step(1, 0, False, True)
    step(2, 0, False, False)
    for _ in range(8):  # the last MFMAs' results before the compiler reads the AGPRs
        e("s_nop 7")
    e(f"s_mov_b32 m0, %{L.m0s}")
    return out, ev


def check(nj, K):
    """Simulate one wave's instruction stream for K (K % 96 == 0) and verify: the pointers
    load K steps 3 .. nk - 1 in order, each into its step's stage, at the LDS offsets that
    make up the stage's X and W rows (every wave-instruction slot of the stage once); every
    read of a stage comes after a vmcnt wait that completed that step's loads; a stage is
    reloaded only after a barrier that follows an lgkmcnt(0) after this wave's last read of
    it; MFMAs use only operand sets whose reads completed, and a set is refilled only
    several MFMAs after its last use."""
    L = Layout(nj)
    out, ev = generate(nj)
    assert K % 96 == 0 and K >= 96
    nk = K // 32
    iters = (nk - 3) // 3
    i_loop = ev.index(("loop",))
    i_back = ev.index(("back",))
    i_tail = ev.index(("tail",))
    seq = list(range(0, i_loop)) + list(range(i_loop, i_back + 1)) * iters + list(range(i_tail, len(out)))
    # the C++ prologue issued the loads of steps 0, 1, 2 before the asm statement
    vmq = [k // L.loads for k in range(3 * L.loads)]    # outstanding loads (their K step), oldest first
    pointers = [L.PA(t) for t in range(5)] + [L.PB(t) for t in range(L.pw)]
    kstep = {p: 3 for p in pointers}
    offsets = {}                                        # K step -> LDS offsets loaded (relative to stage)
    cur_step, n_mfma = 0, 0
    pending = []
    last_read = {0: -1, 1: -1, 2: -1}
    last_wait_after_read = {0: -1, 1: -1, 2: -1}
    last_barrier = -1
    ready = {0: False, 1: False, 2: False}
    last_use = {0: -100, 1: -100, 2: -100}
    for pos, n in enumerate(seq):
        w = ev[n]
        if w is None:
            continue
        kind = w[0]
        if kind == "vm":
            del vmq[:max(0, len(vmq) - w[1])]
        elif kind == "lgkm0":
            for st, b in pending:
                ready[b] = True
                last_wait_after_read[st] = pos
            pending = []
        elif kind == "barrier":
            last_barrier = pos
        elif kind == "read":
            st, b = w[1], w[2]
            held = max(s for s in range(min(cur_step + 2, nk)) if s % 3 == st)
            issued = held < 3 or len(offsets.get(held, ())) == L.loads
            assert issued and held not in vmq, ("read of a stage whose loads may be in flight", nj, K, pos)
            assert n_mfma - last_use[b] >= 4, ("operand set refilled right after its last use", nj, pos)
            ready[b] = False
            pending.append((st, b))
            last_read[st] = pos
        elif kind == "mfma":
            assert ready[w[1]], ("MFMA on an operand set whose reads did not complete", nj, K, pos)
            last_use[w[1]] = n_mfma
            n_mfma += 1
            if n_mfma % (2 * L.n_acc) == 0:
                cur_step += 1
        elif kind == "load":
            st, p, m0 = w[1], w[2], w[3]
            s = kstep[p]
            assert s < nk and st == s % 3, ("load of the wrong step", nj, K, p, s, st)
            assert last_read[st] < last_wait_after_read[st] < last_barrier, ("reload before all reads", nj, pos)
            offsets.setdefault(s, []).append(m0 - st * L.stage_bytes)
            vmq.append(s)
        elif kind == "advance":
            kstep[w[1]] += 1
    assert all(v == nk for v in kstep.values()), kstep
    assert cur_step == nk, (cur_step, nk)
    # each step's loads cover one wave's share of the stage: X instructions 0..19 and W
    # instructions 0..(4 pw - 1) (wave 0; the others are offset by 1 KiB each)
    want = sorted([4096 * t for t in range(5)] + [X_BYTES + 4096 * t for t in range(L.pw)])
    for s in range(3, nk):
        assert sorted(offsets[s]) == want, (nj, s, offsets[s])
    assert 20 * 1024 == X_BYTES and 4 * L.pw * 1024 == L.w_bytes
    return iters


def operand_list(nj):
    L = Layout(nj)
    outs = [f'"+a"(acc[{k}])' for k in range(L.n_acc)]
    outs += [f'"=&v"(F[{b}][{x}])' for b in range(3) for x in range(L.set_size)]
    outs += [f'"+v"(qa[{t}])' for t in range(5)] + [f'"+v"(qb[{t}])' for t in range(L.pw)]
    outs += ['"+s"(iters)', '"=&s"(m0save)']
    ins = [f'"v"(vA[{s}])' for s in range(3)] + [f'"v"(vB[{s}])' for s in range(3)] + ['"s"(sbase)']
    return outs, ins


def header_text():
    parts = ["// Generated by gemm_kloop_gen.py (do not edit): the K loop of gemm_fast_kernel.", "#pragma once", ""]
    for nj in (4, 3):
        out, _ = generate(nj)
        L = Layout(nj)
        outs, ins = operand_list(nj)
        parts.append(f"// NJ = {nj}: {len(out)} instructions; stage {L.stage_bytes} bytes, {L.loads} loads per wave")
        parts.append(f"#define FX_GEMM_STAGE_BYTES_NJ{nj} {L.stage_bytes}")
        parts.append(f"#define FX_GEMM_LOADS_NJ{nj} {L.loads}")
        body = " \\\n    ".join('"' + x + '\\n\\t"' for x in out)
        parts.append(f"#define FX_GEMM_KLOOP_NJ{nj} \\\n    {body}")
        parts.append(f"#define FX_GEMM_KLOOP_OUTS_NJ{nj} \\\n    " + ", \\\n    ".join(outs))
        parts.append(f"#define FX_GEMM_KLOOP_INS_NJ{nj} \\\n    " + ", \\\n    ".join(ins))
        parts.append("")
    return "\n".join(parts)


def main(argv):
    for nj in (4, 3):
        for K in (96, 192, 768, 3072, 9600):
            check(nj, K)
    text = header_text()
    if "--check" in argv:
        with open(OUT) as f:
            assert f.read() == text, "gemm_kloop.h differs from the generator's output"
        print("gemm_kloop.h matches the generator; schedule checks passed")
        return
    with open(OUT, "w") as f:
        f.write(text)
    print(f"wrote {OUT}; schedule checks passed")


if __name__ == "__main__":
    main(sys.argv[1:])
