"""The generated K loops of the whole-tile GEMM kernels (csrc/gemm_asm_gen.py -> gemm_asm.h), on
the CPU: the committed header is the generator's output; the checker, which interprets each
loop's instruction text (branches included) and tracks the data every read, wait, load and MFMA
handles, passes every kind of loop at step counts that enter the loop body at each of its
steps; and it fails loops with a planted mistake of each kind it is meant to catch (a wait too
weak, a barrier or LDS wait missing, a pointer advanced before its load or by another's
stride, a read or load at the wrong place, a wrong entry into the loop, MFMA inputs swapped)."""
import importlib.util
import os
import re

import pytest

from conftest import ROOT

GEN = os.path.join(ROOT, "radeon-igpu-forge_amd", "csrc", "gemm_asm_gen.py")


@pytest.fixture(scope="module")
def gen():
    spec = importlib.util.spec_from_file_location("gemm_asm_gen", GEN)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_header_is_generated(gen):
    with open(gen.OUT) as f:
        assert f.read() == gen.header_text()


@pytest.mark.parametrize("kind", range(6))
@pytest.mark.parametrize("nsteps", [4, 5, 6, 7, 8, 9, 24, 72, 73, 74, 75, 96])
def test_schedule_checks(gen, kind, nsteps):
    kd = gen.KINDS[kind]
    n = gen.loop_steps(kd, nsteps)  # loops of two-step buffers take a leading zero step for odd counts
    assert n % kd.ksteps == 0 and n - nsteps in (0, 1)
    phase, iters = gen.check(kd, n)
    assert (n - 4 + phase) % 4 == 0 and iters == (n - 4 + phase) // 4


def test_layouts(gen):
    # loads per wave and buffer bytes: 4 L wave-instructions of 1 KiB cover both tiles and the
    # pad; loops with a row operand keep two buffers of two K steps (144-byte rows), the weight
    # gradient's four of one step
    for kd in gen.KINDS:
        assert kd.stage == 4 * kd.loads * 1024
        assert kd.region[0][1] + kd.region[1][1] <= kd.stage
        assert kd.bufs * kd.stage <= 160 * 1024 and kd.bufs * kd.ksteps == gen.STAGES
    assert [kd.loads for kd in gen.KINDS] == [18, 16, 18, 16, 9, 8]
    assert [kd.pair for kd in gen.KINDS] == [True] * 4 + [False] * 2


def _first(prog, pred, k=0):
    return [i for i, l in enumerate(prog) if pred(l)][k]


def _vm_weaker(p):
    i = _first(p, lambda l: re.fullmatch(r"s_waitcnt vmcnt\(\d+\)", l) is not None, 1)
    n = int(re.search(r"\d+", p[i])[0])
    p[i] = f"s_waitcnt vmcnt({n + 1})"
    return p


def _drop(line, k):
    def f(p):
        del p[_first(p, lambda l: l == line, k)]
        return p
    return f


def _advance_first(p):
    a = _first(p, lambda l: l.startswith("v_lshl_add_u64"))
    reg = re.search(r"%(\d+)", p[a])[1]
    p.insert(_first(p, lambda x: x == f"global_load_lds_dwordx4 %{reg}, off"), p.pop(a))
    return p


def _other_stride(p):
    i = _first(p, lambda l: l.startswith("v_lshl_add_u64"))
    p[i] = re.sub(r"%(\d+)$", lambda m: f"%{int(m[1]) + 1}", p[i])
    return p


def _read_offset(p):
    i = _first(p, lambda l: l.startswith("ds_read"), 5)
    p[i] = re.sub(r"offset:(\d+)", lambda m: f"offset:{int(m[1]) + 64}", p[i])
    return p


def _load_slot(p):
    i = _first(p, lambda l: l.startswith("s_add_u32 m0"), 4)
    p[i] = re.sub(r", (\d+)$", lambda m: f", {int(m[1]) + 4096}", p[i])
    return p


def _entry(p):
    # the first entry into the loop body past step 0 jumps one step too far
    i = _first(p, lambda l: re.fullmatch(r"s_branch \.Lu[12]%=", l) is not None)
    p[i] = re.sub(r"Lu(\d)", lambda m: f"Lu{int(m[1]) + 1}", p[i])
    return p


def _swap(p):
    i = _first(p, lambda l: l.startswith("v_mfma"), 1)
    m = re.match(r"(v_mfma\S+ %\d+, )(v\[\d+:\d+\]), (v\[\d+:\d+\])(.*)", p[i])
    p[i] = m[1] + m[3] + ", " + m[2] + m[4]
    return p


def _tail_vm(p):
    p[_first(p, lambda l: l == "s_waitcnt vmcnt(0)")] = "s_waitcnt vmcnt(1)"
    return p


@pytest.mark.parametrize("kind", range(6))
@pytest.mark.parametrize("mistake", [_vm_weaker, _drop("s_barrier", 2), _drop("s_waitcnt lgkmcnt(0)", 3),
                                     _advance_first, _other_stride, _read_offset, _load_slot, _entry, _swap,
                                     _tail_vm])
def test_checker_catches_planted_mistakes(gen, monkeypatch, kind, mistake):
    good = gen.generate
    monkeypatch.setattr(gen, "generate", lambda kd: mistake(list(good(kd))))
    caught = 0
    for n in (4, 5, 6, 7, 72, 73, 74, 75):
        try:
            gen.check(gen.KINDS[kind], gen.loop_steps(gen.KINDS[kind], n))
        except (AssertionError, KeyError, TypeError):
            caught += 1
    assert caught > 0
