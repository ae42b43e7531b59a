"""The C-ABI library: it loads, exports every function of include/fx_abi.h, its
struct layouts match the ctypes mirrors, and argument checks reject bad input
before anything reaches the GPU (CPU only)."""
import ctypes
import os
import re
import subprocess
import sys
import tempfile

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "fx_abi.h")


@pytest.fixture(scope="module")
def abi():
    from fxgpu import abi as _abi
    srcs = os.path.join(ROOT, "radeon-igpu-forge_amd", "csrc")
    newest = max(os.path.getmtime(os.path.join(srcs, f)) for f in os.listdir(srcs)
                 if f.endswith((".hip", ".h")))
    newest = max(newest, os.path.getmtime(HEADER))
    if not os.path.exists(_abi.LIB_PATH) or os.path.getmtime(_abi.LIB_PATH) < newest:
        subprocess.run(["python", os.path.join(srcs, "build.py")], check=True)
    return _abi


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|int64_t|char\s*\*|void)\s*\*?\s*(fx_\w+)\s*\(",
                                 text, re.M)))


def test_header_and_ctypes_agree(abi):
    assert header_functions() == sorted(abi.SIGNATURES)


def test_library_exports_every_symbol(abi):
    lib = abi.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (fx_\w+)", out))
    assert set(header_functions()) <= exported
    assert lib.fx_abi_version() == abi.FX_ABI_VERSION


STRUCTS = ["fxCEArgs", "fxTensorList", "fxAdamWState", "fxAttnArgs", "fxAttnDecodeArgs", "fxLinearArgs"]


def test_struct_layout_matches_c(abi, tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for s in STRUCTS:
        cls = getattr(abi, s)
        lines.append(f'printf("{s} %zu\\n", sizeof({s}));')
        for f, _t in cls._fields_:
            lines.append(f'printf("{s}.{f} %zu\\n", offsetof({s}, {f}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.split("\n") if l)
    for s in STRUCTS:
        cls = getattr(abi, s)
        assert int(got[s]) == ctypes.sizeof(cls), s
        for f, _t in cls._fields_:
            assert int(got[f"{s}.{f}"]) == getattr(cls, f).offset, f"{s}.{f}"


def test_argument_checks_reject_before_launch(abi):
    lib = abi.lib()
    fake = ctypes.c_void_p(4096)     # never dereferenced: the checks fail first
    rc = lib.fx_rms_norm_fwd(fake, fake, fake, fake, 4, 7, 1e-6, None)
    assert rc == abi.FX_EINVAL and b"D=7" in lib.fx_last_error()
    assert lib.fx_ce_fwd_grad(None, None) == abi.FX_EINVAL
    a = abi.fxAttnArgs()
    a.D, a.B, a.T, a.H = 96, 1, 1, 1
    assert lib.fx_attn_fwd(ctypes.byref(a), None) == abi.FX_EINVAL
    assert b"head_dim 96" in lib.fx_last_error()
    # masked scores are -inf before scaling: zero, negative or inf scales are rejected
    for bad_scale in (0.0, -0.125, float("inf")):
        a = abi.fxAttnArgs()
        a.D, a.B, a.T, a.H, a.scale = 64, 1, 1, 1, bad_scale
        a.q = a.k = a.v = 0x1000  # never dereferenced: the check fails first
        assert lib.fx_attn_fwd(ctypes.byref(a), None) == abi.FX_EINVAL
        assert b"scale" in lib.fx_last_error()
    tl = abi.fxTensorList()
    tl.count = 65
    st = abi.fxAdamWState()
    assert lib.fx_adamw_step(ctypes.byref(st), ctypes.byref(tl), 1, None) == abi.FX_EINVAL
    # one fp32 dw partial row per backward block: a whole number of rows, far fewer
    # than the batch, and none for an empty batch
    ws = lib.fx_rms_norm_bwd_workspace(65536, 768)
    assert ws > 0 and ws % (768 * 4) == 0 and ws // (768 * 4) <= 65536 // 16
    assert lib.fx_rms_norm_bwd_workspace(3, 768) == 3 * 768 * 4
    assert lib.fx_rms_norm_bwd_workspace(0, 768) == 0


# One invalid call per compute entry point: each returns FX_EINVAL with a message naming the
# entry point before it touches the device (the pointers are fake and never dereferenced).
_F = 4096          # a 16-byte-aligned fake device address
_M = 4098          # a misaligned one


def _bad_calls(abi):
    P = ctypes.c_void_p
    f, m = P(_F), P(_M)
    st = abi.fxAdamWState()          # every state pointer null
    tl = abi.fxTensorList()
    dec = abi.fxAttnDecodeArgs()
    dec.D, dec.B, dec.H, dec.Tmax = 96, 1, 1, 1
    bwd = abi.fxAttnArgs()
    bwd.D, bwd.B, bwd.T, bwd.H, bwd.scale = 64, 1, 64, 1, 0.125
    bwd.q = bwd.k = bwd.v = _F       # o, dout, lse, delta, dq, dk, dv null
    return [
        ("fx_fill_f32", (f, -1, 0.0, None)),
        ("fx_rms_norm_fwd_add", (f, f, f, m, f, f, 4, 8, 1e-6, None)),
        ("fx_rms_norm_bwd", (f, f, f, f, f, None, None, f, 4, 768, None)),
        ("fx_rms_norm_bwd_add", (f, f, None, f, f, f, f, None, f, 4, 768, None)),
        ("fx_ce_inv_nvalid", (f, 4, -100, None, 1.0, None, f, None)),
        ("fx_ce_loss_finalize", (f, 4, None, f, None)),
        ("fx_ce_scale_grad", (f, 8, f, f, 2, None)),
        ("fx_ce_lin_grad_scale", (f, -1, f, 8, f, None, 1.0, f, f, None)),
        ("fx_ce_lin_grad_scale_bf16w", (f, 8, m, 8, f, None, 1.0, f, f, None)),
        ("fx_ce_lin_grad_scale_inplace", (m, 8, f, 8, f, None, 1.0, None)),
        ("fx_adamw_step_noalloc", (ctypes.byref(st), ctypes.byref(tl), 1, None)),
        ("fx_attn_bwd", (ctypes.byref(bwd), None)),
        ("fx_attn_decode", (ctypes.byref(dec), None)),
        ("fx_linear_fwd", (f, 8, None, 0, 0, f, None, f, None, None, 4, 8, 7, 0, None)),
        ("fx_linear_fwd_ex", (None, None)),
        ("fx_gelu_bwd", (f, m, f, 8, None)),
        ("fx_gelu_bwd_gate", (f, m, f, 8, None)),
        ("fx_linear_dgrad", (f, 768, f, 768, None, f, 768, 100, 768, 768, None)),
        ("fx_linear_dgrad_gate", (f, 768, f, 768, None, f, 768, 256, 768, 768, None)),   # no G
        ("fx_linear_wgrad", (f, 12, f, 8, f, 8, None, 12, 8, 16, None)),
        ("fx_lce_fwd", (f, 768, f, f, -100, f, f, f, 256, 1000, 768, None)),
        ("fx_lce_grad", (f, 768, None, f, -100, f, f, f, 768, 256, 768, 768, None)),
    ]


def test_every_entry_point_rejects_bad_arguments_before_launch(abi):
    lib = abi.lib()
    calls = _bad_calls(abi)
    compute = {n for n in abi.SIGNATURES if not n.endswith("_workspace")} - {"fx_abi_version", "fx_last_error"}
    covered = {n for n, _ in calls} | {"fx_rms_norm_fwd", "fx_ce_fwd_grad", "fx_attn_fwd", "fx_adamw_step",
                                       "fx_embedding_bwd"}   # covered by the tests around this one
    assert compute <= covered, sorted(compute - covered)
    for name, args in calls:
        rc = getattr(lib, name)(*args)
        assert rc == abi.FX_EINVAL, (name, rc)
        assert lib.fx_last_error().decode().startswith(name), (name, lib.fx_last_error())


def test_linear_fwd_activation_codes(abi):
    # 0 identity, 1 GELU, 2 GELU with its derivative in H; anything else is refused first
    lib = abi.lib()
    f = ctypes.c_void_p(_F)
    for act in (-1, 3):
        assert lib.fx_linear_fwd(f, 8, None, 0, 0, f, None, f, f, None, 4, 8, 8, act, None) == abi.FX_EINVAL
        assert "act=" in lib.fx_last_error().decode()


def test_embedding_bwd_checks_and_workspace(abi):
    lib = abi.lib()
    fake = ctypes.c_void_p(4096)     # never dereferenced: the checks fail first
    # D must be a multiple of 8, V positive, grad 16-byte aligned, dy rows aligned
    assert lib.fx_embedding_bwd(fake, 4, fake, 12, fake, 10, 12, fake, None) == abi.FX_EINVAL
    assert b"D=12" in lib.fx_last_error()
    assert lib.fx_embedding_bwd(fake, 4, fake, 8, fake, 0, 8, fake, None) == abi.FX_EINVAL
    assert lib.fx_embedding_bwd(fake, 4, fake, 8, ctypes.c_void_p(4098), 10, 8, fake, None) == abi.FX_EINVAL
    assert lib.fx_embedding_bwd(fake, 4, fake, 12, fake, 10, 8, fake, None) == abi.FX_EINVAL
    assert lib.fx_embedding_bwd(fake, -1, fake, 8, fake, 10, 8, fake, None) == abi.FX_EINVAL
    # workspace: per-chunk counts (1024 positions a chunk), offsets, one sum per 256 ids,
    # ranks, the order and the slots' ids, then a head and a tail fp32 row per 32-slot
    # segment, each rounded up to 16 bytes
    ws = lib.fx_embedding_bwd_workspace
    assert ws(0, 100, 8) == 0 and ws(5, 0, 8) == 0 and ws(5, 100, 0) == 0
    assert ws(1024, 100, 8) == 400 + 416 + 16 + 3 * 4096 + 2 * 32 * 8 * 4
    assert ws(1025, 100, 8) == 800 + 416 + 16 + 3 * 4112 + 2 * 33 * 8 * 4
    assert ws(16384, 50304, 768) == (16 * 50304 * 4 + (50305 * 4 + 12) + 800 + 3 * 16384 * 4
                                     + 2 * 512 * 768 * 4)


def test_rms_norm_rejects_misaligned_vectors(abi):
    # x / w / y / dy / dx are read and written as 16-byte vectors: an address that is
    # only 2-byte aligned is rejected before any launch (never dereferenced)
    lib = abi.lib()
    ok, odd = ctypes.c_void_p(4096), ctypes.c_void_p(4096 + 2)
    for args in ((odd, ok, ok), (ok, odd, ok), (ok, ok, odd)):
        x, w, y = args
        assert lib.fx_rms_norm_fwd(x, w, y, ok, 4, 64, 1e-6, None) == abi.FX_EINVAL
        assert b"16-byte aligned" in lib.fx_last_error()
    for i in range(4):   # x, dy, w, dx
        p = [ok, ok, ok, ok]
        p[i] = odd
        x, dy, w, dx = p
        assert lib.fx_rms_norm_bwd(x, dy, w, ok, dx, ok, ok, ok, 4, 64, None) == abi.FX_EINVAL
        assert b"16-byte aligned" in lib.fx_last_error()
        assert lib.fx_rms_norm_bwd_add(x, dy, ok, w, ok, dx, ok, ok, ok, 4, 64, None) == abi.FX_EINVAL


def test_lce_workspace_and_checks(abi):
    # the fused linear-CE kernels take V % 256 or % 192 == 0, K % 32 == 0, K >= 128; the
    # workspace is one (max, sum) fp32 pair per row and column tile plus one fp32 per row
    lib = abi.lib()
    assert lib.fx_lce_workspace(16384, 50304, 768) == 262 * 16384 * 8 + 16384 * 4
    assert lib.fx_lce_workspace(300, 1024, 128) == ((4 * 300 * 8 + 255) // 256 * 256
                                                    + (300 * 4 + 255) // 256 * 256)
    for M, V, K in ((100, 1000, 128), (100, 768, 96), (100, 768, 100), (0, 768, 128)):
        assert lib.fx_lce_workspace(M, V, K) == 0
    fake = ctypes.c_void_p(4096)     # never dereferenced: the checks fail first
    odd = ctypes.c_void_p(4096 + 2)
    assert lib.fx_lce_fwd(fake, 128, fake, fake, -100, fake, fake, fake, 8, 1000, 128, None) == abi.FX_EINVAL
    assert b"V % 256" in lib.fx_last_error()
    assert lib.fx_lce_fwd(odd, 128, fake, fake, -100, fake, fake, fake, 8, 768, 128, None) == abi.FX_EINVAL
    assert b"16-byte aligned" in lib.fx_last_error()
    assert lib.fx_lce_fwd(None, 128, fake, fake, -100, fake, fake, fake, 8, 768, 128, None) == abi.FX_EINVAL
    assert lib.fx_lce_grad(fake, 128, fake, fake, -100, fake, fake, fake, 700, 8, 768, 128, None) == abi.FX_EINVAL
    assert b"row stride" in lib.fx_last_error()
    assert lib.fx_lce_grad(fake, 120, fake, fake, -100, fake, fake, fake, 768, 8, 768, 128, None) == abi.FX_EINVAL
    # an empty batch launches nothing
    assert lib.fx_lce_fwd(fake, 128, fake, fake, -100, None, None, None, 0, 768, 128, None) == 0


def test_wgrad_workspace_follows_the_plan(abi):
    # off a GPU the library plans for 256 CUs.  Fewer whole 256 x 192 tiles than CUs: K split
    # into CUs / tiles slices, one fp32 partial each (qkv: 36 tiles, 7 slices); whole rounds:
    # one slice, no workspace; a partly filled last round: the panels past the full rounds in
    # CUs / (their tiles) slices (the tied head: 788 tiles, the last 20 in 12 slices over its
    # last 1152 rows; 264 tiles of 256 x 256 at N = 1024: the last 8 in 4 slices, capped at a
    # quarter of the 16 64-token steps, over 392 rows); too few tail slices: one product
    lib = abi.lib()
    ws = lib.fx_linear_wgrad_workspace
    assert ws(2304, 768, 16384) == 7 * 2304 * 768 * 4
    assert ws(16384, 3072, 16384) == 0
    assert ws(50304, 768, 16384) == 12 * (50304 - 49152) * 768 * 4
    assert ws(16776, 768, 1024) == 4 * (16776 - 16384) * 768 * 4
    assert ws(16740, 1024, 1024) == 4 * (16740 - 16384) * 1024 * 4
    assert ws(256 * 114, 768, 16384) == 0      # 456 tiles: the 200 past one round get 1 slice each


def test_adamw_workspace_counts_chunks(abi):
    tl = abi.fxTensorList()
    tl.count = 3
    for i, n in enumerate((8192, 8193, 1)):
        tl.n[i] = n
    # 1 + 2 + 1 chunks of 8192 elements, plus the 4-float header
    assert abi.lib().fx_adamw_workspace(ctypes.byref(tl), 1) == (4 + 4) * 4
    # no lists (null pointer) and empty or negative sizes add no chunks
    assert abi.lib().fx_adamw_workspace(None, 3) == 4 * 4
    tl.n[1] = 0
    tl.n[2] = -5
    assert abi.lib().fx_adamw_workspace(ctypes.byref(tl), 1) == (4 + 1) * 4


def test_adamw_noalloc_rejects_lists_beyond_its_scratch(abi):
    # more chunks than the library's scratch holds: FX_EINVAL before the device is looked up
    # or anything is launched (the pointers are never dereferenced)
    lib = abi.lib()
    fake = 4096
    tl = abi.fxTensorList()
    tl.count = 1
    tl.g[0] = fake
    tl.n[0] = 300_000 * 8192                        # 300,000 chunks > 262,140
    st = abi.fxAdamWState()
    st.master = st.m = st.v = st.p16 = fake
    st.step = st.found_inf = st.grad_norm = st.scale = st.growth = fake
    assert lib.fx_adamw_step_noalloc(ctypes.byref(st), ctypes.byref(tl), 1, None) == abi.FX_EINVAL
    assert b"scratch" in lib.fx_last_error()
    # the largest list that fits passes this check (and would go on to the device lookup)
    assert (4 + 262140) * 4 == 1 << 20


def test_workspace_queries_survive_edge_shapes():
    # every workspace query over zero, negative, tiny, odd and large sizes, in a child
    # process so that a crash (an integer division by zero in a size plan) fails this test
    code = r"""
import itertools, sys
sys.path.insert(0, sys.argv[1])
from fxgpu import abi
lib = abi.lib()
vals = [-1, 0, 1, 7, 8, 127, 128, 192, 256, 257, 768, 1024, 3072, 16384, 16385, 50304, 65536]
for M, N, K in itertools.product(vals, vals, vals):
    lib.fx_linear_wgrad_workspace(M, N, K)
    lib.fx_lce_workspace(M, N, K)
    lib.fx_embedding_bwd_workspace(M, N, K)
for a, b in itertools.product(vals, vals):
    lib.fx_rms_norm_bwd_workspace(a, b)
for a, b, c, d in itertools.product([-1, 0, 1, 16], [-1, 0, 12], [-1, 0, 1, 512, 4096], [-1, 0, 64, 128]):
    lib.fx_attn_decode_workspace(a, b, c, d)
print("swept")
"""
    r = subprocess.run([sys.executable, "-c", code, os.path.join(ROOT, "radeon-igpu-forge_amd")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "swept" in r.stdout, (r.returncode, r.stderr[-2000:])
