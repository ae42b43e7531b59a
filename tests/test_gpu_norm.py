"""RMSNorm on the GPU (fx_rms_norm_fwd / fx_rms_norm_bwd) against the oracle and fixtures."""
import pytest
import torch
import torch.nn.functional as F

from golden_util import bf16, f32, load
from oracle import norm as onorm
from tolerances import FRAC_OUT, RTOL_NORM, oracle_close, rel_err

pytestmark = pytest.mark.gpu


def _run(x, w, dy, eps=1e-6):
    from fxlm.norm import rms_norm_bwd_raw, rms_norm_fwd_stats
    y, rstd = rms_norm_fwd_stats(x, w, eps)
    dx, dw32, dw = rms_norm_bwd_raw(x, dy, w, rstd)
    torch.cuda.synchronize()
    return y, rstd, dx, dw32, dw


def test_golden(dev):
    d = load("rms_n7_d768")
    y, rstd, dx, dw32, dw = _run(bf16(d["x"], dev), bf16(d["w"], dev), bf16(d["dy"], dev))
    assert oracle_close(y, f32(d["y"]), FRAC_OUT) and oracle_close(dx, f32(d["dx"]), FRAC_OUT)
    assert rel_err(rstd, f32(d["rstd"])) < RTOL_NORM
    assert rel_err(dw32, f32(d["dw"])) < RTOL_NORM
    assert torch.equal(dw.cpu(), dw32.cpu().bfloat16())


# The backward runs D < 512 on the register kernel (one vector per lane), 512 <= D <= 1536
# on its LDS-ring kernel (1-3 vectors per lane, ring depth 3, or 2 for dres rows past
# D = 1135) and wider rows on the block-per-row kernel (one vector per thread up to
# D = 4096, two up to 8192; more rows than its 512 blocks take the double-buffered row sum
# and the next-row prefetch through several rows per block); _LDS_SHAPES cover the LDS
# kernel's (vectors, depth) combinations with ragged and tiny row counts
_LDS_SHAPES = [(1, 512), (7, 520), (2049, 1024), (33, 1128), (300, 1136), (11, 1536)]
_WIDE_SHAPES = [(7, 1544), (64, 2048), (64, 2056), (1100, 2048), (5, 3000), (64, 4096), (9, 4104),
                (1031, 8192)]


@pytest.mark.parametrize("N,D", [(4, 8), (37, 64), (129, 768), (1000, 512), (300, 8192),
                                 (5, 1032), (3, 96)] + _LDS_SHAPES + _WIDE_SHAPES)
def test_against_oracle(dev, N, D):
    # the reference selftest's cases (ml/fxlm/selftest.py:186-204) plus odd row shapes
    torch.manual_seed(N * 1000 + D)
    x = (torch.randn(N, D) * 3).bfloat16()
    w = (torch.randn(D) * 0.5 + 1).bfloat16()
    dy = torch.randn(N, D).bfloat16()
    y, rstd, dx, dw32, _dw = _run(x.to(dev), w.to(dev), dy.to(dev))
    yr, rr = onorm.rms_norm_fwd(x, w, 1e-6)
    dxr, dwr = onorm.rms_norm_bwd(x, dy, w, rr)
    assert oracle_close(y, yr, FRAC_OUT) and oracle_close(dx, dxr, FRAC_OUT)
    assert rel_err(rstd, rr) < RTOL_NORM and rel_err(dw32, dwr) < RTOL_NORM


def test_autograd_path(dev):
    from fxlm.norm import rms_norm
    torch.manual_seed(1)
    x = torch.randn(2, 9, 768, device=dev).bfloat16().requires_grad_()
    w = (torch.randn(768, device=dev) * 0.1 + 1).bfloat16().requires_grad_()
    y = rms_norm(x, w)
    g = torch.randn_like(y)
    y.backward(g)
    xr, wr = x.detach().float().requires_grad_(), w.detach().float().requires_grad_()
    F.rms_norm(xr, (768,), wr, 1e-6).backward(g.float())
    assert y.shape == x.shape and x.grad.dtype == torch.bfloat16 and w.grad.dtype == torch.bfloat16
    assert oracle_close(x.grad, xr.grad, FRAC_OUT) and oracle_close(w.grad, wr.grad, FRAC_OUT)


def test_empty_batch(dev):
    x = torch.empty(0, 64, device=dev, dtype=torch.bfloat16)
    w = torch.ones(64, device=dev, dtype=torch.bfloat16)
    y, rstd, dx, dw32, dw = _run(x, w, x)
    assert y.shape == (0, 64) and float(dw32.abs().max()) == 0.0


def test_cfg4_full_size(dev):
    # cfg4: x (65536, 768) ~ N(0,1), w ~ N(1, 0.1); checked against fp32 torch math
    g = torch.Generator(device=dev).manual_seed(4)
    N, D = 65536, 768
    x = torch.randn(N, D, device=dev, generator=g).bfloat16()
    w = (torch.randn(D, device=dev, generator=g) * 0.1 + 1).bfloat16()
    dy = torch.randn(N, D, device=dev, generator=g).bfloat16()
    y, rstd, dx, dw32, _ = _run(x, w, dy)
    xr, wr = x.float().requires_grad_(), w.float().requires_grad_()
    yr = F.rms_norm(xr, (D,), wr, 1e-6)
    yr.backward(dy.float())
    rr = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-6)
    assert oracle_close(y, yr, FRAC_OUT) and oracle_close(dx, xr.grad, FRAC_OUT)
    assert rel_err(rstd, rr) < RTOL_NORM and rel_err(dw32, wr.grad) < RTOL_NORM


# ---- the residual block's fused gradient sum (fx_rms_norm_bwd_add / pre_norm) ----------

@pytest.mark.parametrize("N,D", [(129, 768), (300, 8192), (64, 2056), (5, 96), (1100, 2048)] + _LDS_SHAPES)
def test_bwd_add_against_oracle(dev, N, D):
    # dx = dres + (the norm's dx) in one pass; dw is the norm's alone, bit for bit the
    # plain backward's
    from fxgpu.abi import call, lib, ptr, stream_of
    torch.manual_seed(N + D)
    x = (torch.randn(N, D) * 3).bfloat16()
    w = (torch.randn(D) * 0.5 + 1).bfloat16()
    dy = torch.randn(N, D).bfloat16()
    dres = torch.randn(N, D).bfloat16()
    xg, wg, dyg, rg = x.to(dev), w.to(dev), dy.to(dev), dres.to(dev)
    _y, rstd, dx0, dw0, _ = _run(xg, wg, dyg)
    dx = torch.empty_like(xg)
    dw32 = torch.empty(D, device=dev)
    work = torch.empty(max(1, lib().fx_rms_norm_bwd_workspace(N, D) // 4), device=dev)
    call("fx_rms_norm_bwd_add", ptr(xg), ptr(dyg), ptr(rg), ptr(wg), ptr(rstd), ptr(dx), ptr(dw32), None,
         ptr(work), N, D, stream_of(xg))
    torch.cuda.synchronize()
    _yr, rr = onorm.rms_norm_fwd(x, w, 1e-6)
    dxr, _dwr = onorm.rms_norm_bwd(x, dy, w, rr)
    assert oracle_close(dx, dxr + dres.double(), FRAC_OUT)
    assert torch.equal(dw32, dw0)
    with pytest.raises(ValueError, match="null dres"):
        call("fx_rms_norm_bwd_add", ptr(xg), ptr(dyg), None, ptr(wg), ptr(rstd), ptr(dx), ptr(dw32), None,
             ptr(work), N, D, stream_of(xg))


def test_pre_norm_autograd(dev):
    # (x, norm(x)) with both outputs used: x.grad = g_x + the norm's backward of g_y, as
    # fp32 torch autograd computes it; with only the norm used it is the plain backward
    from fxlm.norm import pre_norm, rms_norm
    torch.manual_seed(2)
    x0 = torch.randn(2, 9, 768, device=dev).bfloat16()
    w0 = (torch.randn(768, device=dev) * 0.1 + 1).bfloat16()
    gx = torch.randn(2, 9, 768, device=dev).bfloat16()
    gy = torch.randn(2, 9, 768, device=dev).bfloat16()
    x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    xp, y = pre_norm(x, w)
    assert torch.equal(xp, x0) and y.shape == x0.shape
    torch.autograd.backward([xp, y], [gx, gy])
    xr, wr = x0.float().requires_grad_(), w0.float().requires_grad_()
    yr = F.rms_norm(xr, (768,), wr, 1e-6)
    torch.autograd.backward([xr, yr], [gx.float(), gy.float()])
    assert oracle_close(x.grad, xr.grad, FRAC_OUT) and oracle_close(w.grad, wr.grad, FRAC_OUT)
    x2, w2 = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    _, y2 = pre_norm(x2, w2)
    y2.backward(gy)
    x3, w3 = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    rms_norm(x3, w3).backward(gy)
    assert torch.equal(x2.grad, x3.grad) and torch.equal(w2.grad, w3.grad)


@pytest.mark.parametrize("N,D", [(129, 768), (300, 8192), (64, 2056), (5, 96)])
def test_fwd_add_is_add_then_norm(dev, N, D):
    # fx_rms_norm_fwd_add: the sum rounds like torch's bf16 add and y / rstd are the
    # plain forward's on that sum, bit for bit
    from fxlm.norm import add_pre_norm, rms_norm_fwd_stats
    torch.manual_seed(N + D)
    x = torch.randn(N, D, device=dev).bfloat16()
    r = torch.randn(N, D, device=dev).bfloat16()
    w = (1 + 0.1 * torch.randn(D, device=dev)).bfloat16()
    s, y = add_pre_norm(x, r, w)
    s_ref = x + r
    y_ref, _ = rms_norm_fwd_stats(s_ref, w)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref) and torch.equal(y, y_ref)


def test_add_pre_norm_autograd(dev):
    # gradients equal those of the separate add followed by pre_norm, bit for bit
    from fxlm.norm import add_pre_norm, pre_norm
    torch.manual_seed(11)
    N, D = 200, 768
    x0 = torch.randn(N, D, device=dev).bfloat16()
    r0 = torch.randn(N, D, device=dev).bfloat16()
    w0 = (1 + 0.1 * torch.randn(D, device=dev)).bfloat16()
    gs = torch.randn(N, D, device=dev).bfloat16()
    gy = torch.randn(N, D, device=dev).bfloat16()
    got, ref = [], []
    for fused, out in ((True, got), (False, ref)):
        x, r, w = (t.clone().requires_grad_() for t in (x0, r0, w0))
        if fused:
            s, y = add_pre_norm(x, r, w)
        else:
            s, y = pre_norm(x + r, w)
        torch.autograd.backward([s, y], [gs, gy])
        torch.cuda.synchronize()
        out.extend([s.detach(), y.detach(), x.grad, r.grad, w.grad])
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_misaligned_views_are_accepted(dev):
    # contiguous views at a 2-byte storage offset (the reference accepts any contiguous
    # tensor): the wrappers hand the kernels aligned copies; results equal the aligned run
    from fxlm.norm import add_pre_norm, rms_norm
    torch.manual_seed(21)
    N, D = 37, 256
    base = torch.randn(N * D + 1, device=dev).bfloat16()
    x_odd = base[1:].view(N, D)
    assert x_odd.is_contiguous() and x_odd.data_ptr() % 16 != 0
    wbase = (torch.randn(D + 1, device=dev) * 0.3 + 1).bfloat16()
    w_odd = wbase[1:]
    dy = torch.randn(N, D, device=dev).bfloat16()
    outs = []
    for x, w in ((x_odd, w_odd), (x_odd.clone(), w_odd.clone())):
        xr, wr = x.detach().requires_grad_(), w.detach().requires_grad_()
        y = rms_norm(xr, wr)
        y.backward(dy)
        s, y2 = add_pre_norm(x, x, w)
        outs.append((y, xr.grad, wr.grad, s, y2))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
