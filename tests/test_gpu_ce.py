"""Fused cross-entropy and linear cross-entropy on the GPU against the oracle and fixtures."""
import pytest
import torch
import torch.nn.functional as F

from golden_util import bf16, f32, load
from oracle import cross_entropy as oce
from tolerances import RTOL_LOSS, max_abs

pytestmark = pytest.mark.gpu


def _grad_tol(ref):
    # dlogits are bf16: half an ulp of the largest value, floored for tiny rows
    return max(float(ref.abs().max()) * 2.0 ** -8, 1e-6)


@pytest.mark.parametrize("name", ["ce_n16_v512", "ce_n9_v1000"])
def test_golden(dev, name):
    from fxlm.cross_entropy import fused_cross_entropy
    d = load(name)
    lg = bf16(d["logits"], dev).requires_grad_()
    tg = torch.from_numpy(d["target"]).to(dev)
    loss = fused_cross_entropy(lg, tg)
    loss.backward()
    ref_loss, ref_grad = float(d["loss"]), f32(d["grad"])
    assert abs(float(loss) - ref_loss) <= RTOL_LOSS * abs(ref_loss)
    assert max_abs(lg.grad, ref_grad) <= _grad_tol(ref_grad)
    assert float(lg.grad[2].abs().max()) == 0.0          # out-of-range target row


@pytest.mark.parametrize("N,V", [(5, 32), (100, 512), (301, 8192), (3, 1001), (7, 50304), (2, 8)])
def test_against_oracle(dev, N, V):
    # ml/fxlm/selftest.py:207-226 cases plus odd V (generic kernel) and the cfg3 vocabulary
    from fxlm.cross_entropy import fused_cross_entropy
    torch.manual_seed(N + V)
    lg = (torch.randn(N, V) * 4).bfloat16()
    tg = torch.randint(0, V, (N,))
    tg[::7] = -100
    x = lg.to(dev).requires_grad_()
    loss = fused_cross_entropy(x, tg.to(dev))
    loss.backward()
    rl, rg = oce.fused_cross_entropy(lg, tg)
    assert abs(float(loss) - float(rl)) <= RTOL_LOSS * abs(float(rl))
    assert max_abs(x.grad, rg) <= _grad_tol(rg)


def test_all_ignored_gives_zero(dev):
    from fxlm.cross_entropy import fused_cross_entropy
    lg = torch.randn(6, 64, device=dev).bfloat16().requires_grad_()
    loss = fused_cross_entropy(lg, torch.full((6,), -100, device=dev))
    loss.backward()
    assert float(loss) == 0.0 and float(lg.grad.abs().max()) == 0.0


def test_backward_scales_by_incoming_grad(dev):
    from fxlm.cross_entropy import fused_cross_entropy
    torch.manual_seed(3)
    lg = torch.randn(33, 512, device=dev).bfloat16()
    tg = torch.randint(0, 512, (33,), device=dev)
    a = lg.clone().requires_grad_()
    fused_cross_entropy(a, tg).backward()
    b = lg.clone().requires_grad_()
    (fused_cross_entropy(b, tg) * 4.0).backward()
    assert torch.equal(b.grad, (a.grad.float() * 4.0).bfloat16())


def test_backward_twice_with_retained_graph(dev):
    # the gradient buffer is rescaled in place; the multiplier it carries is tracked in
    # two device slots, so repeated backward calls each see grad * (their g)
    from fxlm.cross_entropy import fused_cross_entropy
    torch.manual_seed(4)
    lg = torch.randn(17, 256, device=dev).bfloat16()
    tg = torch.randint(0, 256, (17,), device=dev)
    ref = lg.clone().requires_grad_()
    fused_cross_entropy(ref, tg).backward()
    c = lg.clone().requires_grad_()
    loss = fused_cross_entropy(c, tg)
    (loss * 2.0).backward(retain_graph=True)
    first = c.grad.clone()
    assert torch.equal(first, (ref.grad.float() * 2.0).bfloat16())
    c.grad = None
    (loss * 2.0).backward(retain_graph=True)  # same g again: no second scaling
    assert torch.equal(c.grad, first)
    c.grad = None
    (loss * 0.5).backward()                   # a different g: rescaled from 2 to 0.5
    assert torch.allclose(c.grad.float(), ref.grad.float() * 0.5, rtol=2 ** -7, atol=1e-6)


def test_cfg3_full_size(dev):
    # cfg3: logits (16384, 50304) ~ N(0, 2), 5% ignored targets; fp32 torch math on the GPU
    from fxlm.cross_entropy import fused_cross_entropy
    g = torch.Generator(device=dev).manual_seed(3)
    N, V = 16384, 50304
    lg = (torch.randn(N, V, device=dev, generator=g) * 2).bfloat16()
    tg = torch.randint(0, V, (N,), device=dev, generator=g)
    tg[torch.rand(N, device=dev, generator=g) < 0.05] = -100
    x = lg.clone().requires_grad_()
    loss = fused_cross_entropy(x, tg)
    loss.backward()
    ref = F.cross_entropy(lg.float(), tg, ignore_index=-100)
    assert abs(float(loss) - float(ref)) <= RTOL_LOSS * abs(float(ref))
    rows = torch.arange(0, N, 1024, device=dev)
    sub = lg[rows].float().requires_grad_()
    tsub = tg[rows]
    nvalid = float((tg != -100).sum())
    (F.cross_entropy(sub, tsub, ignore_index=-100, reduction="sum") / nvalid).backward()
    assert max_abs(x.grad[rows], sub.grad) <= _grad_tol(sub.grad)
    del x, lg


@pytest.mark.parametrize("N,D,V,gs", [(50, 64, 128, 1.0), (301, 256, 8192, 1.0), (1027, 512, 4096, None)])
def test_linear_ce(dev, N, D, V, gs):
    # ml/fxlm/selftest.py:229-253, chunk_rows=128 (does not divide N), tensor grad_scale
    from fxlm.cross_entropy import linear_cross_entropy
    torch.manual_seed(N + D + V)
    x = torch.randn(N, D).bfloat16()
    W = (torch.randn(V, D) * 0.02).bfloat16()
    tg = torch.randint(0, V, (N,))
    tg[::11] = -100
    grad_scale = torch.tensor(65536.0, device=dev) if gs is None else gs
    xq, Wq = x.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    loss = linear_cross_entropy(xq, Wq, tg.to(dev), grad_scale=grad_scale, chunk_rows=128)
    loss.backward()
    rl, rdx, rdW = oce.linear_cross_entropy(x, W, tg)
    assert abs(float(loss) - float(rl)) <= RTOL_LOSS * abs(float(rl))
    assert max_abs(xq.grad, rdx) <= max(2e-2 * float(rdx.abs().max()), 1e-6)
    assert max_abs(Wq.grad, rdW) <= max(2e-2 * float(rdW.abs().max()), 1e-6)


def test_linear_ce_no_grad_path(dev):
    from fxlm.cross_entropy import linear_cross_entropy
    torch.manual_seed(7)
    x = torch.randn(200, 128, device=dev).bfloat16()
    W = (torch.randn(512, 128, device=dev) * 0.02).bfloat16()
    tg = torch.randint(0, 512, (200,), device=dev)
    lg = linear_cross_entropy(x, W, tg, grad_scale=1.0)
    with torch.no_grad():
        ln = linear_cross_entropy(x, W, tg)
    assert ln.grad_fn is None and abs(float(ln) - float(lg)) < 1e-6


@pytest.mark.parametrize("gs", ["tensor", 3.0])
def test_linear_ce_backward_scaling_is_bitwise_torch(dev, gs):
    # fx_ce_lin_grad_scale against the torch ops it replaces (ml/fxlm/cross_entropy.py:141-148),
    # with a device or Python grad_scale and an incoming gradient other than 1
    import fxlm.cross_entropy as ce
    torch.manual_seed(8)
    N, D, V = 301, 256, 1003
    x0 = (torch.randn(N, D, device=dev) * 0.5).bfloat16()
    w0 = (torch.randn(V, D, device=dev) * 0.05).bfloat16()
    t = torch.randint(0, V, (N,), device=dev)
    scale = torch.tensor(8.0, device=dev) if gs == "tensor" else gs
    outs = []
    for fused in (True, False):
        ce._FUSED_LIN_GRAD_SCALE = fused
        try:
            x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
            loss = ce.linear_cross_entropy(x, w, t, grad_scale=scale)
            loss.backward(torch.tensor(0.37, device=dev))
            torch.cuda.synchronize()
            outs.append((x.grad, w.grad))
        finally:
            ce._FUSED_LIN_GRAD_SCALE = True
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
