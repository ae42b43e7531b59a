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
    assert abs(loss.item() - ref_loss) <= RTOL_LOSS * abs(ref_loss)
    assert max_abs(lg.grad, ref_grad) <= _grad_tol(ref_grad)
    assert float(lg.grad[2].abs().max()) == 0.0          # out-of-range target row


@pytest.mark.parametrize("N,V", [(5, 32), (100, 512), (301, 8192), (3, 1001), (7, 50304), (2, 8),
                                 (3, 131072), (2, 140000)])
def test_against_oracle(dev, N, V):
    # ml/fxlm/selftest.py:207-226 cases plus odd V (generic kernel), the cfg3 vocabulary, the
    # widest row the register kernel holds (1024 threads x 16 vectors) and one past it (generic)
    from fxlm.cross_entropy import fused_cross_entropy
    torch.manual_seed(N + V)
    lg = (torch.randn(N, V) * 4).bfloat16()
    tg = torch.randint(0, V, (N,))
    tg[::7] = -100
    x = lg.to(dev).requires_grad_()
    loss = fused_cross_entropy(x, tg.to(dev))
    loss.backward()
    rl, rg = oce.fused_cross_entropy(lg, tg)
    assert abs(loss.item() - float(rl)) <= RTOL_LOSS * abs(float(rl))
    assert max_abs(x.grad, rg) <= _grad_tol(rg)


def test_all_ignored_gives_zero(dev):
    from fxlm.cross_entropy import fused_cross_entropy
    lg = torch.randn(6, 64, device=dev).bfloat16().requires_grad_()
    loss = fused_cross_entropy(lg, torch.full((6,), -100, device=dev))
    loss.backward()
    assert loss.item() == 0.0 and lg.grad.abs().max().item() == 0.0


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
    # the first backward rescales the saved dlogits in place; later backward calls through
    # the retained graph each return a fresh grad * (their g)
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


def test_retained_graph_keeps_earlier_results(dev):
    # torch.autograd.grad through a retained graph: the tensor the first call returned is
    # not changed by the second call
    from fxlm.cross_entropy import fused_cross_entropy
    torch.manual_seed(6)
    lg = torch.randn(9, 384, device=dev).bfloat16().requires_grad_()
    tg = torch.randint(0, 384, (9,), device=dev)
    loss = fused_cross_entropy(lg, tg)
    (g1,) = torch.autograd.grad(loss * 2.0, lg, retain_graph=True)
    keep = g1.clone()
    (g2,) = torch.autograd.grad(loss * 3.0, lg)
    torch.cuda.synchronize()
    assert torch.equal(g1, keep)
    assert g2.data_ptr() != g1.data_ptr()
    assert torch.allclose(g2.float(), keep.float() * 1.5, rtol=2 ** -8, atol=1e-7)


def test_retained_graph_after_zero_grad_raises(dev):
    # a first backward with g = 0 zeroes the saved dlogits: a second backward cannot
    # recover them and says so instead of returning inf * 0 = NaN
    from fxlm.cross_entropy import fused_cross_entropy
    lg = torch.randn(4, 64, device=dev).bfloat16().requires_grad_()
    tg = torch.randint(0, 64, (4,), device=dev)
    loss = fused_cross_entropy(lg, tg)
    (g0,) = torch.autograd.grad(loss * 0.0, lg, retain_graph=True)
    assert float(g0.abs().max()) == 0.0
    with pytest.raises(RuntimeError, match="gradient of 0"):
        torch.autograd.grad(loss, lg)


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
    assert abs(loss.item() - float(ref)) <= RTOL_LOSS * abs(float(ref))
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
    rl, _, _ = oce.linear_cross_entropy(x, W, tg)
    assert abs(loss.item() - float(rl)) <= RTOL_LOSS * abs(float(rl))
    rdx, rdW = _lin_ce_grads_bf16_points(x, W, tg, chunk_rows=128)
    _assert_lin_grads(xq.grad, Wq.grad, rdx, rdW)


@pytest.mark.parametrize("N,V", [(320, 4096), (1024, 1000)])   # V 1000: a 232-row last panel
def test_linear_ce_native_head_weight_gradient(dev, monkeypatch, N, V):
    # the head's weight gradient on fx_linear_wgrad (NATIVE_HEAD_WGRAD, off by default at the
    # cfg5 head where hipBLASLt is faster): the same oracle bounds as the library product
    import fxlm.cross_entropy as ce
    monkeypatch.setattr(ce, "NATIVE_HEAD_WGRAD", True)
    D = 256
    torch.manual_seed(N + V)
    x = torch.randn(N, D).bfloat16()
    W = (torch.randn(V, D) * 0.02).bfloat16()
    tg = torch.randint(0, V, (N,))
    tg[::7] = -100
    xq, Wq = x.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    loss = ce.linear_cross_entropy(xq, Wq, tg.to(dev), grad_scale=256.0)
    loss.backward()
    rl, _, _ = oce.linear_cross_entropy(x, W, tg)
    assert abs(loss.item() - float(rl)) <= RTOL_LOSS * abs(float(rl))
    rdx, rdW = _lin_ce_grads_bf16_points(x, W, tg)
    _assert_lin_grads(xq.grad, Wq.grad, rdx, rdW)


@pytest.mark.parametrize("gs", [1.0, 3.0, None])
def test_lin_grad_scale_bf16_weight_gradient_is_exact(dev, gs):
    # a single chunk keeps its weight-gradient product in bf16: scaling it must give the
    # bits of scaling its fp32 copy, for dx as well, with a float or a tensor grad_scale
    from fxgpu.abi import call, ptr, stream_of
    g = torch.Generator(device=dev).manual_seed(4)
    dw16 = (torch.randn(1003, device=dev, generator=g) * 50).bfloat16()   # odd length: the tail too
    dx = torch.randn(517, device=dev, generator=g).bfloat16()
    gt = torch.tensor(0.37, device=dev)
    gs_t = torch.tensor(1024.0, device=dev) if gs is None else None
    inv = 0.0 if gs is None else 1.0 / gs
    outs = []
    for fn, dw in (("fx_ce_lin_grad_scale", dw16.float()), ("fx_ce_lin_grad_scale_bf16w", dw16)):
        gw, gx = torch.empty_like(dw16), torch.empty_like(dx)
        call(fn, ptr(dw), dw.numel(), ptr(dx), dx.numel(), ptr(gt), ptr(gs_t), inv, ptr(gw), ptr(gx), stream_of(dx))
        outs.append((gw, gx))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("g,gs", [(0.37, 2.0), (0.37, None), (1024.0, None), (3.0, 3.0)])
def test_lin_grad_scale_inplace_matches_out_of_place(dev, g, gs):
    # the first backward's in-place scaling gives the bits of the out-of-place kernel; with a
    # factor of exactly 1 (the training step's g == grad_scale) it leaves both buffers as
    # they were
    from fxgpu.abi import call, ptr, stream_of
    gen = torch.Generator(device=dev).manual_seed(5)
    dw16 = (torch.randn(2003, device=dev, generator=gen) * 50).bfloat16()   # odd length: the tail too
    dx = torch.randn(1029, device=dev, generator=gen).bfloat16()
    gt = torch.tensor(g, device=dev)
    gs_t = torch.tensor(1024.0, device=dev) if gs is None else None
    inv = 0.0 if gs is None else 1.0 / gs
    gw, gx = torch.empty_like(dw16), torch.empty_like(dx)
    call("fx_ce_lin_grad_scale_bf16w", ptr(dw16), dw16.numel(), ptr(dx), dx.numel(), ptr(gt), ptr(gs_t), inv,
         ptr(gw), ptr(gx), stream_of(dx))
    w2, x2 = dw16.clone(), dx.clone()
    call("fx_ce_lin_grad_scale_inplace", ptr(w2), w2.numel(), ptr(x2), x2.numel(), ptr(gt), ptr(gs_t), inv,
         stream_of(dx))
    torch.cuda.synchronize()
    assert torch.equal(w2.view(torch.int16), gw.view(torch.int16))
    assert torch.equal(x2.view(torch.int16), gx.view(torch.int16))
    s = g * (1.0 / 1024.0 if gs is None else inv)
    if s == 1.0:
        assert torch.equal(w2.view(torch.int16), dw16.view(torch.int16))


def test_linear_ce_backward_twice_with_retained_graph(dev):
    # the first backward scales the saved gradients in place and returns them; a second
    # backward through the retained graph returns fresh ones at its own factor, and the
    # first call's results stay as they were
    from fxlm.cross_entropy import linear_cross_entropy
    torch.manual_seed(11)
    N, D, V = 300, 256, 4096
    x = torch.randn(N, D, device=dev).bfloat16().requires_grad_()
    W = (torch.randn(V, D, device=dev) * 0.02).bfloat16().requires_grad_()
    tg = torch.randint(0, V, (N,), device=dev)
    loss = linear_cross_entropy(x, W, tg, grad_scale=4.0)
    g1x, g1w = torch.autograd.grad(loss * 8.0, (x, W), retain_graph=True)
    k1x, k1w = g1x.clone(), g1w.clone()
    g2x, g2w = torch.autograd.grad(loss * 2.0, (x, W))
    torch.cuda.synchronize()
    assert torch.equal(g1x, k1x) and torch.equal(g1w, k1w)
    for a, b in ((g2x, g1x), (g2w, g1w)):
        assert torch.allclose(a.float() * 4.0, b.float(), rtol=2.0 ** -7, atol=1e-30)


def test_linear_ce_retained_graph_after_zero_factor_raises(dev):
    from fxlm.cross_entropy import linear_cross_entropy
    torch.manual_seed(12)
    x = torch.randn(64, 128, device=dev).bfloat16().requires_grad_()
    W = (torch.randn(512, 128, device=dev) * 0.02).bfloat16().requires_grad_()
    tg = torch.randint(0, 512, (64,), device=dev)
    loss = linear_cross_entropy(x, W, tg)
    torch.autograd.grad(loss * 0.0, (x, W), retain_graph=True)
    with pytest.raises(RuntimeError, match="factor of 0"):
        torch.autograd.grad(loss * 1.0, (x, W))


@pytest.mark.parametrize("gs", [1.0, None])
def test_linear_ce_single_chunk(dev, gs):
    # the default chunking holds these rows in one chunk (bf16 weight-gradient product)
    from fxlm.cross_entropy import _auto_chunk, linear_cross_entropy
    N, D, V = 300, 256, 4096
    assert _auto_chunk(D, V) >= N
    torch.manual_seed(9)
    x = torch.randn(N, D).bfloat16()
    W = (torch.randn(V, D) * 0.02).bfloat16()
    tg = torch.randint(0, V, (N,))
    tg[::7] = -100
    grad_scale = torch.tensor(4096.0, device=dev) if gs is None else gs
    xq, Wq = x.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    loss = linear_cross_entropy(xq, Wq, tg.to(dev), grad_scale=grad_scale)
    loss.backward()
    rl, _, _ = oce.linear_cross_entropy(x, W, tg)
    assert abs(loss.item() - float(rl)) <= RTOL_LOSS * abs(float(rl))
    rdx, rdW = _lin_ce_grads_bf16_points(x, W, tg)
    _assert_lin_grads(xq.grad, Wq.grad, rdx, rdW)


def _lin_ce_grads_bf16_points(x, W, tg, rows=None, chunk_rows=None):
    """(dx, dW) in fp64 with the path's rounding points: logits rounded to bf16 (the
    logits GEMM writes bf16), dlogits rounded to bf16 (the CE kernel's output), dW
    products per chunk rounded to bf16 (ml/fxlm/cross_entropy.py:135) and summed in
    fp64.  `rows`: dx only for those rows (dW is then None)."""
    xf, wf = x.double().cpu(), W.double().cpu()
    inv_n = oce.inv_nvalid(tg)
    if rows is not None:
        lg = (xf[rows] @ wf.t()).bfloat16()
        _, dl = oce.ce_rows(lg, tg.cpu()[rows], inv_n)
        return dl.bfloat16().double() @ wf, None
    lg = (xf @ wf.t()).bfloat16()
    _, dl = oce.ce_rows(lg, tg.cpu(), inv_n)
    dl = dl.bfloat16().double()
    N = x.shape[0]
    step = N if chunk_rows is None else chunk_rows
    dW = sum((dl[r:r + step].t() @ xf[r:r + step]).bfloat16().double() for r in range(0, N, step))
    return dl @ wf, dW


def _assert_lin_grads(gx, gw, rdx, rdW):
    # bf16 results: half an ulp of each value plus the fp32 accumulation order and the
    # rare logit rounded the other way (2e-3 of the largest value)
    for ours, ref in ((gx, rdx), (gw, rdW)):
        if ref is None:
            continue
        o, r = ours.double().cpu(), ref.double().cpu()
        tol = 2.0 ** -8 * r.abs() + 2e-3 * float(r.abs().max()) + 1e-9
        assert bool(((o - r).abs() <= tol).all()), float(((o - r).abs() - tol).max())


def test_linear_ce_cfg5_head_one_chunk(dev):
    # the 12-layer model's head: x (16384, 768), tied W (50304, 768).  The default
    # chunking (one chunk here) against the reference's 512-row chunks
    # (ml/fxlm/cross_entropy.py:102-104): the loss against fp32 torch math, dx on sampled
    # rows against the fp64 oracle with the path's rounding points, dW in full
    from fxlm.cross_entropy import _auto_chunk, linear_cross_entropy
    N, D, V = 16384, 768, 50304
    assert _auto_chunk(D, V) >= N
    g = torch.Generator(device=dev).manual_seed(55)
    x0 = torch.randn(N, D, device=dev, generator=g).bfloat16()
    w0 = (torch.randn(V, D, device=dev, generator=g) * 0.02).bfloat16()
    tg = torch.randint(0, V, (N,), device=dev, generator=g)
    tg[torch.rand(N, device=dev, generator=g) < 0.05] = -100
    res = {}
    for chunk in (None, 512):
        x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
        loss = linear_cross_entropy(x, w, tg, grad_scale=1024.0, chunk_rows=chunk)
        loss.backward()
        res[chunk] = (loss.item(), x.grad, w.grad)
    ref = F.cross_entropy(x0.float() @ w0.float().t(), tg, ignore_index=-100)
    for chunk, (l, gx, gw) in res.items():
        assert abs(l - float(ref)) <= RTOL_LOSS * abs(float(ref)), chunk
    assert abs(res[None][0] - res[512][0]) <= 1e-6 * abs(res[None][0])
    rows = torch.arange(7, N, 509)
    rdx, _ = _lin_ce_grads_bf16_points(x0, w0, tg, rows=rows)
    for chunk, (_, gx, _) in res.items():
        _assert_lin_grads(gx[rows.to(dev)], None, rdx, None)
    # dW in full against fp32 torch math on the GPU with the same rounding points (a
    # 16384 x 50304 fp64 reference is too large for the host side of a test)
    inv_n = 1.0 / float((tg != -100).sum())
    p = torch.softmax((x0.float() @ w0.float().t()).bfloat16().float(), dim=-1)
    valid = tg >= 0
    p[valid.nonzero()[:, 0], tg[valid]] -= 1.0
    p[~valid] = 0.0
    dl = (p * inv_n).bfloat16().float()
    del p
    for chunk in (None, 512):
        step = N if chunk is None else chunk
        rdW = torch.zeros(V, D, device=dev, dtype=torch.float32)
        for r in range(0, N, step):
            rdW += (dl[r:r + step].t() @ x0[r:r + step].float()).bfloat16().float()
        o = res[chunk][2].float()
        tol = 2.0 ** -8 * rdW.abs() + 2e-3 * float(rdW.abs().max()) + 1e-9
        assert bool(((o - rdW).abs() <= tol).all()), chunk
