"""FlatAdamW on the GPU (fx_adamw_step) against the oracle, torch AdamW and fixtures.

Tolerance: fp32 master weights within 1e-6 relative (max |err| / max |w|);
grad norm within 1e-3 relative; bf16 params bit-equal to round(master).
"""
import pytest
import torch
from torch import nn

from golden_util import bf16, load
from oracle import adamw as oadam
from tolerances import RTOL_ADAMW, RTOL_NORM

pytestmark = pytest.mark.gpu


class _Params(nn.Module):
    def __init__(self, tensors):
        super().__init__()
        self.ps = nn.ParameterList(nn.Parameter(t.clone()) for t in tensors)


def _p16_matches(opt):
    return all(torch.equal(p, opt.master[o:o + n].view(p.shape).bfloat16())
               for _n, p, o, n, _w in opt._info)


def test_golden_three_steps(dev):
    from fxlm.optim import FlatAdamW
    d = load("adamw_3step")
    shapes = [(64, 32), (37,), (16, 9)]
    params = [torch.from_numpy(d[f"p{i}"]) for i in range(3)]
    m = _Params(params).to(dev)
    opt = FlatAdamW(m, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                    max_grad_norm=0.5, init_scale=8.0, growth_interval=2)
    for st in range(3):
        for i, p in enumerate(m.ps):
            p.grad = bf16(d[f"g{st}_{i}"], dev).view(shapes[i])
        stats = opt.step(lr=1e-3)
        ref = torch.from_numpy(d[f"master{st}"])
        err = float((opt.master.cpu() - ref).abs().max()) / float(ref.abs().max())
        assert err < RTOL_ADAMW, (st, err)
        assert abs(float(stats["grad_norm"]) - float(d[f"norm{st}"])) <= RTOL_NORM * float(d[f"norm{st}"])
        assert float(stats["scale"]) == float(d[f"scale{st}"])
        assert _p16_matches(opt)
    assert int(opt._step_ctr) == int(d["step"])


def test_matches_torch_adamw_and_skip_and_growth(dev):
    # ml/fxlm/selftest.py:219-297 on the GPU
    from fxlm.optim import FlatAdamW
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(256, 512, bias=False), nn.LayerNorm(512),
                          nn.Linear(512, 128, bias=False)).to(dev)
    opt = FlatAdamW(model, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                    max_grad_norm=0.5, init_scale=8.0, growth_interval=4)
    ps = list(model.parameters())
    ref = [nn.Parameter(opt.master[o:o + n].view(p.shape).clone()) for _n, p, o, n, _w in opt._info]
    ropt = torch.optim.AdamW([{"params": [r for r, i in zip(ref, opt._info) if i[4]], "weight_decay": 0.1},
                              {"params": [r for r, i in zip(ref, opt._info) if not i[4]], "weight_decay": 0.0}],
                             lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    torch.manual_seed(1)
    for _ in range(6):
        grads = [torch.randn(p.shape, device=dev).bfloat16() * 0.1 for p in ps]
        scale = float(opt.scale)
        for p, g in zip(ps, grads):
            p.grad = g
        opt.step(lr=1e-3)
        for r, g in zip(ref, grads):
            r.grad = g.float() / scale
        torch.nn.utils.clip_grad_norm_(ref, 0.5)
        ropt.step()
        for (_n, p, o, n, _w), r in zip(opt._info, ref):
            err = float((opt.master[o:o + n].view(p.shape) - r.detach()).abs().max())
            assert err / float(r.detach().abs().max()) < RTOL_ADAMW
        assert _p16_matches(opt)
    # non-finite gradient: step skipped, scale halved, counter unchanged, state bit-equal
    sc0, st0 = float(opt.scale), int(opt._step_ctr)
    m0, mm0, vv0 = opt.master.clone(), opt.m.clone(), opt.v.clone()
    for p in ps:
        p.grad = torch.zeros(p.shape, device=dev).bfloat16()
    ps[0].grad.view(-1)[0] = float("inf")
    stats = opt.step(lr=1e-3)
    assert bool(stats["found_inf"]) and float(stats["scale"]) == sc0 * 0.5
    assert int(opt._step_ctr) == st0
    assert torch.equal(m0, opt.master) and torch.equal(mm0, opt.m) and torch.equal(vv0, opt.v)
    # growth after growth_interval clean steps
    sc0 = float(opt.scale)
    for _ in range(opt.growth_interval):
        for p in ps:
            p.grad = torch.zeros(p.shape, device=dev).bfloat16()
        opt.step(lr=1e-3)
    assert float(opt.scale) == sc0 * 2.0
    # grad accumulation: two backward passes add up
    g1 = torch.randn(ps[0].shape, device=dev).bfloat16()
    ps[0].grad = g1.clone()
    ps[0].grad.add_(g1)
    assert torch.equal(ps[0].grad, (g1.float() * 2).bfloat16())


def test_many_tensors_two_lists_and_missing_grads(dev):
    # 70 parameters -> two 64-entry tensor lists; some without a gradient
    from fxlm.optim import FlatAdamW
    torch.manual_seed(3)
    tensors = [torch.randn((i % 5) + 1, 3 + i) * 0.1 for i in range(70)]
    m = _Params(tensors).to(dev)
    opt = FlatAdamW(m, lr=2e-3, max_grad_norm=1.0, init_scale=1.0)
    ref = oadam.FlatAdamWRef(tensors, lr=2e-3, max_grad_norm=1.0, init_scale=1.0)
    for _ in range(2):
        grads = [None if i % 9 == 4 else (torch.randn(t.shape) * 0.05).bfloat16() for i, t in enumerate(tensors)]
        for p, g in zip(m.ps, grads):
            p.grad = None if g is None else g.to(dev)
        st = opt.step()
        rs = ref.step(grads)
        err = float((opt.master.cpu() - ref.master).abs().max()) / float(ref.master.abs().max())
        assert err < RTOL_ADAMW
        assert abs(float(st["grad_norm"]) - rs["grad_norm"]) <= RTOL_NORM * rs["grad_norm"]


def test_cfg4_full_size(dev):
    # cfg4: one flat fp32 master of 124,373,760 params, bf16 grads ~ N(0, 1e-3),
    # m ~ N(0, 1e-4), v ~ |N(0, 1e-6)|, lr 6e-4, wd 0.1, update at t = 100
    from fxlm.optim import FlatAdamW
    n = 124373760
    g = torch.Generator(device=dev).manual_seed(4)
    w0 = torch.randn(n // 768, 768, device=dev, generator=g) * 0.02
    m = _Params([w0]).to(dev)
    opt = FlatAdamW(m, lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                    max_grad_norm=1.0, init_scale=1.0)
    opt.m.normal_(0, 1e-4, generator=g)
    opt.v.normal_(0, 1e-6, generator=g).abs_()
    opt._step_ctr.fill_(99)
    grad = (torch.randn(n // 768, 768, device=dev, generator=g) * 1e-3).bfloat16()
    m.ps[0].grad = grad
    ref = oadam.FlatAdamWRef([w0.cpu()], lr=6e-4, weight_decay=0.1, max_grad_norm=1.0, init_scale=1.0)
    ref.m.copy_(opt.m.cpu())
    ref.v.copy_(opt.v.cpu())
    ref.step_ctr = 99
    st = opt.step(lr=6e-4)
    rs = ref.step([grad.cpu()], lr=6e-4)
    assert int(opt._step_ctr) == 100
    assert abs(float(st["grad_norm"]) - rs["grad_norm"]) <= RTOL_NORM * rs["grad_norm"]
    err = float((opt.master.cpu() - ref.master).abs().max()) / float(ref.master.abs().max())
    assert err < RTOL_ADAMW
