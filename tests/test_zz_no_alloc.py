"""fx_adamw_step_noalloc (the allocation-free optimiser step, whose workspace is a buffer
inside the library) against fx_adamw_step with a caller-owned workspace: bitwise-equal
optimiser state over several steps, on two calls in a row with the second on a smaller
parameter set (the scratch keeps the first call's contents).  Its size check, which needs no
GPU, is in tests/test_abi.py."""
import ctypes

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu


def _pair(dev, shapes, seed):
    from fxlm.optim import FlatAdamW
    torch.manual_seed(seed)
    tensors = [torch.randn(*s) * 0.1 for s in shapes]
    mods = []
    for _ in range(2):
        m = nn.ParameterList(nn.Parameter(t.clone()) for t in tensors).to(dev)
        mods.append((m, FlatAdamW(m, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                                  max_grad_norm=0.5, init_scale=8.0, growth_interval=2)))
    return mods


def _run_steps(dev, shapes, seed, steps):
    from fxgpu.abi import call, stream_of
    (ma, oa), (mb, ob) = _pair(dev, shapes, seed)
    g = torch.Generator(device=dev).manual_seed(seed)
    for step in range(steps):
        grads = [(torch.randn(p.shape, device=dev, generator=g) * 0.05).bfloat16() for p in ma]
        if step == 1:
            grads[0].view(-1)[3] = float("inf")     # a skipped step and a backoff
        for m in (ma, mb):
            for p, gr in zip(m, grads):
                p.grad = gr.clone()
        oa.step(lr=1e-3)
        lists, nl, _keep = ob._lists()
        st = ob._state(1e-3, None)                  # the workspace pointer is ignored
        call("fx_adamw_step_noalloc", ctypes.byref(st), lists, nl, stream_of(ob.master))
        torch.cuda.synchronize()
        for name in ("master", "m", "v", "flat16", "_step_ctr", "_found_inf", "_norm", "scale", "_growth"):
            assert torch.equal(getattr(oa, name), getattr(ob, name)), (step, name)
    return oa


def test_noalloc_step_matches_workspace_step(dev):
    # first call: 70 tensors (two lists), 3.3 M parameters; then a smaller set of 3
    big = [(512, 256), (1024,), (256, 768)] * 23 + [(3000,)]
    oa = _run_steps(dev, big, seed=1, steps=4)
    assert int(oa._step_ctr) == 3                   # the inf step was skipped
    _run_steps(dev, [(37, 5), (8,), (100,)], seed=2, steps=3)

