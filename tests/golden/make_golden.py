"""Write the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference commits no golden vectors (its tests draw seeded inputs at run
time, ml/fxlm/selftest.py), so these fixtures are produced by the oracle, which
tests/test_oracle.py pins against library routines, brute force and closed
forms.  Shapes follow the reference selftest's cases (ml/fxlm/selftest.py:56-
216) at small sizes, plus the edge cases the kernels special-case (V % 8 != 0,
out-of-range / ignored targets, tail tiles, head_dim 128).  bf16 tensors are
stored as uint16 bit patterns; everything loads with numpy.load(allow_pickle=False).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import adamw as oadam  # noqa: E402
from oracle import attention as oatt  # noqa: E402
from oracle import cross_entropy as oce  # noqa: E402
from oracle import linear as olin  # noqa: E402
from oracle import norm as onorm  # noqa: E402


def bf16_bits(t):
    return t.detach().cpu().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def f32(t):
    # copy: .numpy() of a float32 CPU tensor shares its storage (the optimiser
    # state is updated in place by later steps)
    return t.detach().cpu().to(torch.float32).numpy().copy()


def attention_cases():
    out = {}
    for name, (B, T, H, D, causal, seed) in {
        "attn_t37_d64_causal": (1, 37, 2, 64, True, 11),
        "attn_t33_d128_full": (1, 33, 1, 128, False, 12),
        "attn_t130_d64_causal": (1, 130, 1, 64, True, 13),
    }.items():
        g = torch.Generator().manual_seed(seed)
        q, k, v, do = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(4))
        scale = D ** -0.5
        o, lse = oatt.attn_fwd(q, k, v, causal, scale)
        o_bf = o.to(torch.bfloat16)              # the stored (rounded) forward output
        dq, dk, dv = oatt.attn_bwd(q, k, v, o_bf, lse, do, causal, scale)
        out[name] = dict(q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), do=bf16_bits(do),
                         o=f32(o), lse=f32(lse), dq=f32(dq), dk=f32(dk), dv=f32(dv),
                         causal=np.array(int(causal)), scale=np.array(scale, np.float32))
    return out


def ce_cases():
    out = {}
    for name, (N, V, seed) in {"ce_n16_v512": (16, 512, 21), "ce_n9_v1000": (9, 1000, 22)}.items():
        g = torch.Generator().manual_seed(seed)
        lg = (torch.randn(N, V, generator=g) * 4).bfloat16()
        tg = torch.randint(0, V, (N,), generator=g)
        tg[::7] = -100
        tg[2] = V + 3                             # out of range: counted, no loss, zero row
        loss, grad = oce.fused_cross_entropy(lg, tg)
        out[name] = dict(logits=bf16_bits(lg), target=tg.numpy(), loss=np.array(float(loss)),
                         grad=f32(grad))
    return out


def norm_cases():
    g = torch.Generator().manual_seed(31)
    N, D = 7, 768
    x = (torch.randn(N, D, generator=g) * 3).bfloat16()
    w = (torch.randn(D, generator=g) * 0.5 + 1).bfloat16()
    dy = torch.randn(N, D, generator=g).bfloat16()
    y, rstd = onorm.rms_norm_fwd(x, w, 1e-6)
    dx, dw = onorm.rms_norm_bwd(x, dy, w, rstd)
    return {"rms_n7_d768": dict(x=bf16_bits(x), w=bf16_bits(w), dy=bf16_bits(dy), y=f32(y),
                                rstd=f32(rstd), dx=f32(dx), dw=f32(dw))}


def adamw_cases():
    g = torch.Generator().manual_seed(41)
    shapes = [(64, 32), (37,), (16, 9)]
    params = [torch.randn(s, generator=g) * 0.1 for s in shapes]
    ref = oadam.FlatAdamWRef(params, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                             max_grad_norm=0.5, init_scale=8.0, growth_interval=2)
    d = {f"p{i}": f32(p) for i, p in enumerate(params)}
    for st in range(3):
        grads = [(torch.randn(s, generator=g) * 0.1).bfloat16() for s in shapes]
        stats = ref.step(grads, lr=1e-3)
        for i, gr in enumerate(grads):
            d[f"g{st}_{i}"] = bf16_bits(gr)
        d[f"master{st}"] = f32(ref.master)
        d[f"norm{st}"] = np.array(stats["grad_norm"], np.float32)
        d[f"scale{st}"] = np.array(stats["scale"], np.float32)
    d["step"] = np.array(ref.step_ctr)
    return {"adamw_3step": d}


def linear_cases():
    g = torch.Generator().manual_seed(51)
    R, F, W, B, N = 50, 8, 3, 9, 5
    X = torch.randn(R, F, generator=g).bfloat16()
    idx = torch.randint(0, R - W + 1, (B,), generator=g, dtype=torch.int32)
    Wt = (torch.randn(N, W * F, generator=g) * 0.1).bfloat16()
    bias = (torch.randn(N, generator=g) * 0.1).bfloat16()
    gout = torch.randn(B, N, generator=g).bfloat16()
    out, Xg = olin.gather_linear(X, idx, Wt, bias)
    dW = gout.double().t() @ Xg
    d = dict(X=bf16_bits(X), idx=idx.numpy(), W=bf16_bits(Wt), bias=bf16_bits(bias),
             gout=bf16_bits(gout), out=f32(out), dW=f32(dW), db=f32(gout.double().sum(0)))
    x = torch.randn(12, 64, generator=g).bfloat16()
    Wd = (torch.randn(40, 64, generator=g) * 0.1).bfloat16()
    dy = torch.randn(12, 40, generator=g).bfloat16()
    y, h = olin.linear_act_fwd(x, Wd, None)
    dx, dWd, _db = olin.linear_act_bwd(x, Wd, h, dy)
    return {"gather_linear": d,
            "linear_gelu": dict(x=bf16_bits(x), W=bf16_bits(Wd), dy=bf16_bits(dy), y=f32(y),
                                h=f32(h), dx=f32(dx), dW=f32(dWd))}


def all_cases():
    cases = {}
    for fn in (attention_cases, ce_cases, norm_cases, adamw_cases, linear_cases):
        cases.update(fn())
    return cases


def main():
    for name, d in all_cases().items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
        print("wrote", name)


if __name__ == "__main__":
    main()
