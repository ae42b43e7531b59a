"""Pins of the CPU oracle against independent computations (CPU only).

Each oracle function is checked against a library routine that computes the
same quantity by a different route (torch SDPA / autograd, F.cross_entropy,
F.rms_norm, torch.optim.AdamW + clip_grad_norm_, torch._amp_update_scale_,
Tensor.unfold), against brute-force loops on tiny inputs, and against closed
forms -- so a dropped term, a wrong sign, index or transposed operand in the
oracle fails here.  The reference ships no golden vectors of its own.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import adamw as oadam
from oracle import attention as oatt
from oracle import cross_entropy as oce
from oracle import gpt as ogpt
from oracle import linear as olin
from oracle import norm as onorm

f64 = torch.float64


# ---------------------------------------------------------------- attention

def _sdpa_ref(q, k, v, causal, scale):
    """(B,T,H,D) fp64 SDPA with autograd."""
    o = F.scaled_dot_product_attention(q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3),
                                       v.permute(0, 2, 1, 3), is_causal=causal, scale=scale)
    return o.permute(0, 2, 1, 3)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,T,H,D", [(1, 1, 1, 64), (2, 5, 2, 8), (1, 37, 3, 64), (2, 19, 1, 128)])
def test_attention_matches_sdpa_and_autograd(causal, B, T, H, D):
    torch.manual_seed(T * 7 + D)
    q, k, v, do = (torch.randn(B, T, H, D, dtype=f64) for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    o, lse = oatt.attn_fwd(q, k, v, causal, scale)
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    oref = _sdpa_ref(qr, kr, vr, causal, scale)
    assert torch.allclose(o, oref.detach(), atol=1e-12, rtol=1e-10)
    s = oatt.scores(q, k, causal, scale)
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)
    oref.backward(do)
    dq, dk, dv = oatt.attn_bwd(q, k, v, o, lse, do, causal, scale)
    for ours, ref in ((dq, qr.grad), (dk, kr.grad), (dv, vr.grad)):
        assert torch.allclose(ours, ref, atol=1e-10, rtol=1e-9)


def test_attention_brute_force_loops():
    torch.manual_seed(3)
    B, T, H, D = 1, 4, 2, 3
    q, k, v = (torch.randn(B, T, H, D, dtype=f64) for _ in range(3))
    scale = 0.7
    o, lse = oatt.attn_fwd(q, k, v, True, scale)
    for h in range(H):
        for m in range(T):
            s = [sum(float(q[0, m, h, d]) * float(k[0, n, h, d]) for d in range(D)) * scale
                 for n in range(m + 1)]
            mx = max(s)
            z = sum(math.exp(x - mx) for x in s)
            assert abs(float(lse[0, h, m]) - (mx + math.log(z))) < 1e-12
            for d in range(D):
                ref = sum(math.exp(s[n] - mx) / z * float(v[0, n, h, d]) for n in range(m + 1))
                assert abs(float(o[0, m, h, d]) - ref) < 1e-12


def test_attention_special_cases():
    torch.manual_seed(4)
    q, k, v, do = (torch.randn(2, 1, 3, 64, dtype=f64) for _ in range(4))
    o, lse = oatt.attn_fwd(q, k, v, True)
    assert torch.equal(o, v)                      # one key: O = V
    dq, dk, dv = oatt.attn_bwd(q, k, v, o, lse, do, True)
    assert float(dq.abs().max()) < 1e-12 and float(dk.abs().max()) < 1e-12
    assert torch.allclose(dv, do)
    q, k, v = (torch.randn(1, 9, 2, 64, dtype=f64) for _ in range(3))
    o, _ = oatt.attn_fwd(q, k, v, True)
    assert torch.allclose(o[:, 0], v[:, 0])       # causal row 0 sees only key 0


def test_attention_decode_is_the_last_causal_row():
    # the decode step over the first n keys equals row n-1 of the causal forward, for
    # every n (closed under the forward oracle pinned above)
    g = torch.Generator().manual_seed(3)
    B, T, H, D = 2, 9, 3, 64
    q, k, v = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    o_full, lse_full = oatt.attn_fwd(q, k, v, causal=True)
    for n in range(1, T + 1):
        lens = torch.full((B,), n, dtype=torch.int32)
        o, lse = oatt.attn_decode(q[:, n - 1], k, v, lens)
        assert torch.allclose(o, o_full[:, n - 1], atol=1e-12)
        assert torch.allclose(lse, lse_full[:, :, n - 1], atol=1e-12)
    # per-sequence lengths: sequence 0 empty, sequence 1 at its second token
    q_sel = torch.stack([q[0, 0], q[1, 1]])
    o, lse = oatt.attn_decode(q_sel, k, v, torch.tensor([0, 2], dtype=torch.int32))
    assert float(o[0].abs().max()) == 0 and bool(torch.isinf(lse[0]).all())
    assert torch.allclose(o[1], o_full[1, 1], atol=1e-12)


def test_attention_delta_uses_stored_output():
    # Delta is rowsum(dO * O) of the output handed in (the rounded one), not a recomputed O.
    torch.manual_seed(5)
    q, k, v, do = (torch.randn(1, 6, 1, 64, dtype=f64) for _ in range(4))
    o, lse = oatt.attn_fwd(q, k, v, True)
    o2 = o + 0.5
    a = oatt.attn_bwd(q, k, v, o, lse, do, True)
    b = oatt.attn_bwd(q, k, v, o2, lse, do, True)
    assert not torch.allclose(a[0], b[0])
    assert torch.allclose(a[2], b[2])            # dV does not involve Delta


# ---------------------------------------------------------------- cross-entropy

@pytest.mark.parametrize("N,V", [(5, 32), (100, 512), (301, 8192)])
def test_ce_matches_torch(N, V):
    torch.manual_seed(N + V)
    lg = torch.randn(N, V, dtype=f64) * 4
    tg = torch.randint(0, V, (N,))
    tg[::7] = -100
    loss, grad = oce.fused_cross_entropy(lg, tg)
    lr = lg.clone().requires_grad_()
    ref = F.cross_entropy(lr, tg, ignore_index=-100)
    ref.backward()
    assert abs(float(loss) - float(ref)) < 1e-12
    assert torch.allclose(grad, lr.grad, atol=1e-14)


def test_ce_out_of_range_and_empty():
    torch.manual_seed(1)
    N, V = 12, 40
    lg = torch.randn(N, V, dtype=f64)
    tg = torch.randint(0, V, (N,))
    tg[3] = V + 5          # out of range: counted in n_valid, no loss, zero grad row
    tg[7] = -100
    loss, grad = oce.fused_cross_entropy(lg, tg)
    keep = torch.tensor([i not in (3, 7) for i in range(N)])
    per_row = F.cross_entropy(lg[keep], tg[keep], reduction="none")
    assert abs(float(loss) - float(per_row.sum()) / (N - 1)) < 1e-12
    assert float(grad[3].abs().max()) == 0.0 and float(grad[7].abs().max()) == 0.0
    loss0, grad0 = oce.fused_cross_entropy(lg, torch.full((N,), -100))
    assert float(loss0) == 0.0 and float(grad0.abs().max()) == 0.0


def test_linear_ce_matches_autograd():
    torch.manual_seed(2)
    N, D, V = 50, 16, 30
    x = torch.randn(N, D, dtype=f64)
    W = torch.randn(V, D, dtype=f64) * 0.3
    tg = torch.randint(0, V, (N,))
    tg[::11] = -100
    loss, dx, dW = oce.linear_cross_entropy(x, W, tg)
    xr, Wr = x.clone().requires_grad_(), W.clone().requires_grad_()
    ref = F.cross_entropy(xr @ Wr.t(), tg, ignore_index=-100)
    ref.backward()
    assert abs(float(loss) - float(ref)) < 1e-12
    assert torch.allclose(dx, xr.grad, atol=1e-13) and torch.allclose(dW, Wr.grad, atol=1e-13)


# ---------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("N,D", [(4, 8), (37, 64), (129, 768)])
def test_rms_norm_matches_torch(N, D):
    torch.manual_seed(N * 1000 + D)
    x = torch.randn(N, D, dtype=f64) * 3
    w = torch.randn(D, dtype=f64) * 0.5 + 1
    dy = torch.randn(N, D, dtype=f64)
    y, rstd = onorm.rms_norm_fwd(x, w, 1e-6)
    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    yr = F.rms_norm(xr, (D,), wr, 1e-6)
    yr.backward(dy)
    assert torch.allclose(y, yr.detach(), atol=1e-12)
    dx, dw = onorm.rms_norm_bwd(x, dy, w, rstd)
    assert torch.allclose(dx, xr.grad, atol=1e-11) and torch.allclose(dw, wr.grad, atol=1e-10)


def test_rms_norm_closed_form():
    x = torch.full((3, 16), 2.0, dtype=f64)
    w = torch.ones(16, dtype=f64)
    y, rstd = onorm.rms_norm_fwd(x, w, 1e-6)
    assert torch.allclose(rstd, torch.full((3,), 1 / math.sqrt(4 + 1e-6), dtype=f64))
    assert torch.allclose(y, x / math.sqrt(4 + 1e-6))


# ---------------------------------------------------------------- FlatAdamW

def _params():
    torch.manual_seed(0)
    return [torch.randn(64, 32) * 0.1, torch.randn(37), torch.randn(16, 9) * 0.1]


def test_adamw_layout_align8():
    info, total = oadam.layout([(64, 32), (37,), (16, 9)], 0.1)
    assert info == [(0, 2048, 1), (2048, 37, 0), (2088, 144, 1)] and total == 2232
    info0, _ = oadam.layout([(64, 32)], 0.0)
    assert info0[0][2] == 0          # no decay flag when weight_decay == 0


def test_adamw_matches_torch_adamw_with_clip():
    # grad-injection parity, the procedure of ml/fxlm/selftest.py:219-261
    params = _params()
    ref = oadam.FlatAdamWRef(params, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                             max_grad_norm=0.5, init_scale=8.0, growth_interval=4)
    tp = [torch.nn.Parameter(p.clone()) for p in params]
    topt = torch.optim.AdamW([{"params": [tp[0], tp[2]], "weight_decay": 0.1},
                              {"params": [tp[1]], "weight_decay": 0.0}],
                             lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    torch.manual_seed(1)
    for _ in range(6):
        grads = [(torch.randn(p.shape) * 0.1).bfloat16() for p in params]
        scale = ref.scale
        ref.step(grads)
        for p, g in zip(tp, grads):
            p.grad = g.float() / scale
        torch.nn.utils.clip_grad_norm_(tp, 0.5)
        topt.step()
        for p, (off, n, _wd) in zip(tp, ref.info):
            ours = ref.master[off:off + n]
            err = float((ours - p.detach().reshape(-1)).abs().max())
            assert err / float(p.detach().abs().max()) < 1e-6
    assert ref.step_ctr == 6


def test_adamw_inf_skip_and_growth():
    params = _params()
    ref = oadam.FlatAdamWRef(params, init_scale=8.0, growth_interval=3)
    m0 = ref.master.clone()
    g = [torch.zeros(p.shape).bfloat16() for p in params]
    g[1][5] = float("inf")
    st = ref.step(g)
    assert st["found_inf"] == 1.0 and ref.scale == 4.0 and ref.step_ctr == 0
    assert torch.equal(ref.master, m0) and float(ref.m.abs().max()) == 0.0
    for _ in range(3):
        ref.step([torch.zeros(p.shape).bfloat16() for p in params])
    assert ref.scale == 8.0 and ref.growth == 0 and ref.step_ctr == 3


def test_adamw_scale_update_matches_torch():
    torch.manual_seed(9)
    scale, growth = 1024.0, 0
    ts = torch.tensor(1024.0)
    tg = torch.zeros((), dtype=torch.int32)
    for _ in range(60):
        bad = bool(torch.rand(()) < 0.2)
        scale, growth = oadam.update_scale(scale, growth, bad, 2.0, 0.5, 4)
        torch._amp_update_scale_(ts, tg, torch.tensor(1.0 if bad else 0.0), 2.0, 0.5, 4)
        assert scale == float(ts) and growth == int(tg)


# ---------------------------------------------------------------- linear

def test_gather_matches_unfold():
    # the reference's own gather oracle (ml/fxgpu/selftest.py:35-40)
    torch.manual_seed(0)
    R, Fe, W, B = 200, 8, 5, 33
    X = torch.randn(R, Fe)
    idx = torch.randint(0, R - W + 1, (B,), dtype=torch.int32)
    xb = X.unfold(0, W, 1)[idx.long()].transpose(1, 2).reshape(B, W * Fe)
    assert torch.equal(olin.gather(X, idx, W * Fe), xb)


def test_linear_gelu_matches_autograd():
    torch.manual_seed(1)
    x = torch.randn(20, 12, dtype=f64)
    W = torch.randn(7, 12, dtype=f64) * 0.3
    b = torch.randn(7, dtype=f64)
    dy = torch.randn(20, 7, dtype=f64)
    y, h = olin.linear_act_fwd(x, W, b)
    xr, Wr, br = (t.clone().requires_grad_() for t in (x, W, b))
    yr = F.gelu(F.linear(xr, Wr, br), approximate="tanh")
    yr.backward(dy)
    assert torch.allclose(y, yr.detach(), atol=1e-13)
    dx, dW, db = olin.linear_act_bwd(x, W, h, dy)
    assert torch.allclose(dx, xr.grad, atol=1e-12)
    assert torch.allclose(dW, Wr.grad, atol=1e-12) and torch.allclose(db, br.grad, atol=1e-12)


# ---------------------------------------------------------------- GPT (CPU baseline model)

def test_cpu_gpt_initial_loss_and_learning():
    torch.manual_seed(0)
    m = ogpt.GPT(vocab_size=256, seq_len=32, n_layer=2, n_head=2, d_model=64)
    opt = ogpt.make_optimizer(m, lr=3e-3)
    x = torch.randint(0, 256, (4, 32))
    y = torch.randint(0, 256, (4, 32))
    l0 = ogpt.cpu_train_step(m, opt, x, y)
    assert abs(l0 - math.log(256)) < 0.1      # N(0, 0.02) weights: near-uniform logits
    for _ in range(15):
        l1 = ogpt.cpu_train_step(m, opt, x, y)
    assert l1 < 0.9 * l0


def test_gather_windows_against_unfold_and_outside_zero():
    # in-range windows are the window-major unfold of X; a window leaving X is zeros
    from oracle.linear import gather
    X = torch.randn(30, 8, dtype=torch.float64)
    idx = torch.tensor([0, 26, 13, -1, 27, 5])
    Xg = gather(X, idx, 4 * 8)
    unf = X.unfold(0, 4, 1).transpose(1, 2).reshape(27, 32)   # (R - W + 1, W F)
    for b, st in enumerate(idx.tolist()):
        want = unf[st] if 0 <= st <= 26 else torch.zeros(32, dtype=torch.float64)
        assert torch.equal(Xg[b], want)
