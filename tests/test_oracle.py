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
from oracle import embedding as oemb
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
    assert abs(loss.item() - ref.item()) < 1e-12
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
    assert abs(loss.item() - ref.item()) < 1e-12
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



def test_gelu_tanh_grad_matches_autograd_and_the_sigmoid_form():
    # the oracle's derivative against torch's autograd of F.gelu(approximate="tanh"), over
    # the range where it is not 0 or 1 to double precision, and the form the forward GEMM's
    # epilogue evaluates (fx_linear_fwd act 2): s = sigmoid(2u), gelu = h s,
    # gelu' = s (1 + h (1 - s) (2c + 6c 0.044715 h^2)), c = sqrt(2/pi)
    h = torch.linspace(-12.0, 12.0, 4801, dtype=f64, requires_grad=True)
    F.gelu(h, approximate="tanh").sum().backward()
    hd = h.detach()
    g = olin.gelu_tanh_grad(hd)
    assert torch.allclose(g, h.grad, rtol=0, atol=1e-13)
    c = math.sqrt(2.0 / math.pi)
    s = torch.sigmoid(2 * c * (hd + 0.044715 * hd ** 3))
    assert torch.allclose(hd * s, olin.gelu_tanh(hd), rtol=0, atol=1e-13)
    assert torch.allclose(s * (1 + hd * (1 - s) * (2 * c + 6 * c * 0.044715 * hd * hd)), g, rtol=0, atol=1e-12)
    # a dropped term is caught: without the h (1 - s) u' part the slope misses by up to 0.6
    assert float((s - g).abs().max()) > 0.1


# ---------------------------------------------------------------- GPT (CPU baseline model)

def _tiny_gpt(V=64, T=16, L=2, H=2, D=32, seed=0, dtype=f64):
    torch.manual_seed(seed)
    return ogpt.GPT(vocab_size=V, seq_len=T, n_layer=L, n_head=H, d_model=D).to(dtype)


def _rms(x, w, eps=1e-6):
    """RMSNorm from its definition: x / sqrt(mean(x^2) + eps) * w."""
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * w


def _gelu_tanh(u):
    """GELU with the tanh approximation, from its formula."""
    return 0.5 * u * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (u + 0.044715 * u ** 3)))


@pytest.mark.parametrize("V,T,L,H,D", [(256, 256, 4, 4, 256), (50304, 1024, 12, 12, 768)])
def test_cpu_gpt_param_count_closed_form(V, T, L, H, D):
    # tied head, no biases: V*D (embedding = head) + T*D (positions) + L*(2D norms +
    # 3D^2 qkv + D^2 proj + 4D^2 fc + 4D^2 fc2) + D (final norm); an untied head adds V*D
    with torch.device("meta"):
        m = ogpt.GPT(vocab_size=V, seq_len=T, n_layer=L, n_head=H, d_model=D)
    n = sum(p.numel() for p in m.parameters())
    assert n == V * D + T * D + L * (2 * D + 12 * D * D) + D
    if V == 50304:
        assert n == 124_373_760


def test_cpu_gpt_init_scales():
    # ml/fxlm/model.py:88-99: N(0, 0.02) everywhere, proj / fc2 at 0.02 / sqrt(2 L);
    # norm weights one, positions zero
    L = 4
    m = ogpt.GPT(vocab_size=512, seq_len=64, n_layer=L, n_head=4, d_model=256)
    small = 0.02 / math.sqrt(2 * L)
    for name, p in m.named_parameters():
        if name.endswith(("proj.weight", "fc2.weight")):
            want = small
        elif name.endswith(("qkv.weight", "fc.weight")) or name == "tok_emb.weight":
            want = 0.02
        elif name == "pos_emb":
            assert float(p.detach().abs().max()) == 0.0
            continue
        else:
            assert torch.equal(p, torch.ones_like(p)), name
            continue
        assert abs(p.detach().std().item() / want - 1) < 0.03, name
        assert abs(p.detach().mean().item()) < 0.1 * want, name


def test_cpu_gpt_block_from_definitions():
    # one block restated from its definitions: pre-norm, causal attention (the pinned
    # attention oracle), both residual sums, GELU-tanh MLP (ml/fxlm/model.py:58-72)
    m = _tiny_gpt(L=1)
    blk = m.blocks[0]
    for p in blk.parameters():
        torch.nn.init.normal_(p, std=0.3)
    x = torch.randn(3, 16, 32, dtype=f64)
    H, Dh = 2, 16
    h = _rms(x, blk.ln1_w)
    qkv = (h @ blk.qkv.weight.T).view(3, 16, 3, H, Dh)
    o, _ = oatt.attn_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], True, Dh ** -0.5)
    x1 = x + o.reshape(3, 16, 32) @ blk.proj.weight.T
    want = x1 + _gelu_tanh(_rms(x1, blk.ln2_w) @ blk.fc.weight.T) @ blk.fc2.weight.T
    with torch.no_grad():
        got = blk(x)
    assert torch.allclose(got, want, atol=1e-12, rtol=1e-12)


def test_cpu_gpt_zero_branches_are_identity():
    # with proj and fc2 at zero every block returns its input exactly, and the logits are
    # rms_norm(emb + pos) * lnf_w times the (tied) embedding
    m = _tiny_gpt()
    with torch.no_grad():
        for b in m.blocks:
            b.proj.weight.zero_()
            b.fc2.weight.zero_()
        torch.nn.init.normal_(m.pos_emb, std=0.5)
        torch.nn.init.normal_(m.lnf_w, mean=1.0, std=0.2)
        idx = torch.randint(0, 64, (2, 16))
        x = m.tok_emb(idx) + m.pos_emb[:16]
        for b in m.blocks:
            assert torch.equal(b(x), x)
        want = _rms(x, m.lnf_w) @ m.tok_emb.weight.T
        assert torch.allclose(m(idx), want, atol=1e-12, rtol=1e-12)


def test_cpu_gpt_is_causal():
    # changing the tokens after position t leaves the logits at positions <= t unchanged,
    # and changing the token at t changes the logits at t
    m = _tiny_gpt(L=2)
    idx = torch.randint(0, 64, (2, 16))
    with torch.no_grad():
        base = m(idx)
        for t in (0, 5, 14):
            alt = idx.clone()
            alt[:, t + 1:] = (alt[:, t + 1:] + 7) % 64
            out = m(alt)
            assert torch.allclose(out[:, :t + 1], base[:, :t + 1], atol=1e-12, rtol=0)
            if t + 1 < 16:
                assert not torch.allclose(out[:, t + 1], base[:, t + 1])
            alt2 = idx.clone()
            alt2[:, t] = (alt2[:, t] + 3) % 64
            assert not torch.allclose(m(alt2)[:, t], base[:, t])


def test_cpu_gpt_gradients_match_finite_differences():
    # fp64 gradcheck of the logits over every parameter of a tiny model (the loss path
    # casts the logits to fp32, as the reference does, so it is checked through them)
    m = _tiny_gpt(V=16, T=6, L=1, H=2, D=8, seed=3)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * 0.4 + (1.0 if p.dim() == 1 else 0.0))
    idx = torch.randint(0, 16, (2, 6))
    names = [n for n, _ in m.named_parameters()]
    params = tuple(p.detach().clone().requires_grad_() for p in m.parameters())

    def logits_of(*ps):
        return torch.func.functional_call(m, dict(zip(names, ps)), (idx,))

    assert torch.autograd.gradcheck(logits_of, params, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_cpu_gpt_matches_fxlm_torch_path():
    # the oracle and fxlm.model.GPT with the reference's torch comparator switches
    # (ml/fxlm/selftest.py:305-308) on one state_dict: equal fp32 loss and gradients
    from fxlm.model import GPT as FxGPT, GPTConfig
    cfg = GPTConfig(vocab_size=96, seq_len=24, n_layer=2, n_head=2, d_model=64,
                    attn_impl="sdpa", norm_impl="torch", ce_impl="torch", mlp_impl="torch",
                    linear_impl="torch")
    torch.manual_seed(11)
    fx = FxGPT(cfg)
    m = ogpt.GPT(vocab_size=96, seq_len=24, n_layer=2, n_head=2, d_model=64)
    m.load_state_dict(fx.state_dict())
    with torch.no_grad():
        for p in fx.parameters():       # larger branches than the init gives
            p.add_(torch.randn_like(p) * 0.05)
        m.load_state_dict(fx.state_dict())
    idx = torch.randint(0, 96, (3, 24))
    tgt = torch.randint(0, 96, (3, 24))
    l_fx, l_o = fx(idx, tgt), m(idx, tgt)
    l_fx.backward()
    l_o.backward()
    assert abs(l_fx.item() - l_o.item()) <= 1e-6 * abs(l_o.item())
    op = dict(m.named_parameters())
    for name, p in fx.named_parameters():
        r = op[name].grad
        assert torch.allclose(p.grad, r, atol=1e-6 * float(r.abs().max()) + 1e-9, rtol=1e-4), name


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


def test_cpu_optimizer_decays_matrices_only():
    # zero gradients: Adam's moments stay zero, so the step is exactly the decoupled weight
    # decay, p * (1 - lr wd) on >= 2-D parameters and nothing on the 1-D ones (norm weights,
    # the reference's wd groups, ml/bench/bench10_lm.py:92-99); decay on every parameter, or
    # on none, fails here
    torch.manual_seed(3)
    m = ogpt.GPT(vocab_size=64, seq_len=16, n_layer=2, n_head=2, d_model=32)
    lr, wd = 3e-3, 0.1
    opt = ogpt.make_optimizer(m, lr=lr, weight_decay=wd)
    before = {n: p.detach().clone() for n, p in m.named_parameters()}
    for p in m.parameters():
        p.grad = torch.zeros_like(p)
    opt.step()
    ndim1 = ndim2 = 0
    for n, p in m.named_parameters():
        if p.dim() >= 2:
            assert torch.equal(p.detach(), before[n] * (1 - lr * wd)), n
            ndim2 += 1
        else:
            assert torch.equal(p.detach(), before[n]), n
            ndim1 += 1
    assert ndim1 >= 5 and ndim2 >= 5     # both groups are populated


class _Bilinear(torch.nn.Module):
    """loss = sum(w * x) + sum(b * y): the gradients are exactly x and y."""

    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.full((4, 4), 0.5))
        self.b = torch.nn.Parameter(torch.full((4,), -0.25))

    def forward(self, x, y):
        return (self.w * x).sum() + (self.b * y).sum()


def test_cpu_train_step_clips_the_global_norm_to_one():
    # a gradient of norm 4 is clipped to norm 1 before AdamW sees it
    # (ml/bench/bench10_lm.py:104-111: clip_grad_norm_(1.0) then step): two steps, the first
    # of norm 4 and the second of norm 1/2 (left alone), end where the same steps with the
    # first gradient scaled to norm 1 end.  Unclipped, Adam's moments weigh the two steps
    # differently and the parameters end elsewhere.
    g = torch.Generator().manual_seed(8)
    x1, y1 = torch.randn(4, 4, generator=g), torch.randn(4, generator=g)
    n1 = math.sqrt(float((x1 ** 2).sum() + (y1 ** 2).sum()))
    x1, y1 = x1 * (4 / n1), y1 * (4 / n1)
    x2, y2 = torch.randn(4, 4, generator=g), torch.randn(4, generator=g)
    n2 = math.sqrt(float((x2 ** 2).sum() + (y2 ** 2).sum()))
    x2, y2 = x2 * (0.5 / n2), y2 * (0.5 / n2)

    def run(steps, clip):
        mod = _Bilinear()
        opt = ogpt.make_optimizer(mod, lr=1e-2, weight_decay=0.1)
        for x, y in steps:
            ogpt.cpu_train_step(mod, opt, x, y, clip=clip)
        return torch.cat([mod.w.detach().reshape(-1), mod.b.detach()])

    clipped = run([(x1, y1), (x2, y2)], 1.0)
    prescaled = run([(x1 / 4, y1 / 4), (x2, y2)], 1.0)
    unclipped = run([(x1, y1), (x2, y2)], 1e9)
    assert torch.allclose(clipped, prescaled, rtol=1e-5, atol=1e-7)
    assert float((unclipped - prescaled).abs().max()) > 1e-4


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


# -- token embedding gradient -------------------------------------------------------------

def test_embedding_grad_matches_torch_autograd():
    g = torch.Generator().manual_seed(11)
    V, D = 37, 24
    idx = torch.randint(0, V, (5, 29), generator=g)
    dy = torch.randn(5, 29, D, generator=g, dtype=torch.float64)
    w = torch.zeros(V, D, dtype=torch.float64, requires_grad=True)
    F.embedding(idx, w).backward(dy)
    assert torch.allclose(oemb.embedding_grad(idx, dy, V), w.grad, rtol=0, atol=1e-12)


def test_embedding_grad_special_cases():
    V, D = 6, 8
    dy = torch.arange(4 * D, dtype=torch.float64).reshape(4, D)
    # ids outside [0, V) add nothing; unused ids are zero rows; a single position is its row
    idx = torch.tensor([2, -1, 6, 2])
    got = oemb.embedding_grad(idx, dy, V)
    assert torch.equal(got[2], dy[0] + dy[3])
    assert torch.count_nonzero(got[[0, 1, 3, 4, 5]]) == 0
    one = oemb.embedding_grad(torch.tensor([4]), dy[1:2], V)
    assert torch.equal(one[4], dy[1])


def test_embedding_grad_seq_is_the_position_ordered_fp32_sum():
    g = torch.Generator().manual_seed(12)
    V, D, n = 9, 16, 300
    idx = torch.randint(-2, V, (n,), generator=g)
    dy = torch.randn(n, D, generator=g).bfloat16()
    seq = oemb.embedding_grad_seq(idx, dy, V)
    exact = oemb.embedding_grad(idx, dy, V)
    # within one bf16 rounding plus the fp32 accumulation of up to n terms
    bound = 2.0 ** -8 * exact.abs() + n * 2.0 ** -24 * oemb.embedding_grad(idx, dy.abs(), V) + 1e-30
    assert bool(((seq.double() - exact).abs() <= bound).all())
    # where every id's run is one whole segment (32 positions each, ids in any position
    # order), the result is the plain position-ordered fp32 sum
    perm = torch.randperm(32 * 5, generator=g)
    idx5 = (torch.arange(32 * 5) // 32)[perm]
    dy5 = torch.randn(32 * 5, D, generator=g).bfloat16()
    acc = torch.zeros(5, D, dtype=torch.float32)
    for t in range(32 * 5):
        acc[int(idx5[t])] += dy5[t].float()
    assert torch.equal(oemb.embedding_grad_seq(idx5, dy5, 5), acc.bfloat16())


def _big_small(n, at_one, lead=0):
    """n rows of id 1 after `lead` rows of id 0: 2^24 at id 1's first row, 1 at its row
    `at_one`, -2^24 right after, zeros elsewhere (column 0; the other columns zero)."""
    dy = torch.zeros(lead + n, 8).bfloat16()
    dy[lead, 0] = 2.0 ** 24
    dy[lead + at_one, 0] = 1.0
    dy[lead + at_one + 1, 0] = -(2.0 ** 24)
    idx = torch.tensor([0] * lead + [1] * n)
    return idx, dy


def test_embedding_grad_seq_cuts_runs_at_global_32_slot_segments():
    # 2^24 + 1 rounds back to 2^24 in fp32, so whether the 1 meets 2^24 or -2^24 first
    # decides between a sum of 0 and the exact 1
    # the 1 in the first segment (slot 31): 2^24 + 1 -> 2^24, then -2^24 in the next: 0
    idx, dy = _big_small(64, 31)
    assert float(oemb.embedding_grad_seq(idx, dy, 2)[1, 0]) == 0.0
    # the 1 opens the second segment (slot 32): 1 - 2^24 is exact there, and 2^24 plus that
    # is 1; a position-ordered sum over the whole run would give 0
    idx, dy = _big_small(64, 32)
    assert float(oemb.embedding_grad_seq(idx, dy, 2)[1, 0]) == 1.0
    assert float(oemb.embedding_grad(idx, dy, 2)[1, 0]) == 1.0
    # segments are counted in global slots: after 20 slots of id 0, id 1's 13th row (index 12)
    # is slot 32; cutting at id 1's own 32nd row instead would give 0
    idx, dy = _big_small(40, 12, lead=20)
    assert float(oemb.embedding_grad_seq(idx, dy, 2)[1, 0]) == 1.0
    idx, dy = _big_small(40, 11, lead=20)
    assert float(oemb.embedding_grad_seq(idx, dy, 2)[1, 0]) == 0.0
    # ids outside [0, V) take no slot: 20 of them in front change nothing
    idx, dy = _big_small(64, 32)
    idx = torch.cat([torch.full((20,), -5), idx])
    dy = torch.cat([torch.ones(20, 8).bfloat16(), dy])
    assert float(oemb.embedding_grad_seq(idx, dy, 2)[1, 0]) == 1.0