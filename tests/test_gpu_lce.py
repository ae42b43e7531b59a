"""Fused linear cross-entropy (fx_lce_fwd / fx_lce_grad): the head GEMM with the online CE
in its epilogue, against the oracle's CE of the bf16-rounded logits, and the fused paths of
fxlm.cross_entropy.linear_cross_entropy against the unfused chunk loop."""
import pytest
import torch
import torch.nn.functional as F

from oracle import cross_entropy as oce
from tolerances import RTOL_LOSS

pytestmark = pytest.mark.gpu

# (M, D, V): ragged row counts (the last 256-row tile partly past M), V on 192- and
# 256-column tiles, D from the smallest K the kernels take up to the GPT's; D = 160 and 224
# are odd counts of 32-wide K steps (the loop's leading step of zeros)
SHAPES = [(1, 128, 768), (300, 128, 768), (512, 256, 1536), (777, 128, 1024), (256, 768, 2304), (1000, 384, 4608),
          (300, 160, 768), (512, 224, 1536)]


def _inputs(M, D, V, dev, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).bfloat16()
    w = (torch.randn(V, D, generator=g) * 0.05).bfloat16()
    tg = torch.randint(0, V, (M,), generator=g)
    tg[::7] = -100
    if M > 3:
        tg[3] = V + 5       # out of range: no loss, zero gradient row (ml/fxlm/kernels/ce.hip:43)
        tg[2] = -3
    return x, w, tg, x.to(dev), w.to(dev), tg.to(dev)


def _ref_logits(x, w):
    # the logits as the unfused path stores them: an fp32-exact product rounded to bf16
    return (x.double() @ w.double().t()).bfloat16().double()


def _lce_fwd(xd, wd, td, ignore=-100):
    from fxlm.cross_entropy import _lce_fwd
    row_loss = torch.empty(xd.shape[0], device=xd.device, dtype=torch.float32)
    stat = _lce_fwd(xd, wd, td, ignore, row_loss)
    return row_loss, stat


@pytest.mark.parametrize("M,D,V", SHAPES)
def test_fwd_against_oracle(dev, M, D, V):
    x, w, tg, xd, wd, td = _inputs(M, D, V, dev, M + D + V)
    row_loss, stat = _lce_fwd(xd, wd, td)
    torch.cuda.synchronize()
    lg = _ref_logits(x, w)
    rl, _ = oce.ce_rows(lg, tg, 1.0)
    valid = (tg != -100) & (tg >= 0) & (tg < V)
    # fp32 row losses: 1e-3 relative (a logit rounded to the other bf16 neighbour moves a
    # row's loss by at most its half ulp, ~2e-4 relative here)
    rlc = row_loss.double().cpu()
    assert bool(((rlc - rl).abs() <= RTOL_LOSS * rl.abs() + 1e-6).all()), float((rlc - rl).abs().max())
    assert bool((rlc[~valid] == 0).all())
    # (M, Z) per row: the max exactly (a bf16 value), Z to fp32 accumulation
    m_ref = lg.max(dim=1).values
    z_ref = torch.exp(lg - m_ref[:, None]).sum(dim=1)
    st = stat.double().cpu()
    assert torch.equal(st[:, 0], m_ref) or float((st[:, 0] - m_ref).abs().max()) <= 2.0 ** -8 * float(m_ref.abs().max())
    assert float(((st[:, 1] - z_ref) / z_ref).abs().max()) <= 1e-4


@pytest.mark.parametrize("M,D,V", SHAPES)
@pytest.mark.parametrize("mul", [1.0, 3.0e-3])
def test_grad_against_oracle(dev, M, D, V, mul):
    from fxlm.cross_entropy import _lce_grad
    x, w, tg, xd, wd, td = _inputs(M, D, V, dev, 3 * M + V)
    _, stat = _lce_fwd(xd, wd, td)
    dl = torch.full((M, V + 8), 7.0, device=dev, dtype=torch.bfloat16)[:, :V]   # row stride V + 8
    _lce_grad(xd, wd, td, -100, stat, torch.tensor(mul, device=dev), dl)
    torch.cuda.synchronize()
    _, rdl = oce.ce_rows(_ref_logits(x, w), tg, mul)
    o = dl.double().cpu()
    # bf16 results: half an ulp of each value, plus 2e-3 of the largest for a logit rounded
    # to the other neighbour or a different fp32 summation order of Z
    tol = 2.0 ** -8 * rdl.abs() + 2e-3 * float(rdl.abs().max()) + 1e-12
    assert bool(((o - rdl).abs() <= tol).all()), float(((o - rdl).abs() - tol).max())
    valid = (tg != -100) & (tg >= 0) & (tg < V)
    assert bool((o[~valid] == 0).all())
    # each valid row of softmax - onehot sums to 0 (times mul)
    if bool(valid.any()):
        assert float(o[valid].sum(dim=1).abs().max()) <= 2e-2 * mul


def test_ignore_index_other_than_default(dev):
    x, w, tg, xd, wd, td = _inputs(300, 128, 768, dev, 11)
    tg2 = tg.clone()
    tg2[tg2 == -100] = 5      # 5 is now the ignored class
    row_loss, _ = _lce_fwd(xd, wd, tg2.to(dev), ignore=5)
    rl, _ = oce.ce_rows(_ref_logits(x, w), tg2, 1.0, ignore_index=5)
    assert float((row_loss.double().cpu() - rl).abs().max()) <= RTOL_LOSS * float(rl.abs().max())


def test_unsupported_shapes_fall_back(dev):
    # V not a multiple of 192 or 256, or D below 128: the workspace query says no and
    # linear_cross_entropy runs the unfused loop
    from fxgpu.abi import lib
    from fxlm.cross_entropy import _lce_fused_ok, linear_cross_entropy
    assert int(lib().fx_lce_workspace(100, 1000, 128)) == 0
    assert int(lib().fx_lce_workspace(100, 768, 64)) == 0
    assert int(lib().fx_lce_workspace(100, 768, 128)) > 0
    x = torch.randn(50, 64, device=dev).bfloat16()
    w = (torch.randn(1000, 64, device=dev) * 0.05).bfloat16()
    assert not _lce_fused_ok(x, w)
    tg = torch.randint(0, 1000, (50,), device=dev)
    with torch.no_grad():
        loss = linear_cross_entropy(x, w, tg)
    ref = F.cross_entropy(x.float() @ w.float().t(), tg)
    assert abs(loss.item() - float(ref)) <= RTOL_LOSS * abs(float(ref))


def _run(x0, w0, tg, grad, fused_loss, fused_train, chunk_rows=None, grad_scale=1.0):
    import fxlm.cross_entropy as ce
    old = ce.FUSED_LINEAR_CE_LOSS, ce.FUSED_LINEAR_CE_TRAIN
    ce.FUSED_LINEAR_CE_LOSS, ce.FUSED_LINEAR_CE_TRAIN = fused_loss, fused_train
    try:
        if not grad:
            with torch.no_grad():
                return float(ce.linear_cross_entropy(x0, w0, tg, chunk_rows=chunk_rows)), None, None
        x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
        loss = ce.linear_cross_entropy(x, w, tg, grad_scale=grad_scale, chunk_rows=chunk_rows)
        loss.backward()
        return loss.item(), x.grad, w.grad
    finally:
        ce.FUSED_LINEAR_CE_LOSS, ce.FUSED_LINEAR_CE_TRAIN = old


@pytest.mark.parametrize("N,D,V,chunk", [(1000, 128, 1536, None), (777, 256, 2304, 256), (512, 128, 1024, 100)])
def test_fused_paths_match_unfused(dev, N, D, V, chunk):
    x, w, tg, x0, w0, td = _inputs(N, D, V, dev, N * 7 + V)
    lu, gxu, gwu = _run(x0, w0, td, True, False, False, chunk, grad_scale=256.0)
    lf, gxf, gwf = _run(x0, w0, td, True, False, True, chunk, grad_scale=256.0)
    # the same rounded logits and the same (M, Z) rule: equal losses up to summation order
    assert abs(lf - lu) <= 1e-5 * abs(lu)
    for a, b in ((gxf, gxu), (gwf, gwu)):
        d = (a.double() - b.double()).abs()
        assert float(d.max()) <= 2.0 ** -8 * float(b.double().abs().max()) + 1e-9
    l0, _, _ = _run(x0, w0, td, False, False, False, chunk)
    l1, _, _ = _run(x0, w0, td, False, True, False, chunk)
    assert abs(l1 - l0) <= 1e-5 * abs(l0)
    # the targets include out-of-range values (no loss, but counted in n_valid): the CPU
    # oracle's loss, not torch's F.cross_entropy, which indexes the row by the target
    ref, _, _ = oce.linear_cross_entropy(x, w, tg)
    assert abs(l1 - float(ref)) <= RTOL_LOSS * abs(float(ref))


def test_cfg5_head_fused(dev):
    # the 12-layer model's head, x (16384, 768), tied W (50304, 768): the loss-only path
    # (one fused pass over all rows) and the fused training path against fp32 torch math,
    # and the fused dx / dW against the unfused chunk loop's
    N, D, V = 16384, 768, 50304
    g = torch.Generator(device=dev).manual_seed(56)
    x0 = torch.randn(N, D, device=dev, generator=g).bfloat16()
    w0 = (torch.randn(V, D, device=dev, generator=g) * 0.02).bfloat16()
    tg = torch.randint(0, V, (N,), device=dev, generator=g)
    tg[torch.rand(N, device=dev, generator=g) < 0.05] = -100
    ref = float(F.cross_entropy(x0.float() @ w0.float().t(), tg, ignore_index=-100))
    l_eval, _, _ = _run(x0, w0, tg, False, True, False)
    assert abs(l_eval - ref) <= RTOL_LOSS * abs(ref)
    lf, gxf, gwf = _run(x0, w0, tg, True, True, True, grad_scale=1024.0)
    assert abs(lf - ref) <= RTOL_LOSS * abs(ref)
    lu, gxu, gwu = _run(x0, w0, tg, True, True, False, grad_scale=1024.0)
    assert abs(lf - lu) <= 1e-5 * abs(lu)
    for a, b in ((gxf, gxu), (gwf, gwu)):
        d = (a.float() - b.float()).abs()
        assert float(d.max()) <= 2.0 ** -8 * float(b.float().abs().max()) + 1e-9
