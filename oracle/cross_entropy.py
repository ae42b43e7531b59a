"""Oracle: fused softmax cross-entropy and linear cross-entropy (TEST INFRASTRUCTURE ONLY).

Restates ml/fxlm/kernels/ce.hip:32-116 and ml/fxlm/cross_entropy.py:
  n_valid   (:41-44)   count(target != ignore_index); inv_n = 1/n_valid or 0
  per row   (ce.hip)   valid = t != ignore && 0 <= t < V (ce.hip:43);
                       loss_r = logsumexp(x_r) - x_r[t]; grad_r = (softmax - onehot) * mul,
                       zero rows for invalid targets
  loss                 sum_r loss_r * inv_n (0 when nothing is valid)
  linear CE (:107-149) logits = x W^T; dl = grad with mul = inv_n * grad_scale;
                       dx = dl W, dW = dl^T x (fp32); backward scales both by g/grad_scale
"""
import torch


def inv_nvalid(target, ignore_index=-100):
    nv = int((target.detach().cpu() != ignore_index).sum())
    return 0.0 if nv == 0 else 1.0 / nv


def ce_rows(logits, target, mul, ignore_index=-100, dtype=torch.float64):
    """Returns (row_loss (N,), grad (N,V)) in `dtype`; grad scaled by mul."""
    x = logits.detach().to("cpu", dtype)
    t = target.detach().cpu()
    N, V = x.shape
    valid = (t != ignore_index) & (t >= 0) & (t < V)
    lse = torch.logsumexp(x, -1)
    tc = t.clamp(0, V - 1)
    xt = x.gather(1, tc[:, None]).squeeze(1)
    row_loss = torch.where(valid, lse - xt, torch.zeros_like(lse))
    p = torch.softmax(x, -1)
    p[torch.arange(N), tc] -= 1.0
    grad = torch.where(valid[:, None], p * mul, torch.zeros_like(p))
    return row_loss, grad


def fused_cross_entropy(logits, target, ignore_index=-100, dtype=torch.float64):
    """Returns (loss scalar, dlogits (N,V)) for mean CE over valid rows."""
    inv_n = inv_nvalid(target, ignore_index)
    row_loss, grad = ce_rows(logits, target, inv_n, ignore_index, dtype)
    return row_loss.sum() * inv_n, grad


def linear_cross_entropy(x, weight, target, grad_scale=1.0, ignore_index=-100,
                         dtype=torch.float64):
    """Returns (loss, dx (N,D), dW (V,D)): the gradients of the mean loss."""
    xf = x.detach().to("cpu", dtype)
    wf = weight.detach().to("cpu", dtype)
    logits = xf @ wf.t()
    inv_n = inv_nvalid(target, ignore_index)
    row_loss, dl = ce_rows(logits, target, inv_n, ignore_index, dtype)
    # the kernel path multiplies by grad_scale and the backward divides it back out
    return row_loss.sum() * inv_n, dl @ wf, dl.t() @ xf
