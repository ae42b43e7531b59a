"""Oracle: fused (gather) linear layer (TEST INFRASTRUCTURE ONLY).

Restates ml/fxgpu/gather_gemm.hip:16-180 and ml/fxgpu/fused_linear.py:27-101:
  Xg[b, w*F + f] = X[idx[b] + w, f]      (window-major gather, K = W*F)
  out = Xg @ W^T + bias
  backward: dW = g^T Xg, db = sum_b g (no dX in the reference)
and the dense "fused-linear GELU" form the GPT MLP uses:
  h = x @ W^T (+ bias), y = gelu_tanh(h); dh = dy * gelu_tanh'(h),
  dx = dh @ W, dW = dh^T x, db = sum dh.
"""
import math

import torch


def gather(X, idx, K):
    """Xg (B, K) from X (R, F) and window starts idx (B,).  A window that leaves X
    (idx < 0 or idx + W > R) is all zeros: the reference does not range-check idx
    (ml/fxgpu/gather_gemm.hip:45-46 reads X[idx + w] unchecked), so this build defines
    that case and its kernels follow the definition."""
    Xf = X.detach().cpu()
    R, F = Xf.shape
    W = K // F
    st = idx.detach().cpu().long()
    ok = (st >= 0) & (st + W <= R)
    rows = torch.where(ok, st, 0)[:, None] + torch.arange(W)[None, :]     # (B, W)
    return (Xf[rows] * ok[:, None, None].to(Xf.dtype)).reshape(rows.shape[0], W * F)


def gather_linear(X, idx, weight, bias, dtype=torch.float64):
    Xg = gather(X, idx, weight.shape[1]).to(dtype)
    out = Xg @ weight.detach().to("cpu", dtype).t()
    if bias is not None:
        out = out + bias.detach().to("cpu", dtype)
    return out, Xg


def gelu_tanh(h):
    c = math.sqrt(2.0 / math.pi)
    return 0.5 * h * (1.0 + torch.tanh(c * (h + 0.044715 * h ** 3)))


def gelu_tanh_grad(h):
    c = math.sqrt(2.0 / math.pi)
    u = c * (h + 0.044715 * h ** 3)
    th = torch.tanh(u)
    return 0.5 * (1.0 + th) + 0.5 * h * (1.0 - th * th) * c * (1.0 + 3 * 0.044715 * h * h)


def linear_act_fwd(x, weight, bias=None, act="gelu_tanh", dtype=torch.float64):
    """Returns (y, h): h = x W^T + b, y = act(h)."""
    h = x.detach().to("cpu", dtype) @ weight.detach().to("cpu", dtype).t()
    if bias is not None:
        h = h + bias.detach().to("cpu", dtype)
    y = gelu_tanh(h) if act == "gelu_tanh" else h
    return y, h


def linear_act_bwd(x, weight, h, dy, act="gelu_tanh", dtype=torch.float64):
    """Returns (dx, dW, db) for y = act(x W^T + b)."""
    hf = h.detach().to("cpu", dtype)
    dh = dy.detach().to("cpu", dtype) * (gelu_tanh_grad(hf) if act == "gelu_tanh" else 1.0)
    xf = x.detach().to("cpu", dtype)
    wf = weight.detach().to("cpu", dtype)
    return dh @ wf, dh.t() @ xf, dh.sum(0)
