"""Oracle: RMSNorm forward and backward (TEST INFRASTRUCTURE ONLY).

Restates ml/fxlm/kernels/norm.hip:
  forward  (:32-59)   rstd = rsqrt(mean(x^2) + eps) per row; y = x * rstd * w
  dx       (:63-95)   dx = rstd*w*dy - x * (rstd^3 * sum(x*w*dy) / D)
  dw       (:100-127) dw = sum over rows of x * rstd * dy (fp32, cast to w's dtype
                      by ml/fxlm/norm.py:84)
"""
import torch


def rms_norm_fwd(x, w, eps=1e-6, dtype=torch.float64):
    """Returns (y, rstd) for x (..., D): y (..., D), rstd (N,) in `dtype`."""
    D = x.shape[-1]
    xf = x.detach().to("cpu", dtype).reshape(-1, D)
    wf = w.detach().to("cpu", dtype)
    rstd = torch.rsqrt((xf * xf).mean(-1) + eps)
    y = xf * rstd[:, None] * wf
    return y.reshape(x.shape), rstd


def rms_norm_bwd(x, dy, w, rstd, dtype=torch.float64):
    """Returns (dx (..., D), dw (D,)) in `dtype`."""
    D = x.shape[-1]
    xf = x.detach().to("cpu", dtype).reshape(-1, D)
    dyf = dy.detach().to("cpu", dtype).reshape(-1, D)
    wf = w.detach().to("cpu", dtype)
    r = rstd.detach().to("cpu", dtype)[:, None]
    t = (xf * wf * dyf).sum(-1, keepdim=True)
    dx = r * wf * dyf - xf * (r ** 3 * t / D)
    dw = (xf * r * dyf).sum(0)
    return dx.reshape(x.shape), dw
