"""fxlm.norm: fused RMSNorm (bf16 I/O, fp32 math) on gfx950.

y = x * rsqrt(mean(x^2) + eps) * w.  The forward stores rstd (fp32, one per
row); the backward produces dx and dw from a single pass over x and dy
(fx_rms_norm_bwd).  Surface and checks follow ml/fxlm/norm.py:30-90.  ``pre_norm``
returns the residual stream with the normed input so that the GPT block's two
gradients of x are summed inside that pass (fx_rms_norm_bwd_add).
"""
import torch

from fxgpu.abi import call, lib, ptr, stream_of


def _check(x, w):
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError(f"x and weight must be bfloat16 ({x.dtype}, {w.dtype})")
    if not (x.is_cuda and w.is_cuda):
        raise TypeError("x and weight must be cuda tensors")
    D = x.shape[-1]
    if w.shape != (D,):
        raise ValueError(f"weight must have shape ({D},), got {tuple(w.shape)}")
    if D % 8 != 0 or D > 8192:
        raise ValueError(f"D={D}: needs D % 8 == 0 and D <= 8192")
    if not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("x and weight must be contiguous")
    return D


def _al(t):
    """t itself when its data is 16-byte aligned (the kernels read 16-byte vectors), else
    an aligned copy: a contiguous view at an odd storage offset is accepted, as the
    reference accepts any contiguous tensor."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        D = _check(x, w)
        w = _al(w)
        N = x.numel() // D
        x2 = _al(x.view(N, D))
        y = torch.empty_like(x2)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        call("fx_rms_norm_fwd", ptr(x2), ptr(w), ptr(y), ptr(rstd), N, D, float(eps),
             stream_of(x))
        ctx.save_for_backward(x2, w, rstd)
        ctx.eps = eps
        ctx.oshape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd = ctx.saved_tensors
        dx, dw = _bwd_into(x2, dy, w, rstd)
        return dx.view(ctx.oshape), dw, None


def rms_norm(x, weight, eps=1e-6):
    """x (..., D) bf16, weight (D,) bf16 -> y (..., D) bf16."""
    return _RMSNorm.apply(x, weight, float(eps))


def _bwd_into(x2, dy, w, rstd, dres=None):
    """(dx, dw) of the norm for x2 (N, D); dx += dres in the same pass when given."""
    N, D = x2.shape
    dy2 = _al(dy.contiguous().view(N, D))
    if dy2.dtype != torch.bfloat16:
        dy2 = dy2.to(torch.bfloat16)
    dx = torch.empty_like(x2)
    dw32 = torch.empty(D, device=x2.device, dtype=torch.float32)
    dw = torch.empty(D, device=x2.device, dtype=w.dtype)
    work = torch.empty(max(1, lib().fx_rms_norm_bwd_workspace(N, D) // 4), device=x2.device,
                       dtype=torch.float32)
    if dres is None:
        call("fx_rms_norm_bwd", ptr(x2), ptr(dy2), ptr(w), ptr(rstd), ptr(dx), ptr(dw32),
             ptr(dw), ptr(work), N, D, stream_of(x2))
    else:
        r2 = _al(dres.contiguous().view(N, D))
        if r2.dtype != torch.bfloat16:
            r2 = r2.to(torch.bfloat16)
        call("fx_rms_norm_bwd_add", ptr(x2), ptr(dy2), ptr(r2), ptr(w), ptr(rstd), ptr(dx),
             ptr(dw32), ptr(dw), ptr(work), N, D, stream_of(x2))
    return dx, dw


class _PreNorm(torch.autograd.Function):
    """(x, rms_norm(x)) for a pre-norm residual block, whose input feeds both the norm
    and the residual sum: the backward gets both gradients and forms
    dx = dres + d(norm)/dx in the norm kernel's pass (fx_rms_norm_bwd_add) instead of the
    separate add autograd would run for ml/fxlm/model.py:69,71."""

    @staticmethod
    def forward(ctx, x, w, eps):
        D = _check(x, w)
        w = _al(w)
        N = x.numel() // D
        x2 = _al(x.view(N, D))
        y = torch.empty_like(x2)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        call("fx_rms_norm_fwd", ptr(x2), ptr(w), ptr(y), ptr(rstd), N, D, float(eps),
             stream_of(x))
        ctx.save_for_backward(x2, w, rstd)
        ctx.oshape = x.shape
        ctx.set_materialize_grads(False)
        return x, y.view(x.shape)

    @staticmethod
    def backward(ctx, dres, dy):
        x2, w, rstd = ctx.saved_tensors
        if dy is None:
            return dres, None, None
        dx, dw = _bwd_into(x2, dy, w, rstd, dres)
        return dx.view(ctx.oshape), dw, None


def pre_norm(x, weight, eps=1e-6):
    """(x, rms_norm(x, weight, eps)): the residual stream and the block's normed input,
    with the two gradients of x summed inside the norm's backward kernel."""
    return _PreNorm.apply(x, weight, float(eps))


class _AddPreNorm(torch.autograd.Function):
    """(s, rms_norm(s)) for s = x + r: the residual sum of ml/fxlm/model.py:69,71 done in
    the pass of the norm that reads it (fx_rms_norm_fwd_add; s, y and rstd are bit for
    bit those of the bf16 add followed by the norm).  Both inputs get the gradient of s,
    formed as in _PreNorm."""

    @staticmethod
    def forward(ctx, x, r, w, eps):
        D = _check(x, w)
        if r.shape != x.shape or r.dtype != x.dtype or not r.is_contiguous():
            raise ValueError(f"r must be a contiguous {tuple(x.shape)} {x.dtype} tensor")
        w, r = _al(w), _al(r)
        N = x.numel() // D
        x2 = _al(x.view(N, D))
        s = torch.empty_like(x2)
        y = torch.empty_like(x2)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        call("fx_rms_norm_fwd_add", ptr(x2), ptr(r), ptr(w), ptr(s), ptr(y), ptr(rstd), N, D, float(eps),
             stream_of(x))
        ctx.save_for_backward(s, w, rstd)
        ctx.oshape = x.shape
        ctx.set_materialize_grads(False)
        return s.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, ds, dy):
        s, w, rstd = ctx.saved_tensors
        if dy is None:
            return ds, ds, None, None
        dx, dw = _bwd_into(s, dy, w, rstd, ds)
        dx = dx.view(ctx.oshape)
        return dx, dx, dw, None


def add_pre_norm(x, r, weight, eps=1e-6):
    """(x + r, rms_norm(x + r, weight, eps)) in one pass over x and r; the backward is
    pre_norm's, with the gradient of the sum going to both x and r."""
    return _AddPreNorm.apply(x, r, weight, float(eps))


def rms_norm_fwd_stats(x, weight, eps=1e-6):
    """Forward only, returning (y, rstd): the fp32 per-row rstd for parity checks."""
    D = _check(x, weight)
    weight = _al(weight)
    N = x.numel() // D
    x2 = _al(x.view(N, D))
    y = torch.empty_like(x2)
    rstd = torch.empty(N, device=x.device, dtype=torch.float32)
    call("fx_rms_norm_fwd", ptr(x2), ptr(weight), ptr(y), ptr(rstd), N, D, float(eps),
         stream_of(x))
    return y.view(x.shape), rstd


def rms_norm_bwd_raw(x, dy, weight, rstd):
    """Backward only, returning (dx, dw_f32, dw_bf16) for parity checks."""
    D = _check(x, weight)
    weight = _al(weight)
    N = x.numel() // D
    x2, dy2 = _al(x.view(N, D)), _al(dy.contiguous().view(N, D))
    dx = torch.empty_like(x2)
    dw32 = torch.empty(D, device=x.device, dtype=torch.float32)
    dw = torch.empty(D, device=x.device, dtype=torch.bfloat16)
    work = torch.empty(max(1, lib().fx_rms_norm_bwd_workspace(N, D) // 4), device=x.device,
                       dtype=torch.float32)
    call("fx_rms_norm_bwd", ptr(x2), ptr(dy2), ptr(weight), ptr(rstd), ptr(dx), ptr(dw32),
         ptr(dw), ptr(work), N, D, stream_of(x))
    return dx.view(x.shape), dw32, dw
