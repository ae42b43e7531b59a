"""fxlm.cross_entropy: fused softmax cross-entropy and linear cross-entropy (gfx950).

Surface of ml/fxlm/cross_entropy.py:41-199 with bf16 logits:

* ``fused_cross_entropy(logits, target, ignore_index=-100)``: mean CE over the
  valid rows; the forward kernel also writes dlogits = (softmax - onehot)/n_valid
  (one read and one write of the logits), the backward rescales them by the
  incoming gradient only when it is not 1.
* ``linear_cross_entropy(x, weight, target, grad_scale=1.0, ...)``: CE(x W^T)
  whose backward is computed inside the forward, chunk by chunk; each chunk's
  logits are overwritten in place by their gradient.  Heads whose shape the fused
  kernels take (V % 256 or % 192 == 0, D % 32 == 0, D >= 128) can instead form the
  logits only in MFMA accumulators (fx_lce_fwd: the GEMM with the online
  (max, sum exp) reduction in its epilogue, then fx_lce_grad: the GEMM again with the
  dlogits in its epilogue): always for the loss-only path (FUSED_LINEAR_CE_LOSS), and
  for training with FUSED_LINEAR_CE_TRAIN.

n_valid counts targets != ignore_index (out-of-range targets count, but their
rows get no loss and no gradient); n_valid == 0 gives loss 0 (reference
behaviour, ml/fxlm/cross_entropy.py:41-44 and ml/fxlm/kernels/ce.hip:43).
"""
import ctypes

import torch

from fxgpu.abi import call, fxCEArgs, lib, ptr, stream_of
from fxgpu.fused_linear import linear_wgrad

# rows per linear-CE chunk: bound the chunk's bf16 logits to this many bytes
_CHUNK_BYTES = 2 << 30


def _inv_nvalid(target, ignore_index, grad_scale=None):
    """(inv_n, mul) device scalars: inv_n = 1/n_valid (0 if none), mul = inv_n*grad_scale."""
    dev = target.device
    inv_n = torch.empty((), device=dev, dtype=torch.float32)
    mul = torch.empty((), device=dev, dtype=torch.float32)
    gs_ptr, gs_val = None, 1.0
    if torch.is_tensor(grad_scale):
        gs_t = grad_scale.detach().to(device=dev, dtype=torch.float32).reshape(())
        gs_ptr = ptr(gs_t)
    elif grad_scale is not None:
        gs_val = float(grad_scale)
    call("fx_ce_inv_nvalid", ptr(target), target.numel(), int(ignore_index), gs_ptr,
         float(gs_val), ptr(inv_n), ptr(mul), stream_of(target))
    return inv_n, mul


def _ce_rows(logits, target, grad, row_loss, mul, ignore_index):
    """One launch over the rows of (C, V) logits: per-row loss and, if grad, dlogits."""
    N, V = logits.shape
    a = fxCEArgs()
    a.logits = logits.data_ptr()
    a.target = target.data_ptr()
    a.grad = grad.data_ptr() if grad is not None else None
    a.row_loss = row_loss.data_ptr()
    a.mul = mul.data_ptr()
    a.N, a.V = N, V
    a.ld = logits.stride(0)
    a.ldg = grad.stride(0) if grad is not None else V
    a.ignore_index = int(ignore_index)
    call("fx_ce_fwd_grad", ctypes.byref(a), stream_of(logits))


def _finalize(row_loss, inv_n):
    loss = torch.empty((), device=row_loss.device, dtype=torch.float32)
    call("fx_ce_loss_finalize", ptr(row_loss), row_loss.numel(), ptr(inv_n), ptr(loss),
         stream_of(row_loss))
    return loss


# Fused linear-CE head (fx_lce_fwd / fx_lce_grad), where fx_lce_workspace takes the shape.
# FUSED_LINEAR_CE_LOSS: the no-grad (loss-only) path, which then allocates no logits at all.
# FUSED_LINEAR_CE_TRAIN: the training path; its chunk still holds the bf16 dlogits (the
# dx / dW products read them), and the logits GEMM runs twice (loss pass, gradient pass)
# where the unfused loop runs it once and streams the stored logits through
# fx_ce_fwd_grad, so on MI355X it is the slower of the two at the cfg5 head.
FUSED_LINEAR_CE_LOSS = True
FUSED_LINEAR_CE_TRAIN = False
# True: the head's weight gradient lg^T x on this build's weight-gradient GEMM
# (fx_linear_wgrad: 256 x 192 tiles, a partial last row panel at V = 50304, the 20 tiles past
# three full rounds split over the tokens): at the cfg5 head 1017 us against 1283 us for
# torch.mm (hipBLASLt).  False: torch.mm.
NATIVE_HEAD_WGRAD = True


def _lce_fused_ok(x, weight):
    """True when the fused linear-CE kernels take x (N, D) and weight (V, D)."""
    N, D = x.shape
    V = weight.shape[0]
    return (x.is_cuda and N > 0 and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
            and weight.is_contiguous() and weight.data_ptr() % 16 == 0
            and int(lib().fx_lce_workspace(N, V, D)) > 0)


def _lce_fwd(xc, weight, tc, ignore_index, row_loss):
    """Loss pass of the fused head over the rows of xc: row_loss, and the per-row
    (max, sum exp) pairs the gradient pass needs, as a (C, 2) fp32 tensor."""
    C, D = xc.shape
    V = weight.shape[0]
    nbytes = int(lib().fx_lce_workspace(C, V, D))
    work = torch.empty((nbytes + 3) // 4, device=xc.device, dtype=torch.float32)
    stat = torch.empty(C, 2, device=xc.device, dtype=torch.float32)
    call("fx_lce_fwd", ptr(xc), xc.stride(0), ptr(weight), ptr(tc), int(ignore_index), ptr(work), ptr(stat),
         ptr(row_loss), C, V, D, stream_of(xc))
    return stat


def _lce_grad(xc, weight, tc, ignore_index, stat, mul, dl):
    """Gradient pass of the fused head: dl (C, V) bf16 = the chunk's dlogits times mul."""
    C, D = xc.shape
    V = weight.shape[0]
    call("fx_lce_grad", ptr(xc), xc.stride(0), ptr(weight), ptr(tc), int(ignore_index), ptr(stat), ptr(mul),
         ptr(dl), dl.stride(0), C, V, D, stream_of(xc))


def _check_logits(logits, target):
    if logits.dtype != torch.bfloat16:
        raise TypeError(f"logits must be bfloat16, got {logits.dtype}")
    if not (logits.is_cuda and target.is_cuda):
        raise TypeError("logits and target must be cuda tensors")
    if not logits.is_contiguous() or not target.is_contiguous():
        raise ValueError("logits and target must be contiguous")
    if target.dtype != torch.int64:
        raise TypeError(f"target must be int64, got {target.dtype}")
    if logits.dim() != 2 or target.dim() != 1 or target.shape[0] != logits.shape[0]:
        raise ValueError(f"expected logits (N,V) and target (N,): "
                         f"{tuple(logits.shape)} vs {tuple(target.shape)}")


class _FusedCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, target, ignore_index):
        _check_logits(logits, target)
        N, V = logits.shape
        dev = logits.device
        inv_n, mul = _inv_nvalid(target, ignore_index)
        row_loss = torch.empty(N, device=dev, dtype=torch.float32)
        grad = None
        if ctx.needs_input_grad[0]:
            grad = torch.empty(N, V, device=dev, dtype=torch.bfloat16)
        _ce_rows(logits, target, grad, row_loss, mul, ignore_index)
        ctx.save_for_backward(grad)
        # the first backward's kernel takes the multiplier in grad as written to be 1
        # (src -1) and stores its g in applied[1]
        ctx.applied = torch.empty(2, device=dev, dtype=torch.float32)
        ctx.calls = 0
        return _finalize(row_loss, inv_n)

    @staticmethod
    def backward(ctx, g):
        (grad,) = ctx.saved_tensors
        g32 = g.detach().to(torch.float32).reshape(()).contiguous()
        ctx.calls += 1
        if ctx.calls == 1:
            # the usual single backward: scale the saved dlogits in place (no pass at all
            # when g == 1) and hand them over
            call("fx_ce_scale_grad", ptr(grad), grad.numel(), ptr(g32), ptr(ctx.applied), -1,
                 stream_of(grad))
            return grad, None, None
        # a further backward through a retained graph: a fresh tensor, so the gradient the
        # first backward returned stays as it was
        prev = float(ctx.applied[1])
        if prev == 0.0:
            raise RuntimeError("fused_cross_entropy: the first backward of this graph had an "
                               "incoming gradient of 0, which zeroed the saved dlogits; run the "
                               "forward again")
        return (grad.float() * (g32 / prev)).to(torch.bfloat16), None, None


def fused_cross_entropy(logits, target, ignore_index=-100):
    """logits (N,V) bf16, target (N,) int64 -> fp32 scalar: mean CE over valid rows."""
    return _FusedCE.apply(logits, target, int(ignore_index))


def _auto_chunk(D, V):
    """Rows per chunk so that one chunk's bf16 logits stay within _CHUNK_BYTES.

    The reference sizes chunks for a shared-memory iGPU: at most 4096 rows and
    2.5e10 / (D V) (ml/fxlm/cross_entropy.py:102-104; 512 rows at D 768, V 50304).
    With 288 GB of HBM the limit here is 2 GiB of logits (21,248 rows at V 50304), so
    the 16,384-row batch of the 12-layer model is one chunk: 1.65 GB of logits, three
    large GEMMs, and one pass over the fp32 (V, D) weight-gradient accumulator instead
    of 32 passes (154 MB each) at the reference's chunking."""
    c = (_CHUNK_BYTES // (2 * max(1, V))) // 256 * 256
    return max(256, c)


# the backward's scaling in one kernel (fx_ce_lin_grad_scale); False: the torch ops
_FUSED_LIN_GRAD_SCALE = True


class _LinearCE(torch.autograd.Function):
    """loss = CE(x @ W.T, target); the (N, V) logits never exist beyond one chunk."""

    @staticmethod
    def forward(ctx, x, weight, target, grad_scale, ignore_index, chunk_rows):
        N, D, V = _check_lin(x, weight, target)
        dev = x.device
        if chunk_rows is None:
            chunk_rows = _auto_chunk(D, V)
        inv_n, mul = _inv_nvalid(target, ignore_index, grad_scale)
        row_loss = torch.empty(N, device=dev, dtype=torch.float32)
        dx = torch.empty(N, D, device=dev, dtype=torch.bfloat16)
        dW = None
        fused = FUSED_LINEAR_CE_TRAIN and _lce_fused_ok(x, weight)
        dl_buf = torch.empty(min(chunk_rows, N), V, device=dev, dtype=torch.bfloat16) if fused else None
        for r0 in range(0, N, chunk_rows):
            r1 = min(r0 + chunk_rows, N)
            xc = x[r0:r1]
            if fused:   # the logits only in MFMA accumulators: loss pass, then gradient pass
                stat = _lce_fwd(xc, weight, target[r0:r1], ignore_index, row_loss[r0:r1])
                lg = dl_buf[:r1 - r0]
                _lce_grad(xc, weight, target[r0:r1], ignore_index, stat, mul, lg)
            else:
                lg = torch.mm(xc, weight.t())                   # (C, V) bf16
                _ce_rows(lg, target[r0:r1], lg, row_loss[r0:r1], mul, ignore_index)  # in place
            torch.mm(lg, weight, out=dx[r0:r1])                 # dx_c
            # the reference's dW.add_(torch.mm(dl.t(), xc).float()): a bf16 product,
            # accumulated over the chunks in fp32 (ml/fxlm/cross_entropy.py:135); a single
            # chunk's product stays bf16 (exact in fp32) and the backward reads it as such
            part = linear_wgrad(lg, xc) if NATIVE_HEAD_WGRAD else torch.mm(lg.t(), xc)  # (V, D) bf16
            if dW is None:
                dW = part if r1 >= N else part.float()
            else:
                dW.add_(part)
            del lg
        if dW is None:
            dW = torch.zeros(V, D, device=dev, dtype=torch.float32)
        ctx.save_for_backward(dx, dW)
        ctx.grad_scale = grad_scale
        ctx.wdtype = weight.dtype
        ctx.calls = 0
        return _finalize(row_loss, inv_n)

    @staticmethod
    def backward(ctx, g):
        dx, dW = ctx.saved_tensors
        gs = ctx.grad_scale
        ctx.calls += 1
        if _FUSED_LIN_GRAD_SCALE and ctx.wdtype == torch.bfloat16 and dx.dtype == torch.bfloat16:
            # one pass: the same fp32 reciprocal, products and bf16 rounding as below
            g32 = g.detach().float().reshape(()).contiguous()
            gs_t = gs.detach().float().reshape(()).contiguous() if torch.is_tensor(gs) else None
            inv_value = 0.0 if gs_t is not None else 1.0 / gs
            if dW.dtype == torch.bfloat16 and ctx.calls == 1:
                # the usual single backward (one chunk, so dW is the bf16 product): scale the
                # saved gradients in place and hand them over; in the training step the
                # factor g / grad_scale is exactly 1 and the kernel makes no pass at all
                call("fx_ce_lin_grad_scale_inplace", ptr(dW), dW.numel(), ptr(dx), dx.numel(), ptr(g32),
                     ptr(gs_t), inv_value, stream_of(dx))
                ctx.first = (g32, gs_t, inv_value)
                return dx, dW, None, None, None, None
            if dW.dtype == torch.bfloat16:
                # a further backward through a retained graph: the saved gradients carry the
                # first backward's factor s1; fresh tensors at s / s1
                g1, gs1, inv1 = ctx.first
                s1 = float(g1) * (1.0 / float(gs1) if gs1 is not None else inv1)
                if s1 == 0.0:
                    raise RuntimeError("linear_cross_entropy: the first backward of this graph had a "
                                       "gradient factor of 0, which zeroed the saved gradients; run the "
                                       "forward again")
                s = float(g32) * (1.0 / float(gs_t) if gs_t is not None else inv_value)
                g32 = torch.tensor(s / s1, device=dx.device, dtype=torch.float32)
                gs_t, inv_value = None, 1.0
            gx = torch.empty_like(dx)
            gw = torch.empty(dW.shape, device=dW.device, dtype=torch.bfloat16)
            fn = "fx_ce_lin_grad_scale_bf16w" if dW.dtype == torch.bfloat16 else "fx_ce_lin_grad_scale"
            call(fn, ptr(dW), dW.numel(), ptr(dx), dx.numel(), ptr(g32), ptr(gs_t), inv_value, ptr(gw), ptr(gx),
                 stream_of(dx))
            return gx, gw, None, None, None, None
        inv = torch.reciprocal(gs.float()) if torch.is_tensor(gs) else 1.0 / gs
        gx = dx * (g * inv)
        gw = (dW.float() * (g * inv)).to(ctx.wdtype)
        return gx, gw, None, None, None, None


def _check_lin(x, weight, target):
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("x and weight must be bfloat16")
    if not (x.is_cuda and weight.is_cuda and target.is_cuda):
        raise TypeError("all tensors must be cuda tensors")
    if not (x.is_contiguous() and weight.is_contiguous() and target.is_contiguous()):
        raise ValueError("x, weight and target must be contiguous")
    if target.dtype != torch.int64:
        raise TypeError("target must be int64")
    N, D = x.shape
    V, Dw = weight.shape
    if Dw != D or target.shape != (N,):
        raise ValueError(f"shape mismatch: x{tuple(x.shape)} W{tuple(weight.shape)} "
                         f"t{tuple(target.shape)}")
    return N, D, V


def _linear_ce_loss_only(x, weight, target, ignore_index, chunk_rows):
    """No-grad path: neither dx/dW nor dlogits are allocated."""
    N, D, V = _check_lin(x, weight, target)
    if chunk_rows is None:
        chunk_rows = _auto_chunk(D, V)
    inv_n, _mul = _inv_nvalid(target, ignore_index)
    row_loss = torch.empty(N, device=x.device, dtype=torch.float32)
    if FUSED_LINEAR_CE_LOSS and _lce_fused_ok(x, weight):
        # one pass over all rows: the workspace is a (max, sum) pair per row and column tile
        _lce_fwd(x, weight, target, ignore_index, row_loss)
        return _finalize(row_loss, inv_n)
    for r0 in range(0, N, chunk_rows):
        r1 = min(r0 + chunk_rows, N)
        lg = torch.mm(x[r0:r1], weight.t())
        _ce_rows(lg, target[r0:r1], None, row_loss[r0:r1], _mul, ignore_index)
    return _finalize(row_loss, inv_n)


def linear_cross_entropy(x, weight, target, grad_scale=1.0, ignore_index=-100,
                         chunk_rows=None):
    """x (N,D) bf16, weight (V,D) bf16, target (N,) int64 -> fp32 scalar loss.

    grad_scale: python float or 0-dim fp32 cuda tensor (loss scale); the
    gradients carried through the chunks are multiplied by it and divided
    back out in backward.  chunk_rows: None -> automatic.
    Without grad, the loss-only path is used (no dx/dW buffers).
    """
    if not (torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad)):
        return _linear_ce_loss_only(x, weight, target, ignore_index, chunk_rows)
    return _LinearCE.apply(x, weight, target, grad_scale, int(ignore_index), chunk_rows)
