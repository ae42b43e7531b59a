"""fxgpu.fused_linear: fused (gather) linear layers on gfx950 bf16 MFMA.

* ``FusedGatherLinear.apply(X16, idx32, weight, bias)`` -- surface of
  ml/fxgpu/fused_linear.py:27-101: out[b, n] = bias[n] + sum_k Xg[b, k] W[n, k]
  with Xg[b, w*F + f] = X[idx[b] + w, f] (window-major).  The forward kernel
  also writes Xg when a gradient is needed; the backward is dW = g^T Xg and
  db = sum_b g (no dX, as in the reference).
* ``FusedLinear.apply(x, weight, bias, activation)`` / ``fused_linear`` -- the
  dense form with the activation fused into the GEMM epilogue, used by the
  GPT MLP as fc -> GELU(tanh): y = gelu(x W^T + b).  The pre-activation is kept
  for the backward: dh = dy * gelu'(h) (one elementwise kernel), then dx = dh W
  on the library GEMM and dW = dh^T x on this build's split-K weight-gradient GEMM.
* ``linear(x, weight)`` -- y = x W^T (no bias) with the same backward split: the
  GPT's qkv, proj and fc2 projections.  Forwards of at most FEW_ROWS rows (decode
  steps) run on the few-row kernel behind fx_linear_fwd, the whole_tiles() shapes on
  its whole-tile kernel, the others on the library GEMM.
* ``fused_mlp(x, w1, w2)`` -- gelu_tanh(x w1^T) w2^T as one autograd node: the GELU and
  its derivative g = gelu'(h) in the fc epilogue (g saved in place of the pre-activation),
  the product with g in the fc2 input gradient's epilogue (fx_linear_dgrad_gate).
* ``input_grad(dy, W, g=None)`` -- dx = dy W (and * g) on fx_linear_dgrad(_gate) for whole
  tiles, else the library GEMM (and fx_gelu_bwd_gate).
* ``linear_wgrad(dy, x)`` -- dW = dy^T x for dy (T, N) and x (T, K): the weight
  gradient that ml/fxgpu/fused_linear.py:90-101 computes with rocBLAS.
* ``linear_ex(x, W, bias, residual, norm_weight, eps, activation)`` -- inference
  forward with the input RMSNorm and the output residual folded into the GEMM
  (decoding steps).
"""
import ctypes

import torch

from fxgpu.abi import call, fxLinearArgs, lib, ptr, stream_of

_ACTS = {None: 0, "none": 0, "identity": 0, "gelu_tanh": 1}


def _rows(t):
    """t as a (rows, cols) view whose rows are 16-byte aligned and unit-stride."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


def linear_wgrad(dy, x):
    """dW = dy^T x in bf16 (fp32 accumulation): dy (..., N), x (..., K) bf16 with the
    same leading shape; returns (N, K).  Widths that are not multiples of 8 (the
    kernel stages 16-byte column chunks) take the library GEMM, as the reference's
    rocBLAS dW does for every shape (ml/fxgpu/fused_linear.py:90-101)."""
    if dy.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise TypeError("dy and x must be bfloat16")
    if not (dy.is_cuda and x.is_cuda):
        raise TypeError("dy and x must be cuda tensors")
    dy2, x2 = _rows(dy), _rows(x)
    if dy2.shape[0] != x2.shape[0]:
        raise ValueError(f"dy has {dy2.shape[0]} rows, x has {x2.shape[0]}")
    T, N = dy2.shape
    K = x2.shape[1]
    if N % 8 or K % 8:
        return torch.mm(dy2.t(), x2)
    dW = torch.empty(N, K, device=x.device, dtype=torch.bfloat16)
    nbytes = int(lib().fx_linear_wgrad_workspace(N, K, T))
    work = torch.empty((nbytes + 3) // 4, device=x.device, dtype=torch.float32) if nbytes else None
    call("fx_linear_wgrad", ptr(dy2), dy2.stride(0), ptr(x2), x2.stride(0), ptr(dW), K, ptr(work), N, K, T,
         stream_of(x))
    return dW


# Up to this many rows the forward GEMM is a stream over the weight (decoding, small
# batches) and runs on this build's few-row kernel; above it on the library GEMM, except
# for the shapes of whole_tiles().
FEW_ROWS = 64


def whole_tiles(M, N, K):
    """Shapes that fx_linear_fwd runs on its whole-tile kernel (M % 256 == 0, N % 192 or
    % 256 == 0, K % 32 == 0, K >= 128) and where that kernel measured at least as fast as the
    library GEMM: K up to 1024 (the cfg5 qkv and proj, 62.9 and 22.8 us against 66.8 and
    24.2 us with the operands in the caches, 76.7 and 31.2 against 75.2 and 29.7 us from
    HBM).  With K = 3072 and N = 768 (fc2: one tile per CU) the library GEMM is faster from
    HBM (81.0 against 95.7 us).  Taken only with NATIVE_PROJ_FWD."""
    return M % 256 == 0 and K % 32 == 0 and 128 <= K <= 1024 and (N % 256 == 0 or N % 192 == 0)


# Routing switches, set by interleaved A/Bs of the whole cfg5 training step (24 rounds of 5
# steps, medians, one process).  With the two-step LDS buffers of the whole-tile kernels
# (whole 128-byte lines from HBM), the qkv and proj forwards (whole_tiles()) on fx_linear_fwd
# measured +0.011 ms per step against the library GEMM, within the rounds' spread: they run
# on this build's kernel.  The plain input gradients do not: the qkv one at parity (-0.003
# to +0.005 ms), the proj and fc ones 0.04-0.08 ms slower each (cold operands from HBM, and
# tile epilogues that one workgroup per CU cannot overlap with its MFMA work).  fc2's, with
# the saved GELU derivative multiplied in its epilogue, runs on this build's kernel.
# NATIVE_INPUT_GRAD: input gradients on fx_linear_dgrad where input_grad() takes them;
# NATIVE_PROJ_FWD: the whole_tiles() forwards on fx_linear_fwd.  False: the library GEMM.
NATIVE_INPUT_GRAD = False
NATIVE_PROJ_FWD = True
# NATIVE_GELU_INPUT_GRAD: only the input gradient with the GELU derivative folded in (the
# GPT MLP's fc2, where fx_linear_dgrad_gate also saves fx_gelu_bwd_gate's pass over three
# tensors).  With the derivative stored by the fc forward (fused_mlp) the epilogue only
# multiplies, and the step measured 0.13 ms faster (16 interleaved rounds, every round
# faster); evaluating the derivative from the pre-activation in that epilogue had measured
# 0.04 ms slower than the library GEMM and fx_gelu_bwd.
NATIVE_GELU_INPUT_GRAD = True


def dgrad_tiles(M, N, K):
    """Shapes fx_linear_dgrad takes (whole-tile kernel): dX (M, N) = dY (M, K) W (K, N)."""
    return M % 256 == 0 and (N % 256 == 0 or N % 192 == 0) and K % 32 == 0 and K >= 128


def input_grad(dy2, weight, g=None):
    """dx = dy2 @ weight (bf16), and with g (the GELU(tanh) derivative at the output of the
    layer feeding this one, as fx_linear_fwd with act 2 stores it) bf16(dx) * g.  With
    NATIVE_INPUT_GRAD, on fx_linear_dgrad for dgrad_tiles() shapes where it measured at
    least as fast as the library GEMM with the operands in the caches (input widths up to
    1024 columns: the cfg5 qkv, proj and fc input gradients, 52.1 / 22.9 / 66.0 us against
    60.5 / 25.4 / 67.2 us; from HBM 72.3 / 31.6 / 93.7 against 64.5 / 30.3 / 82.4 us); with
    g and NATIVE_GELU_INPUT_GRAD on fx_linear_dgrad_gate (the product with g in the
    epilogue: 98.8 us against 126.3 for the cfg5 fc2 product on the library GEMM and
    fx_gelu_bwd, 125.5 against 133.6 from HBM); else torch.mm, then fx_gelu_bwd_gate for g."""
    M, K = dy2.shape
    N = weight.shape[1]
    wanted = (NATIVE_INPUT_GRAD and (g is not None or N <= 1024)) or (NATIVE_GELU_INPUT_GRAD and g is not None)
    native = (wanted and dy2.is_cuda and dgrad_tiles(M, N, K)
              and weight.is_contiguous() and weight.data_ptr() % 16 == 0
              and dy2.stride(1) == 1 and dy2.stride(0) % 8 == 0 and dy2.data_ptr() % 16 == 0
              and (g is None or (g.is_contiguous() and g.data_ptr() % 16 == 0)))
    if native:
        dx = torch.empty(M, N, device=dy2.device, dtype=torch.bfloat16)
        if g is None:
            call("fx_linear_dgrad", ptr(dy2), dy2.stride(0), ptr(weight), N, None, ptr(dx), N, M, N, K,
                 stream_of(dy2))
        else:
            call("fx_linear_dgrad_gate", ptr(dy2), dy2.stride(0), ptr(weight), N, ptr(g), ptr(dx), N, M, N,
                 K, stream_of(dy2))
        return dx
    dx = torch.mm(dy2, weight)
    if g is None:
        return dx
    dh = torch.empty_like(dx)
    call("fx_gelu_bwd_gate", ptr(dx), ptr(g), ptr(dh), dh.numel(), stream_of(dx))
    return dh


def _native_fwd(x2, weight):
    """y = x2 W^T on fx_linear_fwd (the few-row kernel for M <= FEW_ROWS, else the tiled ones)."""
    M, K = x2.shape
    y = torch.empty(M, weight.shape[0], device=x2.device, dtype=torch.bfloat16)
    call("fx_linear_fwd", ptr(x2), x2.stride(0), None, 0, 0, ptr(weight), None, ptr(y), None, None,
         M, weight.shape[0], K, 0, stream_of(x2))
    return y


class Linear(torch.autograd.Function):
    """y = x W^T for x (..., K) bf16, weight (N, K) bf16; dW on the split-K GEMM."""

    @staticmethod
    def forward(ctx, x, weight):
        if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
            raise TypeError("x and weight must be bfloat16")
        if weight.dim() != 2 or weight.shape[1] != x.shape[-1]:
            raise ValueError(f"weight must be (N, {x.shape[-1]}), got {tuple(weight.shape)}")
        x2 = _rows(x)
        M, K = x2.shape
        native = x2.is_cuda and weight.is_contiguous() and weight.data_ptr() % 16 == 0 and K % 8 == 0
        if native and (0 < M <= FEW_ROWS or (NATIVE_PROJ_FWD and whole_tiles(M, weight.shape[0], K))):
            y = _native_fwd(x2, weight)
        else:
            y = torch.mm(x2, weight.t())
        ctx.save_for_backward(x2, weight)
        ctx.xshape = x.shape
        return y.view(*x.shape[:-1], weight.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, weight = ctx.saved_tensors
        dy2 = _rows(dy.to(torch.bfloat16) if dy.dtype != torch.bfloat16 else dy)
        dx = input_grad(dy2, weight).view(ctx.xshape) if ctx.needs_input_grad[0] else None
        dW = linear_wgrad(dy2, x2) if ctx.needs_input_grad[1] else None
        return dx, dW


def linear(x, weight):
    """y = x @ weight.T (bf16), the weight gradient on this build's split-K GEMM."""
    return Linear.apply(x, weight)


class FusedGatherLinear(torch.autograd.Function):
    """out[b, n] = sum_k Xg[b, k] * weight[n, k] + bias[n]

    Xg[b, w*F + f] = X[idx[b] + w, f] (window-major flattening).
    X16: (R, F) bf16 contiguous; idx32: (B,) int32 contiguous;
    weight: (N, K) bf16 contiguous, K = W*F; bias: (N,) bf16.
    """

    @staticmethod
    def forward(ctx, X16, idx32, weight, bias):
        F = X16.shape[1]
        K = weight.shape[1]
        if K % F != 0:
            raise ValueError(f"weight.shape[1]={K} is not a multiple of X16.shape[1]={F} "
                             f"(K = window * F)")
        if F % 8 != 0:
            raise ValueError("pad F to a multiple of 8 with zero columns "
                             f"(F={F}; the kernel uses 16-byte loads)")
        if X16.dtype != torch.bfloat16:
            raise TypeError(f"X16 must be bfloat16, got {X16.dtype}")
        if idx32.dtype != torch.int32:
            raise TypeError(f"idx32 must be int32, got {idx32.dtype}")
        if weight.dtype != torch.bfloat16 or bias.dtype != torch.bfloat16:
            raise TypeError("weight and bias must be bfloat16")
        if not (X16.is_cuda and idx32.is_cuda and weight.is_cuda and bias.is_cuda):
            raise TypeError("all tensors must be cuda tensors")
        if not (X16.is_contiguous() and idx32.is_contiguous() and weight.is_contiguous()
                and bias.is_contiguous()):
            raise ValueError("all tensors must be contiguous (call .contiguous())")
        if idx32.dim() != 1:
            raise ValueError(f"idx32 must be (B,), shape={tuple(idx32.shape)}")
        if weight.dim() != 2 or bias.dim() != 1 or bias.shape[0] != weight.shape[0]:
            raise ValueError("weight must be (N,K) and bias (N,)")
        Bsz = idx32.numel()
        N = weight.shape[0]
        C = torch.empty(Bsz, N, device=X16.device, dtype=torch.bfloat16)
        need_grad = any(ctx.needs_input_grad)
        # Xg only serves the backward (dW); inference skips the write-out.
        Xg = torch.empty(Bsz, K, device=X16.device, dtype=torch.bfloat16) if need_grad else None
        call("fx_linear_fwd", ptr(X16), F, ptr(idx32), F, X16.shape[0], ptr(weight), ptr(bias),
             ptr(C), None, ptr(Xg), Bsz, N, K, 0, stream_of(X16))
        if need_grad:
            ctx.save_for_backward(Xg)
        return C

    @staticmethod
    def backward(ctx, g):
        (Xg,) = ctx.saved_tensors
        g = g.contiguous()
        dW = linear_wgrad(g, Xg)          # (N, K)
        db = g.sum(0)
        return None, None, dW, db


def fused_gather_linear(X16, idx32, weight, bias):
    """Thin wrapper over FusedGatherLinear.apply."""
    return FusedGatherLinear.apply(X16, idx32, weight, bias)


class FusedLinear(torch.autograd.Function):
    """y = act(x W^T + b) for x (..., K) bf16, weight (N, K) bf16, bias (N,) bf16 or None."""

    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        if activation not in _ACTS:
            raise ValueError(f"activation {activation!r} not in {sorted(k for k in _ACTS if k)}")
        act = _ACTS[activation]
        if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or (
                bias is not None and bias.dtype != torch.bfloat16):
            raise TypeError("x, weight and bias must be bfloat16")
        if not (x.is_cuda and weight.is_cuda):
            raise TypeError("x and weight must be cuda tensors")
        K = x.shape[-1]
        if weight.dim() != 2 or weight.shape[1] != K:
            raise ValueError(f"weight must be (N, {K}), got {tuple(weight.shape)}")
        if K % 8 != 0:
            raise ValueError(f"in_features={K} must be a multiple of 8")
        if not weight.is_contiguous() or (bias is not None and not bias.is_contiguous()):
            raise ValueError("weight and bias must be contiguous")
        N = weight.shape[0]
        x2 = x.reshape(-1, K)
        if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        M = x2.shape[0]
        y = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
        h = torch.empty_like(y) if (act and any(ctx.needs_input_grad)) else None
        call("fx_linear_fwd", ptr(x2), x2.stride(0), None, 0, 0, ptr(weight), ptr(bias), ptr(y),
             ptr(h), None, M, N, K, act, stream_of(x))
        ctx.save_for_backward(x2, weight, h)
        ctx.act, ctx.has_bias, ctx.xshape = act, bias is not None, x.shape
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, weight, h = ctx.saved_tensors
        N = weight.shape[0]
        dy2 = dy.reshape(-1, N)
        if dy2.dtype != torch.bfloat16:
            dy2 = dy2.to(torch.bfloat16)
        dy2 = dy2.contiguous()
        if ctx.act:
            dh = torch.empty_like(dy2)
            call("fx_gelu_bwd", ptr(dy2), ptr(h), ptr(dh), dh.numel(), stream_of(dy2))
        else:
            dh = dy2
        dx = input_grad(dh, weight).view(ctx.xshape) if ctx.needs_input_grad[0] else None
        dW = linear_wgrad(dh, x2) if ctx.needs_input_grad[1] else None
        db = dh.sum(0) if (ctx.has_bias and ctx.needs_input_grad[2]) else None
        return dx, dW, db, None


def fused_linear(x, weight, bias=None, activation="gelu_tanh"):
    """y = activation(x @ weight.T + bias) with the activation fused into the GEMM."""
    return FusedLinear.apply(x, weight, bias, activation)


class FusedMLP(torch.autograd.Function):
    """y = gelu_tanh(x W1^T) W2^T (no biases): the GPT MLP (ml/fxlm/model.py:64-66,71,
    nn.Linear fc -> F.gelu(approximate="tanh") -> nn.Linear fc2) as one autograd node.  The
    fc forward (fx_linear_fwd, act 2) stores, in place of the pre-activation h, the GELU
    derivative g = gelu'(h) from the fp32 h and the exponential the GELU itself takes; the
    backward's fc2 input gradient multiplies by it in its epilogue (fx_linear_dgrad_gate).
    The forward's outputs are those of fused_linear followed by linear, bit for bit."""

    @staticmethod
    def forward(ctx, x, w1, w2):
        if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
            raise TypeError("x, w1 and w2 must be bfloat16")
        if not (x.is_cuda and w1.is_cuda and w2.is_cuda):
            raise TypeError("x, w1 and w2 must be cuda tensors")
        K = x.shape[-1]
        if w1.dim() != 2 or w1.shape[1] != K or w2.dim() != 2 or w2.shape[1] != w1.shape[0]:
            raise ValueError(f"weights must be (F, {K}) and (N, F), got {tuple(w1.shape)}, {tuple(w2.shape)}")
        if K % 8 or w1.shape[0] % 8:
            raise ValueError("in_features and the hidden width must be multiples of 8")
        if not (w1.is_contiguous() and w2.is_contiguous()):
            raise ValueError("weights must be contiguous")
        x2 = _rows(x)
        M, Fh = x2.shape[0], w1.shape[0]
        u = torch.empty(M, Fh, device=x.device, dtype=torch.bfloat16)
        gd = torch.empty_like(u) if any(ctx.needs_input_grad) else None
        call("fx_linear_fwd", ptr(x2), x2.stride(0), None, 0, 0, ptr(w1), None, ptr(u), ptr(gd), None,
             M, Fh, K, 2, stream_of(x))
        N = w2.shape[0]
        if 0 < M <= FEW_ROWS or (NATIVE_PROJ_FWD and whole_tiles(M, N, Fh)):
            y = _native_fwd(u, w2)
        else:
            y = torch.mm(u, w2.t())
        ctx.save_for_backward(x2, w1, w2, u, gd)
        ctx.xshape = x.shape
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, w1, w2, u, gd = ctx.saved_tensors
        dy2 = _rows(dy.to(torch.bfloat16) if dy.dtype != torch.bfloat16 else dy)
        dh = input_grad(dy2, w2, gd)             # (dy W2) gelu'(h)
        dw2 = linear_wgrad(dy2, u) if ctx.needs_input_grad[2] else None
        dx = input_grad(dh, w1).view(ctx.xshape) if ctx.needs_input_grad[0] else None
        dw1 = linear_wgrad(dh, x2) if ctx.needs_input_grad[1] else None
        return dx, dw1, dw2


def fused_mlp(x, w1, w2):
    """gelu_tanh(x @ w1.T) @ w2.T with the GELU and its derivative in the fc epilogue and the
    product with the derivative in the fc2 input gradient's epilogue."""
    return FusedMLP.apply(x, w1, w2)


def linear_ex(x, weight, bias=None, residual=None, norm_weight=None, eps=1e-6, activation=None):
    """Inference forward y = act(norm(x) @ weight.T + bias) + residual in one launch
    (fx_linear_fwd_ex): norm is an RMSNorm of the rows of x with norm_weight (only for
    at most FEW_ROWS rows), residual a tensor shaped like y.  No autograd."""
    if activation not in _ACTS:
        raise ValueError(f"activation {activation!r} not in {sorted(k for k in _ACTS if k)}")
    for nm, t in (("x", x), ("weight", weight), ("bias", bias), ("residual", residual),
                  ("norm_weight", norm_weight)):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_cuda):
            raise TypeError(f"{nm} must be a bfloat16 cuda tensor")
    K = x.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != K or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous (N, {K}), got {tuple(weight.shape)}")
    if K % 8:
        raise ValueError(f"in_features={K} must be a multiple of 8")
    N = weight.shape[0]
    x2 = _rows(x)
    M = x2.shape[0]
    if norm_weight is not None:
        if norm_weight.shape != (K,) or not norm_weight.is_contiguous():
            raise ValueError(f"norm_weight must be a contiguous ({K},)")
        if M > FEW_ROWS:
            raise ValueError(f"the fused input norm takes at most {FEW_ROWS} rows, got {M}")
    if bias is not None and (bias.shape != (N,) or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous ({N},)")
    r2 = None
    if residual is not None:
        if tuple(residual.shape[:-1]) != tuple(x.shape[:-1]) or residual.shape[-1] != N:
            raise ValueError(f"residual {tuple(residual.shape)} must be shaped like the output")
        r2 = residual.reshape(-1, N)
        if r2.stride(1) != 1:
            r2 = r2.contiguous()
    y = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    a = fxLinearArgs()
    a.X, a.ldx, a.W = x2.data_ptr(), x2.stride(0), weight.data_ptr()
    a.bias = bias.data_ptr() if bias is not None else None
    if r2 is not None:
        a.res, a.ldres = r2.data_ptr(), r2.stride(0)
    a.norm_w = norm_weight.data_ptr() if norm_weight is not None else None
    a.Y = y.data_ptr()
    a.M, a.N, a.K = M, N, K
    a.eps = float(eps)
    a.act = _ACTS[activation]
    call("fx_linear_fwd_ex", ctypes.byref(a), stream_of(x))
    return y.view(*x.shape[:-1], N)
