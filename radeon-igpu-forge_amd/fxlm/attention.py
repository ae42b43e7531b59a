"""fxlm.attention: flash attention (bf16 MFMA, fp32 online softmax) on gfx950.

q, k, v (B,T,H,Dh) bf16 with unit stride along Dh and any other strides (views
of a fused qkv buffer work without a copy).  o (B,T,H,Dh) is returned
contiguous; lse (B,H,T) fp32 is kept for the backward.  Dh in {64, 128}; any
T >= 1 (tail tiles are masked).  Surface, checks and autograd structure follow
ml/fxlm/attention.py:57-199.
"""
import ctypes
import math

import torch

from fxgpu.abi import call, fxAttnArgs, fxAttnDecodeArgs, lib, stream_of


def _check_qkv(q, k, v):
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one 4-D shape: {tuple(q.shape)} "
                         f"{tuple(k.shape)} {tuple(v.shape)}")
    B, T, H, Dh = q.shape
    if Dh not in (64, 128):
        raise ValueError(f"head_dim {Dh} not supported (must be 64 or 128)")
    if T < 1 or B < 1 or H < 1:
        raise ValueError(f"invalid shape: {tuple(q.shape)}")
    for nm, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{nm} must be bfloat16, got {t.dtype}")
        if not t.is_cuda:
            raise TypeError(f"{nm} must be a cuda tensor")
        if t.stride(-1) != 1:
            raise ValueError(f"{nm}: last dim must be contiguous (stride(-1)={t.stride(-1)})")
        if any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
            raise ValueError(f"{nm}: b/t/h strides must be multiples of 8 elements and the "
                             "base 16-byte aligned")
    if q.numel() >= 2 ** 31:
        raise ValueError("tensor too large (2^31 element limit)")
    return B, T, H, Dh


def _strides3(t):
    s = t.stride()
    return s[0], s[1], s[2]


def _args(q, k, v, causal, scale):
    B, T, H, Dh = q.shape
    a = fxAttnArgs()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.qsb, a.qst, a.qsh = _strides3(q)
    a.ksb, a.kst, a.ksh = _strides3(k)
    a.vsb, a.vst, a.vsh = _strides3(v)
    a.B, a.T, a.H, a.D = B, T, H, Dh
    a.scale = scale
    a.causal = int(causal)
    return a


def _fwd(q, k, v, causal, scale):
    B, T, H, Dh = _check_qkv(q, k, v)
    o = torch.empty(B, T, H, Dh, device=q.device, dtype=torch.bfloat16)
    lse = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    a = _args(q, k, v, causal, scale)
    a.o_out, a.lse_out = o.data_ptr(), lse.data_ptr()
    call("fx_attn_fwd", ctypes.byref(a), stream_of(q))
    return o, lse


def _bwd(q, k, v, o, lse, do, causal, scale, dq, dk, dv):
    B, T, H, Dh = q.shape
    do = do.contiguous()
    if do.dtype != torch.bfloat16:
        do = do.to(torch.bfloat16)
    delta = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    a = _args(q, k, v, causal, scale)
    a.o, a.dout = o.data_ptr(), do.data_ptr()
    a.lse, a.delta = lse.data_ptr(), delta.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.dqb, a.dqt, a.dqh = _strides3(dq)
    a.dkb, a.dkt, a.dkh = _strides3(dk)
    a.dvb, a.dvt, a.dvh = _strides3(dv)
    call("fx_attn_bwd", ctypes.byref(a), stream_of(q))
    return dq, dk, dv


class _FlashAttn(torch.autograd.Function):
    """flash_attention(q, k, v): o (B,T,H,Dh) contiguous bf16."""

    @staticmethod
    def forward(ctx, q, k, v, causal, scale):
        o, lse = _fwd(q, k, v, causal, scale)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.causal, ctx.scale = causal, scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        B, T, H, Dh = q.shape
        dq = torch.empty(B, T, H, Dh, device=q.device, dtype=torch.bfloat16)
        dk = torch.empty_like(dq)
        dv = torch.empty_like(dq)
        _bwd(q, k, v, o, lse, do, ctx.causal, ctx.scale, dq, dk, dv)
        return dq, dk, dv, None, None


class _FlashAttnQKV(torch.autograd.Function):
    """flash_attention_qkv(qkv): qkv (B,T,3,H,Dh) bf16 contiguous."""

    @staticmethod
    def forward(ctx, qkv, causal, scale):
        if qkv.dim() != 5 or qkv.shape[2] != 3:
            raise ValueError(f"qkv must be (B,T,3,H,Dh), got {tuple(qkv.shape)}")
        if not qkv.is_contiguous():
            raise ValueError("qkv must be contiguous")
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
        o, lse = _fwd(q, k, v, causal, scale)
        ctx.save_for_backward(qkv, o, lse)
        ctx.causal, ctx.scale = causal, scale
        return o

    @staticmethod
    def backward(ctx, do):
        qkv, o, lse = ctx.saved_tensors
        dqkv = torch.empty_like(qkv)
        _bwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], o, lse, do, ctx.causal, ctx.scale,
             dqkv[:, :, 0], dqkv[:, :, 1], dqkv[:, :, 2])
        return dqkv, None, None


def flash_attention(q, k, v, causal=True, scale=None):
    """q, k, v (B,T,H,Dh) bf16 -> o (B,T,H,Dh) bf16."""
    Dh = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(Dh)
    return _FlashAttn.apply(q, k, v, causal, float(scale))


def flash_attention_qkv(qkv, causal=True, scale=None):
    """qkv (B,T,3,H,Dh) bf16 contiguous -> o (B,T,H,Dh) bf16."""
    if qkv.dim() != 5:
        raise ValueError(f"qkv must be (B,T,3,H,Dh), got {tuple(qkv.shape)}")
    Dh = qkv.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(Dh)
    return _FlashAttnQKV.apply(qkv, causal, float(scale))


def attention_fwd_raw(q, k, v, causal=True, scale=None):
    """Forward only, returning (o, lse): the fp32 logsumexp for parity checks."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _fwd(q, k, v, causal, float(scale))


def decode_attention(q, k_cache, v_cache, lens, scale=None, return_lse=False, k_new=None, v_new=None):
    """One new query per (sequence, head) against a KV cache (inference).

    q (B, H, Dh) bf16; k_cache, v_cache (B, Tmax, H, Dh) bf16 (unit stride along Dh,
    b/t/h strides multiples of 8); lens (B,) int32 cuda: the number of valid cached keys
    of each sequence (the new token's own key included).  Returns o (B, H, Dh) bf16 =
    softmax(scale q K[:lens]^T) V[:lens], and the fp32 logsumexp (B, H) if asked.
    k_new, v_new (B, H, Dh), both or neither: the new token's key and value; the kernel
    uses them as key lens[b] - 1 and writes them into the caches at that row.
    """
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError(f"q (B,H,Dh) and caches (B,Tmax,H,Dh): {tuple(q.shape)} "
                         f"{tuple(k_cache.shape)} {tuple(v_cache.shape)}")
    B, Tmax, H, Dh = k_cache.shape
    if tuple(q.shape) != (B, H, Dh):
        raise ValueError(f"q {tuple(q.shape)} does not match the cache {tuple(k_cache.shape)}")
    if Dh not in (64, 128):
        raise ValueError(f"head_dim {Dh} not supported (must be 64 or 128)")
    for nm, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{nm} must be bfloat16, got {t.dtype}")
        if not t.is_cuda:
            raise TypeError(f"{nm} must be a cuda tensor")
        if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
            raise ValueError(f"{nm}: last dim must be contiguous, other strides multiples of 8 "
                             "elements and the base 16-byte aligned")
    if lens.dtype != torch.int32 or not lens.is_cuda or lens.shape != (B,):
        raise TypeError(f"lens must be an int32 cuda tensor of shape ({B},)")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    for nm, t in (("k_new", k_new), ("v_new", v_new)):
        if t is None:
            continue
        if tuple(t.shape) != (B, H, Dh):
            raise ValueError(f"{nm} {tuple(t.shape)} must be (B, H, Dh) = {(B, H, Dh)}")
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise TypeError(f"{nm} must be a bfloat16 cuda tensor")
        if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
            raise ValueError(f"{nm}: last dim must be contiguous, other strides multiples of 8 "
                             "elements and the base 16-byte aligned")
    if scale is None:
        scale = 1.0 / math.sqrt(Dh)
    lens = lens.contiguous()
    o = torch.empty(B, H, Dh, device=q.device, dtype=torch.bfloat16)
    lse = torch.empty(B, H, device=q.device, dtype=torch.float32) if return_lse else None
    nbytes = int(lib().fx_attn_decode_workspace(B, H, Tmax, Dh))
    work = torch.empty((nbytes + 3) // 4, device=q.device, dtype=torch.float32) if nbytes else None
    a = fxAttnDecodeArgs()
    a.q, a.k, a.v, a.lens, a.o = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), lens.data_ptr(), o.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.work = work.data_ptr() if work is not None else None
    a.qsb, a.qsh = q.stride(0), q.stride(1)
    a.ksb, a.kst, a.ksh = _strides3(k_cache)
    a.vsb, a.vst, a.vsh = _strides3(v_cache)
    a.B, a.H, a.Tmax, a.D = B, H, Tmax, Dh
    a.scale = float(scale)
    if k_new is not None:
        a.knew, a.vnew = k_new.data_ptr(), v_new.data_ptr()
        a.knb, a.knh = k_new.stride(0), k_new.stride(1)
        a.vnb, a.vnh = v_new.stride(0), v_new.stride(1)
    call("fx_attn_decode", ctypes.byref(a), stream_of(q))
    return (o, lse) if return_lse else o
