"""Oracle: causal / non-causal attention forward and backward (TEST INFRASTRUCTURE ONLY).

Restates ml/fxlm/kernels/attention.hip:
  forward  (:103-224)  S = Q K^T * scale, mask key <= query when causal (:165-167),
                       O = softmax(S) V, lse = max + log(sum exp) or -inf for an
                       empty row with O = 0 (:210-223)
  Delta    (:228-251)  rowsum(dO * O) over the *stored* (rounded) output
  backward (:340-364, :487-505)  P = exp(S*scale - lse), dS = P (dP - Delta) scale,
                       dV = P^T dO, dK = dS^T Q, dQ = dS K
Tensors are (B, T, H, D); lse and delta are (B, H, T).  Math in `dtype`
(float64 by default) on the CPU.
"""
import torch


def _bhtd(x, dtype):
    return x.detach().to("cpu", dtype).permute(0, 2, 1, 3)


def scores(q, k, causal, scale, dtype=torch.float64):
    """Masked scaled scores (B, H, T, T); masked entries are -inf."""
    s = _bhtd(q, dtype) @ _bhtd(k, dtype).transpose(-1, -2) * scale
    if causal:
        T = q.shape[1]
        mask = torch.ones(T, T, dtype=torch.bool).triu(1)   # key > query
        s = s.masked_fill(mask, float("-inf"))
    return s


def attn_fwd(q, k, v, causal=True, scale=None, dtype=torch.float64):
    """Returns (o (B,T,H,D), lse (B,H,T)) in `dtype`."""
    D = q.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    s = scores(q, k, causal, scale, dtype)
    m = s.amax(-1, keepdim=True)
    m_use = torch.where(torch.isinf(m), torch.zeros_like(m), m)
    e = torch.exp(s - m_use)
    l = e.sum(-1, keepdim=True)
    o = torch.where(l > 0, e / l.clamp_min(1e-300), torch.zeros_like(e)) @ _bhtd(v, dtype)
    lse = torch.where(l > 0, m_use + torch.log(l.clamp_min(1e-300)),
                      torch.full_like(l, float("-inf")))
    return o.permute(0, 2, 1, 3).contiguous(), lse.squeeze(-1)


def attn_bwd(q, k, v, o, lse, do, causal=True, scale=None, dtype=torch.float64):
    """Returns (dq, dk, dv) (B,T,H,D) in `dtype`.  `o` is the stored forward output."""
    D = q.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    s = scores(q, k, causal, scale, dtype)
    lse_ = lse.detach().to("cpu", dtype).unsqueeze(-1)
    p = torch.exp(s - lse_)
    p = torch.where(torch.isinf(s), torch.zeros_like(p), p)
    dob, ob = _bhtd(do, dtype), _bhtd(o, dtype)
    qb, kb, vb = _bhtd(q, dtype), _bhtd(k, dtype), _bhtd(v, dtype)
    delta = (dob * ob).sum(-1, keepdim=True)
    dp = dob @ vb.transpose(-1, -2)
    ds = p * (dp - delta) * scale
    dv = p.transpose(-1, -2) @ dob
    dk = ds.transpose(-1, -2) @ qb
    dq = ds @ kb
    f = lambda t: t.permute(0, 2, 1, 3).contiguous()
    return f(dq), f(dk), f(dv)


def attn_decode(q, k_cache, v_cache, lens, scale=None, dtype=torch.float64):
    """Decode step: q (B, H, D) against the first lens[b] rows of k_cache / v_cache
    (B, Tmax, H, D).  Returns (o (B, H, D), lse (B, H)) in `dtype`: the last row of the
    causal forward above over those keys (an empty cache gives o = 0, lse = -inf)."""
    B, Tmax, H, D = k_cache.shape
    scale = D ** -0.5 if scale is None else scale
    qd = q.detach().to("cpu", dtype)
    kd, vd = k_cache.detach().to("cpu", dtype), v_cache.detach().to("cpu", dtype)
    lens = [int(x) for x in lens.detach().cpu()]
    o = torch.zeros(B, H, D, dtype=dtype)
    lse = torch.full((B, H), float("-inf"), dtype=dtype)
    for b in range(B):
        n = max(0, min(lens[b], Tmax))
        if n == 0:
            continue
        s = torch.einsum("hd,thd->ht", qd[b], kd[b, :n]) * scale    # (H, n)
        m = s.amax(-1, keepdim=True)
        e = torch.exp(s - m)
        l = e.sum(-1, keepdim=True)
        o[b] = torch.einsum("ht,thd->hd", e / l, vd[b, :n])
        lse[b] = (m + torch.log(l)).squeeze(-1)
    return o, lse
