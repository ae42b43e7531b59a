"""Flash attention on the GPU (fx_attn_fwd / fx_attn_bwd) against the oracle and fixtures.

Tolerance: outputs and gradients within 2e-2 max-abs of the fp64 oracle
(bf16 inputs), lse within 1e-3 relative.
"""
import math

import pytest
import torch

from golden_util import bf16, f32, load
from oracle import attention as oatt
from tolerances import FRAC_GRAD, oracle_close

pytestmark = pytest.mark.gpu


def _fwd_bwd(q, k, v, do, causal, scale):
    from fxlm.attention import attention_fwd_raw, flash_attention
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    o = flash_attention(qq, kk, vv, causal=causal, scale=scale)
    o.backward(do)
    _, lse = attention_fwd_raw(q, k, v, causal, scale)
    torch.cuda.synchronize()
    return o, lse, qq.grad, kk.grad, vv.grad


def _check(got, ref):
    o, lse, dq, dk, dv = got
    ro, rl, rdq, rdk, rdv = ref
    assert oracle_close(o, ro)
    fin = torch.isfinite(rl)
    assert float((lse.cpu().double() - rl.double()).abs()[fin].max()) <= 1e-3 * max(1.0, float(rl[fin].abs().max()))
    for a, b in ((dq, rdq), (dk, rdk), (dv, rdv)):
        assert oracle_close(a, b)


@pytest.mark.parametrize("name", ["attn_t37_d64_causal", "attn_t33_d128_full", "attn_t130_d64_causal"])
def test_golden(dev, name):
    d = load(name)
    q, k, v, do = (bf16(d[x], dev) for x in ("q", "k", "v", "do"))
    got = _fwd_bwd(q, k, v, do, bool(d["causal"]), float(d["scale"]))
    _check(got, [f32(d[x]) for x in ("o", "lse", "dq", "dk", "dv")])


CASES = [(1, 1, 1, 64), (1, 17, 1, 64), (2, 64, 2, 64), (1, 100, 8, 64), (3, 256, 8, 64),
         (2, 513, 2, 64), (1, 130, 4, 128), (2, 200, 8, 128), (1, 33, 1, 128)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,T,H,Dh", CASES)
def test_against_oracle(dev, causal, B, T, H, Dh):
    # ml/fxlm/selftest.py:286-318: q/k/v are strided views of one (B,T,3,H,Dh) buffer
    torch.manual_seed(B * 7 + T * 13 + Dh)
    scale = 1.0 / math.sqrt(Dh)
    qkv = torch.randn(B, T, 3, H, Dh).bfloat16()
    do = torch.randn(B, T, H, Dh).bfloat16()
    qg = qkv.to(dev)
    got = _fwd_bwd(qg[:, :, 0], qg[:, :, 1], qg[:, :, 2], do.to(dev), causal, scale)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    ro, rl = oatt.attn_fwd(q, k, v, causal, scale)
    rdq, rdk, rdv = oatt.attn_bwd(q, k, v, got[0].cpu(), rl, do, causal, scale)
    _check(got, (ro, rl, rdq, rdk, rdv))


@pytest.mark.parametrize("causal", [True, False])
def test_qkv_variant(dev, causal):
    from fxlm.attention import flash_attention_qkv
    torch.manual_seed(5)
    B, T, H, Dh = 2, 100, 4, 64
    qkv = torch.randn(B, T, 3, H, Dh).bfloat16()
    x = qkv.to(dev).requires_grad_()
    o = flash_attention_qkv(x, causal=causal)
    do = torch.randn(B, T, H, Dh).bfloat16()
    o.backward(do.to(dev))
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    ro, rl = oatt.attn_fwd(q, k, v, causal)
    rdq, rdk, rdv = oatt.attn_bwd(q, k, v, o.detach().cpu(), rl, do, causal)
    assert oracle_close(o, ro)
    for i, r in enumerate((rdq, rdk, rdv)):
        assert oracle_close(x.grad[:, :, i], r)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("T,Dh", [(77, 64), (45, 128)])
def test_free_strides(dev, causal, T, Dh):
    # ml/fxlm/attention.py:57-79 accepts any b/t/h strides with a unit-stride last dim:
    # q is a (B,H,T,Dh) buffer seen through transpose(1, 2), k is contiguous, v takes
    # every other head of a (B,T,2H,Dh) buffer, and dO is non-contiguous too
    torch.manual_seed(T + Dh)
    B, H = 2, 3
    qb = torch.randn(B, H, T, Dh).bfloat16()
    k = torch.randn(B, T, H, Dh).bfloat16()
    vb = torch.randn(B, T, 2 * H, Dh).bfloat16()
    dob = torch.randn(B, H, T, Dh).bfloat16()
    q, v, do = qb.transpose(1, 2), vb[:, :, ::2], dob.transpose(1, 2)
    assert not (q.is_contiguous() or v.is_contiguous() or do.is_contiguous())
    got = _fwd_bwd(qb.to(dev).transpose(1, 2), k.to(dev), vb.to(dev)[:, :, ::2], dob.to(dev).transpose(1, 2),
                   causal, 1.0 / math.sqrt(Dh))
    ro, rl = oatt.attn_fwd(q, k, v, causal)
    rdq, rdk, rdv = oatt.attn_bwd(q, k, v, got[0].cpu(), rl, do, causal)
    _check(got, (ro, rl, rdq, rdk, rdv))


def test_single_key_closed_form(dev):
    from fxlm.attention import flash_attention
    torch.manual_seed(2)
    q, k, v = (torch.randn(3, 1, 2, 64, device=dev).bfloat16().requires_grad_() for _ in range(3))
    o = flash_attention(q, k, v)
    o.backward(torch.ones_like(o))
    assert torch.equal(o, v.detach())                     # one key: O = V exactly
    assert float(q.grad.abs().max()) == 0.0 and float(k.grad.abs().max()) == 0.0


def test_cfg2_full_size(dev):
    # cfg2: [16, 12, 1024, 64] causal bf16 ~ N(0,1); fp32 oracle math on two batch entries
    from fxlm.attention import attention_fwd_raw, flash_attention
    g = torch.Generator(device=dev).manual_seed(2)
    B, T, H, Dh = 16, 1024, 12, 64
    q, k, v, do = (torch.randn(B, T, H, Dh, device=dev, generator=g).bfloat16() for _ in range(4))
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    o = flash_attention(qq, kk, vv, causal=True)
    o.backward(do)
    _, lse = attention_fwd_raw(q, k, v, True)
    for b in (0, B - 1):
        sl = slice(b, b + 1)
        ro, rl = oatt.attn_fwd(q[sl], k[sl], v[sl], True, dtype=torch.float32)
        rdq, rdk, rdv = oatt.attn_bwd(q[sl], k[sl], v[sl], o[sl].detach(), rl, do[sl], True,
                                      dtype=torch.float32)
        _check((o[sl], lse[sl], qq.grad[sl], kk.grad[sl], vv.grad[sl]), (ro, rl, rdq, rdk, rdv))


# ---- decode attention (KV cache) ------------------------------------------------------

# one workgroup per (sequence, head) of up to 16 waves streaming 64-key sub-chunks
# (32 at D = 128) once B H >= half the CUs; fewer pairs split the keys into segments
# merged by a second kernel, and segments at or past a sequence's length are skipped
@pytest.mark.parametrize("B,Tmax,H,D,lens", [
    (2, 1024, 12, 64, [1024, 513]),        # 8 segments of 2 waves, ragged second sequence
    (3, 300, 4, 128, [1, 64, 65]),         # segment boundaries at D = 128
    (1, 64, 2, 64, [50]),                  # one wave, one segment: no merge
    (4, 2048, 8, 64, [2048, 1, 1500, 0]),  # an empty sequence
    (16, 1024, 16, 64, [1024 - 61 * i for i in range(16)]),   # one segment, 16 waves
    (32, 300, 64, 64, [300 - 9 * i for i in range(32)]),      # 5 waves, ragged tails
    (16, 256, 128, 128, [256 - 16 * i for i in range(16)]),   # one segment at D = 128
    (8, 2048, 16, 64, [2048 - 97 * i for i in range(8)]),     # waves loop over 2 sub-chunks
])
def test_decode_against_oracle(dev, B, Tmax, H, D, lens):
    from fxlm.attention import decode_attention
    g = torch.Generator(device=dev).manual_seed(B * 1000 + Tmax + D)
    q = torch.randn(B, H, D, device=dev, generator=g).bfloat16()
    k = torch.randn(B, Tmax, H, D, device=dev, generator=g).bfloat16()
    v = torch.randn(B, Tmax, H, D, device=dev, generator=g).bfloat16()
    lt = torch.tensor(lens, dtype=torch.int32, device=dev)
    o, lse = decode_attention(q, k, v, lt, return_lse=True)
    ro, rlse = oatt.attn_decode(q, k, v, lt)
    assert oracle_close(o, ro)
    lse_c = lse.cpu().double()
    fin = torch.isfinite(rlse)
    assert torch.equal(torch.isfinite(lse_c), fin)
    assert float(((lse_c[fin] - rlse[fin]).abs() / rlse[fin].abs().clamp_min(1.0)).max()) <= 1e-3
    assert float(o.float().cpu()[~fin].abs().max() if (~fin).any() else 0.0) == 0.0


def test_decode_matches_forward_last_row(dev):
    # a cache that is the (strided) k / v view of a fused qkv buffer
    from fxlm.attention import attention_fwd_raw, decode_attention
    g = torch.Generator(device=dev).manual_seed(17)
    B, T, H, D = 2, 777, 12, 64
    qkv = torch.randn(B, T, 3, H, D, device=dev, generator=g).bfloat16()
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    o_full, _ = attention_fwd_raw(q, k, v, causal=True)
    for n in (1, 256, 500, T):
        lt = torch.full((B,), n, dtype=torch.int32, device=dev)
        o = decode_attention(q[:, n - 1], k, v, lt)
        assert oracle_close(o, o_full[:, n - 1].float())


def test_decode_rejects_bad_arguments(dev):
    from fxlm.attention import decode_attention
    q = torch.zeros(1, 2, 64, device=dev).bfloat16()
    k = torch.zeros(1, 8, 2, 64, device=dev).bfloat16()
    with pytest.raises(TypeError):
        decode_attention(q, k, k, torch.ones(1, dtype=torch.int64, device=dev))
    with pytest.raises(ValueError):
        decode_attention(torch.zeros(1, 2, 96, device=dev).bfloat16(),
                         torch.zeros(1, 8, 2, 96, device=dev).bfloat16(),
                         torch.zeros(1, 8, 2, 96, device=dev).bfloat16(),
                         torch.ones(1, dtype=torch.int32, device=dev))


@pytest.mark.parametrize("B,Tmax,H,D", [(2, 1024, 12, 64), (16, 512, 12, 64), (3, 300, 4, 128)])
def test_decode_writes_new_key_value(dev, B, Tmax, H, D):
    # k_new / v_new as key lens - 1: the same output, bit for bit, as writing them into
    # the caches first, and the caches hold them afterwards (split segments and one
    # workgroup per (sequence, head) alike)
    from fxlm.attention import decode_attention
    g = torch.Generator(device=dev).manual_seed(B + Tmax + D)
    q = torch.randn(B, H, D, device=dev, generator=g).bfloat16()
    k = torch.randn(B, Tmax, H, D, device=dev, generator=g).bfloat16()
    v = torch.randn(B, Tmax, H, D, device=dev, generator=g).bfloat16()
    qkv_new = torch.randn(B, 3, H, D, device=dev, generator=g).bfloat16()   # strided views
    lens = torch.randint(1, Tmax + 1, (B,), device=dev, generator=g, dtype=torch.int32)
    k2, v2 = k.clone(), v.clone()
    o, lse = decode_attention(q, k, v, lens, return_lse=True, k_new=qkv_new[:, 1], v_new=qkv_new[:, 2])
    rows = (lens.long() - 1)
    bi = torch.arange(B, device=dev)
    k2[bi, rows] = qkv_new[:, 1]
    v2[bi, rows] = qkv_new[:, 2]
    o2, lse2 = decode_attention(q, k2, v2, lens, return_lse=True)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(k, k2) and torch.equal(v, v2)
    with pytest.raises(ValueError):
        decode_attention(q, k, v, lens, k_new=qkv_new[:, 1])
