"""Fused (gather) linear layers on the GPU (fx_linear_fwd / fx_gelu_bwd / fx_linear_dgrad(_gate) /
fx_gelu_bwd_gate / fx_linear_wgrad) against the oracle.

Tolerance (tolerances.oracle_close): |ours - oracle| <= 2^-8 |oracle| + f max|oracle| with
f = 1e-3 for outputs (one rounding of an fp32 product) and f = 4e-3 for gradients (the
bf16 dh between the two backward products).
"""
import pytest
import torch
import torch.nn.functional as F

from golden_util import bf16, f32, load
from oracle import linear as olin
from tolerances import FRAC_GRAD, FRAC_OUT, oracle_close

pytestmark = pytest.mark.gpu


def test_golden_gather(dev):
    from fxgpu.fused_linear import FusedGatherLinear
    d = load("gather_linear")
    X, W, b = bf16(d["X"], dev), bf16(d["W"], dev).requires_grad_(), bf16(d["bias"], dev).requires_grad_()
    idx = torch.from_numpy(d["idx"]).to(dev)
    out = FusedGatherLinear.apply(X, idx, W, b)
    out.backward(bf16(d["gout"], dev))
    assert oracle_close(out, f32(d["out"]), FRAC_OUT)
    assert oracle_close(W.grad, f32(d["dW"]))
    assert oracle_close(b.grad, f32(d["db"]))


def test_golden_linear_gelu(dev):
    from fxgpu.fused_linear import fused_linear
    d = load("linear_gelu")
    x, W = bf16(d["x"], dev).requires_grad_(), bf16(d["W"], dev).requires_grad_()
    y = fused_linear(x, W, None, "gelu_tanh")
    y.backward(bf16(d["dy"], dev))
    assert oracle_close(y, f32(d["y"]), FRAC_OUT)
    assert oracle_close(x.grad, f32(d["dx"]))
    assert oracle_close(W.grad, f32(d["dW"]))


def test_reference_selftest_gather(dev):
    # ml/fxgpu/selftest.py:22-69: R=100k, F=40, W=30, HID=256, B=8192
    from fxgpu.fused_linear import FusedGatherLinear, fused_gather_linear
    torch.manual_seed(0)
    R, Fe, Wn, HID, B = 100_000, 40, 30, 256, 8192
    K = Wn * Fe
    X = torch.randn(R, Fe, device=dev).bfloat16()
    weight = (torch.randn(HID, K, device=dev) * 0.03).bfloat16()
    bias = (torch.randn(HID, device=dev) * 0.01).bfloat16()
    idx = torch.randint(0, R - Wn + 1, (B,), device=dev, dtype=torch.int32)
    xb = X.unfold(0, Wn, 1)[idx.long()].transpose(1, 2).reshape(B, K)
    w_r, b_r = weight.clone().requires_grad_(), bias.clone().requires_grad_()
    out_r = F.linear(xb.float(), w_r.float(), b_r.float())
    w_f, b_f = weight.clone().requires_grad_(), bias.clone().requires_grad_()
    out_f = fused_gather_linear(X, idx, w_f, b_f)
    assert (out_f.detach().double() - out_r.detach().double()).abs().max().item() < 0.05
    g = torch.randn(B, HID, device=dev).bfloat16()
    out_f.backward(g)
    # the reference's backward on the unfolded rows, in fp64: the bf16 dW is its rounding
    # (2^-9 relative) up to the fp32 accumulation order
    from tolerances import bf16_close
    dW_r = g.double().t() @ xb.double()
    assert bf16_close(w_f.grad, dW_r, atol=1e-3 * float(dW_r.abs().max()), rtol=2.0 ** -8)
    assert float((b_f.grad.double() - g.sum(0).double()).abs().max()) < 1e-3
    bad = torch.randn(1000, 37, device=dev).bfloat16()
    with pytest.raises(ValueError, match="multiple of 8"):
        FusedGatherLinear.apply(bad, idx[:8].clamp(max=1000 - Wn),
                                torch.randn(HID, 37 * Wn, device=dev).bfloat16(), bias)
    with torch.no_grad():                # no grad: no Xg write-out, same result
        out_i = fused_gather_linear(X, idx, weight, bias)
    assert torch.equal(out_i, out_f.detach())


def test_gather_window_outside_reads_zero(dev):
    from fxgpu.fused_linear import fused_gather_linear
    X = torch.randn(20, 8, device=dev).bfloat16()
    W = torch.randn(4, 24, device=dev).bfloat16()
    b = torch.zeros(4, device=dev).bfloat16()
    idx = torch.tensor([0, 17, -1, 18], device=dev, dtype=torch.int32)   # windows of 3 rows
    out = fused_gather_linear(X, idx, W, b)
    assert float(out[2].abs().max()) == 0.0 and float(out[3].abs().max()) == 0.0
    assert float(out[1].abs().max()) > 0.0


@pytest.mark.parametrize("M,K,N,bias", [(300, 768, 3072, False), (77, 40, 100, True), (1, 8, 1, True),
                                        (513, 256, 129, False), (300, 200, 300, True)])
def test_linear_gelu_against_oracle(dev, M, K, N, bias):
    from fxgpu.fused_linear import fused_linear
    torch.manual_seed(M + K + N)
    x = torch.randn(M, K).bfloat16()
    W = (torch.randn(N, K) * K ** -0.5).bfloat16()
    b = (torch.randn(N) * 0.1).bfloat16() if bias else None
    dy = torch.randn(M, N).bfloat16()
    xg, Wg = x.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    bg = b.to(dev).requires_grad_() if bias else None
    y = fused_linear(xg, Wg, bg, "gelu_tanh")
    y.backward(dy.to(dev))
    ry, rh = olin.linear_act_fwd(x, W, b)
    rdx, rdW, rdb = olin.linear_act_bwd(x, W, rh, dy)
    assert oracle_close(y, ry, FRAC_OUT)
    assert oracle_close(xg.grad, rdx)
    assert oracle_close(Wg.grad, rdW)
    if bias:
        assert oracle_close(bg.grad, rdb)


def test_cfg5_mlp_shape(dev):
    # the GPT MLP fc at cfg5: (16384 x 768) . (3072 x 768)^T -> GELU, vs fp32 torch math
    from fxgpu.fused_linear import fused_linear
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(16384, 768, device=dev, generator=g).bfloat16()
    W = (torch.randn(3072, 768, device=dev, generator=g) * 0.02).bfloat16()
    y = fused_linear(x, W, None, "gelu_tanh")
    ref = F.gelu(x.float() @ W.float().t(), approximate="tanh")
    assert oracle_close(y, ref, FRAC_OUT)


def test_gather_more_tiles_than_workgroups(dev):
    # 17 x 16 = 272 output tiles of 256 x 256: more than one tile per persistent
    # workgroup, so the next tile's loads run during an epilogue and the gathered rows
    # (Xg) are written by workgroups that hold several tiles; windows of 4 rows x 64
    from fxgpu.fused_linear import FusedGatherLinear
    g = torch.Generator(device=dev).manual_seed(11)
    R, F_, Wn, M, N = 5000, 64, 4, 4352, 4096
    X = torch.randn(R, F_, device=dev, generator=g).bfloat16()
    idx = torch.randint(0, R - Wn + 1, (M,), device=dev, dtype=torch.int32, generator=g)
    W = (torch.randn(N, Wn * F_, device=dev, generator=g) * 0.05).bfloat16().requires_grad_()
    b = torch.randn(N, device=dev, generator=g).bfloat16().requires_grad_()
    out = FusedGatherLinear.apply(X, idx, W, b)
    xg = X.unfold(0, Wn, 1)[idx.long()].transpose(1, 2).reshape(M, Wn * F_)
    ref = xg.float() @ W.detach().float().t() + b.detach().float()
    assert oracle_close(out, ref, FRAC_OUT)
    # dW = g^T Xg uses the gathered rows the forward wrote out
    gy = (torch.randn(M, N, device=dev, generator=g) * 0.01).bfloat16()
    out.backward(gy)
    rdw = gy.float().t() @ xg.float()
    assert oracle_close(W.grad, rdw)


# ---- weight gradient dW = dY^T X (split-K GEMM) --------------------------------------
# Elementwise bound: the bf16 rounding of the result (2^-9 relative, 2^-8 allowed) plus
# 1e-3 of the largest |dW| for the fp32 accumulation over T tokens; a wrong slice,
# transposed operand or dropped K step is off by O(1) relative.

@pytest.mark.parametrize("T,N,K", [
    (16384, 768, 3072),   # cfg5 fc2 dW
    (16384, 3072, 768),   # cfg5 fc dW
    (16384, 2304, 768),   # cfg5 qkv dW
    (16384, 768, 768),    # cfg5 proj dW
    (100, 64, 40),        # one slice, ragged token tail, N and K below a tile
    (1000, 8, 2056),      # several slices, K past a tile boundary
    (333, 264, 520),      # ragged everywhere
    (1, 16, 8),
])
def test_wgrad_against_fp64(dev, T, N, K):
    from fxgpu.fused_linear import linear_wgrad
    from tolerances import bf16_close
    g = torch.Generator(device=dev).manual_seed(T * 7 + N * 3 + K)
    dy = torch.randn(T, N, device=dev, generator=g).bfloat16()
    x = torch.randn(T, K, device=dev, generator=g).bfloat16()
    dW = linear_wgrad(dy, x)
    ref = dy.double().t() @ x.double()
    scale = float(ref.abs().max())
    assert dW.shape == (N, K) and dW.dtype == torch.bfloat16
    assert bf16_close(dW, ref, atol=1e-3 * scale, rtol=2.0 ** -8)


def test_wgrad_strided_rows(dev):
    # dy and x as column windows of wider row-major buffers (row strides > width)
    from fxgpu.fused_linear import linear_wgrad
    from tolerances import bf16_close
    g = torch.Generator(device=dev).manual_seed(5)
    big_dy = torch.randn(2048, 800, device=dev, generator=g).bfloat16()
    big_x = torch.randn(2048, 520, device=dev, generator=g).bfloat16()
    dy, x = big_dy[:, 16:16 + 768], big_x[:, 8:8 + 512]
    dW = linear_wgrad(dy, x)
    ref = dy.double().t() @ x.double()
    assert bf16_close(dW, ref, atol=1e-3 * float(ref.abs().max()), rtol=2.0 ** -8)


def test_wgrad_no_tokens(dev):
    from fxgpu.fused_linear import linear_wgrad
    dW = linear_wgrad(torch.empty(0, 64, device=dev).bfloat16(), torch.empty(0, 32, device=dev).bfloat16())
    assert dW.shape == (64, 32) and int((dW != 0).sum()) == 0


def test_wgrad_rejects_bad_shapes(dev):
    from fxgpu.abi import call, ptr
    from fxgpu.fused_linear import linear_wgrad
    with pytest.raises(ValueError):
        linear_wgrad(torch.zeros(4, 16, device=dev).bfloat16(), torch.zeros(5, 16, device=dev).bfloat16())
    # the C ABI itself refuses widths that are not multiples of 8
    a = torch.zeros(4, 12, device=dev).bfloat16()
    b = torch.zeros(4, 16, device=dev).bfloat16()
    w = torch.zeros(12, 16, device=dev).bfloat16()
    with pytest.raises(ValueError, match="multiples of 8"):
        call("fx_linear_wgrad", ptr(a), 12, ptr(b), 16, ptr(w), 16, None, 12, 16, 4, None)


def test_linear_autograd_against_fp32(dev):
    from fxgpu.fused_linear import linear
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(4, 256, 768, device=dev, generator=g).bfloat16()
    W = (torch.randn(2304, 768, device=dev, generator=g) * 0.02).bfloat16()
    dy = torch.randn(4, 256, 2304, device=dev, generator=g).bfloat16()
    xa, Wa = x.clone().requires_grad_(), W.clone().requires_grad_()
    y = linear(xa, Wa)
    y.backward(dy)
    xr, Wr = x.float().requires_grad_(), W.float().requires_grad_()
    yr = xr @ Wr.t()
    yr.backward(dy.float())
    assert oracle_close(y, yr, FRAC_OUT)
    assert oracle_close(xa.grad, xr.grad)
    assert oracle_close(Wa.grad, Wr.grad)


# ---- few-row forward (M <= 64: decode steps, small batches) ---------------------------

@pytest.mark.parametrize("M,K,N,bias", [
    (1, 768, 2304, False),     # one sequence's decode step (qkv)
    (16, 768, 3072, True),     # batch-16 decode fc: K split over 8 waves
    (16, 3072, 768, False),    # fc2: 16 waves per workgroup
    (17, 40, 100, True),       # K not a multiple of 32, N not of 16, two row tiles of X
    (33, 200, 129, False),
    (64, 8, 1, True),          # the largest few-row M, K = 8
    (16, 768, 50257, False),   # the LM head: two W row tiles per workgroup
])
def test_few_rows_against_oracle(dev, M, K, N, bias):
    from fxgpu.fused_linear import fused_linear
    torch.manual_seed(M * 7 + K + N)
    x = torch.randn(M, K).bfloat16()
    W = (torch.randn(N, K) * K ** -0.5).bfloat16()
    b = (torch.randn(N) * 0.1).bfloat16() if bias else None
    xg, Wg = x.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    bg = b.to(dev).requires_grad_() if bias else None
    y = fused_linear(xg, Wg, bg, "gelu_tanh")      # with a gradient: writes h as well
    ry, rh = olin.linear_act_fwd(x, W, b)
    assert oracle_close(y, ry, FRAC_OUT)
    dy = torch.randn(M, N).bfloat16()
    y.backward(dy.to(dev))                          # dh = dy gelu'(h) reads the stored h
    rdx, rdW, _ = olin.linear_act_bwd(x, W, rh, dy)
    assert oracle_close(xg.grad, rdx)
    assert oracle_close(Wg.grad, rdW)
    with torch.no_grad():                           # identity, no bias: plain x W^T
        from fxgpu.fused_linear import linear
        y0 = linear(x.to(dev), W.to(dev))
    assert oracle_close(y0, x.double() @ W.double().t(), FRAC_OUT)


def test_few_rows_and_tiled_agree_on_golden(dev):
    # the golden fixture (12 rows) through the few-row kernel, and stacked six times
    # (72 rows) through the tiled kernel: every copy matches the reference's values
    from fxgpu.fused_linear import fused_linear
    d = load("linear_gelu")
    x, W = bf16(d["x"], dev), bf16(d["W"], dev)
    with torch.no_grad():
        y_few = fused_linear(x, W, None, "gelu_tanh")
        y_tiled = fused_linear(x.repeat(6, 1), W, None, "gelu_tanh")
    assert oracle_close(y_few, f32(d["y"]), FRAC_OUT)
    for i in range(6):
        assert oracle_close(y_tiled[12 * i:12 * (i + 1)], f32(d["y"]), FRAC_OUT)


def test_few_rows_gather_writes_windows(dev):
    # 40 gathered rows (windows of 6 rows x 16 features), one leaving X: the forward on the
    # few-row kernel, Xg written by its first workgroup and used by the dW of the backward
    from fxgpu.fused_linear import FusedGatherLinear
    g = torch.Generator(device=dev).manual_seed(21)
    R, Fe, Wn, N = 300, 16, 6, 200
    X = torch.randn(R, Fe, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, Fe * Wn, device=dev, generator=g) * 0.1).bfloat16().requires_grad_()
    b = (torch.randn(N, device=dev, generator=g) * 0.1).bfloat16().requires_grad_()
    idx = torch.randint(0, R - Wn + 1, (40,), device=dev, dtype=torch.int32, generator=g)
    idx[7] = R - 2                                     # window leaves X: zeros
    out = FusedGatherLinear.apply(X, idx, W, b)
    ref, Xg = olin.gather_linear(X, idx, W, b)
    assert oracle_close(out, ref, FRAC_OUT)
    gout = torch.randn(40, N, device=dev, generator=g).bfloat16()
    out.backward(gout)
    assert float(Xg[7].abs().max()) == 0.0
    rdW = gout.double().cpu().t() @ Xg
    assert oracle_close(W.grad, rdW)


# ---- inference forward with the input norm and output residual folded in -----------

@pytest.mark.parametrize("M,K,N,norm,res,act", [
    (16, 768, 2304, True, False, None),        # a decode step's qkv: norm inside
    (16, 768, 3072, True, False, "gelu_tanh"),  # fc: norm + GELU
    (16, 768, 768, False, True, None),          # proj: residual inside
    (1, 3072, 768, False, True, None),          # fc2 of one sequence
    (64, 200, 129, True, True, "gelu_tanh"),    # everything, ragged K / N, 64 rows
    (300, 256, 520, False, True, None),         # residual on the tiled kernel (M > 64)
])
def test_linear_ex_against_oracle(dev, M, K, N, norm, res, act):
    from fxgpu.fused_linear import linear_ex
    from oracle import norm as onorm
    torch.manual_seed(M + K + N)
    x = torch.randn(M, K).bfloat16()
    W = (torch.randn(N, K) * K ** -0.5).bfloat16()
    b = (torch.randn(N) * 0.1).bfloat16()
    nw = (torch.randn(K) * 0.1 + 1).bfloat16() if norm else None
    r = (torch.randn(M, N) * 0.5).bfloat16() if res else None
    y = linear_ex(x.to(dev), W.to(dev), bias=b.to(dev), residual=r.to(dev) if res else None,
                  norm_weight=nw.to(dev) if norm else None, eps=1e-6, activation=act)
    # reference: the norm's bf16 output (as the RMSNorm forward writes it), then the GEMM
    h = onorm.rms_norm_fwd(x, nw, 1e-6)[0].to(torch.bfloat16) if norm else x
    z = h.double() @ W.double().t() + b.double()
    if act:
        z = olin.gelu_tanh(z)
    if res:
        z = z + r.double()
    assert oracle_close(y, z, FRAC_OUT)


def test_linear_ex_rejects(dev):
    from fxgpu.fused_linear import linear_ex
    x = torch.zeros(65, 64, device=dev, dtype=torch.bfloat16)
    W = torch.zeros(32, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="at most"):
        linear_ex(x, W, norm_weight=torch.ones(64, device=dev, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        linear_ex(x, W, residual=torch.zeros(65, 31, device=dev, dtype=torch.bfloat16))


# ---- whole-tile kernel (M % 256 == 0, N % 192 or % 256 == 0, K % 96 == 0) ----------------
# fx_linear_fwd takes such shapes on its hand-scheduled kernel.  It computes the same MFMAs
# on the same operands in the same K order as the general tiled kernel and rounds the same
# way, so the two agree bit for bit.  The general kernel's result for an element does not
# depend on M or N, so it is read from the same operands with 8 more rows and columns
# (a shape the whole-tile kernel does not take).

def _linear_fwd(x, W, b, act, want_h):
    from fxgpu.abi import call, ptr, stream_of
    M, K = x.shape
    N = W.shape[0]
    y = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    h = torch.empty_like(y) if want_h else None
    call("fx_linear_fwd", ptr(x), x.stride(0), None, 0, 0, ptr(W), ptr(b), ptr(y), ptr(h), None, M, N, K, act,
         stream_of(x))
    return y, h


@pytest.mark.parametrize("M,K,N,act,bias,want_h,pad_k", [
    (512, 128, 256, 1, True, True, 0),     # 256-wide tiles; 4 K steps: the loop's tail only
    (512, 256, 192, 0, False, False, 0),   # 192-wide tiles, one loop iteration
    (1024, 768, 768, 0, False, False, 64), # proj: 192-wide (a round of 16 tiles), rows of X strided
    (768, 768, 2304, 0, True, False, 0),   # qkv widths
    (256, 3072, 768, 1, False, True, 0),   # fc2 depth
    (16384, 768, 3072, 1, False, True, 0), # the cfg5 MLP fc (256-wide tiles): GELU and the pre-activation
    (512, 160, 256, 1, True, True, 0),     # 5 K steps: a leading zero step makes 6 (entry at the body's third)
    (512, 192, 192, 0, False, False, 8),   # 6 K steps: enters the loop body at its third step
    (512, 224, 256, 0, True, False, 0),    # 7 K steps: 8 with the zero step (the body from its first)
    (256, 288, 192, 1, False, True, 0),    # 9 K steps: 10 with the zero step
])
def test_whole_tile_kernel_matches_general_kernel(dev, M, K, N, act, bias, want_h, pad_k):
    g = torch.Generator(device=dev).manual_seed(M + K + N)
    xs = torch.randn(M + 8, K + pad_k, device=dev, generator=g).bfloat16()
    Ws = (torch.randn(N + 8, K, device=dev, generator=g) * K ** -0.5).bfloat16()
    bs = (torch.randn(N + 8, device=dev, generator=g) * 0.1).bfloat16() if bias else None
    x, W, b = xs[:M, :K], Ws[:N], (bs[:N] if bias else None)
    print(f"whole-tile fwd M={M} K={K} N={N} act={act} bias={bias} h={want_h} ldx={x.stride(0)}", flush=True)
    y, h = _linear_fwd(x, W, b, act, want_h)
    y_gen, h_gen = _linear_fwd(xs[:, :K], Ws, bs, act, want_h)
    torch.cuda.synchronize()
    assert torch.equal(y, y_gen[:M, :N])
    if want_h:
        assert torch.equal(h, h_gen[:M, :N])
    ref = x.float() @ W.float().t() + (b.float() if bias else 0)
    if want_h:
        assert oracle_close(h, ref, FRAC_OUT)
    if act:
        ref = F.gelu(ref, approximate="tanh")
    assert oracle_close(y, ref, FRAC_OUT)


# ---- whole-tile weight gradient (M, N % 256 == 0, T % 32 == 0, T >= 96) -------------------
# Same slices, token ranges and MFMA order as the general split-K kernel, so the two agree bit
# for bit; FX_GEMM_GENERAL=1 (read on every call) routes the product to the general kernel.

@pytest.mark.parametrize("T,M,N,ld_pad", [
    (128, 256, 256, 0),      # 4 steps: the loop's tail only, one slice (bf16 written directly)
    (160, 256, 512, 0),      # 5 steps: enters the loop body at its fourth step
    (192, 512, 256, 8),      # 6 steps: enters at the third; rows of dY and X strided
    (224, 256, 256, 0),      # 7 steps: enters at the second
    (544, 256, 512, 0),      # 2 slices of 8 and 9 steps
    (4096, 768, 768, 0),     # proj-shaped: 9 tiles x 28 slices
    (16384, 3072, 768, 0),   # the cfg5 fc weight (7 slices of 36-37 64-token steps; 5 with 192-wide tiles)
    (2048, 768, 2304, 0),    # qkv widths, 192-wide tiles divide both
    (256, 392, 384, 8),      # M not a multiple of 256: a 136-row last panel (clamped loads, masked rows)
    (1024, 520, 768, 0),     # an 8-row last panel, several slices
    (16384, 50304, 768, 0),  # the cfg5 tied head: 768 tiles in one slice, the last 20 (4.5 panels) in 12
    (1024, 16776, 768, 0),   # 264 tiles: 256 in one slice, the last 1.5 panels in 4 slices
    (1024, 16740, 1024, 0),  # 256 x 256 tiles (N % 192 != 0): 264 tiles, the last 1.4 panels in 4 slices
    (256, 16384, 3072, 0),   # 1024 tiles: four whole rounds, one slice, no tail
])
@pytest.mark.parametrize("tile", ["256", "192"])   # FX_WGRAD_TILE=256: 256 x 256 tiles; else 256 x 192 where N allows
def test_wgrad_whole_tile_kernel_matches_general(dev, monkeypatch, T, M, N, ld_pad, tile):
    if M == 50304 and tile == "256":
        pytest.skip("N = 768 has no 256-wide whole tiles: same as the 192 case")
    from fxgpu.fused_linear import linear_wgrad
    monkeypatch.setenv("FX_WGRAD_TILE", tile)
    g = torch.Generator(device=dev).manual_seed(T + M + N)
    dy = torch.randn(T, M + ld_pad, device=dev, generator=g).bfloat16()[:, :M]
    x = torch.randn(T, N + ld_pad, device=dev, generator=g).bfloat16()[:, :N]
    print(f"whole-tile wgrad T={T} M={M} N={N} ldy={dy.stride(0)} tile={tile}", flush=True)
    dw = linear_wgrad(dy, x)
    monkeypatch.setenv("FX_GEMM_GENERAL", "1")
    dw_gen = linear_wgrad(dy, x)
    monkeypatch.delenv("FX_GEMM_GENERAL")
    torch.cuda.synchronize()
    assert torch.equal(dw, dw_gen)
    ref = dy.double().t() @ x.double()
    from tolerances import bf16_close
    assert bf16_close(dw, ref, atol=1e-3 * float(ref.abs().max()), rtol=2.0 ** -8)


# ---- whole-tile input gradient dX = dY W (fx_linear_dgrad), optionally with the GELU backward -----
# Against the fp32 product (tolerance as for the forward), and with H against the unfused pair
# (fx_linear_dgrad, then fx_gelu_bwd) bit for bit.

def _dgrad(dy, W, h=None):
    from fxgpu.abi import call, ptr, stream_of
    M, K = dy.shape
    N = W.shape[1]
    dx = torch.empty(M, N, device=dy.device, dtype=torch.bfloat16)
    call("fx_linear_dgrad", ptr(dy), dy.stride(0), ptr(W), W.stride(0), ptr(h), ptr(dx), N, M, N, K, stream_of(dy))
    return dx


@pytest.mark.parametrize("M,N,K,pad", [
    (256, 256, 128, 0),      # 256-wide tiles, the loop's tail only
    (512, 192, 160, 0),      # 192-wide tiles, 5 K steps (with the leading zero step, 6)
    (256, 768, 224, 8),      # 7 K steps (8 with the zero step); rows of dY strided
    (256, 256, 192, 0),      # 6 K steps: enters the loop body at its third step
    (512, 192, 256, 8),      # 8 K steps: the body from its first
    (256, 768, 288, 0),      # 9 K steps (10 with the zero step)
    (1024, 3072, 768, 0),    # fc2's input gradient shape (192-wide tiles at this M)
    (16384, 3072, 768, 0),   # cfg5 fc2 (256-wide tiles, 768 tiles)
    (16384, 768, 2304, 0),   # cfg5 qkv
])
def test_dgrad_whole_tile_kernel(dev, M, N, K, pad):
    from fxgpu.abi import call, ptr, stream_of
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    dy = torch.randn(M, K + pad, device=dev, generator=g).bfloat16()[:, :K]
    W = (torch.randn(K, N, device=dev, generator=g) * K ** -0.5).bfloat16()
    h = torch.randn(M, N, device=dev, generator=g).bfloat16()
    print(f"whole-tile dgrad M={M} N={N} K={K} ldy={dy.stride(0)}", flush=True)
    dx = _dgrad(dy, W)
    dh = _dgrad(dy, W, h)
    dh_pair = torch.empty_like(dx)
    call("fx_gelu_bwd", ptr(dx), ptr(h), ptr(dh_pair), dx.numel(), stream_of(dx))
    torch.cuda.synchronize()
    assert torch.equal(dh, dh_pair)
    ref = dy.float() @ W.float()
    assert oracle_close(dx, ref, FRAC_OUT)


def test_dgrad_rejects_partial_tiles(dev):
    from fxgpu.abi import call, ptr, stream_of
    dy = torch.zeros(300, 128, device=dev, dtype=torch.bfloat16)
    W = torch.zeros(128, 256, device=dev, dtype=torch.bfloat16)
    dx = torch.empty(300, 256, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="whole tiles"):
        call("fx_linear_dgrad", ptr(dy), 128, ptr(W), 256, None, ptr(dx), 256, 300, 256, 128, stream_of(dy))
    with pytest.raises(ValueError, match="whole tiles"):      # 3 K steps: fewer than the loop's 4
        call("fx_linear_dgrad", ptr(dy), 128, ptr(W), 256, None, ptr(dx), 256, 256, 256, 96, stream_of(dy))


# ---- the GELU derivative stored by the forward (act 2) and multiplied in the backward --------

@pytest.mark.parametrize("M,K,N,bias,path", [
    (512, 256, 512, True, "whole"),     # 256-wide whole tiles, with bias
    (512, 160, 192, False, "whole"),    # 192-wide whole tiles, 5 K steps (the leading zero step)
    (16384, 768, 3072, False, "whole"), # the cfg5 MLP fc
    (300, 96, 200, True, "general"),    # partial tiles: the general kernel
    (40, 64, 72, True, "few"),          # few rows
])
def test_linear_fwd_gelu_derivative(dev, monkeypatch, M, K, N, bias, path):
    g = torch.Generator(device=dev).manual_seed(M + K + N)
    x = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, K, device=dev, generator=g) * K ** -0.5).bfloat16()
    b = (torch.randn(N, device=dev, generator=g) * 0.3).bfloat16() if bias else None
    print(f"gelu derivative fwd M={M} K={K} N={N} bias={bias} path={path}", flush=True)
    y1, _ = _linear_fwd(x, W, b, 1, True)
    y2, d2 = _linear_fwd(x, W, b, 2, True)
    y3, _ = _linear_fwd(x, W, b, 2, False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, y3)       # the same GELU output, bit for bit
    h = x.double() @ W.double().t() + (b.double() if bias else 0)
    assert oracle_close(d2, olin.gelu_tanh_grad(h.cpu()), FRAC_OUT)
    if path == "whole":   # the general kernel evaluates the same expression
        monkeypatch.setenv("FX_GEMM_GENERAL", "f")
        y4, d4 = _linear_fwd(x, W, b, 2, True)
        torch.cuda.synchronize()
        assert torch.equal(y4, y2) and torch.equal(d4, d2)


def _dgrad_gate(dy, W, gd):
    from fxgpu.abi import call, ptr, stream_of
    M, K = dy.shape
    N = W.shape[1]
    dx = torch.empty(M, N, device=dy.device, dtype=torch.bfloat16)
    call("fx_linear_dgrad_gate", ptr(dy), dy.stride(0), ptr(W), W.stride(0), ptr(gd), ptr(dx), N, M, N, K,
         stream_of(dy))
    return dx


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (512, 192, 160), (256, 768, 224), (16384, 3072, 768)])
def test_dgrad_gate_matches_the_pair(dev, M, N, K):
    from fxgpu.abi import call, ptr, stream_of
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    dy = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(K, N, device=dev, generator=g) * K ** -0.5).bfloat16()
    gd = (torch.rand(M, N, device=dev, generator=g) * 1.3 - 0.15).bfloat16()   # the range of gelu'
    print(f"dgrad gate M={M} N={N} K={K}", flush=True)
    got = _dgrad_gate(dy, W, gd)
    dx = _dgrad(dy, W)
    pair = torch.empty_like(dx)
    call("fx_gelu_bwd_gate", ptr(dx), ptr(gd), ptr(pair), dx.numel(), stream_of(dx))
    torch.cuda.synchronize()
    assert torch.equal(got, pair)
    ref = (dy.double() @ W.double()) * gd.double()
    assert oracle_close(got, ref, FRAC_GRAD)   # two roundings: the bf16 product, then dh


@pytest.mark.parametrize("n", [0, 5, 8 * 997 + 3, 16384 * 3072])
def test_gelu_bwd_gate_is_the_rounded_product(dev, n):
    from fxgpu.abi import call, ptr, stream_of
    g = torch.Generator(device=dev).manual_seed(n)
    a = torch.randn(max(n, 1), device=dev, generator=g).bfloat16()[:n]
    b = torch.randn(max(n, 1), device=dev, generator=g).bfloat16()[:n]
    out = torch.empty_like(a)
    call("fx_gelu_bwd_gate", ptr(a), ptr(b), ptr(out), n, stream_of(a))
    torch.cuda.synchronize()
    # a product of two bf16 values is exact in fp32, so one rounding to nearest even decides
    assert torch.equal(out.cpu(), (a.float().cpu() * b.float().cpu()).bfloat16())


# ---- the GPT MLP as one node (fused_mlp): GELU and its derivative in the fc epilogue, the
# product with the derivative in the fc2 input gradient's epilogue --------------------------------

@pytest.mark.parametrize("native", [True, False])  # the whole-tile kernels where shapes allow, or the library
@pytest.mark.parametrize("M,K,Fh,N", [(512, 256, 1024, 256),     # whole tiles: fx_linear_dgrad_gate
                                      (300, 64, 256, 64),        # partial tiles: library GEMM + fx_gelu_bwd_gate
                                      (16384, 768, 3072, 768)])  # cfg5
def test_fused_mlp_against_composition_and_fp32(dev, monkeypatch, native, M, K, Fh, N):
    import fxgpu.fused_linear as FL
    monkeypatch.setattr(FL, "NATIVE_INPUT_GRAD", native)
    monkeypatch.setattr(FL, "NATIVE_PROJ_FWD", native)
    monkeypatch.setattr(FL, "NATIVE_GELU_INPUT_GRAD", native)
    g = torch.Generator(device=dev).manual_seed(M + Fh)
    x = torch.randn(M, K, device=dev, generator=g).bfloat16()
    w1 = (torch.randn(Fh, K, device=dev, generator=g) * K ** -0.5).bfloat16()
    w2 = (torch.randn(N, Fh, device=dev, generator=g) * Fh ** -0.5).bfloat16()
    dy = torch.randn(M, N, device=dev, generator=g).bfloat16()
    print(f"fused_mlp M={M} K={K} F={Fh} N={N}", flush=True)
    xa, w1a, w2a = (t.clone().requires_grad_() for t in (x, w1, w2))
    y = FL.fused_mlp(xa, w1a, w2a)
    y.backward(dy)
    xb, w1b, w2b = (t.clone().requires_grad_() for t in (x, w1, w2))
    yb = FL.linear(FL.fused_linear(xb, w1b, None, "gelu_tanh"), w2b)
    yb.backward(dy)
    assert torch.equal(y, yb)                      # the same forward kernels
    xr, w1r, w2r = (t.float().requires_grad_() for t in (x, w1, w2))
    yr = F.gelu(xr @ w1r.t(), approximate="tanh") @ w2r.t()
    yr.backward(dy.float())
    assert oracle_close(y, yr, 4e-3)               # through the bf16 GELU output
    for ours, comp, ref in ((xa.grad, xb.grad, xr.grad), (w1a.grad, w1b.grad, w1r.grad),
                            (w2a.grad, w2b.grad, w2r.grad)):
        assert oracle_close(ours, ref)
        assert oracle_close(comp, ref)
