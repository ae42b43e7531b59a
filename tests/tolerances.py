"""Parity tolerances of this build's kernels against the oracle, stated once for every test.

* Attention and linear outputs / gradients (bf16 results of bf16 inputs):
  |ours - oracle| <= 2^-8 |oracle| + f * max|oracle| elementwise (`oracle_close`), with
  f = FRAC_OUT = 1e-3 for a product rounded once (linear outputs) and f = FRAC_GRAD =
  4e-3 for results that pass through bf16 intermediates (attention's P and dS, the
  linear backward's dh): twice the largest excess measured over the test shapes
  (2.0e-3 for attention dQ, 2.2e-3 for a linear dW), so that a systematic error of a
  percent of the largest value anywhere fails.
* RMSNorm y / dx / dw (bf16, each one rounding of an fp32 result): `oracle_close` with
  f = FRAC_OUT.
* fp32 scalars and fp32 norm quantities (CE loss, rstd, fp32 dw, grad norm):
  relative error <= 1e-3.
* FlatAdamW fp32 master update: max |ours - oracle| / max |oracle| <= 1e-6.
"""
ATOL_BF16 = 2e-2
RTOL_BF16 = 2.0 ** -8
RTOL_LOSS = 1e-3
RTOL_NORM = 1e-3
RTOL_ADAMW = 1e-6


def max_abs(a, b):
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max()) if a.numel() else 0.0


def bf16_close(ours, ref, atol=ATOL_BF16, rtol=RTOL_BF16):
    """True when |ours - ref| <= atol + rtol |ref| elementwise."""
    o, r = ours.detach().double().cpu(), ref.detach().double().cpu()
    return bool(((o - r).abs() <= atol + rtol * r.abs()).all())


FRAC_OUT = 1e-3
FRAC_GRAD = 4e-3


def oracle_close(ours, ref, frac=FRAC_GRAD):
    """|ours - ref| <= 2^-8 |ref| + frac * max|ref| elementwise (bf16 results)."""
    r = ref.detach().double().cpu()
    return bf16_close(ours, r, atol=frac * float(r.abs().max()) + 1e-9, rtol=RTOL_BF16)


def rel_err(ours, ref):
    o, r = ours.detach().double().cpu(), ref.detach().double().cpu()
    den = r.abs().max().clamp_min(1e-30)
    return float((o - r).abs().max() / den)
