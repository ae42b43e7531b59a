"""Parity tolerances of this build's kernels against the oracle, stated once for every test.

* Attention and linear outputs / gradients (bf16 results of bf16 inputs):
  max |ours - fp32 oracle| <= 2e-2.
* bf16 results of larger magnitude (RMSNorm y/dx on N(0, 3) inputs, the
  reference selftest's distribution): |ours - oracle| <= 2e-2 + 2^-8 |oracle|
  (the bf16 rounding of the result alone is up to 2^-9 |oracle|).
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
    return float((a.double().cpu() - b.double().cpu()).abs().max()) if a.numel() else 0.0


def bf16_close(ours, ref, atol=ATOL_BF16, rtol=RTOL_BF16):
    """True when |ours - ref| <= atol + rtol |ref| elementwise."""
    o, r = ours.double().cpu(), ref.double().cpu()
    return bool(((o - r).abs() <= atol + rtol * r.abs()).all())


def rel_err(ours, ref):
    o, r = ours.double().cpu(), ref.double().cpu()
    den = r.abs().max().clamp_min(1e-30)
    return float((o - r).abs().max() / den)
