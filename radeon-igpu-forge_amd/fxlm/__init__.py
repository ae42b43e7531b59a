"""fxlm: small-GPT training hot path on MI355X (gfx950).

Hand-written HIP kernels behind the reference's Python surface
(ml/fxlm/__init__.py:13-46):
  - flash attention fwd/bwd (bf16 I/O, fp32 softmax, MFMA)
  - fused cross-entropy and linear cross-entropy
  - fused RMSNorm
  - FlatAdamW (fp32 master + bf16 params + dynamic loss scale)

Lazy exports: ``from fxlm.env import setup_lm_env`` does not import torch.
"""

__all__ = [
    "setup_lm_env",
    "require_gpu",
    "flash_attention",
    "flash_attention_qkv",
    "fused_cross_entropy",
    "linear_cross_entropy",
    "rms_norm",
    "FlatAdamW",
    "GPT",
    "GPTConfig",
]


def __getattr__(name):
    if name in ("setup_lm_env", "require_gpu"):
        from . import env as _m
        return getattr(_m, name)
    if name in ("flash_attention", "flash_attention_qkv"):
        from . import attention as _m
        return getattr(_m, name)
    if name in ("fused_cross_entropy", "linear_cross_entropy"):
        from . import cross_entropy as _m
        return getattr(_m, name)
    if name == "rms_norm":
        from .norm import rms_norm
        return rms_norm
    if name == "FlatAdamW":
        from .optim import FlatAdamW
        return FlatAdamW
    if name in ("GPT", "GPTConfig"):
        from . import model as _m
        return getattr(_m, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
