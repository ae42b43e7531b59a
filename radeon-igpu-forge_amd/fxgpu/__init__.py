"""fxgpu: MI355X (gfx950) kernel loader and the fused (gather) linear layer.

Lazy exports, as in ml/fxgpu/__init__.py:10-27: modules that need torch are
imported on first attribute access, so ``from fxgpu.env import setup_env``
works before torch is imported.
"""

__all__ = [
    "FusedGatherLinear",
    "fused_gather_linear",
    "FusedLinear",
    "fused_linear",
    "FusedMLP",
    "fused_mlp",
    "setup_env",
    "require_gpu",
]


def __getattr__(name):
    if name in ("FusedGatherLinear", "fused_gather_linear", "FusedLinear", "fused_linear", "FusedMLP", "fused_mlp"):
        from . import fused_linear as _m
        return getattr(_m, name)
    if name in ("setup_env", "require_gpu"):
        from . import env as _m
        return getattr(_m, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
