"""fxgpu.env: environment defaults and the gfx950 device check.

Counterpart of ml/fxgpu/env.py:8-45 for MI355X.  ``setup_env()`` must run
before ``import torch``; this module does not import torch at import time.
"""
import os

ENV_DEFAULTS = {
    # hipBLASLt picks its kernels by heuristics on gfx950; TunableOp stays off
    # unless a caller opts in.
    "PYTORCH_TUNABLEOP_ENABLED": "0",
}

ARCH = "gfx950"


def setup_env():
    """Set the environment defaults with setdefault (existing values win)."""
    for k, v in ENV_DEFAULTS.items():
        os.environ.setdefault(k, v)


def require_gpu():
    """Return torch.device("cuda") when device 0 is a gfx950; SystemExit otherwise."""
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("no GPU: torch.cuda.is_available() is False")
    props = torch.cuda.get_device_properties(0)
    arch = str(getattr(props, "gcnArchName", "?"))
    if not arch.startswith(ARCH):
        raise SystemExit(f"expected {ARCH}, found {arch} ({props.name}); the kernels "
                         f"are built for {ARCH} only")
    print(f"torch {torch.__version__} | HIP {torch.version.hip} | {props.name} ({arch})")
    return torch.device("cuda")
