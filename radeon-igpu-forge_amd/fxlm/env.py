"""fxlm.env: environment defaults and the gfx950 device check for LM training.

Counterpart of ml/fxlm/env.py:11-48.  ``setup_lm_env()`` must run before
``import torch``; this module does not import torch at import time.
"""
import os

from fxgpu.env import require_gpu  # noqa: F401  (same check for both packages)


def setup_lm_env(tunable=False, tune_file=None):
    """Set TunableOp on/off (overrides existing values) and its CSV path."""
    os.environ["PYTORCH_TUNABLEOP_ENABLED"] = "1" if tunable else "0"
    os.environ.setdefault("PYTORCH_TUNABLEOP_MAX_TUNING_DURATION_MS", "100")
    if tune_file is not None:
        os.environ["PYTORCH_TUNABLEOP_FILENAME"] = str(tune_file)
