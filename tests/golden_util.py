"""Loading helpers for the golden fixtures (numpy, allow_pickle=False)."""
import os

import numpy as np
import torch

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf16(a, device="cpu"):
    """uint16 bit patterns -> bf16 tensor."""
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(device)


def f32(a, device="cpu"):
    return torch.from_numpy(np.asarray(a, dtype=np.float32).copy()).to(device)
