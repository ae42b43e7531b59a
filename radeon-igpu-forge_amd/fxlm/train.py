"""fxlm.train: the data format, LR schedule and checkpoints of the fxlm training loop.

Library form of what ml/fxlm/train_lm.py and ml/fxlm/prepare_bytes.py do around the
GPU step (their argparse front ends are fxlm.train_lm and fxlm.prepare_bytes):

* byte-level token files: ``<prefix>_train.bin`` / ``<prefix>_val.bin`` (uint16, one
  token per byte value) and ``<prefix>.json`` {vocab_size, tokenizer, n_train, n_val,
  n_files} (ml/fxlm/prepare_bytes.py:84-97); ``read_meta`` / ``load_tokens`` read them
  as train_lm does (ml/fxlm/train_lm.py:95-118);
* ``get_batch``: B random windows of T + 1 tokens (ml/fxlm/train_lm.py:148-152);
* ``lr_at``: linear warm-up, then cosine decay to ``min_lr_frac`` of the peak
  (ml/fxlm/train_lm.py:154-160);
* ``save_checkpoint`` / ``load_checkpoint``: the reference's checkpoint dict (fp32
  master weights by parameter name, the FlatAdamW state, config, step, meta, args),
  written to a temporary file and renamed into place (ml/fxlm/train_lm.py:162-174,
  resumed as at :134-138).  Everything in it is tensors, numbers, strings, lists and
  dicts, so ``torch.load(..., weights_only=True)`` reads it back.
"""
import json
import math
import os

import numpy as np
import torch

BYTE_VOCAB = 256


def write_byte_tokens(raw, out_prefix, val_frac=0.01, n_files=1):
    """Write bytes `raw` as byte-level tokens: the last max(1, int(n * val_frac)) tokens
    are the validation split.  Returns the meta dict (also written as <prefix>.json)."""
    toks = np.frombuffer(bytes(raw), dtype=np.uint8).astype(np.uint16)
    n = toks.size
    if n < 2:
        raise ValueError("need at least two bytes (one train and one val token)")
    n_val = max(1, int(n * val_frac))
    n_tr = n - n_val
    d = os.path.dirname(os.path.abspath(out_prefix))
    os.makedirs(d, exist_ok=True)
    toks[:n_tr].tofile(out_prefix + "_train.bin")
    toks[n_tr:].tofile(out_prefix + "_val.bin")
    meta = {"vocab_size": BYTE_VOCAB, "tokenizer": "bytes", "n_train": int(n_tr),
            "n_val": int(n_val), "n_files": int(n_files)}
    with open(out_prefix + ".json", "w", encoding="utf-8") as f:
        json.dump(meta, f, indent=2)
    return meta


def data_prefix(data_path):
    """<prefix> of a token file: `x_train.bin` -> `x`, any other `x.ext` -> `x`."""
    if data_path.endswith("_train.bin"):
        return data_path[:-len("_train.bin")]
    return os.path.splitext(data_path)[0]


def read_meta(data_path):
    """The meta dict next to a token file ({} when there is none) and its vocab size
    (65536, the uint16 range, when the meta does not give one)."""
    meta_path = data_prefix(data_path) + ".json"
    meta = {}
    if os.path.exists(meta_path):
        with open(meta_path, "r", encoding="utf-8") as f:
            meta = json.load(f)
    return meta, int(meta.get("vocab_size", 65536))


def load_tokens(path, device="cpu"):
    """A uint16 token file as an int32 tensor on `device`."""
    return torch.from_numpy(np.fromfile(path, dtype=np.uint16).astype(np.int32)).to(device)


def val_path(data_path, meta):
    """The validation file train_lm falls back to: <prefix>_val.bin when the meta
    counts validation tokens and the file exists, else None."""
    if not meta.get("n_val"):
        return None
    p = data_prefix(data_path) + "_val.bin"
    return p if os.path.exists(p) else None


def get_batch(src, batch, seq_len, generator=None):
    """(x, y) int64 (batch, seq_len): windows of seq_len + 1 tokens at uniform random
    offsets in [0, len(src) - seq_len - 1); y is x shifted by one token."""
    if src.numel() < seq_len + 2:
        raise ValueError(f"{src.numel()} tokens cannot hold a window of {seq_len + 1}")
    offs = torch.randint(0, src.numel() - seq_len - 1, (batch,), device=src.device, generator=generator)
    ar = torch.arange(seq_len + 1, device=src.device)
    seq = src[offs[:, None] + ar[None, :]].long()
    return seq[:, :-1], seq[:, 1:]


def lr_at(step, lr, warmup, steps, min_lr_frac=0.1):
    """Learning rate of optimizer step `step` (0-based): lr (step + 1) / warmup during
    the warm-up, then lr (min_lr_frac + (1 - min_lr_frac) (1 + cos(pi t)) / 2) with
    t = (step - warmup) / max(1, steps - warmup) clamped to 1."""
    if step < warmup:
        return lr * (step + 1) / warmup
    t = (step - warmup) / max(1, steps - warmup)
    c = 0.5 * (1.0 + math.cos(math.pi * min(1.0, t)))
    return lr * (min_lr_frac + (1.0 - min_lr_frac) * c)


def _cpu(v):
    return v.detach().cpu() if torch.is_tensor(v) else v


def checkpoint_dict(opt, config, step, meta=None, args=None):
    """The reference's checkpoint layout, every tensor on the host."""
    return {
        "model": {k: v.detach().to("cpu", torch.float32) for k, v in opt.master_state_dict().items()},
        "opt": {k: _cpu(v) for k, v in opt.state_dict().items()},
        "config": dict(config if isinstance(config, dict) else vars(config)),
        "step": int(step),
        "meta": dict(meta or {}),
        "args": dict(args or {}),
    }


def save_checkpoint(out_dir, opt, config, step, meta=None, args=None, tag="last"):
    """Write <out_dir>/ckpt_<tag>.pt atomically (a .tmp file renamed over the old one,
    so a crash mid-write leaves the previous checkpoint intact).  Returns its path."""
    os.makedirs(out_dir, exist_ok=True)
    tmp = os.path.join(out_dir, f"ckpt_{tag}.tmp")
    final = os.path.join(out_dir, f"ckpt_{tag}.pt")
    torch.save(checkpoint_dict(opt, config, step, meta, args), tmp)
    os.replace(tmp, final)
    return final


def load_checkpoint(path, opt=None, map_location="cpu"):
    """Read a checkpoint with torch.load(weights_only=True) (nothing in the file is
    executed); when `opt` is given, restore its master / m / v / step / scale state and
    refresh the bf16 parameters from the master.  Returns the checkpoint dict."""
    sd = torch.load(path, map_location=map_location, weights_only=True)
    if opt is not None:
        opt.load_state_dict(sd["opt"])
    return sd
