"""fxlm.train: byte-token files, LR schedule, batches and atomic checkpoints (CPU).

Pinned against the reference's formulas (ml/fxlm/train_lm.py:95-174,
ml/fxlm/prepare_bytes.py:84-97) through their closed forms and properties."""
import json
import math
import os

import pytest
import torch

from fxlm import train as tr


def test_lr_warmup_then_cosine_to_floor():
    lr, warm, steps, floor = 6e-4, 10, 110, 0.1
    assert tr.lr_at(0, lr, warm, steps, floor) == pytest.approx(lr / warm)
    assert tr.lr_at(9, lr, warm, steps, floor) == pytest.approx(lr)
    assert tr.lr_at(10, lr, warm, steps, floor) == pytest.approx(lr)               # t = 0: cos = 1
    assert tr.lr_at(60, lr, warm, steps, floor) == pytest.approx(lr * (floor + (1 - floor) * 0.5))
    assert tr.lr_at(110, lr, warm, steps, floor) == pytest.approx(lr * floor)       # t = 1
    assert tr.lr_at(500, lr, warm, steps, floor) == pytest.approx(lr * floor)       # t clamps to 1
    after = [tr.lr_at(s, lr, warm, steps, floor) for s in range(warm, steps + 1)]
    assert all(a >= b for a, b in zip(after, after[1:]))
    # a quarter of the way: (1 + cos(pi / 4)) / 2
    q = (1 + math.cos(math.pi / 4)) / 2
    assert tr.lr_at(35, lr, warm, steps, floor) == pytest.approx(lr * (floor + (1 - floor) * q))


def test_byte_tokens_round_trip(tmp_path):
    raw = bytes(range(256)) * 3 + b"hello, world\n"
    prefix = str(tmp_path / "sub" / "demo")
    meta = tr.write_byte_tokens(raw, prefix, val_frac=0.01, n_files=2)
    n = len(raw)
    n_val = max(1, int(n * 0.01))
    assert meta == {"vocab_size": 256, "tokenizer": "bytes", "n_train": n - n_val, "n_val": n_val, "n_files": 2}
    with open(prefix + ".json", encoding="utf-8") as f:
        assert json.load(f) == meta
    t = tr.load_tokens(prefix + "_train.bin")
    v = tr.load_tokens(prefix + "_val.bin")
    assert t.dtype == torch.int32 and bytes(t.tolist() + v.tolist()) == raw
    assert os.path.getsize(prefix + "_train.bin") == 2 * (n - n_val)       # uint16 on disk
    m2, vocab = tr.read_meta(prefix + "_train.bin")
    assert m2 == meta and vocab == 256
    assert tr.val_path(prefix + "_train.bin", m2) == prefix + "_val.bin"
    with pytest.raises(ValueError):
        tr.write_byte_tokens(b"x", prefix)


def test_prefix_and_missing_meta(tmp_path):
    assert tr.data_prefix("/d/x_train.bin") == "/d/x"
    assert tr.data_prefix("/d/y.bin") == "/d/y"
    meta, vocab = tr.read_meta(str(tmp_path / "none.bin"))
    assert meta == {} and vocab == 65536
    assert tr.val_path(str(tmp_path / "none.bin"), {"n_val": 0}) is None


def test_get_batch_windows():
    src = torch.arange(1000, dtype=torch.int32)
    g = torch.Generator().manual_seed(3)
    x, y = tr.get_batch(src, 8, 64, generator=g)
    assert x.shape == (8, 64) and y.shape == (8, 64) and x.dtype == torch.int64
    assert torch.equal(x[:, 1:], y[:, :-1])                         # y is x shifted by one
    assert torch.equal(y[:, -1] - x[:, 0], torch.full((8,), 64))    # consecutive tokens
    assert int(x.min()) >= 0 and int(y.max()) <= 999
    with pytest.raises(ValueError):
        tr.get_batch(src[:10], 2, 9)


class _FakeOpt:
    """The FlatAdamW state API on host tensors."""

    def __init__(self, seed):
        g = torch.Generator().manual_seed(seed)
        self.master = torch.randn(40, generator=g)
        self.m, self.v = torch.randn(40, generator=g), torch.rand(40, generator=g)
        self.step_ctr, self.scale = torch.tensor(7.0), torch.tensor(65536.0)

    def state_dict(self):
        return {"master": self.master, "m": self.m, "v": self.v, "step": self.step_ctr, "scale": self.scale,
                "offsets": [("w", 0, 32), ("b", 32, 8)]}

    def load_state_dict(self, sd):
        for k in ("master", "m", "v"):
            getattr(self, k).copy_(sd[k])
        self.step_ctr.copy_(sd["step"])
        self.scale.copy_(sd["scale"])

    def master_state_dict(self):
        return {"w": self.master[:32].view(4, 8), "b": self.master[32:]}


def test_checkpoint_round_trip_and_atomic_replace(tmp_path):
    a = _FakeOpt(1)
    cfg = {"vocab_size": 256, "n_layer": 2}
    p = tr.save_checkpoint(str(tmp_path), a, cfg, 12, meta={"tokenizer": "bytes"}, args={"lr": 3e-4})
    assert p.endswith("ckpt_last.pt") and not os.path.exists(str(tmp_path / "ckpt_last.tmp"))
    b = _FakeOpt(2)
    sd = tr.load_checkpoint(p, b)                                   # weights_only=True
    assert sd["step"] == 12 and sd["config"] == cfg and sd["meta"] == {"tokenizer": "bytes"}
    assert torch.equal(b.master, a.master) and torch.equal(b.v, a.v) and float(b.step_ctr) == 7.0
    assert torch.equal(sd["model"]["w"], a.master[:32].view(4, 8))
    assert sd["opt"]["offsets"] == [("w", 0, 32), ("b", 32, 8)]
    # a save that fails while writing leaves the previous checkpoint in place
    with pytest.raises(Exception):
        tr.save_checkpoint(str(tmp_path), a, cfg, 13, args={"bad": lambda: 0})
    assert tr.load_checkpoint(p)["step"] == 12
