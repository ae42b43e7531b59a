"""The training front ends on the CPU: prepare_bytes (ml/fxlm/prepare_bytes.py:19-99) and
train_lm's argument checks, loop, evaluation cadence, checkpoints and resume rules
(ml/fxlm/train_lm.py:24-228), with the model's torch paths and an AdamW stand-in for
FlatAdamW (whose step needs the GPU; the GPU test runs the real one)."""
import json
import os

import numpy as np
import pytest
import torch

from fxlm import prepare_bytes as pb
from fxlm import train as tr
from fxlm import train_lm


def test_prepare_bytes_walks_filters_and_truncates(tmp_path):
    d = tmp_path / "src"
    (d / "sub").mkdir(parents=True)
    (d / "a.txt").write_bytes(b"hello world\n" * 10)
    (d / "sub" / "b.md").write_bytes(b"# title\n" * 5)
    (d / "sub" / "c.bin").write_bytes(b"\x00\x01\x02" * 10)          # wrong suffix: not walked
    (d / "d.py").write_bytes(b"x = 1\x00\n")                           # a NUL byte: binary
    extra = tmp_path / "e.log"
    extra.write_bytes(b"log line\n")                                 # explicit file: taken as given
    out = str(tmp_path / "data" / "demo")
    meta = pb.main([str(d), str(extra), "--out", out, "--val-frac", "0.1"])
    want = b"hello world\n" * 10 + b"# title\n" * 5 + b"log line\n"
    toks = np.concatenate([np.fromfile(out + "_train.bin", dtype=np.uint16),
                           np.fromfile(out + "_val.bin", dtype=np.uint16)])
    assert toks.tobytes() == np.frombuffer(want, dtype=np.uint8).astype(np.uint16).tobytes()
    assert meta == json.load(open(out + ".json"))
    assert meta["n_files"] == 3 and meta["n_val"] == max(1, int(len(want) * 0.1))
    meta2 = pb.main([str(d / "a.txt"), "--out", out + "2", "--max-bytes", "30"])
    assert meta2["n_train"] + meta2["n_val"] == 30
    with pytest.raises(SystemExit):
        pb.main([str(tmp_path / "missing*.txt"), "--out", out + "3"])
    with pytest.raises(SystemExit):
        pb.main([str(d / "d.py"), "--out", out + "4"])


def test_prepare_bytes_directory_order_is_sorted_top_down(tmp_path):
    # the walk order rule: a directory's files in sorted name order, then its subdirectories
    # in sorted name order, each walked the same way (top-down, depth first); files are
    # created in the reverse of that order so that a listing-order walk would differ
    d = tmp_path / "corpus"
    want_order = ["A.txt", "b.txt", "z.md", "a/1.txt", "a/y.txt", "a/x/0.md", "a/x/deep/q.txt",
                  "b/0.txt", "c c/n.md"]
    for rel in reversed(want_order):
        f = d / rel
        f.parent.mkdir(parents=True, exist_ok=True)
        f.write_bytes(f"<{rel}>".encode())
    (d / "a" / "skip.bin").write_bytes(b"not walked")
    got = pb.collect_files([str(d)], (".txt", ".md"))
    assert [os.path.relpath(p, d).replace(os.sep, "/") for p in got] == want_order
    out = str(tmp_path / "tok")
    pb.main([str(d), "--out", out, "--val-frac", "0.05"])
    toks = np.concatenate([np.fromfile(out + "_train.bin", dtype=np.uint16),
                           np.fromfile(out + "_val.bin", dtype=np.uint16)])
    assert toks.astype(np.uint8).tobytes() == b"".join(f"<{r}>".encode() for r in want_order)
    # inputs keep their given order; a glob's matches are sorted; the cut is exact
    g = pb.collect_files([str(d / "b.txt"), str(d / "a" / "*.txt")], (".txt",))
    assert [os.path.basename(p) for p in g] == ["b.txt", "1.txt", "y.txt"]
    assert pb.read_bytes(g, max_bytes=9) == b"<b.txt><a"


def test_train_lm_refuses_bad_arguments(tmp_path):
    p = train_lm.build_parser()
    with pytest.raises(SystemExit, match="tokens per micro-step"):
        train_lm.check_args(p.parse_args(["--data", "x.bin", "--out", "o", "--batch", "64",
                                          "--seq-len", "8192"]))
    with pytest.raises(SystemExit, match="--out"):
        train_lm.check_args(p.parse_args(["--data", "x.bin"]))
    a = p.parse_args(["--data", "x.bin", "--out", "o"])
    assert (a.attn, a.norm, a.ce, a.lr, a.warmup, a.seq_len) == ("flash", "fused", "fused", 6e-4, 100, 256)


class CpuAdamW:
    """FlatAdamW's interface over torch.optim.AdamW on the CPU (test stand-in)."""

    def __init__(self, model, lr=3e-4, weight_decay=0.1, max_grad_norm=1.0, init_scale=2.0 ** 16):
        self.model, self.max_grad_norm = model, max_grad_norm
        self.scale = torch.tensor(float(init_scale))
        self.opt = torch.optim.AdamW(model.parameters(), lr=lr, weight_decay=weight_decay)
        self.steps = 0

    def backward(self, loss):
        (loss * self.scale).backward()

    def step(self, lr=None):
        for p in self.model.parameters():
            if p.grad is not None:
                p.grad /= self.scale
        norm = torch.nn.utils.clip_grad_norm_(self.model.parameters(), self.max_grad_norm)
        for g in self.opt.param_groups:
            g["lr"] = lr
        self.opt.step()
        self.steps += 1
        return {"grad_norm": norm, "found_inf": torch.tensor(0.0), "scale": self.scale}

    def zero_grad(self):
        self.opt.zero_grad(set_to_none=True)

    def master_state_dict(self):
        return {n: p.detach().float() for n, p in self.model.named_parameters()}

    def state_dict(self):
        return {"params": [p.detach().clone() for p in self.model.parameters()],
                "step": torch.tensor(self.steps), "scale": self.scale.clone()}

    def load_state_dict(self, sd):
        with torch.no_grad():
            for p, q in zip(self.model.parameters(), sd["params"]):
                p.copy_(q)
        self.steps = int(sd["step"])


def _corpus(tmp_path):
    raw = b"the quick brown fox jumps over the lazy dog. " * 300
    tr.write_byte_tokens(raw, str(tmp_path / "corpus"), val_frac=0.1)
    return str(tmp_path / "corpus_train.bin")


def _args(data, out, *extra):
    return train_lm.build_parser().parse_args(
        ["--data", data, "--out", out, "--seq-len", "32", "--layers", "1", "--heads", "2", "--dim", "32",
         "--batch", "4", "--accum", "2", "--lr", "3e-3", "--warmup", "2", "--eval-every", "3",
         "--eval-batches", "2", "--log-every", "2", "--attn", "sdpa", "--norm", "torch", "--ce", "torch",
         "--mlp", "torch", "--linear", "torch", *extra])


def test_train_lm_loop_checkpoints_and_resume(tmp_path):
    data, out = _corpus(tmp_path), str(tmp_path / "run")
    lines = []
    r = train_lm.train(_args(data, out, "--steps", "7"), device=torch.device("cpu"), log=lines.append,
                       optimizer_cls=CpuAdamW)
    steps_logged = [int(l.split()[1]) for l in lines if l.startswith("step ")]
    evals = [int(l.split()[2][:-1]) for l in lines if l.strip().startswith("eval @")]
    assert steps_logged == [1, 2, 4, 6] and evals == [3, 6, 7]
    assert r["step"] == 7 and r["val_loss"] is not None and r["loss"] < 5.6   # ln 256 = 5.55 at init
    sd = tr.load_checkpoint(r["ckpt"])
    assert sd["step"] == 7 and sd["args"]["accum"] == 2 and sd["config"]["seq_len"] == 32
    assert sd["meta"]["vocab_size"] == 256
    # a second run into the same directory is refused unless it resumes
    with pytest.raises(SystemExit, match="already exists"):
        train_lm.train(_args(data, out, "--steps", "9"), device=torch.device("cpu"), log=lines.append,
                       optimizer_cls=CpuAdamW)
    lines2 = []
    r2 = train_lm.train(_args(data, out, "--steps", "9", "--resume", r["ckpt"]), device=torch.device("cpu"),
                        log=lines2.append, optimizer_cls=CpuAdamW)
    assert any(l.startswith("resume:") and "@ step 7" in l for l in lines2)
    assert r2["step"] == 9 and [int(l.split()[1]) for l in lines2 if l.startswith("step ")] == [8]
    assert tr.load_checkpoint(r2["ckpt"])["step"] == 9
