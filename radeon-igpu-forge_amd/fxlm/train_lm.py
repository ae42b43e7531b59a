"""fxlm.train_lm: train the small GPT on a byte-token file (the user's entry point).

    python radeon-igpu-forge_amd/fxlm/prepare_bytes.py --out data/demo corpus/
    python radeon-igpu-forge_amd/fxlm/train_lm.py --data data/demo_train.bin --out runs/demo

Front end of ml/fxlm/train_lm.py:24-228 with the same arguments and loop:
* the token file stays on the GPU and a batch is B random windows gathered by index
  arithmetic (no DataLoader); FlatAdamW (fp32 master, bf16 params, dynamic loss scale);
* `--accum` micro-steps per optimiser step, each loss divided by the count;
* warm-up + cosine learning rate; one host synchronisation per `--log-every` steps;
* evaluation on the validation split every `--eval-every` steps and at the end, with a
  checkpoint after each evaluation and at the end, written atomically (tmp + rename);
* `--out` is required and an existing `<out>/ckpt_last.pt` is refused unless `--resume`
  names the checkpoint to continue from.
Differences, all for MI355X: bf16 in place of fp16; RMSNorm defaults to the fused
kernel (`--norm fused`: the gfx950 kernel is the faster one); checkpoints load with
torch.load(weights_only=True); the per-micro-step token limit, a guard against
overloading the reference's shared-memory iGPU at 16,384 tokens, is `--max-tokens`
(default 262,144: 16 sequences of the cfg5 model's 1024 tokens fill 5 % of the HBM).
"""
import argparse
import os
import sys
import time


def build_parser():
    ap = argparse.ArgumentParser(description="train the fxlm GPT on a uint16 token file")
    ap.add_argument("--data", required=True, help="uint16 token .bin (prepare_bytes.py output)")
    ap.add_argument("--val", default=None, help="validation .bin (default: <prefix>_val.bin if the meta counts one)")
    ap.add_argument("--seq-len", type=int, default=256)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--dim", type=int, default=512)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--accum", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--lr", type=float, default=6e-4)
    ap.add_argument("--min-lr-frac", type=float, default=0.1)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--wd", type=float, default=0.1)
    ap.add_argument("--clip", type=float, default=1.0)
    ap.add_argument("--init-scale", type=float, default=2.0 ** 16)
    ap.add_argument("--eval-every", type=int, default=200)
    ap.add_argument("--eval-batches", type=int, default=20)
    ap.add_argument("--log-every", type=int, default=20)
    ap.add_argument("--out", default=None, help="checkpoint directory (required)")
    ap.add_argument("--resume", default=None, help="checkpoint file to continue from")
    ap.add_argument("--tunable", action="store_true", help="let TunableOp tune the library GEMMs")
    ap.add_argument("--attn", choices=["flash", "sdpa"], default="flash")
    ap.add_argument("--norm", choices=["fused", "torch"], default="fused")
    ap.add_argument("--ce", choices=["fused", "torch"], default="fused")
    # beyond the reference's switches: the MLP's fused linear + GELU and the qkv / proj / fc2
    # projections (the reference always runs those in torch)
    ap.add_argument("--mlp", choices=["fused", "torch"], default="fused")
    ap.add_argument("--linear", choices=["fused", "torch"], default="fused")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--max-tokens", type=int, default=262144, help="limit on batch * seq-len per micro-step")
    return ap


def check_args(args):
    """The reference's refusals before any work (ml/fxlm/train_lm.py:56-63)."""
    if args.batch * args.seq_len > args.max_tokens:
        raise SystemExit(f"batch * seq_len = {args.batch * args.seq_len} > {args.max_tokens} tokens per "
                         "micro-step: lower --batch or use --accum")
    if args.out is None:
        raise SystemExit("--out <checkpoint directory> is required")


def train(args, device=None, log=print, optimizer_cls=None):
    """The training loop of ml/fxlm/train_lm.py:79-228.  Returns {"step", "loss", "val_loss",
    "skipped", "ckpt"} (the last logged loss, the last validation loss or None).  `device`
    defaults to the checked gfx950 GPU; `optimizer_cls` to FlatAdamW (its constructor and
    backward / step / zero_grad / scale / state_dict / load_state_dict / master_state_dict)."""
    import torch

    from fxlm import train as tr
    from fxlm.model import GPT, GPTConfig

    check_args(args)
    if device is None:
        from fxlm.env import require_gpu
        device = require_gpu()
    if optimizer_cls is None:
        from fxlm.optim import FlatAdamW as optimizer_cls
    torch.manual_seed(args.seed)

    meta, vocab = tr.read_meta(args.data)
    log(f"meta: {tr.data_prefix(args.data)}.json -> vocab_size={vocab} tokenizer={meta.get('tokenizer', '?')}")
    tokens = tr.load_tokens(args.data, device)
    vpath = args.val or tr.val_path(args.data, meta)
    vt = tr.load_tokens(vpath, device) if vpath else None
    log(f"train {tokens.numel():,} tokens" + (f" | val {vt.numel():,}" if vt is not None else ""))

    cfg = GPTConfig(vocab_size=vocab, seq_len=args.seq_len, n_layer=args.layers, n_head=args.heads,
                    d_model=args.dim, attn_impl=args.attn, norm_impl=args.norm, ce_impl=args.ce,
                    mlp_impl=args.mlp, linear_impl=args.linear)
    model = GPT(cfg).to(device)
    log(f"GPT params: {model.num_params():,} ({model.num_params() / 1e6:.1f}M)")
    opt = optimizer_cls(model, lr=args.lr, weight_decay=args.wd, max_grad_norm=args.clip,
                        init_scale=args.init_scale)

    ckpt_path = os.path.join(args.out, "ckpt_last.pt")
    start = 0
    if args.resume:
        sd = tr.load_checkpoint(args.resume, opt, map_location=device)
        start = int(sd["step"])
        log(f"resume: {args.resume} @ step {start}")
    elif os.path.exists(ckpt_path):
        raise SystemExit(f"{ckpt_path} already exists: keep the earlier run (choose another --out) "
                         "or continue it with --resume")
    os.makedirs(args.out, exist_ok=True)

    B, T, acc_n = args.batch, args.seq_len, args.accum

    def evaluate():
        model.eval()
        tot = torch.zeros((), device=device)
        with torch.inference_mode():
            for _ in range(args.eval_batches):
                x, y = tr.get_batch(vt, B, T)
                tot += model(x, y)
        model.train()
        return float(tot) / args.eval_batches

    def save(step):
        return tr.save_checkpoint(args.out, opt, cfg, step, meta=meta, args=vars(args))

    log(f"steps: {args.steps} | micro-batch {B}x{T} x{acc_n} accum | lr {args.lr} warmup {args.warmup}")
    loss_acc = torch.zeros((), device=device)
    skipped, nb, t0, step = 0, 0, None, start
    last_loss, val_loss = None, None
    while step < args.steps:
        if t0 is None:
            if device.type == "cuda":
                torch.cuda.synchronize()
            t0 = time.perf_counter()
        lr = tr.lr_at(step, args.lr, args.warmup, args.steps, args.min_lr_frac)
        for _ in range(acc_n):
            x, y = tr.get_batch(tokens, B, T)
            loss = model(x, y, grad_scale=opt.scale)
            opt.backward(loss / acc_n)
            loss_acc += loss.detach() / acc_n
            nb += 1
        stats = opt.step(lr=lr)
        opt.zero_grad()
        step += 1
        if step % args.log_every == 0 or step == 1:
            if device.type == "cuda":
                torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            skipped += int(bool(stats["found_inf"]))
            last_loss = float(loss_acc) / nb
            log(f"step {step:5d} | loss {last_loss:.4f} | lr {lr:.2e} | {nb * B * T / dt:,.0f} tok/s | "
                f"gnorm {float(stats['grad_norm']):.3f} | scale {float(stats['scale']):.0f} | skip {skipped}")
            loss_acc = torch.zeros((), device=device)
            nb, t0 = 0, None
        if vt is not None and (step % args.eval_every == 0 or step == args.steps):
            val_loss = evaluate()
            log(f"  eval @ {step}: val_loss {val_loss:.4f}")
            save(step)
    path = save(step)
    log(f"done: checkpoint -> {path}")
    return {"step": step, "loss": last_loss, "val_loss": val_loss, "skipped": skipped, "ckpt": path}


def main(argv=None):
    args = build_parser().parse_args(argv)
    check_args(args)
    tune_file = os.path.join(args.out, "tunable_gemms.csv") if args.tunable else None
    from fxlm.env import setup_lm_env
    setup_lm_env(tunable=args.tunable, tune_file=tune_file)  # before torch is imported
    return train(args)


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    main()
