"""Benchmark: the fxlm GPT 12L-d768 training step on one MI355X, plus the hot-path kernels.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --only {attention,ce,norm,adamw,linear,wgrad,head,library,step,copy,decode,embedding,cpu,
                            fc-ours,fc-library,fc-ours-cold,fc-library-cold}   (profiling runs)
    python bench.py --counter-table p_counter_collection.csv [...]   (per-kernel counter table)
    python bench.py --traffic-table FETCH.csv WRITE.csv COPY_FETCH.csv COPY_WRITE.csv
    python bench.py --trace-table kernel_trace.csv [ONCE_PER_STEP_KERNEL]   (kernel-trace table)
    python bench.py --pmc-summary FETCH.csv WRITE.csv COPY_FETCH.csv COPY_WRITE.csv

Workload (the headline metric's fifth config): GPT with 12 layers, d_model 768, 12 heads of
64, RMSNorm (fused), fused-linear GELU MLP 3072, vocab 50304, causal S=1024,
batch 16, tied head; all bf16 with FlatAdamW (fp32 master, lr 6e-4, betas
(0.9, 0.95), eps 1e-8, wd 0.1, clip 1.0).  Tokens are uniform random from a
seed, weights N(0, 0.02): synthetic data, random init.  One step = forward +
backward + optimiser step over 16,384 tokens; K steps are timed after W
warm-up steps, bracketed by torch.cuda.synchronize().

Also measured in the same run, each with HIP events on the stream the kernels
are launched on (torch's current stream):
  attention cfg2 [16,12,1024,64] causal: fx_attn_fwd and fx_attn_bwd
  cross-entropy cfg3 [16384, 50304]: fused forward + backward
  RMSNorm cfg4 [65536, 768]: forward and backward
  FlatAdamW cfg4: one step over 124,373,760 parameters
  fused linear + GELU: the cfg5 MLP fc (16384 x 768 x 3072)
  weight gradients: the four cfg5 dW = dy^T x products over 16384 tokens
  linear-CE head: the cfg5 tied head, unfused chunk loop against the fused kernels
  library comparisons: attention, CE, RMSNorm and the optimizer step next to SDPA,
    F.cross_entropy, F.rms_norm and fused torch AdamW at the same shapes (each kernel
    line's "library" entry)
and, on the host CPU, the reference's naive-PyTorch fp32 training step
(oracle/gpt.py) on a bounded sample.  Prints ONE JSON line.
"""
import argparse
import gc
import json
import math
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "radeon-igpu-forge_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA, TFLOP/s

CFG5 = dict(vocab_size=50304, seq_len=1024, n_layer=12, n_head=12, d_model=768, batch=16)


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_us(torch, fn, iters=20, warm=5, warm_ms=200.0, rounds=5):
    """Steady-state duration (us) of fn(): the median over `rounds` of the average of
    `iters` runs (HIP events on the current stream), after warm-up calls that fill at least
    `warm_ms` of GPU time.  The GPU's clocks ramp up over the first ~100 ms of sustained
    load: timed from idle, the attention backward measured 157 us, and 133-134 us once
    warm (the training step's kernels run under sustained load)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    s, e = _events(torch)
    s.record()
    fn()
    e.record()
    torch.cuda.synchronize()
    n = int(min(5000, max(1.0, warm_ms / max(s.elapsed_time(e), 1e-3))))
    for _ in range(n):
        fn()
    res = []
    for _ in range(rounds):
        torch.cuda.synchronize()
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        res.append(s.elapsed_time(e) / iters * 1e3)
    return sorted(res)[len(res) // 2]


def graph_time_us(torch, fn, reps=20, iters=10):
    """Average duration (us) of fn() captured `reps` times in one HIP graph and replayed
    `iters` times: the GPU time of short launches without the host's per-call cost."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = _events(torch)
    t0.record()
    for _ in range(iters):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (iters * reps) * 1e3


def bench_attention(torch):
    from fxlm.attention import _bwd, _fwd
    B, T, H, D = 16, 1024, 12, 64
    g = torch.Generator(device="cuda").manual_seed(2)
    q, k, v, do = (torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16() for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    o, lse = _fwd(q, k, v, True, scale)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    t_fwd = time_us(torch, lambda: _fwd(q, k, v, True, scale))
    t_bwd = time_us(torch, lambda: _bwd(q, k, v, o, lse, do, True, scale, dq, dk, dv))
    f_fwd = 4.0 * B * H * T * T * D * 0.5          # causal half of QK^T and PV
    f_bwd = 2.5 * f_fwd                            # dV, dP, dK, dQ (+ recomputed S)
    return {
        "shape": [B, T, H, D], "causal": True,
        "fwd_us": round(t_fwd, 2), "bwd_us": round(t_bwd, 2),
        "fwd_tflops": round(f_fwd / t_fwd / 1e6, 1), "bwd_tflops": round(f_bwd / t_bwd / 1e6, 1),
        "fwdbwd_tflops": round((f_fwd + f_bwd) / (t_fwd + t_bwd) / 1e6, 1),
        "fwdbwd_frac_of_bf16_peak": round((f_fwd + f_bwd) / (t_fwd + t_bwd) / 1e6 / BF16_PEAK_TFLOPS, 4),
        "flop_fwd": f_fwd, "flop_bwd": f_bwd,
    }


def bench_ce(torch):
    from fxlm.cross_entropy import fused_cross_entropy
    N, V = 16384, 50304
    g = torch.Generator(device="cuda").manual_seed(3)
    lg = (torch.randn(N, V, device="cuda", generator=g) * 2).bfloat16().requires_grad_()
    tg = torch.randint(0, V, (N,), device="cuda", generator=g)
    tg[torch.rand(N, device="cuda", generator=g) < 0.05] = -100

    def fb():
        fused_cross_entropy(lg, tg).backward()
        lg.grad = None
    t = time_us(torch, fb, iters=10, warm=3)
    n_valid = int((tg != -100).sum())
    # algorithmic work of the config: logits read once, dlogits written once, targets
    nbytes = 2 * N * V * 2 + N * 8
    # what the kernel moves: rows with an ignored target get a zero gradient row
    # without their logits being read
    moved = (n_valid + N) * V * 2 + N * 8
    del lg
    return {"shape": [N, V], "fwdbwd_us": round(t, 2), "gbs": round(nbytes / t / 1e3, 1),
            "frac_of_hbm": round(nbytes / t / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes,
            "moved_bytes": moved, "moved_gbs": round(moved / t / 1e3, 1)}


def bench_norm(torch):
    from fxlm.norm import rms_norm_bwd_raw, rms_norm_fwd_stats
    N, D = 65536, 768
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(N, D, device="cuda", generator=g).bfloat16()
    w = (torch.randn(D, device="cuda", generator=g) * 0.1 + 1).bfloat16()
    dy = torch.randn(N, D, device="cuda", generator=g).bfloat16()
    _, rstd = rms_norm_fwd_stats(x, w)
    tf = time_us(torch, lambda: rms_norm_fwd_stats(x, w))
    tb = time_us(torch, lambda: rms_norm_bwd_raw(x, dy, w, rstd))
    bf = N * D * 2 * 2 + N * 4 + D * 2             # x read, y write, rstd, w
    bb = N * D * 2 * 3 + N * 4 + D * 2 + D * 4     # x, dy read, dx write, rstd, w, dw
    return {"shape": [N, D], "fwd_us": round(tf, 2), "bwd_us": round(tb, 2),
            "fwd_gbs": round(bf / tf / 1e3, 1), "bwd_gbs": round(bb / tb / 1e3, 1),
            "fwd_frac_of_hbm": round(bf / tf / 1e3 / HBM_PEAK_GBS, 4),
            "bwd_frac_of_hbm": round(bb / tb / 1e3 / HBM_PEAK_GBS, 4)}


def _zipf_ids(torch, n, V, seed, a=1.1):
    g = torch.Generator().manual_seed(seed)
    p = 1.0 / torch.arange(1, V + 1, dtype=torch.float64) ** a
    return torch.multinomial(p / p.sum(), n, replacement=True, generator=g)


def _byte_text_ids(torch, n):
    """n byte-level tokens (V = 256) of this repository's own prose (its top-level markdown
    documents; a fixed English sentence when those are absent): the space byte holds ~15 % of
    them."""
    text = b""
    for name in ("DESIGN.md", "README.md", "INTEGRATION.md"):
        try:
            with open(os.path.join(ROOT, name), "rb") as fh:
                text += fh.read()
        except OSError:
            pass
    if len(text) < n:
        text += b"the quick brown fox jumps over the lazy dog " * (n // 44 + 1)
    return torch.tensor(list(text[:n]), dtype=torch.int64)


def bench_embedding(torch):
    """The token-embedding weight gradient at the cfg5 step's lookup (16,384 ids, D 768):
    fx_embedding_bwd against torch's embedding backward on the same ids and rows, for three id
    distributions: uniform ids over V 50,304 (the bench's synthetic batches), Zipf ids over
    V 50,304 (exponent 1.1, as BPE token counts fall off) and byte-level text over V 256 (the
    reference's prepare_bytes tokens: the space byte alone is ~15 % of the positions).
    Algorithmic bytes: dy read once and the (V, D) gradient written once."""
    from fxlm.embedding import embedding_grad
    n, D = 16384, 768
    g = torch.Generator(device="cuda").manual_seed(6)
    dy = torch.randn(n, D, device="cuda", generator=g).bfloat16()
    cases = {"uniform": (50304, torch.randint(0, 50304, (n,), device="cuda", generator=g)),
             "zipf": (50304, _zipf_ids(torch, n, 50304, 6).cuda()),
             "byte_text": (256, _byte_text_ids(torch, n).cuda())}
    out = {}
    for name, (V, idx) in cases.items():
        t = time_us(torch, lambda: embedding_grad(idx, dy, V))
        tl = time_us(torch, lambda: torch.ops.aten.embedding_dense_backward(dy, idx, V, -1, False))
        b = n * D * 2 + V * D * 2
        top = int(torch.bincount(idx, minlength=V).max())
        out[name] = {"shape_nVD": [n, V, D], "max_positions_per_id": top, "bwd_us": round(t, 2), "bytes": b,
                     "gbs": round(b / t / 1e3, 1), "frac_of_hbm": round(b / t / 1e3 / HBM_PEAK_GBS, 4),
                     "library": {"torch_embedding_backward_us": round(tl, 2), "speedup": round(tl / t, 2)}}
    res = dict(out["uniform"])
    res["id_distributions"] = out
    return res


def bench_adamw(torch):
    from torch import nn

    from fxlm.optim import FlatAdamW
    n = 124373760

    class Flat(nn.Module):
        def __init__(self):
            super().__init__()
            self.w = nn.Parameter(torch.empty(n // 768, 768, device="cuda").normal_(0, 0.02))

    m = Flat()
    opt = FlatAdamW(m, lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0,
                    init_scale=1.0)
    g = torch.Generator(device="cuda").manual_seed(5)
    opt.m.normal_(0, 1e-4, generator=g)
    opt.v.normal_(0, 1e-6, generator=g).abs_()
    opt._step_ctr.fill_(99)
    m.w.grad = (torch.randn(n // 768, 768, device="cuda", generator=g) * 1e-3).bfloat16()
    t = time_us(torch, lambda: opt.step(lr=6e-4), iters=10, warm=3)
    nbytes = 30 * n
    del opt, m
    return {"params": n, "step_us": round(t, 2), "gbs": round(nbytes / t / 1e3, 1),
            "frac_of_hbm": round(nbytes / t / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes}


def bench_library(torch):
    """Each bandwidth / attention op next to its PyTorch equivalent at the same shape, as the
    reference's microbench compares them (ml/fxlm/bench_kernels.py:49-190): flash attention
    against scaled_dot_product_attention, fused CE against F.cross_entropy (on fp32 logits, as
    the reference times it, and on the bf16 logits), RMSNorm against F.rms_norm, and the
    FlatAdamW step against GradScaler unscale + clip_grad_norm_ + fused torch AdamW.  Both
    sides go through autograd where the reference's do (fwd + bwd).  SDPA runs on its flash or
    memory-efficient backend only: its math backend is never timed here (its bf16 batched
    products take transposed operands, which this GPU's library path is not trusted with)."""
    import torch.nn.functional as Fn

    from fxlm.attention import flash_attention
    from fxlm.cross_entropy import fused_cross_entropy
    from fxlm.norm import rms_norm
    out = {}
    g = torch.Generator(device="cuda").manual_seed(6)

    # attention, cfg2: this build's autograd op against SDPA (B, H, T, D) on the same values
    B, T, H, D = 16, 1024, 12, 64
    q, k, v, do = (torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16() for _ in range(4))
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))

    def ours_fwd():
        with torch.no_grad():
            flash_attention(qa, ka, va, causal=True)

    def ours_fb():
        flash_attention(qa, ka, va, causal=True).backward(do)
        qa.grad = ka.grad = va.grad = None
    att = {"ours_fwd_us": round(time_us(torch, ours_fwd), 2), "ours_fwdbwd_us": round(time_us(torch, ours_fb), 2)}
    qs, ks, vs = (t.transpose(1, 2).contiguous().requires_grad_() for t in (q, k, v))
    dos = do.transpose(1, 2).contiguous()
    from torch.nn.attention import SDPBackend, sdpa_kernel
    err = None
    for be, name in ((SDPBackend.FLASH_ATTENTION, "flash"), (SDPBackend.EFFICIENT_ATTENTION, "efficient")):
        try:
            with sdpa_kernel([be]):
                def s_fwd():
                    with torch.no_grad():
                        Fn.scaled_dot_product_attention(qs, ks, vs, is_causal=True)

                def s_fb():
                    Fn.scaled_dot_product_attention(qs, ks, vs, is_causal=True).backward(dos)
                    qs.grad = ks.grad = vs.grad = None
                s_fb()
                torch.cuda.synchronize()
                att.update({"sdpa_backend": name, "sdpa_fwd_us": round(time_us(torch, s_fwd), 2),
                            "sdpa_fwdbwd_us": round(time_us(torch, s_fb), 2)})
            err = None
            break
        except RuntimeError as e:
            err = str(e).splitlines()[0][:160]
    if err:
        att["sdpa_error"] = err
    elif "sdpa_fwd_us" in att:
        att["speedup_fwd"] = round(att["sdpa_fwd_us"] / att["ours_fwd_us"], 2)
        att["speedup_fwdbwd"] = round(att["sdpa_fwdbwd_us"] / att["ours_fwdbwd_us"], 2)
    out["attention_cfg2"] = att
    del q, k, v, do, qa, ka, va, qs, ks, vs, dos

    # cross-entropy, cfg3
    N, V = 16384, 50304
    lg = (torch.randn(N, V, device="cuda", generator=g) * 2).bfloat16().requires_grad_()
    tg = torch.randint(0, V, (N,), device="cuda", generator=g)
    tg[torch.rand(N, device="cuda", generator=g) < 0.05] = -100

    def ce_ours():
        fused_cross_entropy(lg, tg).backward()
        lg.grad = None

    def ce_f32():
        Fn.cross_entropy(lg.float(), tg, ignore_index=-100).backward()
        lg.grad = None

    def ce_bf16():
        Fn.cross_entropy(lg, tg, ignore_index=-100).backward()
        lg.grad = None
    ce = {"ours_fwdbwd_us": round(time_us(torch, ce_ours, iters=10, warm=3), 1),
          "torch_fp32_fwdbwd_us": round(time_us(torch, ce_f32, iters=10, warm=3), 1),
          "torch_bf16_fwdbwd_us": round(time_us(torch, ce_bf16, iters=10, warm=3), 1)}
    ce["speedup_vs_fp32"] = round(ce["torch_fp32_fwdbwd_us"] / ce["ours_fwdbwd_us"], 2)
    ce["speedup_vs_bf16"] = round(ce["torch_bf16_fwdbwd_us"] / ce["ours_fwdbwd_us"], 2)
    out["cross_entropy_cfg3"] = ce
    del lg, tg
    torch.cuda.empty_cache()

    # RMSNorm, cfg4
    N, D = 65536, 768
    x = torch.randn(N, D, device="cuda", generator=g).bfloat16().requires_grad_()
    w = (torch.randn(D, device="cuda", generator=g) * 0.1 + 1).bfloat16().requires_grad_()
    dy = torch.randn(N, D, device="cuda", generator=g).bfloat16()

    def n_ours_f():
        with torch.no_grad():
            rms_norm(x, w, 1e-6)

    def n_ours_fb():
        rms_norm(x, w, 1e-6).backward(dy)
        x.grad = w.grad = None

    def n_t_f():
        with torch.no_grad():
            Fn.rms_norm(x, (D,), w, 1e-6)

    def n_t_fb():
        Fn.rms_norm(x, (D,), w, 1e-6).backward(dy)
        x.grad = w.grad = None
    nm = {"ours_fwd_us": round(time_us(torch, n_ours_f), 2), "ours_fwdbwd_us": round(time_us(torch, n_ours_fb), 2),
          "torch_fwd_us": round(time_us(torch, n_t_f), 2), "torch_fwdbwd_us": round(time_us(torch, n_t_fb), 2)}
    nm["speedup_fwd"] = round(nm["torch_fwd_us"] / nm["ours_fwd_us"], 2)
    nm["speedup_fwdbwd"] = round(nm["torch_fwdbwd_us"] / nm["ours_fwdbwd_us"], 2)
    out["rmsnorm_cfg4"] = nm
    del x, w, dy

    # optimizer, cfg4 size: the reference's torch comparator (fp32 params and gradients,
    # GradScaler unscale, clip to 1.0, fused AdamW, scaler update)
    n = 124373760
    p = torch.nn.Parameter(torch.empty(n // 768, 768, device="cuda").normal_(0, 0.02, generator=g))
    p.grad = torch.randn(n // 768, 768, device="cuda", generator=g) * 1e-3
    opt2 = torch.optim.AdamW([p], lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, fused=True)
    scaler = torch.amp.GradScaler("cuda", init_scale=1.0)
    dummy = torch.ones((), device="cuda")

    def t_step():
        scaler.scale(dummy)
        scaler.unscale_(opt2)
        torch.nn.utils.clip_grad_norm_([p], 1.0)
        scaler.step(opt2)
        scaler.update()
    out["flat_adamw_cfg4"] = {"torch_fused_adamw_clip_scaler_us": round(time_us(torch, t_step, iters=10, warm=3), 1)}
    del p, opt2, scaler
    torch.cuda.empty_cache()
    return out


def bench_linear(torch):
    from fxgpu.fused_linear import fused_linear
    M, K, N = 16384, 768, 3072
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(M, K, device="cuda", generator=g).bfloat16()
    W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).bfloat16()
    with torch.no_grad():
        t = time_us(torch, lambda: fused_linear(x, W, None, "gelu_tanh"))
        t_ref = time_us(torch, lambda: torch.nn.functional.gelu(x @ W.t(), approximate="tanh"))
    # the training step's form: the GELU output and, in place of the pre-activation, its
    # derivative (fx_linear_fwd act 2, fused_mlp's fc)
    from fxgpu.abi import call, ptr, stream_of
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    gd = torch.empty_like(y)
    t_d = time_us(torch, lambda: call("fx_linear_fwd", ptr(x), K, None, 0, 0, ptr(W), None, ptr(y), ptr(gd), None,
                                      M, N, K, 2, stream_of(x)))
    f = 2.0 * M * K * N
    del W, y, gd
    # the block's projections (y = x W^T): this build's routing (linear) against torch.mm
    from fxgpu.fused_linear import linear
    proj = {}
    for name, (n, kk) in {"qkv": (2304, 768), "proj": (768, 768), "fc2": (768, 3072)}.items():
        xp = torch.randn(M, kk, device="cuda", generator=g).bfloat16()
        wp = (torch.randn(n, kk, device="cuda", generator=g) * 0.02).bfloat16()
        with torch.no_grad():
            t_o = time_us(torch, lambda: linear(xp, wp))
            t_l = time_us(torch, lambda: torch.mm(xp, wp.t()))
        proj[name] = {"us": round(t_o, 2), "tflops": round(2.0 * M * n * kk / t_o / 1e6, 1),
                      "library_mm_us": round(t_l, 2)}
        del xp, wp
    return {"shape": [M, K, N], "fwd_us": round(t, 2), "tflops": round(f / t / 1e6, 1),
            "frac_of_bf16_peak": round(f / t / 1e6 / BF16_PEAK_TFLOPS, 4),
            "hipblaslt_mm_plus_gelu_us": round(t_ref, 2), "with_derivative_us": round(t_d, 2), "projections": proj}


def bench_wgrad(torch):
    """The GPT's weight gradients dW = dy^T x at cfg5 (16384 tokens) on fx_linear_wgrad
    (the whole-tile kernel with the split-K reduce), beside the general kernel
    (FX_GEMM_GENERAL=w) and the library's torch.mm(dy.t(), x)."""
    from fxgpu.fused_linear import linear_wgrad
    T = 16384
    g = torch.Generator(device="cuda").manual_seed(8)
    out = {}
    for name, (M, N) in {"qkv": (2304, 768), "proj": (768, 768), "fc": (3072, 768), "fc2": (768, 3072)}.items():
        dy = torch.randn(T, M, device="cuda", generator=g).bfloat16()
        x = torch.randn(T, N, device="cuda", generator=g).bfloat16()
        t = time_us(torch, lambda: linear_wgrad(dy, x))
        prev = os.environ.get("FX_GEMM_GENERAL")
        os.environ["FX_GEMM_GENERAL"] = "w"
        try:
            t_gen = time_us(torch, lambda: linear_wgrad(dy, x))
        finally:
            if prev is None:
                os.environ.pop("FX_GEMM_GENERAL", None)
            else:
                os.environ["FX_GEMM_GENERAL"] = prev
        t_mm = time_us(torch, lambda: torch.mm(dy.t(), x))
        f = 2.0 * T * M * N
        out[name] = {"shape_TMN": [T, M, N], "us": round(t, 2), "tflops": round(f / t / 1e6, 1),
                     "frac_of_bf16_peak": round(f / t / 1e6 / BF16_PEAK_TFLOPS, 4),
                     "general_kernel_us": round(t_gen, 2), "library_mm_us": round(t_mm, 2)}
        del dy, x
    return out


def bench_wgrad_step(torch, rounds=12, warm_ms=300.0):
    """For profiler runs: the cfg5 step's 48 layer weight gradients (12 rounds of the qkv,
    proj, fc and fc2 products over 16384 tokens), after warm-up rounds that fill `warm_ms` of
    GPU time (the clocks ramp up over the first ~100 ms), so that per-dispatch averages over
    the last 48 dispatches weigh the four shapes as the step does and match bench.py's timing
    (--trace-table ... --trace-last 48)."""
    from fxgpu.fused_linear import linear_wgrad
    T = 16384
    g = torch.Generator(device="cuda").manual_seed(8)
    ops = []
    for M, N in ((2304, 768), (768, 768), (3072, 768), (768, 3072)):
        ops.append((torch.randn(T, M, device="cuda", generator=g).bfloat16(),
                    torch.randn(T, N, device="cuda", generator=g).bfloat16()))
    for dy, x in ops:
        linear_wgrad(dy, x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for dy, x in ops:
            linear_wgrad(dy, x)
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(rounds):
        for dy, x in ops:
            linear_wgrad(dy, x)
    torch.cuda.synchronize()
    return {"launches": 4 * rounds, "wall_us_per_launch": round((time.perf_counter() - t0) / (4 * rounds) * 1e6, 2)}


def bench_gemm_kernels(torch, reps=10, warm_ms=300.0):
    """For counter runs: this build's three whole-tile GEMM kernels at the cfg5 layer shapes,
    16384 tokens: the forward (fx_linear_fwd, gemm_fast_kernel) at the qkv / proj / fc2
    shapes, the input gradient (fx_linear_dgrad, gemm_dgrad_fast_kernel) at the qkv / proj /
    fc / fc2 shapes, the weight gradient (fx_linear_wgrad) at all four, `reps` times each
    after warm-up rounds filling `warm_ms` of GPU time."""
    from fxgpu.abi import call, ptr, stream_of
    from fxgpu.fused_linear import _native_fwd, linear_wgrad
    T = 16384
    g = torch.Generator(device="cuda").manual_seed(9)
    R = lambda *s: (torch.randn(*s, device="cuda", generator=g) * 0.5).bfloat16()  # noqa: E731
    ops = []
    for N, K in ((2304, 768), (768, 768), (768, 3072)):       # y (T, N) = x (T, K) W^T
        x, w = R(T, K), R(N, K)
        ops.append(lambda x=x, w=w: _native_fwd(x, w))
    for N, K in ((768, 2304), (768, 768), (768, 3072), (3072, 768)):   # dx (T, N) = dy (T, K) W (K, N)
        dy, w = R(T, K), R(K, N)
        dx = torch.empty(T, N, device="cuda", dtype=torch.bfloat16)
        ops.append(lambda dy=dy, w=w, dx=dx, N=N, K=K: call(
            "fx_linear_dgrad", ptr(dy), K, ptr(w), N, None, ptr(dx), N, T, N, K, stream_of(dy)))
    for M, N in ((2304, 768), (768, 768), (3072, 768), (768, 3072)):  # dW (M, N) = dy^T x
        dy, x = R(T, M), R(T, N)
        ops.append(lambda dy=dy, x=x: linear_wgrad(dy, x))
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for f in ops:
            f()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        for f in ops:
            f()
    torch.cuda.synchronize()
    return {"launches": reps * len(ops), "wall_us_per_launch": round((time.perf_counter() - t0) / (reps * len(ops)) * 1e6, 2)}


def wgrad_roofline(wg):
    """fx_linear_wgrad over the step's four layer shapes (each 12 times per step): algorithmic
    FLOPs 2 T M N per product, over the measured launch times (kernel plus split-K reduce)."""
    flop = sum(2.0 * v["shape_TMN"][0] * v["shape_TMN"][1] * v["shape_TMN"][2] for v in wg.values())
    us = sum(v["us"] for v in wg.values())
    return flop / len(wg), us / len(wg)


def bench_head(torch):
    """The cfg5 tied head, linear_cross_entropy over x (16384, 768) and E (50304, 768): the
    unfused chunk loop (library logits GEMM, fx_ce_fwd_grad, dx and dW GEMMs) against the
    fused kernels (fx_lce_fwd: the GEMM with the online CE in its epilogue; fx_lce_grad: the
    GEMM again with the dlogits in its epilogue), for training (forward + backward) and for
    the loss-only path (no grad)."""
    import fxlm.cross_entropy as ce
    N, D, V = 16384, 768, 50304
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn(N, D, device="cuda", generator=g).bfloat16().requires_grad_()
    w = (torch.randn(V, D, device="cuda", generator=g) * 0.02).bfloat16().requires_grad_()
    tg = torch.randint(0, V, (N,), device="cuda", generator=g)
    old = ce.FUSED_LINEAR_CE_LOSS, ce.FUSED_LINEAR_CE_TRAIN

    def train():
        ce.linear_cross_entropy(x, w, tg).backward()
        x.grad = w.grad = None

    def loss_only():
        with torch.no_grad():
            ce.linear_cross_entropy(x, w, tg)
    out = {"shape_NDV": [N, D, V], "gemm_flop": 2 * N * D * V}
    try:
        for fused in (False, True):
            ce.FUSED_LINEAR_CE_LOSS = ce.FUSED_LINEAR_CE_TRAIN = fused
            tag = "fused" if fused else "unfused"
            out[f"train_{tag}_us"] = round(time_us(torch, train, iters=5, warm=2), 1)
            out[f"loss_only_{tag}_us"] = round(time_us(torch, loss_only, iters=5, warm=2), 1)
        # the fused loss pass alone: the logits GEMM with its online-CE epilogue + the merge
        row_loss = torch.empty(N, device="cuda", dtype=torch.float32)
        xd = x.detach()
        t = time_us(torch, lambda: ce._lce_fwd(xd, w.detach(), tg, -100, row_loss), iters=10, warm=3)
        out["lce_fwd_us"] = round(t, 1)
        out["lce_fwd_tflops"] = round(out["gemm_flop"] / t / 1e6, 1)
        out["lce_fwd_frac_of_bf16_peak"] = round(out["gemm_flop"] / t / 1e6 / BF16_PEAK_TFLOPS, 4)
        t_mm = time_us(torch, lambda: torch.mm(xd, w.detach().t()), iters=10, warm=3)
        out["library_logits_mm_us"] = round(t_mm, 1)
    finally:
        ce.FUSED_LINEAR_CE_LOSS, ce.FUSED_LINEAR_CE_TRAIN = old
    del x, w
    return out


def bench_decode(torch):
    """Inference: decode attention over a KV cache (HBM-bound kernel) and one cached
    token step of the cfg5 model against the reference sampler's full-context re-run."""
    from fxlm.attention import decode_attention
    from fxlm.model import GPT, GPTConfig
    B, T, H, D = 16, 1024, 12, 64
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(B, H, D, device="cuda", generator=g).bfloat16()
    k = torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16()
    v = torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16()
    lens = torch.full((B,), T, dtype=torch.int32, device="cuda")
    t_k = graph_time_us(torch, lambda: decode_attention(q, k, v, lens))
    nbytes = 2 * B * T * H * D * 2 + 2 * B * H * D * 2           # K and V read once, q, o
    del q, k, v
    # the step's few-row GEMMs (16 rows): this build's kernel against the library GEMM
    from fxgpu.fused_linear import fused_linear, linear
    gemms = {}
    for name, (n, kk) in {"qkv": (2304, 768), "fc_gelu": (3072, 768), "fc2": (768, 3072),
                          "head": (CFG5["vocab_size"], 768)}.items():
        x = torch.randn(B, kk, device="cuda", generator=g).bfloat16()
        w = (torch.randn(n, kk, device="cuda", generator=g) * 0.02).bfloat16()
        ours = (lambda: fused_linear(x, w, None, "gelu_tanh")) if name == "fc_gelu" else (lambda: linear(x, w))
        with torch.no_grad():
            t_o = graph_time_us(torch, ours)
            t_l = graph_time_us(torch, lambda: torch.mm(x, w.t()))
        gemms[name] = {"us": round(t_o, 2), "library_mm_us": round(t_l, 2),
                       "weight_gbs": round(n * kk * 2 / t_o / 1e3, 1)}
        del x, w
    c = CFG5
    torch.manual_seed(0)
    m = GPT(GPTConfig(vocab_size=c["vocab_size"], seq_len=c["seq_len"], n_layer=c["n_layer"],
                      n_head=c["n_head"], d_model=c["d_model"])).cuda().bfloat16().eval()
    ctx = 512
    idx = torch.randint(0, c["vocab_size"], (B, ctx + 1), device="cuda", generator=g)
    cache = m.init_cache(B, ctx + 1)
    with torch.no_grad():
        m.prefill(idx[:, :ctx], cache)
        t_step = time_us(torch, lambda: m.decode_step(idx[:, ctx], cache, ctx), iters=10, warm=3)
        # the recompute before the graph exists (its private memory pool would make the
        # recompute's 0.8 GB of logits reallocate on every call)
        t_full = time_us(torch, lambda: m(idx[:, 1:ctx + 1])[:, -1, :].float(), iters=10, warm=3)
        step = m.decode_graph(cache, B)
        t_graph = time_us(torch, lambda: step(idx[:, ctx], ctx), iters=50, warm=5)
    del m, cache, step
    return {"kernel_shape": [B, T, H, D], "kernel_us": round(t_k, 2), "kernel_gbs": round(nbytes / t_k / 1e3, 1),
            "kernel_frac_of_hbm": round(nbytes / t_k / 1e3 / HBM_PEAK_GBS, 4), "kernel_bytes": nbytes,
            "few_row_gemms": gemms,
            "model": f"cfg5 GPT, batch {B}, context {ctx}", "cached_step_us": round(t_step, 1),
            "cached_graph_step_us": round(t_graph, 1), "recompute_step_us": round(t_full, 1),
            "tok_s_cached_graph": round(B / t_graph * 1e6, 1), "tok_s_cached": round(B / t_step * 1e6, 1),
            "tok_s_recompute": round(B / t_full * 1e6, 1)}


def gpu_step_bench(torch, steps, warmup):
    from fxlm.model import GPT, GPTConfig
    from fxlm.optim import FlatAdamW
    c = CFG5
    torch.manual_seed(0)
    cfg = GPTConfig(vocab_size=c["vocab_size"], seq_len=c["seq_len"], n_layer=c["n_layer"],
                    n_head=c["n_head"], d_model=c["d_model"])
    model = GPT(cfg).cuda()
    opt = FlatAdamW(model, lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    B, T = c["batch"], c["seq_len"]
    g = torch.Generator(device="cuda").manual_seed(1234)
    data = torch.randint(0, c["vocab_size"], (4 * B, T + 1), device="cuda", generator=g)

    def step(i):
        s = data[(i % 4) * B:(i % 4 + 1) * B]
        loss = model(s[:, :-1], s[:, 1:], grad_scale=opt.scale)
        opt.backward(loss)
        opt.step(lr=6e-4)
        opt.zero_grad()
        return loss

    # Host side: move everything allocated so far (torch, the model) out of the cyclic
    # garbage collector's reach.  Each step's autograd graph creates Python objects, and a
    # full collection over the whole heap, when one falls due, stalls the launching thread
    # for about 40 ms (one 58 ms step among 19.7 ms ones).
    gc.collect()
    gc.freeze()
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        loss = step(i)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"ms_per_step": dt * 1e3, "tok_s": B * T / dt, "loss": float(loss.detach()),
            "params": model.num_params(), "found_inf": float(opt._found_inf)}


def _lscpu():
    """CPU model, sockets, physical cores and threads per core from lscpu (host facts for the
    baseline's report)."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass

    def num(k):
        try:
            return int(info.get(k, ""))
        except ValueError:
            return None
    sockets, per_socket, tpc = num("Socket(s)"), num("Core(s) per socket"), num("Thread(s) per core")
    return {"cpu_model": info.get("Model name", ""),
            "physical_cores": sockets * per_socket if sockets and per_socket else None,
            "threads_per_core": tpc, "logical_cpus": num("CPU(s)")}


def cpu_baseline(torch):
    """The reference's naive-PyTorch fp32 step (oracle/gpt.py) on the host cores: the cfg5
    model at the cfg5 batch (16 x 1024 tokens, 1 warm-up + 2 timed steps) and cfg1."""
    from oracle import gpt as ogpt
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    host = _lscpu()
    c = CFG5
    torch.manual_seed(0)
    m = ogpt.GPT(c["vocab_size"], c["seq_len"], c["n_layer"], c["n_head"], c["d_model"])
    opt = ogpt.make_optimizer(m, lr=6e-4)
    Bc, T = c["batch"], c["seq_len"]
    gen = torch.Generator().manual_seed(1234)
    data = torch.randint(0, c["vocab_size"], (Bc, T + 1), generator=gen)
    x, y = data[:, :-1], data[:, 1:]
    ogpt.cpu_train_step(m, opt, x, y)          # warm-up
    n = 2
    t0 = time.perf_counter()
    for _ in range(n):
        ogpt.cpu_train_step(m, opt, x, y)
    dt = (time.perf_counter() - t0) / n
    del m, opt, data, x, y
    # cfg1, the reference's CPU-runnable case: 4L-d256 H4 V256, T256, batch 32, lr 3e-4
    torch.manual_seed(0)
    m1 = ogpt.GPT(256, 256, 4, 4, 256)
    opt1 = ogpt.make_optimizer(m1, lr=3e-4)
    d1 = torch.randint(0, 256, (32, 257), generator=gen)
    x1, y1 = d1[:, :-1], d1[:, 1:]
    ogpt.cpu_train_step(m1, opt1, x1, y1)      # warm-up
    n1, t1 = 0, time.perf_counter()
    while n1 < 3 or (time.perf_counter() - t1 < 5.0 and n1 < 10):
        ogpt.cpu_train_step(m1, opt1, x1, y1)
        n1 += 1
    dt1 = (time.perf_counter() - t1) / n1
    return {"value": round(Bc * T / dt, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle/gpt.py naive-PyTorch fp32 GPT 12L-d768 V50304 (SDPA, F.rms_norm, "
                       f"F.cross_entropy, AdamW + clip 1.0) at the cfg5 batch {Bc} x {T} tokens, "
                       f"1 warm-up + {n} timed steps ({dt:.2f} s/step) on {threads} threads"),
            "host": host,
            "cfg1_tok_s": round(32 * 256 / dt1, 1),
            "cfg1_sample": (f"cfg1 4L-d256 H4 V256 T256 B32 fp32 step, 1 warm-up + {n1} timed steps "
                            f"({dt1:.3f} s/step) on {threads} threads")}


def bench_copy(torch):
    """Calibration workload for the HBM byte counters: torch's copy of 1 GiB."""
    n = 1 << 29
    a = torch.empty(n, device="cuda", dtype=torch.bfloat16).fill_(1.0)
    b = torch.empty_like(a)
    t = time_us(torch, lambda: b.copy_(a), iters=5, warm=2)
    return {"bytes_read": n * 2, "bytes_written": n * 2, "us": round(t, 2)}


def bench_fc_product(torch, which, cold):
    """Profiling workload: the cfg5 fc product y = x W^T (16384 x 768 x 3072) 12 times, on
    this build's whole-tile kernel (`ours`) or torch.mm (hipBLASLt, `library`); with `cold`
    a 1 GiB buffer is written before each call, so the operands come from HBM."""
    from fxgpu.abi import call, ptr, stream_of
    M, K, N = 16384, 768, 3072
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(M, K, device="cuda", generator=g).bfloat16()
    W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).bfloat16()
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    flush = torch.empty(1 << 29, device="cuda", dtype=torch.bfloat16)
    for i in range(12):
        if cold:
            flush.fill_(i)
        if which == "ours":
            call("fx_linear_fwd", ptr(x), K, None, 0, 0, ptr(W), None, ptr(y), None, None, M, N, K, 0,
                 stream_of(x))
        else:
            torch.mm(x, W.t(), out=y)
    torch.cuda.synchronize()
    return {"product": which, "cold": cold, "calls": 12}


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "attn_bwd_cfg2_traffic.json")
_TRAFFIC_KERNELS = ("attn_bwd_dq_kernel", "attn_bwd_dkv_kernel")
# fx_linear_wgrad: the whole-tile kernel and its split-K reduce, averaged over the step's
# 48 layer products (bench.py --only wgrad-step runs each of the four shapes equally often)
WGRAD_TRAFFIC_JSON = os.path.join(ROOT, "profiles", "wgrad_cfg5_traffic.json")
_WGRAD_TRAFFIC_KERNELS = ("gemm_wgrad_fast_kernel", "wgrad_reduce_kernel")


def _pmc_per_dispatch(csv_path, counter, name_filter):
    """Average of `counter` (KiB) per dispatch of kernels whose name contains name_filter,
    from a rocprofv3 --pmc counter_collection.csv."""
    import csv
    vals = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter or name_filter not in r["Kernel_Name"]:
                continue
            vals.setdefault(r["Dispatch_Id"], 0.0)
            vals[r["Dispatch_Id"]] += float(r["Counter_Value"])
    if not vals:
        raise SystemExit(f"{csv_path}: no {counter} rows for kernels matching {name_filter!r}")
    return sum(vals.values()) / len(vals), len(vals)


def pmc_summary(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, kernels=_TRAFFIC_KERNELS):
    """HBM bytes per launch of an entry point made of `kernels` (one dispatch of each per
    launch: fx_attn_bwd's two, or fx_linear_wgrad's kernel and reduce) from FETCH_SIZE /
    WRITE_SIZE (KiB per dispatch), each scaled by what the counter reads for torch's 1 GiB
    copy (known bytes)."""
    known = 1 << 30
    cf, _ = _pmc_per_dispatch(copy_fetch_csv, "FETCH_SIZE", "copy")
    cw, _ = _pmc_per_dispatch(copy_write_csv, "WRITE_SIZE", "copy")
    sf, sw = known / (cf * 1024.0), known / (cw * 1024.0)
    out = {"scale_fetch": sf, "scale_write": sw, "kernels": {}}
    tot = 0.0
    for k in kernels:
        f, nf = _pmc_per_dispatch(fetch_csv, "FETCH_SIZE", k)
        w, nw = _pmc_per_dispatch(write_csv, "WRITE_SIZE", k)
        fb, wb = f * 1024.0 * sf, w * 1024.0 * sw
        out["kernels"][k] = {"fetch_kib": f, "write_kib": w, "dispatches": [nf, nw],
                             "fetch_bytes": fb, "write_bytes": wb}
        tot += fb + wb
    out["traffic_bytes_per_launch"] = tot
    return out


def counter_table(csv_paths, top=12):
    """Per-kernel averages per dispatch from rocprofv3 --pmc counter_collection.csv files,
    as a markdown table: MFMA busy % of the SIMDs (SQ_VALU_MFMA_BUSY_CYCLES over the
    dispatch's active cycles x 1024 SIMDs; the csv's GRBM_GUI_ACTIVE is summed over the 8
    XCDs, so one XCD's count is an eighth of it), issued bf16 MFMA TFLOP/s
    (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 flops over the dispatch time), or FETCH_SIZE /
    WRITE_SIZE in KiB, whichever the files hold."""
    import csv
    agg = {}
    for path in csv_paths:
        with open(path) as f:
            for r in csv.DictReader(f):
                k = r["Kernel_Name"]
                d = agg.setdefault(k, {})
                disp = d.setdefault(r["Dispatch_Id"], {"_t": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))})
                disp[r["Counter_Name"]] = disp.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    rows = []
    for k, disps in agg.items():
        n = len(disps)
        avg = {}
        for dd in disps.values():
            for c, v in dd.items():
                avg[c] = avg.get(c, 0.0) + v / n
        rows.append((k, n, avg))
    rows.sort(key=lambda r: -r[2]["_t"] * r[1])
    names = sorted({c for _, _, a in rows for c in a if c != "_t"})
    hdr = ["kernel", "dispatches", "avg µs"] + names
    mf = "SQ_VALU_MFMA_BUSY_CYCLES" in names and "GRBM_GUI_ACTIVE" in names
    bf = "SQ_INSTS_VALU_MFMA_MOPS_BF16" in names
    if mf:
        hdr.append("MFMA busy %")
    if bf:
        hdr.append("issued bf16 TFLOP/s")
    # per-CU and per-SIMD ratios of the issue / LDS / memory-pipeline counters, when present:
    # a count of CU cycles over GRBM_GUI_ACTIVE / 8 x 256 CUs, a count of wave quad-cycles
    # (x 4) over GRBM_GUI_ACTIVE / 8 x 1024 SIMDs, and the mean L2 read latency in cycles
    per_cu = [c for c in ("SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "TA_TA_BUSY", "TD_TD_BUSY",
                          "TCP_PENDING_STALL_CYCLES") if c in names]
    per_simd = [c for c in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS") if c in names]
    lat = "TCP_TCC_READ_REQ_LATENCY" in names and "TCP_TCC_READ_REQ" in names
    grbm = "GRBM_GUI_ACTIVE" in names
    if grbm:
        hdr += [f"{c} % of CU cycles" for c in per_cu] + [f"{c} % of SIMD cycles" for c in per_simd]
    if lat:
        hdr.append("L2 read latency (cycles)")
    lines = ["| " + " | ".join(hdr) + " |", "|" + "---|" * len(hdr)]
    for k, n, a in rows[:top]:
        kn = k if len(k) < 70 else k[:67] + "..."
        cells = [f"`{kn}`", str(n), f"{a['_t'] / 1e3:.1f}"] + [f"{a.get(c, 0):.0f}" for c in names]
        if mf:
            cells.append(f"{100 * a['SQ_VALU_MFMA_BUSY_CYCLES'] / max(1.0, a['GRBM_GUI_ACTIVE'] / 8 * 1024):.1f}")
        if bf:
            cells.append(f"{a['SQ_INSTS_VALU_MFMA_MOPS_BF16'] * 512 / max(1.0, a['_t']) / 1e3:.1f}")
        if grbm:
            cu_cycles = max(1.0, a["GRBM_GUI_ACTIVE"] / 8 * 256)
            cells += [f"{100 * a[c] / cu_cycles:.1f}" for c in per_cu]
            cells += [f"{100 * 4 * a[c] / (cu_cycles * 4):.1f}" for c in per_simd]
        if lat:
            cells.append(f"{a['TCP_TCC_READ_REQ_LATENCY'] / max(1.0, a['TCP_TCC_READ_REQ']):.0f}")
        lines.append("| " + " | ".join(cells) + " |")
    return "\n".join(lines)


def trace_table(trace_csv, per_step=None, skip=2, top=40, last=None):
    """Per-kernel durations from a rocprofv3 --kernel-trace kernel_trace.csv as a markdown
    table.  With per_step (a kernel name fragment that runs once per training step, e.g. the
    CE row kernel), only the windows between consecutive dispatches of that kernel count,
    after `skip` windows: each holds one step's kernels, and the table is per step, with the
    span (first start to last end) beside the summed kernel time.  With `last`, only the last
    `last` dispatches of each kernel count: the timed rounds of a bench.py kernel line (5 x 20
    launches after the warm-up ones, whose early launches run before the clocks ramp up)."""
    import csv
    rows = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    if last:
        seen, keep = {}, []
        for r in reversed(rows):
            seen[r[2]] = seen.get(r[2], 0) + 1
            if seen[r[2]] <= last:
                keep.append(r)
        rows = keep[::-1]
    note = f"{len(rows)} dispatches" + (f" (the last {last} of each kernel)" if last else "")
    if per_step:
        marks = [i for i, (_, _, k) in enumerate(rows) if per_step in k]
        wins = list(zip(marks[skip:], marks[skip + 1:]))
        if not wins:
            raise SystemExit(f"fewer than {skip + 2} dispatches of {per_step!r}")
        sel = [rows[i] for a, b in wins for i in range(a, b)]
        nwin = len(wins)
        span = sum(rows[b][0] - rows[a][0] for a, b in wins) / nwin / 1e3
        note = (f"{nwin} steps (windows between consecutive `{per_step}` dispatches, the first {skip} "
                f"skipped): {sum(e - s for s, e, _ in sel) / nwin / 1e3:.1f} µs of kernels per step in a "
                f"span of {span:.1f} µs, {len(sel) / nwin:.0f} dispatches per step")
    else:
        sel, nwin = rows, 1
    agg = {}
    for s, e, k in sel:
        d = agg.setdefault(k, [0, 0, float("inf"), 0])
        d[0] += 1
        d[1] += e - s
        d[2] = min(d[2], e - s)
        d[3] = max(d[3], e - s)
    total = sum(d[1] for d in agg.values())
    unit = "per step" if per_step else "total"
    lines = [note, "", f"| kernel | calls {unit} | avg µs | min µs | max µs | µs {unit} | % |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for k, (n, t, lo, hi) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]:
        kn = k if len(k) < 90 else k[:87] + "..."
        lines.append(f"| `{kn}` | {n / nwin:.1f} | {t / n / 1e3:.2f} | {lo / 1e3:.2f} | {hi / 1e3:.2f} | "
                     f"{t / nwin / 1e3:.1f} | {100 * t / total:.1f} |")
    return "\n".join(lines)


def traffic_table(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, top=12):
    """HBM bytes per dispatch of every kernel in a FETCH_SIZE and a WRITE_SIZE pass, each
    scaled by what the same counter reads for torch's 1 GiB copy (bench.py --only copy), as a
    markdown table with the achieved GB/s over the dispatch time of the FETCH pass."""
    import csv
    known = 1 << 30
    cf, _ = _pmc_per_dispatch(copy_fetch_csv, "FETCH_SIZE", "copy")
    cw, _ = _pmc_per_dispatch(copy_write_csv, "WRITE_SIZE", "copy")
    sf, sw = known / (cf * 1024.0), known / (cw * 1024.0)
    per = {}
    for path, ctr in ((fetch_csv, "FETCH_SIZE"), (write_csv, "WRITE_SIZE")):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != ctr:
                    continue
                d = per.setdefault(r["Kernel_Name"], {}).setdefault(ctr, {})
                e = d.setdefault(r["Dispatch_Id"], [0.0, int(r["End_Timestamp"]) - int(r["Start_Timestamp"])])
                e[0] += float(r["Counter_Value"])
    lines = [f"Calibration: FETCH_SIZE x{sf:.4f}, WRITE_SIZE x{sw:.4f} (torch copy of 1 GiB).", "",
             "| kernel | dispatches | fetch MB | write MB | total MB | µs (fetch pass) | GB/s |",
             "|---|---|---|---|---|---|---|"]
    rows = []
    for k, d in per.items():
        if "FETCH_SIZE" not in d or "WRITE_SIZE" not in d:
            continue
        fv = list(d["FETCH_SIZE"].values())
        wv = list(d["WRITE_SIZE"].values())
        fb = sum(v for v, _ in fv) / len(fv) * 1024 * sf
        wb = sum(v for v, _ in wv) / len(wv) * 1024 * sw
        us = sum(t for _, t in fv) / len(fv) / 1e3
        rows.append((k, len(fv), fb, wb, us))
    rows.sort(key=lambda r: -(r[2] + r[3]) * r[1])
    for k, n, fb, wb, us in rows[:top]:
        kn = k if len(k) < 70 else k[:67] + "..."
        lines.append(f"| `{kn}` | {n} | {fb / 1e6:.1f} | {wb / 1e6:.1f} | {(fb + wb) / 1e6:.1f} | {us:.1f} | "
                     f"{(fb + wb) / max(us, 1e-9) / 1e3:.0f} |")
    return "\n".join(lines)


def _traffic(path=TRAFFIC_JSON):
    try:
        with open(path) as f:
            return round(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    # 4 warm-up steps: one pass over each of the 4 synthetic batches the step cycles through,
    # so that no batch's first step (and no first allocation of a size) falls in the timed steps
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-CPU baseline")
    ap.add_argument("--only", choices=["attention", "ce", "norm", "adamw", "linear", "wgrad", "wgrad-step",
                                       "gemm-kernels", "head",
                                       "library", "step", "copy",
                                       "decode", "embedding",
                                       "cpu", "fc-ours", "fc-library", "fc-ours-cold", "fc-library-cold"],
                    help="run one workload and print its figures (for profiling runs)")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                                                       "COPY_WRITE_CSV"),
                    help="write the fx_attn_bwd HBM traffic from rocprofv3 --pmc csv files")
    ap.add_argument("--pmc-summary-wgrad", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                                                             "COPY_WRITE_CSV"),
                    help="write the fx_linear_wgrad HBM traffic (bench.py --only wgrad-step runs)")
    ap.add_argument("--counter-table", nargs="+", metavar="CSV",
                    help="print per-kernel counter averages from rocprofv3 --pmc csv files")
    ap.add_argument("--trace-table", nargs="+", metavar=("TRACE_CSV", "PER_STEP_KERNEL"),
                    help="print per-kernel durations from a rocprofv3 --kernel-trace csv (per step when a "
                         "once-per-step kernel name is given)")
    ap.add_argument("--trace-last", type=int, default=None, metavar="N",
                    help="--trace-table: only the last N dispatches of each kernel (bench.py's timed rounds: 100)")
    ap.add_argument("--traffic-table", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                                                         "COPY_WRITE_CSV"),
                    help="print per-kernel HBM bytes from FETCH_SIZE / WRITE_SIZE passes")
    args = ap.parse_args()
    if args.counter_table:
        print(counter_table(args.counter_table))
        return
    if args.traffic_table:
        print(traffic_table(*args.traffic_table))
        return
    if args.trace_table:
        print(trace_table(args.trace_table[0], args.trace_table[1] if len(args.trace_table) > 1 else None,
                          last=args.trace_last))
        return
    if args.pmc_summary or args.pmc_summary_wgrad:
        wg = bool(args.pmc_summary_wgrad)
        res = pmc_summary(*(args.pmc_summary_wgrad if wg else args.pmc_summary),
                          kernels=_WGRAD_TRAFFIC_KERNELS if wg else _TRAFFIC_KERNELS)
        with open(WGRAD_TRAFFIC_JSON if wg else TRAFFIC_JSON, "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the fxlm hot path is "
              "measured on a single GPU; multi-GPU sharding is designed, not built.", file=sys.stderr)
        sys.exit(2)
    import torch
    from fxgpu.abi import lib
    lib()
    if args.only:
        fn = {"attention": bench_attention, "ce": bench_ce, "norm": bench_norm, "adamw": bench_adamw,
              "linear": bench_linear, "wgrad": bench_wgrad, "wgrad-step": bench_wgrad_step,
              "gemm-kernels": bench_gemm_kernels,
              "head": bench_head, "copy": bench_copy,
              "library": bench_library,
              "decode": bench_decode, "embedding": bench_embedding,
              "cpu": cpu_baseline,
              "step": lambda t: gpu_step_bench(t, args.steps, args.warmup),
              "fc-ours": lambda t: bench_fc_product(t, "ours", False),
              "fc-library": lambda t: bench_fc_product(t, "library", False),
              "fc-ours-cold": lambda t: bench_fc_product(t, "ours", True),
              "fc-library-cold": lambda t: bench_fc_product(t, "library", True)}[args.only]
        r = fn(torch)
        print(json.dumps({k: v for k, v in r.items() if not k.startswith("flop")}))
        return

    attn = bench_attention(torch)
    ce = bench_ce(torch)
    norm = bench_norm(torch)
    adamw = bench_adamw(torch)
    lin = bench_linear(torch)
    wg = bench_wgrad(torch)
    head = bench_head(torch)
    torch.cuda.empty_cache()
    libs = bench_library(torch)
    attn["library"] = libs["attention_cfg2"]
    ce["library"] = libs["cross_entropy_cfg3"]
    norm["library"] = libs["rmsnorm_cfg4"]
    adamw["library"] = dict(libs["flat_adamw_cfg4"],
                            speedup=round(libs["flat_adamw_cfg4"]["torch_fused_adamw_clip_scaler_us"]
                                          / adamw["step_us"], 2))
    dec = bench_decode(torch)
    emb = bench_embedding(torch)
    torch.cuda.empty_cache()
    step = gpu_step_bench(torch, args.steps, args.warmup)
    torch.cuda.empty_cache()

    # the dominant kernel of the step among this build's own: fx_linear_wgrad (48 launches,
    # ~3.3 ms of the step's kernel time against ~1.75 ms for the attention backward), per
    # average launch of the step's mix; the attention figures stay under kernels
    wf, wus = wgrad_roofline(wg)
    roofline = {
        "kernel": "fx_linear_wgrad (gemm_wgrad_fast_kernel<3> + wgrad_reduce), the cfg5 step's layer "
                  "weight gradients dW = dy^T x over 16384 tokens (qkv, proj, fc, fc2), per average launch",
        "bound": "mfma", "achieved": round(wf / wus / 1e6, 1),
        "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": round(wf / wus / 1e6 / BF16_PEAK_TFLOPS, 4),
        # HBM bytes per average launch: rocprofv3 FETCH_SIZE + WRITE_SIZE of the kernel and
        # its reduce, calibrated on a copy of known size (profiles/wgrad_cfg5_traffic.*)
        "traffic": _traffic(WGRAD_TRAFFIC_JSON),
        "flop_per_launch": round(wf),
    }
    attn_roof = {"kernel": "fx_attn_bwd (attn_bwd_dq + attn_bwd_dkv), cfg2 [16,12,1024,64] causal",
                 "achieved": round(attn["flop_bwd"] / attn["bwd_us"] / 1e6, 1),
                 "frac": round(attn["flop_bwd"] / attn["bwd_us"] / 1e6 / BF16_PEAK_TFLOPS, 4),
                 "traffic": _traffic()}
    cpu = None if args.no_cpu else cpu_baseline(torch)
    out = {
        "metric": "train tokens/sec (GPT 12L-d768, S=1024) + attn fwd/bwd TFLOPS, % roofline",
        "value": round(step["tok_s"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step["ms_per_step"], 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform random tokens, seed 1234; random-init weights N(0,0.02))",
        "config": {"workload": "GPT 12L-d768 H12 V50304 S1024 B16 bf16 train step "
                               "(fwd+bwd+FlatAdamW), fused attention/RMSNorm/linear-CE/MLP/AdamW",
                   "global_batch": 16, "seq_len": 1024, "tokens_per_step": 16384,
                   "params": step["params"], "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gpu_over_cpu": (round(step["tok_s"] / cpu["value"], 1) if cpu else None),
        "kernels": {"attention_cfg2": dict({k: v for k, v in attn.items() if not k.startswith("flop")},
                                           bwd_roofline=attn_roof),
                    "cross_entropy_cfg3": ce, "rmsnorm_cfg4": norm, "flat_adamw_cfg4": adamw,
                    "fused_linear_gelu_cfg5_fc": lin, "linear_wgrad_cfg5": wg,
                    "linear_ce_head_cfg5": head, "decode": dec,
                    "embedding_grad_cfg5": emb},
        "final_loss": round(step["loss"], 4),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
