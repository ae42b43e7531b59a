"""Oracle: FlatAdamW step semantics (TEST INFRASTRUCTURE ONLY).

Restates ml/fxlm/optim.py:61-173 and ml/fxlm/kernels/optim.hip:25-162:
  layout    each parameter at an 8-aligned offset of one flat buffer (optim.py:46-47,85);
            weight decay only for ndim >= 2 when weight_decay != 0 (:82-84)
  sumsq     sum of squares of the (scaled) low-precision gradients; bad = any non-finite
            gradient or a non-finite sum (optim.hip:44-51, :81)
  final     norm = sqrt(sumsq)/scale; clip = bad ? 0 : min(1, max_norm/(norm + 1e-6));
            step += 1 only when not bad (optim.hip:77-93)
  update    skipped when bad; g = grad * clip / scale; w -= lr*wd*w (flagged);
            m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
            w -= lr * (m / (1 - b1^step)) / (sqrt(v / (1 - b2^step)) + eps); p16 = round(w)
            (optim.hip:95-162) -- fp32 arithmetic
  scale     torch._amp_update_scale_ semantics: bad -> scale *= backoff, growth = 0;
            else growth += 1 and at growth_interval scale *= growth_factor (if finite),
            growth = 0 (optim.py:170-171)
"""
import math

import torch


def align8(n):
    return (n + 7) & ~7


def layout(shapes, weight_decay):
    """[(offset, numel, wd_flag)] and the flat size for parameters of `shapes`."""
    out, total = [], 0
    for shp in shapes:
        n = int(math.prod(shp))
        out.append((total, n, 1 if (len(shp) >= 2 and weight_decay != 0) else 0))
        total += align8(n)
    return out, total


def update_scale(scale, growth, found_inf, growth_factor=2.0, backoff=0.5, interval=1000):
    """Returns (scale, growth) after one step (fp32 scale)."""
    scale = torch.tensor(scale, dtype=torch.float32)
    if found_inf:
        return float(scale * backoff), 0
    ok = growth + 1
    if ok == interval:
        ns = scale * growth_factor
        return (float(ns) if math.isfinite(float(ns)) else float(scale)), 0
    return float(scale), ok


class FlatAdamWRef:
    """Flat-buffer AdamW with clip, skip-on-inf and dynamic loss scale (fp32 CPU)."""

    def __init__(self, params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                 max_grad_norm=1.0, init_scale=2.0 ** 16, growth_interval=1000):
        self.shapes = [tuple(p.shape) for p in params]
        self.info, total = layout(self.shapes, weight_decay)
        self.master = torch.zeros(total, dtype=torch.float32)
        for p, (off, n, _wd) in zip(params, self.info):
            self.master[off:off + n] = p.detach().cpu().float().reshape(-1)
        self.m = torch.zeros(total, dtype=torch.float32)
        self.v = torch.zeros(total, dtype=torch.float32)
        self.lr, self.betas, self.eps = lr, betas, eps
        self.weight_decay, self.max_grad_norm = weight_decay, max_grad_norm
        self.scale, self.growth, self.step_ctr = float(init_scale), 0, 0
        self.growth_interval = growth_interval

    def flat16(self):
        return self.master.to(torch.bfloat16)

    def step(self, grads, lr=None):
        """grads: list (same order as params) of gradient tensors or None."""
        lr = self.lr if lr is None else lr
        f32 = torch.float32
        sumsq = 0.0
        for g in grads:
            if g is not None:
                gf = g.detach().cpu().to(f32)
                sumsq += float((gf * gf).to(torch.float64).sum())
        sumsq_f = float(torch.tensor(sumsq, dtype=f32))
        bad = not math.isfinite(sumsq_f)
        scale = torch.tensor(self.scale, dtype=f32)
        norm = torch.sqrt(torch.tensor(sumsq_f, dtype=f32)) / scale
        clip = torch.tensor(0.0, dtype=f32) if bad else torch.clamp(
            torch.tensor(self.max_grad_norm, dtype=f32) / (norm + 1e-6), max=1.0)
        if not bad:
            self.step_ctr += 1
            b1, b2 = torch.tensor(self.betas[0], dtype=f32), torch.tensor(self.betas[1], dtype=f32)
            bc1 = 1 - b1 ** self.step_ctr
            bc2 = 1 - b2 ** self.step_ctr
            inv = clip / scale
            lr_t, wd_t = torch.tensor(lr, dtype=f32), torch.tensor(self.weight_decay, dtype=f32)
            for g, (off, n, wd) in zip(grads, self.info):
                if g is None:
                    continue
                gg = g.detach().cpu().to(f32).reshape(-1) * inv
                w = self.master[off:off + n]
                if wd:
                    w = w - lr_t * wd_t * w
                m = self.m[off:off + n] * b1 + (1 - b1) * gg
                v = self.v[off:off + n] * b2 + (1 - b2) * gg * gg
                w = w - lr_t * (m / bc1) / (torch.sqrt(v / bc2) + self.eps)
                self.master[off:off + n] = w
                self.m[off:off + n] = m
                self.v[off:off + n] = v
        found = 1.0 if bad else 0.0
        self.scale, self.growth = update_scale(self.scale, self.growth, bad,
                                               interval=self.growth_interval)
        return {"grad_norm": float(norm), "found_inf": found, "scale": self.scale}
