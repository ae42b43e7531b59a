"""Oracle: the reference's naive-PyTorch GPT training step on the CPU (TEST INFRASTRUCTURE ONLY).

Restates fxlm's GPT with its plain-PyTorch implementations selected
(ml/fxlm/model.py:22-130 with attn_impl="sdpa", norm_impl="torch",
ce_impl="torch"; the configuration ml/fxlm/selftest.py:305-308 uses as its
comparator) and the baseline optimiser loop of ml/bench/bench10_lm.py:92-111
(AdamW with weight decay on ndim >= 2 parameters, clip_grad_norm_(1.0)).
Pre-norm blocks, no biases, GELU-tanh MLP, tied LM head, init N(0, 0.02) with
proj/fc2 at 0.02/sqrt(2L).  Parameter names match fxlm.model.GPT so one
state_dict loads into both.

bench.py times `cpu_train_step` on the host as the CPU baseline.
"""
import math

import torch
import torch.nn.functional as F
from torch import nn


class Block(nn.Module):
    def __init__(self, D, H, mlp_ratio, eps):
        super().__init__()
        self.n_head, self.eps = H, eps
        self.ln1_w = nn.Parameter(torch.ones(D))
        self.ln2_w = nn.Parameter(torch.ones(D))
        self.qkv = nn.Linear(D, 3 * D, bias=False)
        self.proj = nn.Linear(D, D, bias=False)
        self.fc = nn.Linear(D, mlp_ratio * D, bias=False)
        self.fc2 = nn.Linear(mlp_ratio * D, D, bias=False)

    def forward(self, x):
        B, T, D = x.shape
        h = F.rms_norm(x, (D,), self.ln1_w, self.eps)
        qkv = self.qkv(h).view(B, T, 3, self.n_head, D // self.n_head)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + self.proj(y.transpose(1, 2).reshape(B, T, D))
        h = F.rms_norm(x, (D,), self.ln2_w, self.eps)
        return x + self.fc2(F.gelu(self.fc(h), approximate="tanh"))


class GPT(nn.Module):
    def __init__(self, vocab_size, seq_len, n_layer, n_head, d_model, mlp_ratio=4, eps=1e-6):
        super().__init__()
        self.vocab_size, self.eps = vocab_size, eps
        self.tok_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Parameter(torch.zeros(seq_len, d_model))
        self.blocks = nn.ModuleList(Block(d_model, n_head, mlp_ratio, eps) for _ in range(n_layer))
        self.lnf_w = nn.Parameter(torch.ones(d_model))
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, std=0.02)
        s = 0.02 / math.sqrt(2 * n_layer)
        for b in self.blocks:
            nn.init.normal_(b.proj.weight, std=s)
            nn.init.normal_(b.fc2.weight, std=s)

    def forward(self, idx, targets=None):
        """Mean CE over every position, or the logits (B, T, V) without targets
        (ml/fxlm/model.py:114-130)."""
        T = idx.shape[1]
        x = self.tok_emb(idx) + self.pos_emb[:T]
        for blk in self.blocks:
            x = blk(x)
        x = F.rms_norm(x, (x.shape[-1],), self.lnf_w, self.eps)
        logits = F.linear(x, self.tok_emb.weight)
        if targets is None:
            return logits
        return F.cross_entropy(logits.float().view(-1, logits.shape[-1]), targets.reshape(-1))


def make_optimizer(model, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1):
    decay = [p for p in model.parameters() if p.dim() >= 2]
    other = [p for p in model.parameters() if p.dim() < 2]
    return torch.optim.AdamW([{"params": decay, "weight_decay": weight_decay},
                              {"params": other, "weight_decay": 0.0}],
                             lr=lr, betas=betas, eps=1e-8)


def cpu_train_step(model, opt, x, y, clip=1.0):
    """One fp32 training step (forward, backward, clip, AdamW); returns the loss."""
    loss = model(x, y)
    opt.zero_grad(set_to_none=True)
    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), clip)
    opt.step()
    return float(loss.detach())
