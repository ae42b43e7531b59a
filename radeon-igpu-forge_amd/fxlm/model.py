"""fxlm.model: GPTConfig + GPT -- pre-norm transformer trained in bf16 on gfx950.

Block: RMSNorm -> qkv Linear(D -> 3D, no bias) -> flash_attention_qkv on the
(B,T,3,H,Dh) view (no permute) -> proj Linear -> residual; RMSNorm -> fused
linear+GELU(tanh) (D -> 4D) -> fc2 -> residual.  Final RMSNorm; LM head = tied
embedding (or a separate Linear).  Same structure, names and initialisation
as ml/fxlm/model.py:22-130.  Implementation switches pick the gfx950 kernels
("flash" / "fused") or the plain PyTorch paths ("sdpa" / "torch") for
ablation and parity; mlp_impl covers the fused linear layer the reference
computes as fc followed by F.gelu.
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as Fn
from torch import nn

from fxgpu.fused_linear import FEW_ROWS, fused_linear, fused_mlp, linear, linear_ex

from .attention import decode_attention, flash_attention_qkv
from .cross_entropy import linear_cross_entropy
from .embedding import token_embedding
from .norm import add_pre_norm, pre_norm, rms_norm


@dataclass
class GPTConfig:
    vocab_size: int
    seq_len: int
    n_layer: int
    n_head: int
    d_model: int
    mlp_ratio: int = 4
    tie_embeddings: bool = True
    attn_impl: str = "flash"      # "flash" | "sdpa"
    norm_impl: str = "fused"      # "fused" | "torch"
    ce_impl: str = "fused"        # "fused" | "torch"
    mlp_impl: str = "fused"       # "fused" | "torch"
    linear_impl: str = "fused"    # qkv / proj / fc2 (split-K dW) and tok_emb's gradient: "fused" | "torch"
    eps: float = 1e-6


class Block(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        D, H = cfg.d_model, cfg.n_head
        self.n_head = H
        self.head_dim = D // H
        self.attn_impl = cfg.attn_impl
        self.norm_impl = cfg.norm_impl
        self.mlp_impl = cfg.mlp_impl
        self.linear_impl = cfg.linear_impl
        self.eps = cfg.eps
        self.ln1_w = nn.Parameter(torch.ones(D))
        self.ln2_w = nn.Parameter(torch.ones(D))
        self.qkv = nn.Linear(D, 3 * D, bias=False)
        self.proj = nn.Linear(D, D, bias=False)
        self.fc = nn.Linear(D, cfg.mlp_ratio * D, bias=False)
        self.fc2 = nn.Linear(cfg.mlp_ratio * D, D, bias=False)

    def _norm(self, x, w):
        if self.norm_impl == "fused":
            return rms_norm(x, w, self.eps)
        return Fn.rms_norm(x, (x.shape[-1],), w, self.eps)

    def _prenorm(self, x, w):
        """(x, norm(x)); the fused form sums x's two gradients in the norm's backward."""
        if self.norm_impl == "fused":
            return pre_norm(x, w, self.eps)
        return x, self._norm(x, w)

    def _lin(self, x, layer):
        if self.linear_impl == "fused":
            return linear(x, layer.weight)
        return layer(x)

    def _mlp_out(self, h):
        """fc2(gelu(fc(h))) (ml/fxlm/model.py:64-66,71): one node (fused_mlp) when both the
        MLP and the projections take the fused kernels"""
        if self.mlp_impl == "fused" and self.linear_impl == "fused" and h.is_cuda:
            return fused_mlp(h, self.fc.weight, self.fc2.weight)
        if self.mlp_impl == "fused":
            u = fused_linear(h, self.fc.weight, None, "gelu_tanh")
        else:
            u = Fn.gelu(self.fc(h), approximate="tanh")
        return self._lin(u, self.fc2)

    def _mlp(self, x):
        x, h = self._prenorm(x, self.ln2_w)
        return x + self._mlp_out(h)

    def _add_prenorm(self, x, r, w):
        """(x + r, norm(x + r)); the fused form adds inside the norm's own pass."""
        if self.norm_impl == "fused":
            return add_pre_norm(x, r, w, self.eps)
        x = x + r
        return x, self._norm(x, w)

    def forward(self, x, kv=None):
        """kv: optional (k_cache, v_cache) (B, Tmax, H, Dh) that receive this block's
        keys and values at positions 0..T-1 (the prompt of a cached generation)."""
        x, out = self.forward_pair(x, None, kv)
        return x + out

    def forward_pair(self, x, branch=None, kv=None):
        """(x', out) with the block's output x' + out (ml/fxlm/model.py:58-72), the last
        residual sum left to the next norm that reads it; `branch`, the previous block's
        `out`, is added to x inside this block's first norm."""
        B, T, D = x.shape
        if branch is None:
            x, h = self._prenorm(x, self.ln1_w)
        else:
            x, h = self._add_prenorm(x, branch, self.ln1_w)
        qkv = self._lin(h, self.qkv).view(B, T, 3, self.n_head, self.head_dim)
        if kv is not None:
            kv[0][:, :T].copy_(qkv[:, :, 1])
            kv[1][:, :T].copy_(qkv[:, :, 2])
        if self.attn_impl == "flash":
            y = flash_attention_qkv(qkv, causal=True)
        else:
            q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))   # (B,H,T,Dh)
            y = Fn.scaled_dot_product_attention(q, k, v, is_causal=True)
            y = y.transpose(1, 2)
        x, h = self._add_prenorm(x, self._lin(y.reshape(B, T, D), self.proj), self.ln2_w)
        return x, self._mlp_out(h)

    def step(self, x, kv, pos, lens):
        """One new token per sequence: x (B, 1, D) at position lens[b] - 1 (lens (B,) int32
        on the device, pos (1,) int64 the same position); attention over the first
        lens[b] keys, the new key and value written into the caches by the attention
        kernel.  No host value depends on the position, so a step can be captured once in
        a HIP graph and replayed for every token."""
        B, _, D = x.shape
        if self._fused_step(B):
            # four projections and the attention: the norms run inside qkv / fc, the
            # residual sums inside proj / fc2
            qkv = linear_ex(x, self.qkv.weight, norm_weight=self.ln1_w, eps=self.eps)
            qkv = qkv.view(B, 1, 3, self.n_head, self.head_dim)
            y = decode_attention(qkv[:, 0, 0], kv[0], kv[1], lens, k_new=qkv[:, 0, 1], v_new=qkv[:, 0, 2])
            x = linear_ex(y.reshape(B, 1, D), self.proj.weight, residual=x)
            u = linear_ex(x, self.fc.weight, norm_weight=self.ln2_w, eps=self.eps, activation="gelu_tanh")
            return linear_ex(u, self.fc2.weight, residual=x)
        h = self._norm(x, self.ln1_w)
        qkv = self._lin(h, self.qkv).view(B, 1, 3, self.n_head, self.head_dim)
        # the attention kernel writes the new key and value into the caches at lens - 1
        y = decode_attention(qkv[:, 0, 0], kv[0], kv[1], lens, k_new=qkv[:, 0, 1], v_new=qkv[:, 0, 2])
        x = x + self._lin(y.reshape(B, 1, D), self.proj)
        return self._mlp(x)

    def _fused_step(self, rows):
        return (self.norm_impl == "fused" and self.linear_impl == "fused" and self.mlp_impl == "fused"
                and rows <= FEW_ROWS)


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        if cfg.d_model % cfg.n_head:
            raise ValueError("d_model must be a multiple of n_head")
        self.cfg = cfg
        D = cfg.d_model
        self.tok_emb = nn.Embedding(cfg.vocab_size, D)
        self.pos_emb = nn.Parameter(torch.zeros(cfg.seq_len, D))
        self.blocks = nn.ModuleList(Block(cfg) for _ in range(cfg.n_layer))
        self.lnf_w = nn.Parameter(torch.ones(D))
        if not cfg.tie_embeddings:
            self.head = nn.Linear(D, cfg.vocab_size, bias=False)
        self.apply(self._init)
        # small init for the residual projections (depth scaling)
        s = 0.02 / math.sqrt(2 * cfg.n_layer)
        for b in self.blocks:
            nn.init.normal_(b.proj.weight, std=s)
            nn.init.normal_(b.fc2.weight, std=s)

    @staticmethod
    def _init(m):
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, std=0.02)

    def _head(self, x):
        """Logits of a few rows (prefill's last position, decode steps)."""
        if self.cfg.linear_impl == "fused" and x.is_cuda:
            return linear(x, self._head_w())
        return Fn.linear(x, self._head_w())

    def _norm_f(self, x):
        if self.cfg.norm_impl == "fused":
            return rms_norm(x, self.lnf_w, self.cfg.eps)
        return Fn.rms_norm(x, (x.shape[-1],), self.lnf_w, self.cfg.eps)

    def _norm_f_add(self, x, r):
        """Final norm of x + r (the last block's residual sum, added in the norm's pass);
        r is None when there are no blocks."""
        if r is None:
            return self._norm_f(x)
        if self.cfg.norm_impl == "fused":
            return add_pre_norm(x, r, self.lnf_w, self.cfg.eps)[1]
        return self._norm_f(x + r)

    def _tok(self, idx):
        """tok_emb(idx) (ml/fxlm/model.py:118); on the fused path its weight gradient is
        fx_embedding_bwd's (deterministic, launch sizes independent of the ids)."""
        w = self.tok_emb.weight
        if (self.cfg.linear_impl == "fused" and idx.is_cuda and w.dtype == torch.bfloat16
                and w.shape[1] % 8 == 0):
            return token_embedding(idx, w)
        return self.tok_emb(idx)

    def _head_w(self):
        return self.tok_emb.weight if self.cfg.tie_embeddings else self.head.weight

    def num_params(self):
        return sum(p.numel() for p in self.parameters())

    def forward(self, idx, targets=None, grad_scale=1.0):
        B, T = idx.shape
        if T > self.cfg.seq_len:
            raise ValueError(f"T={T} > seq_len={self.cfg.seq_len}")
        x = self._tok(idx) + self.pos_emb[:T]
        branch = None
        for blk in self.blocks:
            x, branch = blk.forward_pair(x, branch)
        x = self._norm_f_add(x, branch)
        if targets is None:
            return Fn.linear(x, self._head_w())
        if self.cfg.ce_impl == "fused":
            return linear_cross_entropy(x.reshape(-1, x.shape[-1]), self._head_w(),
                                        targets.reshape(-1), grad_scale=grad_scale)
        logits = Fn.linear(x, self._head_w())
        return Fn.cross_entropy(logits.float().view(-1, logits.shape[-1]), targets.reshape(-1))

    # -- cached inference ------------------------------------------------------------
    # The reference's sampler re-runs the whole (cropped) context for every new token
    # (ml/fxlm/sample.py:62-73).  Here the prompt runs once through the blocks, which
    # leave their keys and values in a bf16 cache, and each new token runs the blocks
    # on one row per sequence with decode attention over the cache.

    def init_cache(self, batch, max_len=None):
        """Per-layer (k, v) caches (batch, max_len, H, Dh) bf16 on the model's device."""
        cfg = self.cfg
        T = cfg.seq_len if max_len is None else min(int(max_len), cfg.seq_len)
        H, Dh = cfg.n_head, cfg.d_model // cfg.n_head
        dev = self.pos_emb.device
        return [(torch.empty(batch, T, H, Dh, device=dev, dtype=torch.bfloat16),
                 torch.empty(batch, T, H, Dh, device=dev, dtype=torch.bfloat16))
                for _ in self.blocks]

    @torch.no_grad()
    def prefill(self, idx, cache):
        """Run the prompt idx (B, T) and fill the caches; returns the last position's
        logits (B, V) in fp32."""
        if self.cfg.attn_impl != "flash":
            raise ValueError("cached inference needs attn_impl='flash'")
        B, T = idx.shape
        if T > cache[0][0].shape[1]:
            raise ValueError(f"prompt of {T} tokens exceeds the cache ({cache[0][0].shape[1]})")
        x = self.tok_emb(idx) + self.pos_emb[:T]
        for blk, kv in zip(self.blocks, cache):
            x = blk(x, kv)
        x = self._norm_f(x[:, -1:].contiguous())
        return self._head(x[:, 0]).float()

    def _decode(self, tok, cache, pos, lens):
        """Cached step with the position in device memory: tok (B,) int64, pos (1,) int64,
        lens (B,) int32 = pos + 1; returns the logits (B, V) fp32."""
        B = tok.shape[0]
        x = self.tok_emb(tok.view(B, 1)) + self.pos_emb.index_select(0, pos)
        for blk, kv in zip(self.blocks, cache):
            x = blk.step(x, kv, pos, lens)
        if self.blocks and self.blocks[0]._fused_step(B):   # final norm inside the head GEMM
            return linear_ex(x[:, 0], self._head_w(), norm_weight=self.lnf_w, eps=self.cfg.eps).float()
        x = self._norm_f(x)
        return self._head(x[:, 0]).float()

    @torch.no_grad()
    def decode_step(self, tok, cache, pos):
        """tok (B,) int64 at position pos (< the cache length, every sequence at the same
        position); returns its logits (B, V) in fp32."""
        B = tok.shape[0]
        if pos >= cache[0][0].shape[1]:
            raise ValueError(f"position {pos} is past the cache ({cache[0][0].shape[1]})")
        p = torch.full((1,), pos, dtype=torch.int64, device=tok.device)
        lens = torch.full((B,), pos + 1, dtype=torch.int32, device=tok.device)
        return self._decode(tok, cache, p, lens)

    def decode_graph(self, cache, batch):
        """A HIP graph of one cached step for `cache` (the launches of ~14 ops per layer
        otherwise cost more host time than the step's GPU work).  Call the returned
        object as step(tok, pos) -> logits (B, V) fp32; the logits tensor is reused by
        the next call."""
        return _DecodeGraph(self, cache, batch)

    @torch.no_grad()
    def generate(self, idx, max_new, temperature=0.8, top_k=50, generator=None, graph=True):
        """Sample max_new tokens after idx (B, T) as ml/fxlm/sample.py:62-73 does
        (temperature, top-k, multinomial); returns (B, max_new) int64.  While the
        context fits seq_len each token is one cached step (replayed from a HIP graph
        when `graph`); past it, as in the reference, the model re-runs the last seq_len
        tokens."""
        x = idx
        B = idx.shape[0]
        L = self.cfg.seq_len
        cache = self.init_cache(B, min(L, idx.shape[1] + max_new)) if idx.shape[1] < L else None
        logits = self.prefill(idx, cache) if cache is not None else None
        step = None
        if cache is not None and max_new > 1:
            step = self.decode_graph(cache, B) if graph else (lambda t, p: self.decode_step(t, cache, p))
        out = []
        for _ in range(max_new):
            if logits is None:  # context beyond seq_len: re-run the cropped window
                logits = self(x[:, -L:])[:, -1, :].float()
            logits = logits / max(temperature, 1e-5)
            if top_k > 0:
                v, _ = torch.topk(logits, min(top_k, logits.shape[-1]))
                logits = logits.masked_fill(logits < v[:, -1:], -float("inf"))
            nxt = torch.multinomial(torch.softmax(logits, dim=-1), 1, generator=generator)
            out.append(nxt)
            x = torch.cat([x, nxt], dim=1)
            pos = x.shape[1] - 1
            if len(out) == max_new:
                break
            logits = step(nxt[:, 0], pos) if step is not None and pos < cache[0][0].shape[1] else None
        return torch.cat(out, dim=1) if out else idx.new_zeros(B, 0)


class _DecodeGraph:
    """One cached decode step captured in a HIP graph (torch.cuda.CUDAGraph).  Inputs
    are copied into static device tensors before each replay; the kernels read the
    position from them, so one capture serves every position of the cache."""

    def __init__(self, model, cache, batch):
        dev = cache[0][0].device
        self.cache_len = cache[0][0].shape[1]
        self.tok = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int64, device=dev)
        self.lens = torch.ones(batch, dtype=torch.int32, device=dev)
        with torch.no_grad():
            # warm-up off the capture (library handles, workspaces), as torch requires;
            # position 0 only rewrites a cache row the real prompt fills again
            # copies of the cache rows the warm-up writes, queued before the side stream
            # waits on the current one: the warm-up then runs after them
            saved = [(k[:, :1].clone(), v[:, :1].clone()) for k, v in cache]
            s = torch.cuda.Stream(device=dev)
            s.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(s):
                for _ in range(2):
                    model._decode(self.tok, cache, self.pos, self.lens)
            torch.cuda.current_stream(dev).wait_stream(s)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.logits = model._decode(self.tok, cache, self.pos, self.lens)
            for (k, v), (k0, v0) in zip(cache, saved):
                k[:, :1].copy_(k0)
                v[:, :1].copy_(v0)

    def __call__(self, tok, pos):
        if pos >= self.cache_len:
            raise ValueError(f"position {pos} is past the cache ({self.cache_len})")
        self.tok.copy_(tok)
        self.pos.fill_(pos)
        self.lens.fill_(pos + 1)
        self.graph.replay()
        return self.logits
