"""Oracle: token-embedding weight gradient (TEST INFRASTRUCTURE ONLY).

Restates the gradient of the reference's tok_emb(idx) (ml/fxlm/model.py:82,118: nn.Embedding,
whose backward torch computes): grad[v] = sum of dy[t] over the positions t with idx[t] == v;
rows no position selects are zero.  Ids outside [0, V) add nothing (torch's lookup rejects
them; the GPU kernel skips them).

embedding_grad_seq sums in increasing t in fp32 and rounds once to bf16, the order the GPU
kernel (fx_embedding_bwd) uses, so the two agree bit for bit; embedding_grad gives the exact
sum in fp64.  Both are pinned in tests/test_oracle.py against torch's own embedding backward.
"""
import numpy as np
import torch


def embedding_grad(idx, dy, V, dtype=torch.float64):
    """(V, D) in `dtype`: the per-id sums of the rows of dy (..., D), ids idx (...)."""
    D = dy.shape[-1]
    ids = idx.detach().to("cpu").reshape(-1)
    rows = dy.detach().to("cpu", dtype).reshape(-1, D)
    keep = (ids >= 0) & (ids < V)
    out = torch.zeros(V, D, dtype=dtype)
    out.index_add_(0, ids[keep], rows[keep])
    return out


def embedding_grad_seq(idx, dy, V):
    """(V, D) bf16: each id's rows of dy summed one by one in increasing position in fp32,
    then rounded to bf16 (round to nearest even)."""
    D = dy.shape[-1]
    ids = idx.detach().to("cpu").reshape(-1).numpy()
    rows = dy.detach().to("cpu", torch.float32).reshape(-1, D).numpy()
    acc = np.zeros((V, D), dtype=np.float32)
    for t in range(ids.shape[0]):
        v = int(ids[t])
        if 0 <= v < V:
            acc[v] += rows[t]          # one fp32 add per element, in position order
    return torch.from_numpy(acc).to(torch.bfloat16)
