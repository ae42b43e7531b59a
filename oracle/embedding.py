"""Oracle: token-embedding weight gradient (TEST INFRASTRUCTURE ONLY).

Restates the gradient of the reference's tok_emb(idx) (ml/fxlm/model.py:82,118: nn.Embedding,
whose backward torch computes): grad[v] = sum of dy[t] over the positions t with idx[t] == v;
rows no position selects are zero.  Ids outside [0, V) add nothing (torch's lookup rejects
them; the GPU kernel skips them).

embedding_grad_seq restates the summation order of the GPU kernel (fx_embedding_bwd), so the
two agree bit for bit: the valid positions sorted stably by id form slots 0, 1, ...; the slots
are cut into segments of SEG = 32 (at global slot multiples of 32, not per id); an id's rows
are summed in fp32 in increasing position within each segment, its segment sums are added in
segment order, and the total is rounded once to bf16.  embedding_grad gives the exact sum in
fp64.  Both are pinned in tests/test_oracle.py: against torch's own embedding backward, and the
segment rule by fp32 sums that come out differently under any other cut or order.
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


SEG = 32  # slots per segment (kEmbSeg in embedding.hip)


def embedding_grad_seq(idx, dy, V, seg=SEG):
    """(V, D) bf16: per id, fp32 sums of its rows in increasing position over each segment of
    `seg` id-sorted slots, the segment sums added in segment order, rounded once to bf16 (round
    to nearest even)."""
    D = dy.shape[-1]
    ids = idx.detach().to("cpu").reshape(-1).numpy()
    rows = dy.detach().to("cpu", torch.float32).reshape(-1, D).numpy()
    valid = np.nonzero((ids >= 0) & (ids < V))[0]
    order = valid[np.argsort(ids[valid], kind="stable")]  # slot s -> position, (id, t) order
    out = np.zeros((V, D), dtype=np.float32)
    s = 0
    while s < order.shape[0]:
        v = int(ids[order[s]])
        e = s
        while e < order.shape[0] and int(ids[order[e]]) == v:
            e += 1
        total = None
        a = s
        while a < e:                    # pieces of the run [s, e) cut at multiples of seg
            b = min(e, (a // seg + 1) * seg)
            piece = np.zeros(D, dtype=np.float32)
            for k in range(a, b):
                piece += rows[order[k]]  # one fp32 add per element, in position order
            total = piece if total is None else total + piece
            a = b
        out[v] = total
        s = e
    return torch.from_numpy(out).to(torch.bfloat16)
