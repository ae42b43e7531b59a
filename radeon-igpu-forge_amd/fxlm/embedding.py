"""fxlm.embedding: the token embedding with this build's weight gradient.

``token_embedding(idx, weight)`` is ``torch.nn.functional.embedding(idx, weight)`` in the
forward (a row gather of the table); its weight gradient comes from ``fx_embedding_bwd``: a
deterministic counting sort of the ids, sums of each id's rows of dy in increasing position
over segments of 32 sorted slots, and the segments' fp32 sums added in order, rounded once to
bf16 (no wave sums more than 32 rows, so a skewed id distribution costs no long serial walk).
It stands in for torch's nn.Embedding backward behind the reference's ``tok_emb(idx)``
(ml/fxlm/model.py:82,118), which sorts the ids and sizes its segment kernels from counts it
reads back from the device, so its launches depend on the ids; these do not.
"""
import torch
import torch.nn.functional as Fn

from fxgpu.abi import call, lib, ptr, stream_of


class _TokenEmbedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, idx, weight):
        ctx.save_for_backward(idx)
        ctx.V = weight.shape[0]
        return Fn.embedding(idx, weight)

    @staticmethod
    def backward(ctx, dy):
        if not ctx.needs_input_grad[1]:
            return None, None
        (idx,) = ctx.saved_tensors
        return None, embedding_grad(idx, dy, ctx.V)


def embedding_grad(idx, dy, V):
    """(V, D) bf16 weight gradient of an embedding lookup: row v = the sum of the rows of dy
    (..., D) whose id in idx (same leading shape, int64) is v, in fp32 (increasing position
    within each 32-slot segment of the id-sorted positions, the segments in order), rounded
    once; zero rows for ids no position has; ids outside [0, V) add nothing."""
    if idx.dtype != torch.int64:
        raise TypeError(f"idx must be int64, got {idx.dtype}")
    if not (idx.is_cuda and dy.is_cuda):
        raise TypeError("idx and dy must be cuda tensors")
    D = dy.shape[-1]
    if D % 8:
        raise ValueError(f"embedding width {D} must be a multiple of 8")
    dy2 = dy.reshape(-1, D)
    if dy2.dtype != torch.bfloat16:
        dy2 = dy2.to(torch.bfloat16)
    if dy2.stride(1) != 1 or dy2.stride(0) % 8 or dy2.data_ptr() % 16:
        dy2 = dy2.contiguous()
    ids = idx.reshape(-1)
    if not ids.is_contiguous():
        ids = ids.contiguous()
    n = ids.numel()
    if n != dy2.shape[0]:
        raise ValueError(f"{n} ids for {dy2.shape[0]} rows of dy")
    grad = torch.empty(V, D, device=dy.device, dtype=torch.bfloat16)
    nbytes = int(lib().fx_embedding_bwd_workspace(n, V, D))
    work = torch.empty(max(1, (nbytes + 3) // 4), device=dy.device, dtype=torch.float32)
    call("fx_embedding_bwd", ptr(ids), n, ptr(dy2), dy2.stride(0), ptr(grad), V, D, ptr(work), stream_of(dy2))
    return grad


def token_embedding(idx, weight):
    """Fn.embedding(idx, weight) for a bf16 (V, D) cuda table with D a multiple of 8, whose
    weight gradient is embedding_grad's."""
    if weight.dtype != torch.bfloat16 or not weight.is_cuda or weight.dim() != 2:
        raise TypeError("weight must be a 2-D bfloat16 cuda tensor")
    if weight.shape[1] % 8:
        raise ValueError(f"embedding width {weight.shape[1]} must be a multiple of 8")
    return _TokenEmbedding.apply(idx, weight)
