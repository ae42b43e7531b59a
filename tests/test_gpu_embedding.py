"""fx_embedding_bwd (the GPT's token-embedding gradient) against the oracle, through the C ABI.

The kernel sums each id's rows of dy in increasing position in fp32 and rounds once, which is
exactly oracle.embedding.embedding_grad_seq, so the comparison is bitwise."""
import pytest
import torch

from oracle import embedding as oemb

pytestmark = pytest.mark.gpu


def _case(n, V, D, lo=0, seed=0, ld=None, same=None):
    g = torch.Generator().manual_seed(seed)
    idx = torch.full((n,), same, dtype=torch.int64) if same is not None else torch.randint(lo, V, (n,), generator=g)
    rows = torch.randn(n, ld or D, generator=g).bfloat16()
    return idx, rows


@pytest.mark.parametrize("n,V,D,lo,same,ld", [
    (3000, 50, 64, 0, None, None),       # three chunks, the last partial
    (2500, 7, 16, 0, 3, None),           # every position the same id: one sum of 2500 rows
    (1030, 8, 24, -3, None, None),       # ids outside [0, V) add nothing
    (1, 5, 8, 0, None, None),
    (1024, 1, 8, 0, None, None),         # one chunk exactly, one id
    (700, 300, 40, 0, None, 48),         # rows of dy strided (ld 48 > D 40)
    (16384, 50304, 768, 0, None, None),  # the cfg5 step's lookup
])
def test_matches_position_ordered_sum(n, V, D, lo, same, ld):
    from fxlm.embedding import embedding_grad
    idx, rows = _case(n, V, D, lo=lo, same=same, ld=ld)
    dy = rows.cuda()[:, :D]
    got = embedding_grad(idx.cuda(), dy, V)
    ref = oemb.embedding_grad_seq(idx, rows[:, :D], V)
    torch.cuda.synchronize()
    assert got.shape == (V, D) and got.dtype == torch.bfloat16
    assert torch.equal(got.cpu(), ref)


def test_deterministic_and_leading_shape():
    from fxlm.embedding import embedding_grad
    idx, rows = _case(4 * 1024, 97, 32, seed=3)
    i2, d2 = idx.view(4, 1024).cuda(), rows.view(4, 1024, 32).cuda()
    a = embedding_grad(i2, d2, 97)
    b = embedding_grad(i2, d2, 97)
    assert torch.equal(a, b)
    assert torch.equal(a.cpu(), oemb.embedding_grad_seq(idx, rows, 97))


def test_no_positions_gives_zeros():
    from fxlm.embedding import embedding_grad
    got = embedding_grad(torch.empty(0, dtype=torch.int64, device="cuda"),
                         torch.empty(0, 16, dtype=torch.bfloat16, device="cuda"), 33)
    assert got.shape == (33, 16) and int(torch.count_nonzero(got)) == 0


def test_token_embedding_autograd():
    from fxlm.embedding import token_embedding
    g = torch.Generator().manual_seed(5)
    V, D = 64, 32
    w = (torch.randn(V, D, generator=g) * 0.02).bfloat16().cuda().requires_grad_()
    idx = torch.randint(0, V, (3, 50), generator=g)
    dy = torch.randn(3, 50, D, generator=g).bfloat16()
    y = token_embedding(idx.cuda(), w)
    assert torch.equal(y, torch.nn.functional.embedding(idx.cuda(), w.detach()))
    y.backward(dy.cuda())
    assert torch.equal(w.grad.cpu(), oemb.embedding_grad_seq(idx, dy, V))


def test_rejects_bad_inputs():
    from fxlm.embedding import embedding_grad, token_embedding
    with pytest.raises(TypeError):
        embedding_grad(torch.zeros(4, dtype=torch.int32, device="cuda"),
                       torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda"), 10)
    with pytest.raises(ValueError):
        embedding_grad(torch.zeros(4, dtype=torch.int64, device="cuda"),
                       torch.zeros(4, 12, dtype=torch.bfloat16, device="cuda"), 10)
    with pytest.raises(TypeError):
        token_embedding(torch.zeros(4, dtype=torch.int64, device="cuda"),
                        torch.zeros(10, 8, dtype=torch.float32, device="cuda"))


def test_workspace_and_output_contents_do_not_matter():
    # every workspace word the kernels read is written first in the same call, and every
    # gradient row is stored: buffers filled with garbage give the same bits
    from fxgpu.abi import call, lib, ptr, stream_of
    idx, rows = _case(5000, 600, 48, lo=-2, seed=9)
    ids, dy = idx.cuda(), rows.cuda()
    nbytes = int(lib().fx_embedding_bwd_workspace(5000, 600))
    ref = oemb.embedding_grad_seq(idx, rows, 600)
    for fill in (-1, 0x3F800000, 7):
        work = torch.full(((nbytes + 3) // 4,), fill, dtype=torch.int32, device="cuda")
        grad = torch.full((600, 48), float("nan"), dtype=torch.bfloat16, device="cuda")
        call("fx_embedding_bwd", ptr(ids), 5000, ptr(dy), 48, ptr(grad), 600, 48, ptr(work), stream_of(dy))
        torch.cuda.synchronize()
        assert torch.equal(grad.cpu(), ref)
