"""fx_embedding_bwd (the GPT's token-embedding gradient) against the oracle, through the C ABI.

The kernel sums each id's rows of dy in fp32 in increasing position within 32-slot segments of
the id-sorted positions and adds the segment sums in order, rounding once: exactly
oracle.embedding.embedding_grad_seq, so the comparison is bitwise.  Skewed id distributions
(one id at most positions, Zipf ids, byte-level text) split long runs over many segments."""
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
    (0, 10, 16, 0, None, None),          # no positions: every row zero
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


def _zipf_ids(n, V, seed, a=1.1):
    g = torch.Generator().manual_seed(seed)
    p = 1.0 / torch.arange(1, V + 1, dtype=torch.float64) ** a
    return torch.multinomial(p / p.sum(), n, replacement=True, generator=g)


@pytest.mark.parametrize("kind", ["zipf_50304", "bytes_256", "one_id_16384", "two_ids"])
def test_skewed_ids(kind):
    from fxlm.embedding import embedding_grad
    g = torch.Generator().manual_seed(21)
    if kind == "zipf_50304":
        V, D, idx = 50304, 768, _zipf_ids(16384, 50304, 4)
    elif kind == "bytes_256":
        # byte-level English-like text: the space and a few letters hold most positions
        V, D = 256, 768
        text = (b"the quick brown fox jumps over the lazy dog and then some more words " * 300)[:16384]
        idx = torch.tensor(list(text), dtype=torch.int64)
    elif kind == "one_id_16384":
        V, D, idx = 1000, 64, torch.full((16384,), 17, dtype=torch.int64)
    else:
        V, D = 3, 32
        idx = torch.randint(0, 2, (5000,), generator=g)
    rows = torch.randn(idx.numel(), D, generator=g).bfloat16()
    got = embedding_grad(idx.cuda(), rows.cuda(), V)
    assert torch.equal(got.cpu(), oemb.embedding_grad_seq(idx, rows, V))


@pytest.mark.parametrize("at_one,lead,want", [(31, 0, 0.0), (32, 0, 1.0), (12, 20, 1.0), (11, 20, 0.0)])
def test_segment_cut_matches_the_oracle_rule(at_one, lead, want):
    # 2^24 + 1 rounds to 2^24 in fp32: the sum is 0 or the exact 1 depending on which side of a
    # global 32-slot boundary the 1 falls (the oracle's rule, pinned on the CPU)
    from fxlm.embedding import embedding_grad
    n = 64 if lead == 0 else 40
    dy = torch.zeros(lead + n, 8).bfloat16()
    dy[lead, 0] = 2.0 ** 24
    dy[lead + at_one, 0] = 1.0
    dy[lead + at_one + 1, 0] = -(2.0 ** 24)
    idx = torch.tensor([0] * lead + [1] * n)
    got = embedding_grad(idx.cuda(), dy.cuda(), 2)
    assert float(got[1, 0]) == want
    assert torch.equal(got.cpu(), oemb.embedding_grad_seq(idx, dy, 2))


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
    nbytes = int(lib().fx_embedding_bwd_workspace(5000, 600, 48))
    ref = oemb.embedding_grad_seq(idx, rows, 600)
    for fill in (-1, 0x3F800000, 7):
        work = torch.full(((nbytes + 3) // 4,), fill, dtype=torch.int32, device="cuda")
        grad = torch.full((600, 48), float("nan"), dtype=torch.bfloat16, device="cuda")
        call("fx_embedding_bwd", ptr(ids), 5000, ptr(dy), 48, ptr(grad), 600, 48, ptr(work), stream_of(dy))
        torch.cuda.synchronize()
        assert torch.equal(grad.cpu(), ref)
