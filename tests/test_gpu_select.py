"""GPU parity, read-set top-k (session.py:1429-1438): on identical scores the HIP
selection is bit-exact against the oracle's brute-force order (value descending, ties by
ascending index), returned ascending."""

import pytest
import torch

from maskahead_amd.kernels import topk_ascending
from oracle import selection as OS

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(1, 1), (37, 0), (37, 37), (1000, 99), (4096, 512), (32768, 2048), (65536, 8192),
                                 (50001, 1234)])
def test_topk_bit_exact(gpu, n, k):
    g = torch.Generator().manual_seed(n + k)
    rows = 4
    x = torch.rand((rows, n), generator=g)
    # heavy ties: quantize half of each row to a few levels, plus +/-0 and -inf
    x[:, ::2] = (x[:, ::2] * 8).floor() / 8
    x[:, 1::7] = -0.0
    x[:, 3::11] = float("-inf")
    mask = (torch.rand((rows, n), generator=g) > 0.1).to(torch.uint8)
    got = topk_ascending(x.to(gpu), k, mask.to(gpu))
    want = OS.topk_ascending(x, k, mask)
    assert torch.equal(got.cpu(), want)
    vals = torch.empty((rows, k), device=gpu)
    got2 = topk_ascending(x.to(gpu), k, mask.to(gpu), values=vals)
    assert torch.equal(got2.cpu(), want)
    ref_vals = torch.where(mask.bool(), x, torch.tensor(float("-inf"))).gather(1, want)
    assert torch.equal(vals.cpu(), ref_vals)


def test_topk_batched_shape(gpu):
    g = torch.Generator().manual_seed(9)
    x = torch.rand((2, 3, 5000), generator=g)
    got = topk_ascending(x.to(gpu), 100)
    assert got.shape == (2, 3, 100)
    want = x.topk(100, dim=-1).indices.sort(dim=-1).values
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("n,k,rows", [(131072, 2048, 4), (1_100_003, 70001, 2)])
def test_topk_large_rows(gpu, n, k, rows):
    """Rows past one workgroup's reach: 128 chunks of 1024 (config 4's longest prefix), and
    the 4096-element chunks used above 1M entries."""
    g = torch.Generator().manual_seed(n)
    x = torch.randn((rows, n), generator=g).exp()
    x[:, ::5] = (x[:, ::5] * 4).round() / 4           # ties across chunks
    mask = (torch.rand((rows, n), generator=g) > 0.05).to(torch.uint8)
    got = topk_ascending(x.to(gpu), k, mask.to(gpu))
    assert torch.equal(got.cpu(), OS.topk_ascending(x, k, mask))


def test_topk_all_equal_and_special_values(gpu):
    """Every key in the boundary bin (the whole row equal), ties taken across many
    chunks in index order; NaN above +inf; -inf rows; -0.0 == +0.0."""
    n = 20000
    rows = torch.zeros((6, n))
    rows[1] = 1.5                                      # all equal: candidates = the row
    rows[2] = float("-inf")                            # all dead-equivalent
    rows[3, ::3] = float("nan")
    rows[3, 1::3] = float("inf")
    rows[4, ::2] = -0.0                                # +0.0 / -0.0 mix
    rows[5] = torch.arange(n, dtype=torch.float32) % 7
    for k in (1, 999, 12345, n):
        got = topk_ascending(rows.to(gpu), k)
        assert torch.equal(got.cpu(), OS.topk_ascending(rows, k)), k


def test_topk_workspace_reuse_and_unaligned(gpu):
    """Consecutive calls of different row counts and sizes share one state buffer (each
    call leaves its rows' blocks zero); an unaligned, strided row view takes the scalar
    load path."""
    g = torch.Generator().manual_seed(5)
    base = torch.rand((7, 40001), generator=g)
    for rows, n, k in ((3, 40000, 3000), (7, 777, 50), (1, 40000, 1), (5, 5000, 5000), (7, 40000, 39999),
                       (2, 12345, 600)):
        x = base[:rows, 1:n + 1]
        want = OS.topk_ascending(x.contiguous(), k)
        got = topk_ascending(x.to(gpu), k)                    # contiguous copy, 16-byte loads
        assert torch.equal(got.cpu(), want), (rows, n, k)
        xg = base.to(gpu)[:rows, 1:n + 1]                     # 4-byte offset, row stride 40001
        got = topk_ascending(xg, k)
        assert torch.equal(got.cpu(), want), (rows, n, k, "view")


@pytest.mark.parametrize("n,k", [(32768, 2048), (40000, 3000), (65536, 700)])
def test_topk_ties_spread_over_chunks(gpu, n, k):
    """Rows of at most 64 chunks whose boundary bin holds a few keys per chunk, so every
    workgroup of the emit kernel reads its candidates speculatively: keys equal to the k-th
    value in several chunks (ties taken in index order across chunks), in one chunk only,
    and a row whose one chunk holds more boundary-bin keys than its speculative slots
    (the emit kernel's general path for that row)."""
    g = torch.Generator().manual_seed(n + k)
    rows = 4
    # values over ~20 octaves: a 13-bit bin (16 per octave) holds few keys, so the boundary
    # bin has a few candidates per chunk
    x = (torch.randn((rows, n), generator=g) * 3.0).exp()
    kth = x.sort(dim=-1, descending=True).values[:, k - 1:k]
    pos = torch.arange(n)
    x[0, pos % 4099 == 17] = kth[0, 0]                # the k-th value repeated in every chunk
    x[1, (pos >= 3000) & (pos < 3040)] = kth[1, 0]    # 40 copies inside one chunk
    x[2, (pos >= 5000) & (pos < 5400)] = kth[2, 0] * (1 + 1e-6 * torch.arange(400) / 400)  # one dense chunk
    got = topk_ascending(x.to(gpu), k)
    assert torch.equal(got.cpu(), OS.topk_ascending(x, k))
    mask = (torch.rand((rows, n), generator=g) > 0.02).to(torch.uint8)
    got = topk_ascending(x.to(gpu), k, mask.to(gpu))
    assert torch.equal(got.cpu(), OS.topk_ascending(x, k, mask))
