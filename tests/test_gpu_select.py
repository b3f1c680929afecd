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
