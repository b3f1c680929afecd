"""GPU parity of PackedKVCache.load_dynamic_cache (the reference's cache.py:568-606, called
by both generators at prefill): a prefill cache object read through each of the three
access forms the reference accepts (tuple indexing, key_cache / value_cache lists,
layers[i].keys / .values) lands in the packed planes bit-exactly as the oracle quantizer
writes it (whole 32-token key groups 4-bit, the rest as the bf16 residual), and a failing
layer aborts the append and leaves the cache empty."""

from types import SimpleNamespace

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from oracle import attention as OA

pytestmark = pytest.mark.gpu

L, B, H, D = 3, 1, 2, 128


class _Tuple:
    """Indexable like a transformers DynamicCache: cache[i] -> (K, V)."""

    def __init__(self, kv):
        self.kv = kv

    def get_seq_length(self):
        return self.kv[0][0].shape[2]

    def __getitem__(self, i):
        return self.kv[i]


class _Lists:
    """key_cache / value_cache lists (indexing raises)."""

    def __init__(self, kv):
        self.key_cache = [k for k, _ in kv]
        self.value_cache = [v for _, v in kv]

    def get_seq_length(self):
        return self.key_cache[0].shape[2]


class _Layers:
    """transformers 5.x: layers[i].keys / .values (indexing raises)."""

    def __init__(self, kv):
        self.layers = [SimpleNamespace(keys=k, values=v) for k, v in kv]

    def get_seq_length(self):
        return self.layers[0].keys.shape[2]


def _prefill(dev, n, seed):
    g = torch.Generator().manual_seed(seed)
    kv = []
    for _ in range(L):
        k = torch.randn(B, H, n + 5, D, generator=g) * torch.exp(0.5 * torch.randn(1, H, 1, D, generator=g))
        v = torch.randn(B, H, n + 5, D, generator=g)
        kv.append((k.to(torch.bfloat16), v.to(torch.bfloat16)))
    # the objects hold 5 tokens more than get_seq_length (a cropped cache): only n are read
    gpu = [(k.to(dev), v.to(dev)) for k, v in kv]
    return kv, gpu


@pytest.mark.parametrize("form", [_Tuple, _Lists, _Layers])
def test_load_dynamic_cache_bit_exact(gpu, form):
    n = 200                                    # 5 whole key groups (160) + a 40-token bf16 residual
    kv, dev_kv = _prefill(gpu, n, seed=5)
    dyn = form(dev_kv)
    dyn.get_seq_length = lambda n=n: n
    c = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=1024,
                      quant=QuantizationConfig(), device=gpu)
    c.load_dynamic_cache(dyn)
    nq = (n - 32) // 32 * 32                   # at least residual_tokens (32) stay bf16
    assert (c.length, c.quantized_length, c.residual_length) == (n, nq, n - nq)
    torch.cuda.synchronize()
    for layer, (k, v) in enumerate(kv):
        kq, ks, kz = OA.quantize_keys(k[:, :, :nq])
        vq, vs, vz = OA.quantize_values(v[:, :, :nq])
        view = c.layer_view(layer)
        assert torch.equal(view.k_q.cpu(), kq) and torch.equal(view.k_scale.cpu(), ks) \
            and torch.equal(view.k_zero.cpu(), kz), f"layer {layer}: keys"
        assert torch.equal(view.v_q.cpu(), vq) and torch.equal(view.v_scale.cpu(), vs) \
            and torch.equal(view.v_zero.cpu(), vz), f"layer {layer}: values"
        assert torch.equal(view.k_residual.cpu(), k[:, :, nq:n]) and torch.equal(view.v_residual.cpu(), v[:, :, nq:n])
    with pytest.raises(RuntimeError, match="requires an empty cache"):
        c.load_dynamic_cache(dyn)


def test_load_dynamic_cache_errors_abort(gpu):
    _, dev_kv = _prefill(gpu, 64, seed=6)
    c = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=100,
                      quant=QuantizationConfig(), device=gpu)
    c.load_dynamic_cache(None)
    assert c.length == 0

    class _Bad(_Tuple):
        def __getitem__(self, i):
            if i == 2:
                raise IndexError(i)
            return self.kv[i]

    with pytest.raises(TypeError, match="cannot read layer 2"):
        c.load_dynamic_cache(_Bad(dev_kv))
    assert c.length == 0 and not c.append_in_progress
    big = _Tuple(dev_kv)
    big.get_seq_length = lambda: 101
    with pytest.raises(RuntimeError, match="exceeds capacity 100"):
        c.load_dynamic_cache(big)
    dyn = _Tuple(dev_kv)
    dyn.get_seq_length = lambda: 64
    c.load_dynamic_cache(dyn)                  # the aborted appends left it usable
    assert (c.length, c.quantized_length, c.residual_length) == (64, 32, 32)
