"""GPU parity, byte/integer work: dequant, gather and the 4-bit quantizers are
bit-exact against the CPU oracle (and, for the quantizers, against the golden vectors
the reference itself wrote)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from maskahead_amd.kernels import dequantize_prefix, gather_packed_kv, quantize_key_groups_into, quantize_values_into
from maskahead_amd.kernels.splitk import Prefix
from oracle import attention as OA
from oracle import codec

from _util import dequant_cpu, gpu_prefix, layer_inputs, packed_cpu

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden" / "golden_vectors.npz"


class _View:
    """Minimal LayerCacheView stand-in (cache.py:37-60 fields used by gather)."""

    def __init__(self, p: Prefix, d: int):
        self.k_bits = self.v_bits = 4
        self.length, self.quantized_length, self.residual_length = p.n, p.nq, p.nf
        self.key_token_group = self.value_channel_group = 32
        self.k_q, self.k_scale, self.k_zero = p.kq, p.ks, p.kz
        self.v_q, self.v_scale, self.v_zero = p.vq, p.vs, p.vz
        self.k_fp = self.v_fp = None
        self.k_residual, self.v_residual = p.kf, p.vf
        self.head_dim = d
        self.key_mode = "channel"


def _setup(dev, n=320, tail=40, d=128, seed=21):
    _, k, v, _, _ = layer_inputs(hq=4, hkv=2, d=d, n=n + tail, t=4, seed=seed, dtype=torch.bfloat16)
    store, nq = packed_cpu(k[:, :, :n], v[:, :, :n], pad_groups=3, pad_tokens=70)
    kt, vt = k[:, :, n:], v[:, :, n:]
    p = gpu_prefix(store, nq, dev, kf=kt, vf=vt)
    kd, vd = dequant_cpu(store, nq)
    k_all = torch.cat([kd.to(torch.bfloat16), kt], 2)
    v_all = torch.cat([vd.to(torch.bfloat16), vt], 2)
    return p, k_all, v_all, kd, vd


@pytest.mark.parametrize("d", [128, 64])
def test_dequant_prefix_bit_exact(gpu, d):
    p, k_all, v_all, kd, vd = _setup(gpu, d=d)
    ko, vo = dequantize_prefix(p, 1, 2, d, dtype=torch.bfloat16)
    assert torch.equal(ko.cpu(), k_all) and torch.equal(vo.cpu(), v_all)
    ko32, vo32 = dequantize_prefix(p, 1, 2, d, dtype=torch.float32)
    assert torch.equal(ko32[:, :, :320].cpu(), kd) and torch.equal(vo32[:, :, :320].cpu(), vd)
    # the C oracle agrees on the bf16 bits too
    _, k16 = codec.dequant_keys4(p.kq.cpu().numpy(), p.ks.cpu().numpy(), p.kz.cpu().numpy())
    assert np.array_equal(ko[:, :, :320].cpu().view(torch.int16).numpy().view(np.uint16), k16)


def test_gather_bit_exact(gpu):
    p, k_all, v_all, _, _ = _setup(gpu)
    g = torch.Generator().manual_seed(5)
    idx = torch.stack([torch.randperm(360, generator=g)[:97].sort().values for _ in range(2)]).unsqueeze(0)
    idx[0, 1, -1] = 400                   # out of range: zeros, never a fault
    out_k = torch.full((1, 2, 100, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    ok, ov = gather_packed_kv(_View(p, 128), idx.to(gpu), out_key=out_k[:, :, :97], out_value=None)
    ref_idx = idx.clamp_max(359).unsqueeze(-1).expand(-1, -1, -1, 128)
    want_k = torch.gather(k_all, 2, ref_idx)
    want_v = torch.gather(v_all, 2, ref_idx)
    want_k[0, 1, -1] = 0
    want_v[0, 1, -1] = 0
    assert torch.equal(ok.cpu(), want_k) and torch.equal(ov.cpu(), want_v)
    assert torch.all(out_k[:, :, 97:].cpu() == 7.0)        # writes stay inside the view


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quantizers_bit_exact(gpu, dtype):
    x = (layer_inputs(hq=4, hkv=2, d=128, n=256, t=4, seed=31)[1]).to(dtype)
    kq, ks, kz = OA.quantize_keys(x)
    vq, vs, vz = OA.quantize_values(x)
    xg = x.to(gpu)
    gkq = torch.empty((1, 2, 10, 128, 16), dtype=torch.uint8, device=gpu)[:, :, 1:9]   # strided view
    gks = torch.empty((1, 2, 8, 128), dtype=torch.float16, device=gpu)
    gkz = torch.empty_like(gks)
    quantize_key_groups_into(xg, gkq, gks, gkz, bits=4, token_group=32)
    gvq = torch.empty((1, 2, 256, 4, 16), dtype=torch.uint8, device=gpu)
    gvs = torch.empty((1, 2, 256, 4), dtype=torch.float16, device=gpu)
    gvz = torch.empty_like(gvs)
    quantize_values_into(xg, gvq, gvs, gvz, bits=4, channel_group=32)
    assert torch.equal(gkq.cpu(), kq) and torch.equal(gks.cpu(), ks) and torch.equal(gkz.cpu(), kz)
    assert torch.equal(gvq.cpu(), vq) and torch.equal(gvs.cpu(), vs) and torch.equal(gvz.cpu(), vz)


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_quantizers_match_reference_golden(gpu, tag):
    z = np.load(GOLD)
    x = z[f"q_{tag}_x"]
    xt = (torch.from_numpy(x.view(np.int16)).view(torch.bfloat16) if tag == "bf16" else torch.from_numpy(x)).to(gpu)
    kq = torch.empty((1, 2, 2, 128, 16), dtype=torch.uint8, device=gpu)
    ks = torch.empty((1, 2, 2, 128), dtype=torch.float16, device=gpu)
    kz = torch.empty_like(ks)
    quantize_key_groups_into(xt, kq, ks, kz, bits=4, token_group=32)
    vq = torch.empty((1, 2, 64, 4, 16), dtype=torch.uint8, device=gpu)
    vs = torch.empty((1, 2, 64, 4), dtype=torch.float16, device=gpu)
    vz = torch.empty_like(vs)
    quantize_values_into(xt, vq, vs, vz, bits=4, channel_group=32)
    u16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(kq.cpu().numpy(), z[f"q_{tag}_kq"])
    assert np.array_equal(u16(ks), z[f"q_{tag}_ks"]) and np.array_equal(u16(kz), z[f"q_{tag}_kz"])
    assert np.array_equal(vq.cpu().numpy(), z[f"q_{tag}_vq"])
    assert np.array_equal(u16(vs), z[f"q_{tag}_vs"]) and np.array_equal(u16(vz), z[f"q_{tag}_vz"])
