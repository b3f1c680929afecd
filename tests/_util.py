"""Shared helpers of the GPU parity tests: seeded inputs, packed prefixes built on the
CPU with the oracle's quantizer, and copies of them on the GPU."""

from __future__ import annotations

import torch

from maskahead_amd.kernels.splitk import Prefix
from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA


def packed_cpu(key: torch.Tensor, value: torch.Tensor, *, pad_groups: int = 0, pad_tokens: int = 0):
    """Quantize [B,H,n,D] K/V with the oracle's rule into capacity-padded storage (so the
    kernels see non-dense strides) and return (dict of padded tensors, nq)."""
    kq, ks, kz = OA.quantize_keys(key)
    vq, vs, vz = OA.quantize_values(value)
    b, h, n, d = key.shape

    def pad(x, axis, extra):
        if not extra:
            return x
        shape = list(x.shape)
        shape[axis] += extra
        out = torch.zeros(shape, dtype=x.dtype)
        out.narrow(axis, 0, x.shape[axis]).copy_(x)
        return out

    store = dict(kq=pad(kq, 2, pad_groups), ks=pad(ks, 2, pad_groups), kz=pad(kz, 2, pad_groups),
                 vq=pad(vq, 2, pad_tokens), vs=pad(vs, 2, pad_tokens), vz=pad(vz, 2, pad_tokens))
    return store, n


def gpu_prefix(store: dict, nq: int, dev, *, kf=None, vf=None, mask=None) -> Prefix:
    """Views of the first nq tokens of GPU copies of `store` (+ optional 16-bit tail)."""
    g = {k: v.to(dev) for k, v in store.items()}
    gq = nq // 32
    p = Prefix(kq=g["kq"][:, :, :gq], ks=g["ks"][:, :, :gq], kz=g["kz"][:, :, :gq],
               vq=g["vq"][:, :, :nq], vs=g["vs"][:, :, :nq], vz=g["vz"][:, :, :nq],
               kf=None if kf is None else kf.to(dev), vf=None if vf is None else vf.to(dev),
               nq=nq, nf=0 if kf is None else kf.shape[2], kb=4, vb=4, kg=32, vg=32,
               mask=None if mask is None else mask.to(dev))
    return p


def dequant_cpu(store: dict, nq: int):
    """Oracle dequant of the first nq tokens -> f32 K, V [B,H,nq,D]."""
    gq = nq // 32
    k = OA.dequantize_keys(store["kq"][:, :, :gq], store["ks"][:, :, :gq], store["kz"][:, :, :gq])
    v = OA.dequantize_values(store["vq"][:, :, :nq], store["vs"][:, :, :nq], store["vz"][:, :, :nq])
    return k, v


def rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.double().cpu(), want.double().cpu()
    return float(((got - want).abs() / want.abs().clamp_min(1e-30)).max())


def assert_attention_close(got: torch.Tensor, want: torch.Tensor, atol=2e-2, rtol=1e-2):
    """The north star's attention tolerance: 2e-2 absolute / 1e-2 relative (bf16)."""
    got, want = got.double().cpu(), want.double().cpu()
    bad = (got - want).abs() > atol + rtol * want.abs()
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance, max abs diff {(got - want).abs().max():.3e}"


__all__ = ["layer_inputs", "packed_cpu", "gpu_prefix", "dequant_cpu", "rel_err", "assert_attention_close"]
