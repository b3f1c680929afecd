"""The oracle's byte / integer half (oracle/codec.c) pinned by closed forms and by
independent library routines (numpy float16, torch bfloat16)."""

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import codec


def test_pack_closed_form():
    # reference.py:35-45: element 2i in bits 0-3, element 2i+1 in bits 4-7
    codes = np.array([[1, 2, 15, 0, 7, 9]], dtype=np.uint8)
    assert codec.pack4(codes).tolist() == [[0x21, 0x0F, 0x97]]
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, size=(3, 5, 64), dtype=np.uint8)
    assert np.array_equal(codec.unpack4(codec.pack4(c)), c)


def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = codec.f16_bits_to_f32(bits)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4000),
        # exact ties: 1 + 2^-8 (-> 1, even), 1 + 3*2^-8 (-> 1 + 2^-6, even)
        np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), np.inf, -np.inf, 0.0, -0.0,
                  3.0e38, 1e-40], dtype=np.float32),
    ])
    got = codec.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _rand_packed(seed, b=1, h=2, n=96, d=128):
    rng = np.random.default_rng(seed)
    kq = rng.integers(0, 256, size=(b, h, n // 32, d, 16), dtype=np.uint8)
    ks = (rng.random((b, h, n // 32, d)) * 0.5 + 1e-3).astype(np.float16)
    kz = (rng.standard_normal((b, h, n // 32, d)) * 3).astype(np.float16)
    vq = rng.integers(0, 256, size=(b, h, n, d // 32, 16), dtype=np.uint8)
    vs = (rng.random((b, h, n, d // 32)) * 0.5 + 1e-3).astype(np.float16)
    vz = (rng.standard_normal((b, h, n, d // 32)) * 3).astype(np.float16)
    return kq, ks, kz, vq, vs, vz


def test_dequant_closed_form_and_two_implementations():
    kq, ks, kz, vq, vs, vz = _rand_packed(2)
    k32, k16 = codec.dequant_keys4(kq, ks, kz)
    v32, v16 = codec.dequant_values4(vq, vs, vz)
    # closed form: code*scale is exact, so f32(code*scale + zero) is the correctly
    # rounded f64 value -- one rounding, fused or not (reference.py:168-179, 259-268)
    codes_k = np.stack([kq & 15, kq >> 4], -1).reshape(*kq.shape[:-1], 32)       # [b,h,g,d,32]
    exact_k = codes_k.astype(np.float64) * ks[..., None].astype(np.float64) + kz[..., None].astype(np.float64)
    exact_k = np.swapaxes(exact_k, -1, -2).reshape(k32.shape).astype(np.float32)
    assert np.array_equal(k32.view(np.uint32), exact_k.view(np.uint32))
    codes_v = np.stack([vq & 15, vq >> 4], -1).reshape(*vq.shape[:-1], 32)
    exact_v = (codes_v.astype(np.float64) * vs[..., None] + vz[..., None].astype(np.float64))
    exact_v = exact_v.reshape(v32.shape).astype(np.float32)
    assert np.array_equal(v32.view(np.uint32), exact_v.view(np.uint32))
    # the torch restatement agrees bit for bit, and bf16 rounding is torch's RNE
    tk = OA.dequantize_keys(torch.from_numpy(kq), torch.from_numpy(ks), torch.from_numpy(kz))
    tv = OA.dequantize_values(torch.from_numpy(vq), torch.from_numpy(vs), torch.from_numpy(vz))
    assert np.array_equal(tk.numpy().view(np.uint32), k32.view(np.uint32))
    assert np.array_equal(tv.numpy().view(np.uint32), v32.view(np.uint32))
    assert np.array_equal(tk.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16), k16)
    assert np.array_equal(tv.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16), v16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantizer_invariants(dtype):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((1, 2, 64, 128), generator=g) * 2).to(dtype)
    kq, ks, kz = OA.quantize_keys(x)
    vq, vs, vz = OA.quantize_values(x)
    k = OA.dequantize_keys(kq, ks, kz)
    v = OA.dequantize_values(vq, vs, vz)
    xf = x.float()
    # reconstruction error within half a step, plus the f16 rounding of scale/zero and,
    # for bf16 input, the bf16 rounding of (x - min) / scale (up to 15 * 2^-8 of a step)
    half = 0.5 if dtype == torch.float32 else 0.5 + 16 * 2 ** -8
    kstep = ks.float().repeat_interleave(32, dim=2)
    assert ((k - xf).abs() <= half * kstep * 1.01 + 1e-2 * xf.abs().clamp_min(1)).all()
    vstep = vs.float().repeat_interleave(32, dim=-1)
    assert ((v - xf).abs() <= half * vstep * 1.01 + 1e-2 * xf.abs().clamp_min(1)).all()
    # zero point is the group minimum (stored in f16)
    grp_min = x.reshape(1, 2, 2, 32, 128).amin(3)
    assert torch.equal(kz, grp_min.to(torch.float16))
