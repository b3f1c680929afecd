"""Seeded synthetic inputs for the benchmark configurations of the read/keep path.

The distribution follows the benchmark definition: Q, K, V ~ N(0, 1) drawn from
torch.Generator("cpu").manual_seed(seed) (the reference's default seed 1234,
config.py:263), keys scaled per (KV head, channel) by LogNormal(0, 0.5), and the first
`sinks` prefix keys multiplied by 8 (attention-sink tokens).  Tensors are created on the
CPU (so every host draws the same numbers) and moved by the caller.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class LayerShape:
    name: str
    b: int
    hq: int
    hkv: int
    d: int
    n: int            # prefix entries
    t: int            # block (query) positions
    read_k: int       # read budget per KV head
    keep_k: int       # keep budget per KV head (0: no eviction step)
    packed: bool      # int4 k4v4 cache


# BASELINE configs 0-3 (config 4 is a ragged batch of config-2 layers)
CONFIGS = {
    "c0": LayerShape("c0_fp32_n4096", 1, 28, 4, 128, 4096, 32, 512, 1024, False),
    "c1": LayerShape("c1_bf16_n32768", 1, 28, 4, 128, 32768, 32, 2048, 0, False),
    "c2": LayerShape("c2_k4v4_n32768", 1, 28, 4, 128, 32768, 32, 2048, 0, True),
    "c3": LayerShape("c3_bf16_n65536_keep", 1, 32, 8, 128, 65536, 96, 0, 8192, False),
}


def layer_inputs(shape: LayerShape | None = None, *, b=1, hq=28, hkv=4, d=128, n=4096, t=32, seed=1234,
                 sinks=4, sink_scale=8.0, dtype=torch.float32):
    """(query [B,Hq,T,D], key, value [B,Hkv,n,D], current_key, current_value [B,Hkv,T,D])."""
    if shape is not None:
        b, hq, hkv, d, n, t = shape.b, shape.hq, shape.hkv, shape.d, shape.n, shape.t
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn((b, hq, t, d), generator=g)
    k = torch.randn((b, hkv, n, d), generator=g)
    v = torch.randn((b, hkv, n, d), generator=g)
    kc = torch.randn((b, hkv, t, d), generator=g)
    vc = torch.randn((b, hkv, t, d), generator=g)
    chan = torch.empty((1, hkv, 1, d)).log_normal_(0.0, 0.5, generator=g)
    k = k * chan
    kc = kc * chan
    k[:, :, :sinks] *= sink_scale
    return tuple(x.to(dtype) for x in (q, k, v, kc, vc))


def packed_layout(b: int, hkv: int, n: int, d: int, *, device, kg: int = 32, vg: int = 32):
    """Empty packed-int4 cache tensors in the reference's layout (cache.py:154-189):
    kq [B,H,n/KG,D,KG/2] u8, ks/kz [B,H,n/KG,D] f16, vq [B,H,n,D/VG,VG/2] u8,
    vs/vz [B,H,n,D/VG] f16."""
    gn = n // kg
    return dict(
        kq=torch.empty((b, hkv, gn, d, kg // 2), dtype=torch.uint8, device=device),
        ks=torch.empty((b, hkv, gn, d), dtype=torch.float16, device=device),
        kz=torch.empty((b, hkv, gn, d), dtype=torch.float16, device=device),
        vq=torch.empty((b, hkv, n, d // vg, vg // 2), dtype=torch.uint8, device=device),
        vs=torch.empty((b, hkv, n, d // vg), dtype=torch.float16, device=device),
        vz=torch.empty((b, hkv, n, d // vg), dtype=torch.float16, device=device),
    )
