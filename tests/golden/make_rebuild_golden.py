"""Write the golden vectors of the packed eviction rebuild.

Run in the build container (where /root/reference exists):

    python tests/golden/make_rebuild_golden.py

It imports the reference package (brain-lab-research/MaskAhead, src/maskahead) and
runs, on small seeded CPU caches, the two steps whose slot layout no closed form fixes:

  * the lazy / full plan of the session's eviction (runtime/session.py:270-361,
    ``BitSieveSession._evict_to``), called on a stand-in object that carries only the
    attributes that method reads (cache, eviction state and settings, next position);
  * ``PackedKVCache.rebuild`` (cache.py:236-335), which that plan drives: kept key
    groups copied as they are, sparse groups and decided bf16 entries quantized into
    fresh groups, undecided entries kept in bf16, the slot remap.

Only inputs and outputs are written (rebuild_vectors.npz): the cache tensors before
and after (raw bits), the eviction state's positions and slots, the keep sets and the
settings.  Nothing of the reference is copied.  tests/test_oracle_golden.py checks the
CPU oracle (oracle/rebuild.py) against these vectors; the GPU tests check the HIP
kernels against the oracle and against the vectors.
"""

from __future__ import annotations

import sys
import types
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference/src")
OUT = Path(__file__).resolve().parent / "rebuild_vectors.npz"

L, B, H, D = 2, 1, 2, 64


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _snapshot(cache) -> dict[str, np.ndarray]:
    """The written part of every storage tensor, plus the lengths."""
    gk = cache.quant.key_token_group
    ng, ql, rl = cache.quantized_length // gk, cache.quantized_length, cache.residual_length
    return {
        "kq": cache.k_q[:, :, :, :ng].numpy().copy(),
        "ks": _bits16(cache.k_scale[:, :, :, :ng]), "kz": _bits16(cache.k_zero[:, :, :, :ng]),
        "vq": cache.v_q[:, :, :, :ql].numpy().copy(),
        "vs": _bits16(cache.v_scale[:, :, :, :ql]), "vz": _bits16(cache.v_zero[:, :, :, :ql]),
        "kr": _bits16(cache.k_residual[:, :, :, :rl]), "vr": _bits16(cache.v_residual[:, :, :, :rl]),
        "lens": np.array([cache.length, cache.quantized_length, cache.residual_length, cache.dropped], np.int64),
    }


def _append(cache, g, n):
    k = (torch.randn((L, B, H, n, D), generator=g) *
         torch.empty((L, B, H, 1, D)).log_normal_(0, 0.5, generator=g)).to(torch.bfloat16)
    v = torch.randn((L, B, H, n, D), generator=g).to(torch.bfloat16)
    cache.begin_append(n)
    for layer in range(L):
        cache.stage_layer(layer, k[layer], v[layer])
    cache.commit_append()


def _keep(st, g, capacity, window, dense_groups):
    """Survivors [L, B, H, C] in position order: the window, then the best of a score that
    favours a few key groups per lane (dense_groups[lane], lanes in (layer, batch, head)
    order), so some groups keep most of their entries and the lanes' lists differ in
    length (the shorter ones padded)."""
    live = st.live
    pos = st.pos[..., :live].to(torch.int64)
    score = torch.rand((L, B, H, live), generator=g)
    grp_of = st.phys[..., :live] // 32
    for lane, groups in enumerate(dense_groups):
        li, bi, hi = lane // (B * H), (lane // H) % B, lane % H
        for grp in groups:
            score[li, bi, hi] += 2.0 * (grp_of[li, bi, hi] == grp)
    w = min(window, capacity)
    newest = pos >= pos.topk(w, dim=-1).values.amin(-1, keepdim=True) if w else torch.zeros_like(pos, dtype=bool)
    score = torch.where(newest, torch.full_like(score, 1e9), score)
    keep = score.topk(capacity, dim=-1).indices
    return keep.gather(-1, pos.gather(-1, keep).argsort(dim=-1))


def main() -> None:
    sys.path.insert(0, str(REF))
    from maskahead.cache import PackedKVCache                    # noqa: E402
    from maskahead.config import QuantizationConfig              # noqa: E402
    from maskahead.eviction import EvictionConfig, EvictionState  # noqa: E402
    from maskahead.runtime.session import BitSieveSession         # noqa: E402

    g = torch.Generator("cpu").manual_seed(1234)
    out: dict[str, np.ndarray] = {}

    def run(tag, cache, st, next_pos, keep, ecfg):
        before = _snapshot(cache)
        pos0, phys0, live0 = st.pos[..., :st.live].clone(), st.phys[..., :st.live].clone(), st.live
        fake = types.SimpleNamespace(_eviction=st, config=types.SimpleNamespace(eviction=ecfg), _attn_log=None,
                                     _phys_compact=True, cache=cache, _next_position=next_pos,
                                     trace=types.SimpleNamespace(add_counter=lambda *a, **k: None))
        BitSieveSession._evict_to(fake, keep)
        after = _snapshot(cache)
        for k, v in before.items():
            out[f"{tag}_in_{k}"] = v
        for k, v in after.items():
            out[f"{tag}_out_{k}"] = v
        out[f"{tag}_pos"] = pos0.numpy().astype(np.int64)
        out[f"{tag}_phys"] = phys0.numpy().astype(np.int64)
        out[f"{tag}_keep"] = keep.numpy().astype(np.int64)
        out[f"{tag}_out_phys"] = st.phys[..., :st.live].numpy().astype(np.int64)
        out[f"{tag}_cfg"] = np.array([live0, next_pos, int(cache.stage), ecfg.recent_window,
                                      {"lazy": 0, "full": 1}[ecfg.compaction],
                                      int(round(ecfg.repack_below * 1000))], np.int64)
        print(tag, "live", live0, "->", st.live, "lens", before["lens"], "->", after["lens"])

    def new_cache(residual_tokens):
        q = QuantizationConfig(k_bits=4, v_bits=4, key_token_group=32, value_channel_group=32,
                               residual_tokens=residual_tokens)
        return PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=4096, quant=q,
                             device="cpu", compute_dtype=torch.bfloat16, backend="torch")

    def new_state():
        return EvictionState(num_layers=L, batch_size=B, num_kv_heads=H, capacity=64, device="cpu")

    # lazy: 7 quantized groups + 32 residual; groups with >= 16 survivors stay as they are;
    # then a second eviction on the rebuilt cache after one more block
    cache, st = new_cache(32), new_state()
    _append(cache, g, 224)
    _append(cache, g, 32)
    st.append(range(256))
    ecfg = EvictionConfig(policy="recent", recent_window=16, capacity_floor=16, compaction="lazy", repack_below=0.5)
    run("lazy", cache, st, 256, _keep(st, g, 96, 16, ((1, 4), (1,), (), (4, 5, 6))), ecfg)
    n0 = cache.get_seq_length()
    _append(cache, g, 32)
    st.append(range(n0, n0 + 32), phys=torch.arange(cache.length - 32, cache.length))
    run("lazy2", cache, st, n0 + 32, _keep(st, g, 80, 16, ((0, 2), (2,), (0, 1, 2), ())), ecfg)

    # full: every survivor outside the window re-quantized
    cache, st = new_cache(32), new_state()
    _append(cache, g, 160)
    _append(cache, g, 32)
    st.append(range(192))
    run("full", cache, st, 192, _keep(st, g, 70, 8, ((2,), (), (1,), (3, 4))),
        EvictionConfig(policy="recent", recent_window=8, capacity_floor=8, compaction="full"))

    # staged bf16 entries and a stored-but-unadmitted tail (appended to the bf16 stage)
    cache, st = new_cache(32), new_state()
    _append(cache, g, 128)
    cache.stage = True
    _append(cache, g, 32)
    _append(cache, g, 32)
    _append(cache, g, 32)
    st.append(range(cache.length - 32))
    run("stage", cache, st, cache.length - 32, _keep(st, g, 60, 16, ((1,), (0, 3), (), (2,))),
        EvictionConfig(policy="recent", recent_window=16, capacity_floor=16, compaction="lazy", repack_below=0.75))

    # no residual, a tail of two whole unadmitted groups placed after the rebuilt ones
    cache, st = new_cache(0), new_state()
    _append(cache, g, 128)
    _append(cache, g, 64)
    st.append(range(128))
    run("tail", cache, st, 128, _keep(st, g, 50, 0, ((0, 3), (1,), (), (0, 1, 3))),
        EvictionConfig(policy="recent", recent_window=0, capacity_floor=8, compaction="lazy", repack_below=0.5))

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
