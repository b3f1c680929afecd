"""CPU oracle of the packed eviction rebuild -- TEST INFRASTRUCTURE ONLY.

Restates, with torch CPU ops, what the reference does when an eviction brings a packed
(4-bit) cache in line with the surviving entries:

  * ``plan`` -- the lazy / full plan of runtime/session.py:288-345 (``_evict_to``):
    which old key groups are copied as they are, which old slots are quantized into
    fresh groups, which stay in bf16, and the groups of a stored-but-unadmitted tail;
  * ``rebuild`` -- ``PackedKVCache.rebuild`` (cache.py:236-335): the new storage
    [kept groups | encoded | tail groups] + the bf16 stage, and the slot remap;
  * ``evict`` -- both, after the eviction state's compaction (eviction.py:411-418).

Storage is a dict of CPU tensors over all layers, [L, B, H, ...]:
kq u8 [.., G, D, 16], ks / kz f16 [.., G, D], vq u8 [.., N, D/32, 16], vs / vz f16
[.., N, D/32], kr / vr bf16 [.., R, D] (the residual), with lengths (length,
quantized_length, residual_length, dropped).

Pinned by tests/golden/rebuild_vectors.npz, written by the reference's own
``_evict_to`` / ``rebuild`` on seeded caches (tests/test_oracle_golden.py); the
dequantizer and quantizer it calls are pinned on their own (oracle/attention.py).
"""

from __future__ import annotations

import math

import torch

from .attention import dequantize_keys, dequantize_values, quantize_keys, quantize_values

GK = 32
BIG = 1 << 62


def _dequantize_all(store: dict, lens: tuple) -> tuple[torch.Tensor, torch.Tensor]:
    """Every stored entry of every layer as bf16 [L, B, H, length, D]: the quantized
    prefix dequantized (reference.py:168-179, 259-268), then the residual
    (cache.py:680-741)."""
    length, ql, rl = lens[0], lens[1], lens[2]
    L, B, H = store["kq"].shape[:3]
    parts_k, parts_v = [], []
    if ql:
        ng = ql // GK
        k = dequantize_keys(store["kq"][:, :, :, :ng].reshape(L * B, H, ng, *store["kq"].shape[4:]),
                            store["ks"][:, :, :, :ng].reshape(L * B, H, ng, -1),
                            store["kz"][:, :, :, :ng].reshape(L * B, H, ng, -1))
        v = dequantize_values(store["vq"][:, :, :, :ql].reshape(L * B, H, ql, *store["vq"].shape[4:]),
                              store["vs"][:, :, :, :ql].reshape(L * B, H, ql, -1),
                              store["vz"][:, :, :, :ql].reshape(L * B, H, ql, -1))
        parts_k.append(k.to(torch.bfloat16).reshape(L, B, H, ql, -1))
        parts_v.append(v.to(torch.bfloat16).reshape(L, B, H, ql, -1))
    if rl:
        parts_k.append(store["kr"][:, :, :, :rl])
        parts_v.append(store["vr"][:, :, :, :rl])
    assert sum(p.shape[3] for p in parts_k) == length
    return torch.cat(parts_k, 3), torch.cat(parts_v, 3)


def _gather_tokens(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x [L, B, H, n, *row], idx [L, B, H, m] (-1 = dead: zero rows) -> [L, B, H, m, *row]."""
    safe = idx.clamp_min(0)
    e = safe.view(*safe.shape, *([1] * (x.dim() - 4))).expand(*safe.shape, *x.shape[4:])
    out = x.gather(3, e)
    dead = (idx < 0).view(*idx.shape, *([1] * (x.dim() - 4)))
    return out.masked_fill(dead, 0)


def rebuild(store: dict, lens: tuple, groups_before: torch.Tensor, encode: torch.Tensor,
            groups_after: torch.Tensor, stage: torch.Tensor):
    """cache.py:236-335.  Index tensors [L, B, H, n] int64, -1 = padding.  Returns
    (new store, new lens, remap [L, B, H, old length]: new slot of every old slot, -1 if
    dropped).  A padding key group holds a copy of old group 0 (the reference gathers
    clamped ids); padding encoded / staged entries are zeros."""
    length, ql, rl, dropped = lens
    L, B, H = store["kq"].shape[:3]
    g1, m, g3, st = groups_before.shape[-1], encode.shape[-1], groups_after.shape[-1], stage.shape[-1]
    g2 = -(-m // GK)
    nql = (g1 + g2 + g3) * GK
    new_len = nql + st
    ar = torch.arange(GK)
    remap = torch.full((L, B, H, length + 1), -1, dtype=torch.int64)   # last: sink of the padding

    def groups(gid: torch.Tensor, at: int):
        """Old key groups gid copied bit-exactly to new groups at, at + 1, ..."""
        n = gid.shape[-1]
        safe = gid.clamp_min(0)
        kq = store["kq"].gather(3, safe.view(L, B, H, n, 1, 1).expand(-1, -1, -1, -1, *store["kq"].shape[4:]))
        ks = store["ks"].gather(3, safe.view(L, B, H, n, 1).expand(-1, -1, -1, -1, store["ks"].shape[4]))
        kz = store["kz"].gather(3, safe.view(L, B, H, n, 1).expand(-1, -1, -1, -1, store["kz"].shape[4]))
        tok = (safe.unsqueeze(-1) * GK + ar).reshape(L, B, H, n * GK)
        vq = store["vq"].gather(3, tok.view(L, B, H, -1, 1, 1).expand(-1, -1, -1, -1, *store["vq"].shape[4:]))
        vs = store["vs"].gather(3, tok.view(L, B, H, -1, 1).expand(-1, -1, -1, -1, store["vs"].shape[4]))
        vz = store["vz"].gather(3, tok.view(L, B, H, -1, 1).expand(-1, -1, -1, -1, store["vz"].shape[4]))
        new_slot = ((torch.arange(n) + at).view(n, 1) * GK + ar).expand(L, B, H, n, GK)
        src = torch.where((gid >= 0).unsqueeze(-1), tok.view(L, B, H, n, GK), length)
        remap.scatter_(-1, src.reshape(L, B, H, -1), new_slot.reshape(L, B, H, -1))
        return kq, ks, kz, vq, vs, vz

    parts = [groups(groups_before, 0)]
    d = store["kq"].shape[4]
    if m or st:
        k_all, v_all = _dequantize_all(store, lens)
    if m:
        sk = _gather_tokens(k_all, encode)
        sv = _gather_tokens(v_all, encode)
        pad = g2 * GK - m
        sk = torch.nn.functional.pad(sk, (0, 0, 0, pad)).reshape(L * B, H, g2 * GK, d)
        sv = torch.nn.functional.pad(sv, (0, 0, 0, pad)).reshape(L * B, H, g2 * GK, d)
        pk = quantize_keys(sk, bits=4, token_group=GK)
        pv = quantize_values(sv, bits=4, channel_group=32)
        parts.append(tuple(t.reshape(L, B, H, *t.shape[2:]) for t in (*pk, *pv)))
        slot = (torch.arange(m) + g1 * GK).expand(L, B, H, m)
        remap.scatter_(-1, torch.where(encode >= 0, encode, length), slot)
    parts.append(groups(groups_after, g1 + g2))
    new = {}
    for i, name in enumerate(("kq", "ks", "kz", "vq", "vs", "vz")):
        new[name] = torch.cat([p[i] for p in parts], 3)
    if st:
        new["kr"] = _gather_tokens(k_all, stage)
        new["vr"] = _gather_tokens(v_all, stage)
        slot = (torch.arange(st) + nql).expand(L, B, H, st)
        remap.scatter_(-1, torch.where(stage >= 0, stage, length), slot)
    else:
        new["kr"] = store["kr"][:, :, :, :0]
        new["vr"] = store["vr"][:, :, :, :0]
    new_lens = (new_len, nql, st, dropped + length - new_len)
    return new, new_lens, remap[..., :length]


def _packed(sel: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """Per lane: key where sel, ascending, padded with -1 to the largest count of any lane
    (session.py:328-332)."""
    n = int(sel.sum(-1).max()) if sel.numel() else 0
    k2 = torch.where(sel, key, BIG).sort(dim=-1).values[..., :n]
    return torch.where(k2 >= BIG, -1, k2)


def plan(phys: torch.Tensor, pos: torch.Tensor, lens: tuple, *, tail: int, stage_mode: bool, mode: str,
         repack_below: float, recent_window: int):
    """The lists of session.py:288-345 for live entries phys / pos [L, B, H, live] (after
    the state's compaction).  Returns (groups_before, encode, groups_after, stage)."""
    length, ql, rl, _ = lens
    L, B, H, live = phys.shape
    phys = phys.to(torch.int64)
    pos = pos.to(torch.int64)
    tail_slots = torch.arange(length - tail, length).expand(L, B, H, tail)
    in_q = phys < ql
    ng = max(1, ql // GK)
    grp = torch.where(in_q, phys // GK, ng)
    counts = torch.zeros((L, B, H, ng + 1), dtype=torch.int32)
    counts.scatter_add_(-1, grp, torch.ones_like(grp, dtype=torch.int32))
    counts = counts[..., :ng]
    if mode == "lazy":
        keep_g = counts >= max(1, int(math.ceil(repack_below * GK)))
    else:
        keep_g = torch.zeros_like(counts, dtype=torch.bool)
    tail_groups = 0
    if tail and not stage_mode:
        if rl or (length - tail) % GK:
            raise RuntimeError("unadmitted tail must be whole key groups")
        tail_groups = tail // GK
        keep_g[..., ng - tail_groups:] = False
    in_kept = in_q & keep_g.gather(-1, grp.clamp_max(ng - 1)) & (grp < ng)
    w = min(recent_window, live)
    if w:
        thr = pos.topk(w, dim=-1).values.amin(-1, keepdim=True)
    else:
        thr = torch.full((L, B, H, 1), 1 << 60, dtype=torch.int64)
    undecided = ~in_q & (pos >= thr)
    encode = ~in_kept & ~undecided

    def by_pos(sel):
        k2 = _packed(sel, pos * (1 << 24) + phys)
        return torch.where(k2 < 0, -1, k2 % (1 << 24))

    groups_before = _packed(keep_g, torch.arange(ng).expand(L, B, H, ng))
    enc = by_pos(encode)
    stage = by_pos(undecided)
    empty = torch.empty((L, B, H, 0), dtype=torch.int64)
    if tail and stage_mode:
        stage = torch.cat([stage, tail_slots], -1)
        after = empty
    elif tail:
        after = torch.arange(ng - tail_groups, ng).expand(L, B, H, tail_groups)
    else:
        after = empty
    return groups_before, enc, after, stage


def evict(store: dict, lens: tuple, pos: torch.Tensor, phys: torch.Tensor, keep: torch.Tensor, *,
          next_position: int, stage_mode: bool, mode: str, repack_below: float, recent_window: int):
    """Survivors keep [L, B, H, C] (live-axis indices) of the state's pos / phys
    [L, B, H, live]: the state's compaction (eviction.py:411-418), the plan and the
    rebuild (session.py:270-361).  Returns (new store, new lens, new phys [L, B, H, C])."""
    pos = pos.gather(-1, keep)
    phys = phys.to(torch.int64).gather(-1, keep)
    tail = lens[0] + lens[3] - next_position
    lists = plan(phys, pos, lens, tail=tail, stage_mode=stage_mode, mode=mode, repack_below=repack_below,
                 recent_window=recent_window)
    new, new_lens, remap = rebuild(store, lens, *lists)
    new_phys = remap.gather(-1, phys)
    if bool((new_phys < 0).any()):
        raise AssertionError("rebuild lost a live entry")
    return new, new_lens, new_phys
