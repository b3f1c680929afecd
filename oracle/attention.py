"""Floating-point half of the CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

torch on the CPU.  The split-K / scoring restatements compute in float64 and keep the
reference fast path's deterministic rounding points (inputs cast to bf16 before the dot
products, O_p rounded to the query dtype before the value centre is taken); the
per-tile bf16 rounding of p inside the reference's PV dot depends on its tiling and is
not modelled (it is below the stated tolerances).  Shapes follow the reference:
Q [B, Hq, T, D], prefix K/V [B, Hkv, n, D], rows r = g*T + t of KV head h, G = Hq/Hkv.
"""

from __future__ import annotations

import math

import torch

from . import codec

F64 = torch.float64


# ---------------------------------------------------------------- codec (torch form)

def _round_half_even(x: torch.Tensor) -> torch.Tensor:
    return torch.round(x)          # torch.round rounds half to even


def quantize_keys(key: torch.Tensor, *, bits: int = 4, token_group: int = 32,
                  param_dtype: torch.dtype = torch.float16):
    """KIVI key quantization, per channel over token groups (reference.py:58-90).

    Arithmetic stays in key.dtype (min, max, range/levels, (x - min)/scale, round half
    to even), scale and zero are stored in param_dtype.  Returns
    (payload u8 [B,H,G,D,KG/2], scale [B,H,G,D], zero [B,H,G,D]).
    Pinned by tests/golden (vectors written by the reference's own quantize_keys)."""
    b, h, t, d = key.shape
    if t % token_group:
        raise ValueError("token count must be a multiple of token_group")
    levels = float((1 << bits) - 1)
    grouped = key.reshape(b, h, t // token_group, token_group, d).transpose(-1, -2)
    lo = grouped.amin(dim=-1, keepdim=True)
    hi = grouped.amax(dim=-1, keepdim=True)
    step = ((hi - lo) / levels).clamp_min(1e-8)
    codes = _round_half_even((grouped - lo) / step).clamp_(0, levels).to(torch.uint8)
    payload = (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()
    return payload, step.squeeze(-1).to(param_dtype).contiguous(), lo.squeeze(-1).to(param_dtype).contiguous()


def quantize_values(value: torch.Tensor, *, bits: int = 4, channel_group: int = 32,
                    param_dtype: torch.dtype = torch.float16):
    """Per-token value quantization over channel groups (reference.py:182-213).
    Returns (payload u8 [B,H,N,D/VG,VG/2], scale [B,H,N,D/VG], zero [B,H,N,D/VG])."""
    b, h, t, d = value.shape
    if d % channel_group:
        raise ValueError("head_dim must be a multiple of channel_group")
    levels = float((1 << bits) - 1)
    grouped = value.reshape(b, h, t, d // channel_group, channel_group)
    lo = grouped.amin(dim=-1, keepdim=True)
    hi = grouped.amax(dim=-1, keepdim=True)
    step = ((hi - lo) / levels).clamp_min(1e-8)
    codes = _round_half_even((grouped - lo) / step).clamp_(0, levels).to(torch.uint8)
    payload = (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()
    return payload, step.squeeze(-1).to(param_dtype).contiguous(), lo.squeeze(-1).to(param_dtype).contiguous()


def dequantize_keys(payload: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """[B,H,G,D,KG/2] -> f32 [B,H,G*KG,D] (reference.py:168-179; cast to bf16 by the caller).
    Cross-checked element by element against oracle/codec.c."""
    lo_nib = (payload & 15).to(torch.float32)
    hi_nib = (payload >> 4).to(torch.float32)
    codes = torch.stack([lo_nib, hi_nib], dim=-1).flatten(-2)          # [B,H,G,D,KG]
    x = codes * scale.float().unsqueeze(-1)
    x = x + zero.float().unsqueeze(-1)
    b, h, g, d, kg = x.shape
    return x.transpose(-1, -2).reshape(b, h, g * kg, d)


def dequantize_values(payload: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """[B,H,N,D/VG,VG/2] -> f32 [B,H,N,D] (reference.py:259-268)."""
    lo_nib = (payload & 15).to(torch.float32)
    hi_nib = (payload >> 4).to(torch.float32)
    codes = torch.stack([lo_nib, hi_nib], dim=-1).flatten(-2)          # [B,H,N,NG,VG]
    x = codes * scale.float().unsqueeze(-1)
    x = x + zero.float().unsqueeze(-1)
    b, h, n, ng, vg = x.shape
    return x.reshape(b, h, n, ng * vg)


# ---------------------------------------------------------------- attention

def _rows_view(query: torch.Tensor, hkv: int) -> torch.Tensor:
    """[B, Hq, T, D] -> [B, Hkv, R = G*T, D] with r = g*T + t (splitk.py:131-138)."""
    b, hq, t, d = query.shape
    return query.reshape(b, hkv, (hq // hkv) * t, d)


def splitk_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                     current_key: torch.Tensor, current_value: torch.Tensor, *,
                     mask: torch.Tensor | None = None, scale: float | None = None,
                     causal_block: int = 0, q_pos0: int = 0, c_pos0: int = 0):
    """Softmax attention over [prefix | current] for every query row, plus the
    prefix-only statistics (splitk.py:493-579, kernels 116-318).

    query [B,Hq,T,D]; key/value: the prefix [B,Hkv,n,D] as the kernel reads it (the
    dequantized bf16 prefix for packed caches); current_* [B,Hkv,Tc,D]; mask uint8
    [B,Hkv,n] (0 = dead slot).  Q, K, V are rounded to bf16 (splitk.py:139, 152, 164),
    everything after that is float64.  A current key j is visible to query t only if
    (c_pos0+j)//causal_block <= (q_pos0+t)//causal_block (splitk.py:175-176).

    Returns out [B,Hq,T,D] (query dtype), M_p, L_p f32 [B,Hkv,R] (prefix max of the
    scaled logits and sum of exp(s - M_p); -inf / 0 when no prefix entry is live), and
    O_p [B,Hkv,R,D] = prefix-only output in the query dtype (0 when L_p = 0)."""
    b, hq, t, d = query.shape
    hkv = current_key.shape[1]
    g = hq // hkv
    sc = d ** -0.5 if scale is None else scale
    q = _rows_view(query.to(torch.bfloat16).to(F64), hkv)              # [B,Hkv,R,D]
    k = key.to(torch.bfloat16).to(F64)
    v = value.to(torch.bfloat16).to(F64)
    kc = current_key.to(torch.bfloat16).to(F64)
    vc = current_value.to(torch.bfloat16).to(F64)
    n = k.shape[2]

    s = torch.matmul(q, k.transpose(-1, -2)) * sc                      # [B,Hkv,R,n]
    if mask is not None and n:
        s = s.masked_fill(~mask.bool()[:, :, None, :], -math.inf)
    if n:
        m_p = s.amax(dim=-1)
    else:
        m_p = torch.full(q.shape[:3], -math.inf, dtype=F64)
    m_safe = torch.where(torch.isinf(m_p) & (m_p < 0), torch.zeros_like(m_p), m_p)
    e = torch.exp(s - m_safe.unsqueeze(-1))
    l_p = e.sum(dim=-1)
    acc_p = torch.matmul(e, v)
    o_p = acc_p / torch.where(l_p > 0, l_p, torch.ones_like(l_p)).unsqueeze(-1)

    sc_cur = torch.matmul(q, kc.transpose(-1, -2)) * sc                # [B,Hkv,R,Tc]
    if causal_block > 0:
        tq = torch.arange(g * t) % t
        tc = torch.arange(kc.shape[2])
        ok = ((c_pos0 + tc)[None, :] // causal_block) <= ((q_pos0 + tq)[:, None] // causal_block)
        sc_cur = sc_cur.masked_fill(~ok, -math.inf)
    m_c = sc_cur.amax(dim=-1) if kc.shape[2] else torch.full_like(m_p, -math.inf)
    m_all = torch.maximum(m_p, m_c)
    m_all_safe = torch.where(torch.isinf(m_all) & (m_all < 0), torch.zeros_like(m_all), m_all)
    w_p = torch.exp(m_safe - m_all_safe)
    e_c = torch.exp(sc_cur - m_all_safe.unsqueeze(-1))
    den = l_p * w_p + e_c.sum(dim=-1)
    num = acc_p * w_p.unsqueeze(-1) + torch.matmul(e_c, vc)
    out = num / torch.where(den > 0, den, torch.ones_like(den)).unsqueeze(-1)
    out = out.reshape(b, hq, t, d).to(query.dtype)
    return out, m_p.float(), l_p.float(), o_p.to(query.dtype)


def prefix_scores(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor | None,
                  m_p: torch.Tensor, l_p: torch.Tensor, o_p: torch.Tensor | None,
                  q_rows, *, mask: torch.Tensor | None = None, value_aware: bool,
                  scale: float | None = None):
    """Per prefix entry j of KV head h (splitk.py:582-614, kernel 321-371):

        a_j = (1 / (G*T2)) * sum over g < G, t in q_rows of exp(s_rj - M_p[r]) / L_p[r]
        score_j = a_j * || v_j - c ||,  c = mean over the same rows of f32(O_p[r])

    with s the scaled bf16-input logits and r = g*T + t.  Dead slots (mask 0) get
    a = 0 and score = 0.  `value` is the prefix as the distance sees it (bf16-rounded
    when the reference unpacks the prefix, splitk.py:513-516 + 592).  float64 inside;
    returns (mass f32 [B,Hkv,n], score f32 [B,Hkv,n] or None)."""
    b, hq, t, d = query.shape
    hkv = m_p.shape[1]
    g = hq // hkv
    sc = d ** -0.5 if scale is None else scale
    rows = torch.as_tensor(list(q_rows), dtype=torch.int64)
    rf = (torch.arange(g)[:, None] * t + rows[None, :]).reshape(-1)    # [G*T2]
    q = _rows_view(query.to(torch.bfloat16).to(F64), hkv)[:, :, rf, :]
    k = key.to(torch.bfloat16).to(F64)
    s = torch.matmul(q, k.transpose(-1, -2)) * sc                      # [B,Hkv,R2,n]
    mp = m_p.to(F64)[:, :, rf]
    lp = l_p.to(F64)[:, :, rf]
    p = torch.exp(s - mp.unsqueeze(-1)) / torch.where(lp > 0, lp, torch.ones_like(lp)).unsqueeze(-1)
    a = p.mean(dim=2)
    if mask is not None:
        a = torch.where(mask.bool(), a, torch.zeros_like(a))
    if not value_aware:
        return a.float(), None
    centre = o_p[:, :, rf, :].float().to(F64).mean(dim=2)              # [B,Hkv,D]
    dist = (value.to(F64) - centre.unsqueeze(2)).norm(dim=-1)
    score = a * dist
    if mask is not None:
        score = torch.where(mask.bool(), score, torch.zeros_like(score))
    return a.float(), score.float()


def selector_importance(query: torch.Tensor, key: torch.Tensor, query_indices, *,
                        live_mask: torch.Tensor | None = None, scale: float | None = None):
    """Mean prefix-softmax mass over the G grouped heads and the selection rows, dead
    entries removed before the softmax (reference.py:318-366, domain "prefix", score
    "softmax"), in float64 on the inputs as given.  Closed-form twin of prefix_scores'
    mass: tests check the two agree."""
    b, hq, t, d = query.shape
    hkv = key.shape[1]
    g = hq // hkv
    sc = d ** -0.5 if scale is None else scale
    idx = torch.as_tensor(list(query_indices), dtype=torch.int64)
    q = query[:, :, idx, :].to(F64).reshape(b, hkv, g, len(idx), d)
    logits = torch.einsum("bhgmd,bhnd->bhgmn", q, key.to(F64)) * sc
    if live_mask is not None:
        logits = logits.masked_fill(~live_mask.bool()[:, :, None, None, :], -math.inf)
    return torch.softmax(logits, dim=-1).mean(dim=(2, 3))


def dense_attention(query, old_key, old_value, current_key, current_value, *, scale=None):
    """Softmax attention over [old | current] with GQA head repetition, float64
    (reference.py:279-296; compact_attention_reference 299-315 is the same call)."""
    hq = query.shape[1]
    k = torch.cat([old_key, current_key], dim=2).to(F64)
    v = torch.cat([old_value, current_value], dim=2).to(F64)
    rep = hq // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    sc = query.shape[-1] ** -0.5 if scale is None else scale
    p = torch.softmax(torch.matmul(query.to(F64), k.transpose(-1, -2)) * sc, dim=-1)
    return torch.matmul(p, v)


# ---------------------------------------------------------------- keep-path score

def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(F64)


def value_score_bf16(a: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Keep score a_i * ||v_i - c||, c = sum_j w_j v_j / sum_j w_j, with the bf16
    rounding points of session.py:38-40 (the default, non-diagnostic branch):
    w = bf16(a); numerator and denominator each rounded to bf16 after an exact
    accumulation; c = bf16(num / max(den, 1e-12)); v - c rounded to bf16; the norm
    rounded to bf16; the product with a in f32.  a [..., n] f32, v [..., n, D] bf16.
    Pinned by tests/golden (vectors written by the reference's own value_score)."""
    w = _bf16(a.float())
    vv = v.to(torch.bfloat16).to(F64)
    num = _bf16((w.unsqueeze(-1) * vv).sum(dim=-2))                    # [..., D]
    den = _bf16(w.sum(dim=-1, keepdim=True))
    den = torch.maximum(den, _bf16(torch.tensor(1e-12, dtype=F64)))
    c = _bf16(num / den)
    diff = _bf16(vv - c.unsqueeze(-2))
    norm = _bf16(diff.pow(2).sum(dim=-1).sqrt())
    return (a.float() * norm.float())


def value_score_fp32(a: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """The BITSIEVE_VSCORE_FP32 branch of session.py:34-37, float64 inside."""
    vv = v.to(F64)
    w = a.to(F64)
    c = (w.unsqueeze(-1) * vv).sum(-2, keepdim=True) / w.sum(-1, keepdim=True).clamp_min(1e-12).unsqueeze(-1)
    return (w * (vv - c).norm(dim=-1)).float()


# ---------------------------------------------------------------- CPU baseline

def reference_cpu_step(query, key, value, current_key, current_value, *, query_indices,
                       topk: int, scale: float | None = None):
    """The reference's CPU torch path for step 0 of one sparse layer, in the reference's
    own float32 arithmetic, for timing as the CPU baseline (not a parity oracle):
    dense step-0 attention (reference.py:279-296), selector importance
    (reference.py:318-366), value-aware rescoring with the attention-weighted centre
    (session.py:870-954), top-k + ascending sort (session.py:965-967) and the gather of
    the selected bf16 K/V (reference.py:396-400).  key/value are the dequantized prefix."""
    b, hq, t, d = query.shape
    hkv = key.shape[1]
    g = hq // hkv
    sc = d ** -0.5 if scale is None else scale
    kk = torch.cat([key, current_key], dim=2).float().repeat_interleave(g, dim=1)
    vv = torch.cat([value, current_value], dim=2).float().repeat_interleave(g, dim=1)
    out = torch.matmul(torch.softmax(torch.matmul(query.float(), kk.transpose(-1, -2)) * sc, dim=-1), vv)
    idx = torch.as_tensor(list(query_indices), dtype=torch.int64)
    q = query[:, :, idx, :].float().reshape(b, hkv, g, len(idx), d)
    logits = torch.einsum("bhgmd,bhnd->bhgmn", q, key.float()) * sc
    imp = torch.softmax(logits, dim=-1).mean(dim=(2, 3))
    v32 = value.float()
    centre = (imp.unsqueeze(-1) * v32).sum(dim=2, keepdim=True) / imp.sum(-1, keepdim=True).clamp_min(1e-12).unsqueeze(-1)
    score = imp * (v32 - centre).norm(dim=-1)
    sel = torch.topk(score, min(topk, key.shape[2]), dim=-1).indices.sort(dim=-1).values
    gi = sel.unsqueeze(-1).expand(-1, -1, -1, d)
    return out.to(query.dtype), sel, torch.gather(key, 2, gi), torch.gather(value, 2, gi)
