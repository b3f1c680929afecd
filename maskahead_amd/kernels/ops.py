"""Kernel-op API of the read path (the reference's ``maskahead.kernels.ops``).

Same names and arguments as ops.py:130-860 of the reference, served by the gfx950
kernels.  ``backend``: "auto", "triton" and "hip" all select the HIP kernels; "torch"
(the reference's CPU path) is not part of this package -- it lives in the test oracle --
and raises KernelUnavailableError, as does any variant this build does not implement.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _native as N
from .._native import KernelUnavailableError
from .select import topk_ascending
from .splitk import Prefix, prefix_scores, splitk_attention

__all__ = [
    "KernelUnavailableError",
    "_selected_queries",
    "SelectorResult",
    "SelectorScratch",
    "dense_packed_attention",
    "gather_packed_kv",
    "quantize_key_groups_into",
    "quantize_values_into",
    "selector_topk",
    "hip_available",
    "triton_available",
]


def hip_available() -> bool:
    """Whether the gfx950 kernels can run here: the library loads and a GPU is present."""
    try:
        N.load()
    except KernelUnavailableError:
        return False
    return torch.cuda.is_available()


# the reference's name for "the GPU kernels can run" (ops.py:23-24); callers that probe
# it before choosing a backend get the HIP answer
triton_available = hip_available


def _choose_backend(backend: str, tensor: torch.Tensor) -> str:
    """ops.py:44-53: every GPU backend name maps to HIP; the CPU path is not shipped."""
    if backend == "torch":
        raise KernelUnavailableError("backend='torch' is the reference's CPU path; this package runs the HIP "
                                     "kernels only (the CPU restatement is the test oracle)")
    if backend not in ("auto", "triton", "hip"):
        raise ValueError(f"unknown backend {backend!r}")
    N.require_gpu(tensor)
    return "hip"


def _view_heads(view) -> int:
    for t in (view.k_fp, view.k_q, view.k_residual):
        if t is not None:
            return int(t.shape[1])
    raise ValueError("empty view")


def _view_head_dim(view, out_key=None, out_value=None) -> int:
    """ops.py:525-567: one head dim from every source that states it."""
    dims = set()
    if getattr(view, "head_dim", None):
        dims.add(int(view.head_dim))
    for t in (out_key, out_value, view.k_fp, view.v_fp, view.k_residual, view.v_residual):
        if t is not None:
            dims.add(int(t.shape[-1]))
    if view.k_q is not None:
        dims.add(int(view.k_q.shape[-2]))
    if len(dims) != 1:
        raise ValueError(f"cannot infer one KV head dimension: {sorted(dims)}")
    return dims.pop()


def dense_packed_attention(query, view, current_key, current_value, *, scaling=None, backend="auto",
                           kernel_variant="blocked"):
    """Attention over [cache view | current block] (ops.py:130-264, 766-787)."""
    _choose_backend(backend, query)
    prefix = Prefix.from_view(view)
    out, _ = splitk_attention(query, prefix, current_key, current_value, scaling=scaling)
    return out


@dataclass(slots=True)
class SelectorResult:
    indices: torch.Tensor
    values: torch.Tensor
    importance: torch.Tensor | None = None


class SelectorScratch:
    """Kept for API compatibility (ops.py:274-317); the HIP selector needs no logits
    buffer -- scores are reduced in registers -- so it holds nothing."""

    def tensors(self, **_):
        raise KernelUnavailableError("the HIP selector has no logits scratch")


def _selected_queries(query: torch.Tensor, query_indices, hkv: int) -> torch.Tensor:
    """[B, Hq, T, D] -> [B, Hkv, G*len(idx), D] (ops.py:320-330)."""
    if not query_indices:
        raise ValueError("query_indices cannot be empty")
    b, hq, _, d = query.shape
    if hq % hkv:
        raise ValueError("Hq must be divisible by Hkv")
    q = query[:, :, list(query_indices), :]          # [B, Hq, T2, D]; rows g * T2 + t2 per KV head
    return q.reshape(b, hkv, -1, d).contiguous()


def selector_topk(query, view, *, query_indices, topk, current_key=None, domain="prefix", score_kind="softmax",
                  sort_indices=True, scaling=None, backend="auto", live_mask=None, return_importance=False,
                  scratch=None, kernel_variant="blocked", logits_dtype=torch.float16) -> SelectorResult:
    """Top-k prefix entries per KV head by mean prefix-softmax mass of the selection
    queries (ops.py:333-521, 790-832).  live_mask [B, Hkv, n] bool: False = evicted
    (removed before the softmax, never selected).  Indices come back ascending."""
    if view.length <= 0:
        raise ValueError("selector requires a non-empty prefix")
    if not query_indices:
        raise ValueError("query_indices cannot be empty")
    if domain != "prefix" or score_kind != "softmax":
        raise KernelUnavailableError(f"selector domain={domain!r} score_kind={score_kind!r} is not built "
                                     "(fast path: prefix / softmax)")
    _choose_backend(backend, query)
    hkv = _view_heads(view)
    k = min(int(topk), view.length)
    prefix = Prefix.from_view(view)
    if live_mask is not None:
        prefix.mask = live_mask.to(torch.uint8).contiguous()
    empty = query.new_empty((query.shape[0], hkv, 0, query.shape[-1]))
    _, stats = splitk_attention(query, prefix, empty, empty, scaling=scaling, want_prefix=True)
    rows = torch.as_tensor(list(query_indices), dtype=torch.int32, device=query.device)
    importance, _ = prefix_scores(query, prefix, stats, rows, value=False, scaling=scaling)
    values = torch.empty((*importance.shape[:-1], k), device=query.device, dtype=torch.float32)
    indices = topk_ascending(importance, k, prefix.mask, values=values)
    return SelectorResult(indices=indices, values=values,
                          importance=importance.clone() if return_importance else None)


def gather_packed_kv(view, indices, *, dtype=torch.bfloat16, backend="auto", out_key=None, out_value=None):
    """Selected entries of a cache view, dequantized, as [B, Hkv, k, D] K and V
    (ops.py:570-662, 835-855).  Indices outside the view produce zeros.  ``view`` may also
    be the view's Prefix (its mask is not used)."""
    if indices.ndim != 3:
        raise ValueError("indices must have shape [B,Hkv,K]")
    _choose_backend(backend, indices)
    b, hkv, k = indices.shape
    if isinstance(view, Prefix):
        prefix = view
        src = prefix.kq if prefix.nq else prefix.kf
        d = int(src.shape[-2] if prefix.nq else src.shape[-1])
        if out_key is not None and int(out_key.shape[-1]) != d:
            raise ValueError("output head_dim differs from the prefix's")
    else:
        d = _view_head_dim(view, out_key=out_key, out_value=out_value)
        prefix = Prefix.from_view(view)
    if out_key is None:
        out_key = torch.empty((b, hkv, k, d), device=indices.device, dtype=dtype)
    if out_value is None:
        out_value = torch.empty_like(out_key)
    if tuple(out_key.shape) != (b, hkv, k, d) or tuple(out_value.shape) != (b, hkv, k, d):
        raise ValueError("output buffer has the wrong shape")
    idx = indices if indices.dtype == torch.int64 else indices.to(torch.int64)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    prefix.check_mask(b, hkv)
    lib = N.load()
    rc = lib.ma_gather_kv(prefix.native(), b, hkv, d, idx.data_ptr(), N.i64arr(idx.stride(0), idx.stride(1)), k,
                          N.t4(out_key), N.t4(out_value), N.stream_of(idx))
    N.check(rc, "ma_gather_kv")
    return out_key, out_value


def quantize_key_groups_into(source, out_payload, out_scale, out_zero, *, bits, token_group, backend="auto"):
    """4-bit key groups of `source` [B,H,T,D] into payload [B,H,T/KG,D,KG/2] and f16
    scale/zero [B,H,T/KG,D] (ops.py:665-713; rule reference.py:58-90)."""
    _choose_backend(backend, source)
    if bits != 4:
        raise KernelUnavailableError(f"{bits}-bit keys are not built")
    if out_scale.dtype != torch.float16 or out_zero.dtype != torch.float16:
        raise KernelUnavailableError("only float16 scale/zero are built")
    b, h, t, d = source.shape
    if t % token_group or out_payload.shape[2] != t // token_group:
        raise ValueError("invalid key quantization output geometry")
    if out_zero.stride() != out_scale.stride():
        raise ValueError("scale and zero must share strides")
    lib = N.load()
    rc = lib.ma_quantize_keys(N.t4(source), b, h, t, d, int(token_group), out_payload.data_ptr(),
                              N.i64arr(*out_payload.stride()[:4]), out_scale.data_ptr(), out_zero.data_ptr(),
                              N.i64arr(*out_scale.stride()[:3]), N.stream_of(source))
    N.check(rc, "ma_quantize_keys")


def quantize_values_into(source, out_payload, out_scale, out_zero, *, bits, channel_group, backend="auto"):
    """4-bit per-token values of `source` [B,H,T,D] into payload [B,H,T,D/VG,VG/2] and
    f16 scale/zero [B,H,T,D/VG] (ops.py:716-758; rule reference.py:182-213)."""
    _choose_backend(backend, source)
    if bits != 4:
        raise KernelUnavailableError(f"{bits}-bit values are not built")
    if out_scale.dtype != torch.float16 or out_zero.dtype != torch.float16:
        raise KernelUnavailableError("only float16 scale/zero are built")
    b, h, t, d = source.shape
    if out_zero.stride() != out_scale.stride():
        raise ValueError("scale and zero must share strides")
    lib = N.load()
    rc = lib.ma_quantize_values(N.t4(source), b, h, t, d, int(channel_group), out_payload.data_ptr(),
                                N.i64arr(*out_payload.stride()[:4]), out_scale.data_ptr(), out_zero.data_ptr(),
                                N.i64arr(*out_scale.stride()[:3]), N.stream_of(source))
    N.check(rc, "ma_quantize_values")
