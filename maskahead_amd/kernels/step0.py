"""Step 0 of a sparse layer in one library call (the reference session's _fast_step0,
session.py:1403-1454): split-K attention with the prefix statistics, the value-aware
prefix scores, the read-set top-k (ascending indices) and the gather of the selected
entries, enqueued by ``ma_step0`` -- the same launches and results as splitk_attention +
prefix_scores_topk + gather_packed_kv, without the per-op Python, ctypes packing and
allocation.  ``Step0Buffers`` holds one layer's outputs and workspace between calls, so
a call allocates nothing once its buffers have grown to the layer's sizes.
"""

from __future__ import annotations

import torch

from .. import _native as N
from .select import _state
from .splitk import Prefix, splitk_attention


def _unpacked(prefix: Prefix, r: int, query: torch.Tensor) -> bool:
    """Whether the reference reads this packed prefix through a copy unpacked to the
    query dtype (splitk.py:513-516), as splitk_attention does."""
    return bool(prefix.nq) and (r > 256 or prefix.n > 256) and query.dtype != torch.float32


def _vround(prefix: Prefix, r: int, query: torch.Tensor) -> int:
    """The dtype of that copy, as splitk_attention records it in its statistics (bf16
    queries; an f16 copy is made and read instead, see _staged)."""
    return N.dtype_code(query.dtype) if _unpacked(prefix, r, query) else 0


def _staged(query, prefix, current_key, current_value, rows, k, value, scale, out_key, out_value):
    """Step 0 as its stages, for f16 queries over an unpacked packed prefix: splitk_attention
    makes the f16 copy the reference reads (K and V rounded f32 -> f16, then f16 -> bf16 at
    every dot) and the scores, the read set and the gather read that copy."""
    from .ops import gather_packed_kv
    from .select import prefix_scores_topk

    out, stats = splitk_attention(query, prefix, current_key, current_value, scaling=scale, want_prefix=True)
    mass, score, idx = prefix_scores_topk(query, prefix, stats, rows, k, value=value,
                                          rank="score" if value else "mass", scaling=scale)
    if out_key is not None or out_value is not None:
        gather_packed_kv(stats[3], idx, dtype=(out_key if out_key is not None else out_value).dtype,
                         out_key=out_key, out_value=out_value)
    return out, stats, mass, score, idx


class Step0Buffers:
    """One layer's step-0 outputs and workspace, grown to fit and reused: out [B, Hq, T, D]
    (query dtype), M_p / L_p [B, Hkv, R] f32, O_p [B, Hkv, R, D], mass / score [B, Hkv, n]
    f32, idx [B, Hkv, k] int64 (views into storage of the largest sizes seen).  A later
    call of the same layer overwrites them."""

    def __init__(self):
        self._store: dict = {}
        # the last call's checked arguments and ctypes argument list (step0_select reuses
        # them while the prefix object, the shapes, the selection rows, the output views,
        # the workspace owner and the stream are the same: only the three operands' pointers
        # change from call to call)
        self._plan: tuple | None = None

    def take(self, name: str, numel: int, dtype: torch.dtype, device: torch.device, shape: tuple) -> torch.Tensor:
        t = self._store.get(name)
        if t is None or t.numel() < numel or t.dtype != dtype or t.device != device:
            t = torch.empty((max(numel, 1),), dtype=dtype, device=device)
            self._store[name] = t
        return t[:numel].view(shape)


def step0_select(bufs: Step0Buffers, query: torch.Tensor, prefix: Prefix, current_key: torch.Tensor,
                 current_value: torch.Tensor, rows, k: int, *, value: bool, scaling: float | None = None,
                 out_key: torch.Tensor | None = None, out_value: torch.Tensor | None = None,
                 workspace: Step0Buffers | None = None):
    """(out, (M_p, L_p, O_p, prefix_used), mass, score, idx) of one step 0, in one library
    call.  rows: the selection rows (a host list -- 0 .. T2-1 in order needs no table --
    or an int32 device tensor).  out_key / out_value (optional): [B, Hkv, k, D] views the
    selected entries are gathered into (the layer's compact buffer).  workspace: where the
    scratch workspace lives (default bufs); layers run one after another on a stream can
    share one."""
    stream = N.stream_of(query)
    rows_key = rows if isinstance(rows, torch.Tensor) else tuple(rows)
    views = tuple(None if x is None else (x.data_ptr(), x.shape, x.stride(), x.dtype) for x in (out_key, out_value))
    key = (query.shape, query.stride(), query.dtype, current_key.shape, current_key.stride(), current_value.stride(),
           current_key.dtype, current_value.dtype, int(k), bool(value), scaling, views, stream)
    plan = bufs._plan
    # (prefix.native() returns the same descriptor object while the prefix's tensors and
    # mask are the ones it was built from)
    if (plan is not None and plan[0] is prefix and plan[1] is workspace and plan[2] == key
            and (plan[3] is rows_key if isinstance(rows_key, torch.Tensor) else plan[3] == rows_key)
            and plan[4][5] is prefix.native()):
        args, result = plan[4], plan[5]
        # the same shapes, strides and dtypes (the key): only the operands' addresses change
        args[0].ptr = query.data_ptr()
        if current_key.shape[2]:
            args[7].ptr, args[8].ptr = current_key.data_ptr(), current_value.data_ptr()
        N.check(N.load().ma_step0(*args), "ma_step0")
        return result
    if query.ndim != 4 or current_key.ndim != 4:
        raise ValueError("query and current_key must be [B, H, T, D]")
    N.require_gpu(query, "query")
    b, hq, t, d = query.shape
    hkv = current_key.shape[1]
    if hq % hkv:
        raise ValueError("Hq must be divisible by Hkv")
    r = (hq // hkv) * t
    n = prefix.n
    k = int(k)
    if n <= 0 or not 0 < k <= n:
        raise ValueError(f"read budget k={k} outside [1, {n}]")
    prefix.check_mask(b, hkv)
    if isinstance(rows, torch.Tensor) and rows.is_cuda:
        q_rows = rows.to(torch.int32).contiguous()
        t2 = int(q_rows.numel())
    else:
        host = tuple(int(x) for x in (rows.tolist() if isinstance(rows, torch.Tensor) else rows))
        if any(x < 0 or x >= t for x in host):
            raise ValueError(f"q_rows must be block positions in [0, {t})")
        from .splitk import _row_table

        q_rows = None if host == tuple(range(len(host))) else _row_table(host, query.device)
        t2 = len(host)
    if t2 == 0:
        raise ValueError("q_rows cannot be empty")
    if query.dtype == torch.float16 and _unpacked(prefix, r, query):
        return _staged(query, prefix, current_key, current_value, rows, k, value,
                       float(scaling) if scaling is not None else d ** -0.5, out_key, out_value)
    dev = query.device
    nat = prefix.native()
    vround = _vround(prefix, r, query)
    used = prefix.with_vround(vround) if vround else prefix
    out = bufs.take("out", query.numel(), query.dtype, dev, tuple(query.shape))
    mp = bufs.take("mp", b * hkv * r, torch.float32, dev, (b, hkv, r))
    lp = bufs.take("lp", b * hkv * r, torch.float32, dev, (b, hkv, r))
    op = bufs.take("op", b * hkv * r * d, query.dtype, dev, (b, hkv, r, d))
    mass = bufs.take("mass", b * hkv * n, torch.float32, dev, (b, hkv, n))
    score = bufs.take("score", b * hkv * n, torch.float32, dev, (b, hkv, n)) if value else None
    idx = bufs.take("idx", b * hkv * k, torch.int64, dev, (b, hkv, k))
    ws_bytes = N.size_query("ma_step0_workspace_bytes", b, hkv, hq, t, d, prefix.nq, prefix.nf)
    if ws_bytes <= 0:
        raise N.KernelUnavailableError(f"ma_step0: no workspace size for n={n}")
    ws = (workspace or bufs).take("ws", ws_bytes, torch.uint8, dev, (ws_bytes,))
    st = _state(dev, N.size_query("ma_topk_state_bytes", b * hkv), stream)
    scale = float(scaling) if scaling is not None else d ** -0.5
    tc = current_key.shape[2]
    args = [N.t4(query), b, hq, t, d, nat, hkv, N.t4(current_key if tc else None),
            N.t4(current_value if tc else None), tc, scale, N.t4(out), mp.data_ptr(), lp.data_ptr(), op.data_ptr(),
            N.ptr(q_rows), t2, 1 if value else 0, 2 if value else 1, vround, mass.data_ptr(), N.ptr(score), k,
            idx.data_ptr(), N.t4(out_key), N.t4(out_value), st.data_ptr(), st.numel(), ws.data_ptr(), ws_bytes,
            stream]
    N.check(N.load().ma_step0(*args), "ma_step0")
    result = (out, (mp, lp, op, used), mass, score, idx)
    # the plan keeps every tensor its pointers name alive: q_rows (a cached device table, or
    # None), the select state and the workspace (which another layer sharing the owner may
    # have replaced by a larger one since)
    bufs._plan = (prefix, workspace, key, rows_key, args, result, q_rows, st, ws)
    return result
