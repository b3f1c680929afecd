"""Split-K attention and prefix scoring over a packed-int4 or 16-bit KV prefix.

Drop-in for the reference's ``maskahead.kernels.splitk`` (splitk.py:408-614): same
names, arguments and return values, served by hand-written gfx950 kernels in
libmaskahead_hip.so.

    out, stats = splitk_attention(q, prefix, kc, vc, want_prefix=True)
    mass, score = prefix_scores(q, prefix, stats, q_rows, value=True)

Differences in mechanism (not in results): the packed prefix is never unpacked to a
bf16 copy -- nibble unpack and scale/zero dequant happen in the load path of every
kernel -- and the split count is chosen for 256 CUs, not from the Triton tile sizes.
The Triton tuning arguments (block_m, block_n, num_warps, fused_max) are accepted and
ignored; dequant_rows / packed_direct_max still decide, as in the reference, whether
the value distance reads V rounded to the query dtype (the reference's unpacked copy)
or in f32.
"""

from __future__ import annotations

import torch

from .. import _native as N


class Prefix:
    """The prefix a kernel reads: packed (+ 16-bit residual tail) or plain 16-bit,
    [B, Hkv, n, D] (splitk.py:408-462).  ``mask``: optional uint8 [B, Hkv, n],
    0 = dead slot.  ``vround``: 0, or the dtype code (MA_BF16 / MA_F16) of the unpacked
    copy the reference would read this packed prefix through (splitk.py:513-516); only
    the copy splitk_attention hands back in its statistics carries it."""

    __slots__ = ("kq", "ks", "kz", "vq", "vs", "vz", "kf", "vf", "nq", "nf", "kb", "vb", "kg", "vg", "mask",
                 "kmode", "kch", "vround", "_nat")

    def __init__(self, *, kq=None, ks=None, kz=None, vq=None, vs=None, vz=None, kf=None, vf=None,
                 nq=0, nf=0, kb=16, vb=16, kg=32, vg=32, mask=None, kmode=0, kch=None):
        self.mask = mask
        self.kmode, self.kch = kmode, kch
        self.kq, self.ks, self.kz, self.vq, self.vs, self.vz = kq, ks, kz, vq, vs, vz
        self.kf, self.vf, self.nq, self.nf = kf, vf, int(nq), int(nf)
        self.kb, self.vb, self.kg, self.vg = kb, vb, kg, vg
        self.vround = 0
        self._nat = None   # (key, descriptor) of the last native()

    def with_vround(self, code: int) -> "Prefix":
        """A copy (same tensors) whose packed values are read rounded to dtype `code`."""
        p = Prefix(kq=self.kq, ks=self.ks, kz=self.kz, vq=self.vq, vs=self.vs, vz=self.vz, kf=self.kf, vf=self.vf,
                   nq=self.nq, nf=self.nf, kb=self.kb, vb=self.vb, kg=self.kg, vg=self.vg, mask=self.mask,
                   kmode=self.kmode, kch=self.kch)
        p.vround = int(code)
        p._nat = self._nat   # same tensors: the same descriptor
        return p

    def check_mask(self, b: int, hkv: int) -> None:
        """The kernels index the mask as (b * Hkv + h) * n + j: it must be exactly [B, Hkv, n]."""
        m = self.mask
        if m is not None and tuple(m.shape) != (b, hkv, self.n):
            raise ValueError(f"prefix mask must have shape {(b, hkv, self.n)}, got {tuple(m.shape)}")

    @property
    def n(self) -> int:
        return self.nq + self.nf

    @classmethod
    def from_view(cls, view) -> "Prefix":
        if view.k_bits == 16 and view.v_bits == 16:
            return cls(kf=view.k_fp, vf=view.v_fp, nf=view.length)
        if view.k_bits == 16 or view.v_bits == 16:
            raise NotImplementedError("mixed 16-bit / packed K,V")
        return cls(kq=view.k_q, ks=view.k_scale, kz=view.k_zero, vq=view.v_q, vs=view.v_scale, vz=view.v_zero,
                   kf=view.k_residual, vf=view.v_residual, nq=view.quantized_length, nf=view.residual_length,
                   kb=view.k_bits, vb=view.v_bits, kg=view.key_token_group, vg=view.value_channel_group,
                   kmode=1 if getattr(view, "key_mode", "channel") == "token" else 0,
                   kch=getattr(view, "k_chan", None))

    @classmethod
    def dense(cls, key: torch.Tensor, value: torch.Tensor, mask=None) -> "Prefix":
        return cls(kf=key, vf=value, nf=key.shape[2], mask=mask)

    def device(self) -> torch.device:
        for t in (self.kq, self.kf):
            if t is not None:
                return t.device
        return torch.device("cuda")

    def _native_key(self):
        ts = (self.kq, self.ks, self.kz, self.vq, self.vs, self.vz, self.kf, self.vf, self.mask)
        return (self.nq, self.nf, self.kb, self.vb, self.kg, self.vg, self.kmode,
                tuple(None if t is None else (id(t), t.data_ptr()) for t in ts))

    def native(self) -> N.MaPrefix:
        """The C-ABI descriptor (pointers, strides); validates layouts.  Built once per set
        of tensors: a later call with the same tensor objects and storage returns the same
        descriptor (a host-side saving of ~10 us per kernel call).  The tensors' strides
        are read when it is built; a tensor whose strides change in place afterwards
        (transpose_, as_strided_) needs a new Prefix."""
        key = self._native_key()
        if self._nat is not None and self._nat[0] == key:
            return self._nat[1]
        p = self._build_native()
        self._nat = (key, p)
        return p

    def _build_native(self) -> N.MaPrefix:
        if self.kmode:
            raise N.KernelUnavailableError("quant.key_mode='token' prefixes are not built in this library")
        p = N.MaPrefix()
        p.nq, p.nf = self.nq, self.nf
        p.kbits, p.vbits, p.kgroup, p.vgroup = int(self.kb), int(self.vb), int(self.kg), int(self.vg)
        if self.nq:
            kq, ks, kz, vq, vs, vz = self.kq, self.ks, self.kz, self.vq, self.vs, self.vz
            for name, t, nd in (("k_q", kq, 5), ("k_scale", ks, 4), ("k_zero", kz, 4), ("v_q", vq, 5),
                                ("v_scale", vs, 4), ("v_zero", vz, 4)):
                if t is None or t.ndim != nd:
                    raise ValueError(f"packed prefix: {name} must be a {nd}-d tensor")
                N.require_gpu(t, name)
                if t.stride(-1) != 1:
                    raise ValueError(f"packed prefix: {name} innermost dim must be contiguous")
            if kz.stride()[:3] != ks.stride()[:3] or vz.stride()[:3] != vs.stride()[:3]:
                raise ValueError("packed prefix: zero must share the scale's strides")
            if ks.dtype != torch.float16 or vs.dtype != torch.float16:
                raise N.KernelUnavailableError("packed prefix: only float16 scale/zero (param_dtype) is built")
            p.kq, p.ks, p.kz = kq.data_ptr(), ks.data_ptr(), kz.data_ptr()
            p.vq, p.vs, p.vz = vq.data_ptr(), vs.data_ptr(), vz.data_ptr()
            for i in range(4):
                p.skq[i] = kq.stride(i)
                p.svq[i] = vq.stride(i)
            for i in range(3):
                p.sks[i] = ks.stride(i)
                p.svs[i] = vs.stride(i)
        if self.nf:
            kf, vf = self.kf, self.vf
            if kf is None or vf is None or kf.ndim != 4 or vf.ndim != 4:
                raise ValueError("16-bit prefix: kf/vf must be 4-d")
            N.require_gpu(kf, "kf")
            if kf.stride(-1) != 1 or vf.stride(-1) != 1:
                raise ValueError("16-bit prefix: innermost dim must be contiguous")
            if kf.dtype != vf.dtype:
                raise ValueError("16-bit prefix: K and V dtypes differ")
            p.kf, p.vf = kf.data_ptr(), vf.data_ptr()
            p.fdtype = N.dtype_code(kf.dtype)
            for i in range(3):
                p.skf[i] = kf.stride(i)
                p.svf[i] = vf.stride(i)
        if self.mask is not None:
            m = self.mask
            if m.dtype != torch.uint8 or not m.is_contiguous() or m.shape[-1] != self.n:
                raise ValueError("prefix mask must be a contiguous uint8 [B, Hkv, n] tensor")
            p.mask = m.data_ptr()
        return p


def dequantize_prefix(prefix: Prefix, b: int, hkv: int, d: int, dtype=torch.bfloat16, block_n: int = 64):
    """The whole prefix as contiguous [B, Hkv, n, D] tensors (splitk.py:465-480)."""
    n = prefix.n
    ko = torch.empty((b, hkv, n, d), device=prefix.device(), dtype=dtype)
    vo = torch.empty_like(ko)
    if n == 0:
        return ko, vo
    lib = N.load()
    N.check(lib.ma_dequant_prefix(prefix.native(), b, hkv, d, N.t4(ko), N.t4(vo), N.stream_of(ko)),
            "ma_dequant_prefix")
    return ko, vo


def _check_query(query: torch.Tensor, current_key: torch.Tensor):
    if query.ndim != 4 or current_key.ndim != 4:
        raise ValueError("query and current_key must be [B, H, T, D]")
    N.require_gpu(query, "query")
    b, hq, t, d = query.shape
    hkv = current_key.shape[1]
    if hq % hkv:
        raise ValueError("Hq must be divisible by Hkv")
    return b, hq, t, d, hkv


def splitk_attention(query, prefix: Prefix, current_key, current_value, *, scaling=None,
                     causal_block: int = 0, q_pos0: int = 0, c_pos0: int = 0, want_prefix: bool = False,
                     block_m: int = 64, block_n: int = 32, num_warps: int = 4,
                     dequant_rows: int = 256, packed_direct_max: int = 256, fused_max: int = 1200,
                     split_tokens: int = 0):
    """softmax over [prefix | current] for every query row (splitk.py:493-579).

    Returns (out, stats); stats (want_prefix) = (M_p, L_p, O_p, prefix): prefix-only
    max of the scaled logits, sum of exp, and normalized output per row r = g*T + t of
    each KV head ([B,Hkv,R] f32, [B,Hkv,R] f32, [B,Hkv,R,D] query dtype).
    causal_block > 0: query at q_pos0+t sees current key c_pos0+j only if
    (c_pos0+j)//causal_block <= (q_pos0+t)//causal_block."""
    b, hq, t, d, hkv = _check_query(query, current_key)
    g = hq // hkv
    r = g * t
    prefix.check_mask(b, hkv)
    # the reference unpacks such a prefix to query.dtype and reads that copy from here on
    # (splitk.py:513-516).  For bf16 queries the copy holds what the kernels read anyway
    # (each dequantized value rounded to bf16 once): the statistics carry a descriptor
    # that marks the value distance to round V to bf16 too.  For f16 queries the copy's
    # values are rounded f32 -> f16 and every dot rounds them again, f16 -> bf16: the
    # copy is made (ma_dequant_prefix) and read from here on, as the reference does.
    used = prefix
    nat = prefix.native()   # built before the copy below, which then shares it
    if prefix.nq and (r > dequant_rows or prefix.n > packed_direct_max) and query.dtype != torch.float32:
        if query.dtype == torch.float16:
            used = Prefix.dense(*dequantize_prefix(prefix, b, hkv, d, dtype=torch.float16), mask=prefix.mask)
            nat = used.native()
        else:
            used = prefix.with_vround(N.dtype_code(query.dtype))
    dev = query.device
    scale = float(scaling) if scaling is not None else d ** -0.5
    out = torch.empty_like(query)
    if want_prefix:
        mp = torch.empty((b, hkv, r), device=dev, dtype=torch.float32)
        lp = torch.empty_like(mp)
        op = torch.empty((b, hkv, r, d), device=dev, dtype=query.dtype)
    else:
        mp = lp = op = None
    lib = N.load()
    n = prefix.n
    ws_bytes = N.size_query("ma_splitk_workspace_bytes", b, hkv, hq, t, d, prefix.nq, prefix.nf, int(split_tokens))
    if ws_bytes < 0:
        raise ValueError("bad splitk_attention geometry")
    ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
    tc = current_key.shape[2]
    rc = lib.ma_splitk_attention(
        N.t4(query), b, hq, t, d, nat, hkv, N.t4(current_key if tc else None),
        N.t4(current_value if tc else None), tc, int(causal_block), int(q_pos0), int(c_pos0), scale,
        N.t4(out), N.ptr(mp), N.ptr(lp), N.ptr(op), int(split_tokens), ws.data_ptr(), ws_bytes,
        N.stream_of(query))
    N.check(rc, "ma_splitk_attention")
    return out, ((mp, lp, op, used) if want_prefix else None)


_ROW_TABLES: dict = {}


def _row_table(rows: tuple, device: torch.device) -> torch.Tensor:
    """The int32 device copy of a host list of selection rows, made once per (device, list)
    by a synchronous copy and kept, so that a call under HIP graph capture finds it
    resident: a copy recorded during capture would read its host source again at every
    replay, after that temporary was freed.  Raises under capture for a list not seen
    before (pass the rows as a device tensor there)."""
    key = (device.index, rows)
    t = _ROW_TABLES.get(key)
    if t is None:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("q_rows given as a host list that was not used before graph capture: pass an int32 "
                             "device tensor, or make one call with these rows before capturing")
        if len(_ROW_TABLES) >= 64:
            _ROW_TABLES.pop(next(iter(_ROW_TABLES)))
        t = torch.tensor(rows, dtype=torch.int32, device=device)
        _ROW_TABLES[key] = t
    return t


def prefix_scores(query, prefix: Prefix, stats, q_rows: torch.Tensor, *, value: bool, scaling=None,
                  block_m: int = 64, block_n: int = 64, _topk_hist=None):
    """Per prefix entry: mass a_j (mean prefix-softmax over the selection rows) and, with
    value=True, a_j * ||v_j - c|| with c the mean of O_p over those rows
    (splitk.py:582-614).  q_rows: block positions of the selection queries -- an int
    tensor (on the GPU: used as given) or a host sequence / CPU tensor (checked; the whole
    block in order takes the kernels' row-table-free path; any other host list is copied
    to the device once and kept, see _row_table).
    Returns (mass, score) as [B, Hkv, n] f32 (score None when value=False); dead slots 0.
    _topk_hist = (rank, state): also build the read-set top-k's first-level histogram of the
    mass (rank 1) or score (rank 2) into that select state (select.prefix_scores_topk pairs
    this with the select that empties it again)."""
    b, hq, t, d = query.shape
    mp, lp, op, used = stats
    prefix = used if used is not None else prefix
    hkv = mp.shape[1]
    g = hq // hkv
    n = prefix.n
    prefix.check_mask(b, hkv)
    # host-side rows (a sequence, or a CPU tensor) are checked here; 0 .. T2-1 in order
    # needs no row table at all (mode "all"); device rows are clamped into the block in-kernel
    if not isinstance(q_rows, torch.Tensor) or not q_rows.is_cuda:
        host = tuple(int(x) for x in (q_rows.tolist() if isinstance(q_rows, torch.Tensor) else q_rows))
        if any(x < 0 or x >= t for x in host):
            raise ValueError(f"q_rows must be block positions in [0, {t})")
        q_rows = None if host == tuple(range(len(host))) else _row_table(host, query.device)
        t2 = len(host)
    else:
        q_rows = q_rows.to(dtype=torch.int32).contiguous()
        t2 = int(q_rows.numel())
    if t2 == 0:
        raise ValueError("q_rows cannot be empty")
    mass = torch.empty((b, hkv, n), device=query.device, dtype=torch.float32)
    score = torch.empty_like(mass) if value else None
    lib = N.load()
    st = N.stream_of(query)
    if n == 0:
        return mass, score
    if value and (not op.is_contiguous() or tuple(op.shape) != (b, hkv, g * t, d)):
        raise ValueError("stats O_p must be a contiguous [B, Hkv, R, D] tensor")
    scale = float(scaling) if scaling is not None else d ** -0.5
    vround = int(prefix.vround) if prefix.nq else 0
    args = (N.t4(query), b, hq, t, d, prefix.native(), hkv, N.ptr(q_rows), t2, mp.data_ptr(), lp.data_ptr(),
            op.data_ptr() if value else None, N.dtype_code(op.dtype) if value else 0, scale, 1 if value else 0,
            vround, mass.data_ptr(), N.ptr(score))
    if _topk_hist is None:
        N.check(lib.ma_prefix_scores(*args, st), "ma_prefix_scores")
    else:
        rank, state = _topk_hist
        N.check(lib.ma_prefix_scores_hist(*args, int(rank), state.data_ptr(), state.numel(), st),
                "ma_prefix_scores_hist")
    return mass, score
