// LDS tile staging shared by the split-K attention and the score pass: 64 tokens of one
// (batch, KV head) lane, dequantized (packed int4) or converted (16/32-bit) to bf16 and
// laid out for the MFMA operand reads:
//   Ks[t][d]  (row stride KS = D + 8 bf16)  -> 16-byte fragments along d
//   Vt[d][t]  (row stride VS = 64 + 4 bf16) -> 8-byte fragments along tokens
// okmask bit t = token t is usable (inside the range and live).  Dead or out-of-range
// tokens are staged as zero values, so stale codes or NaN of an evicted slot never
// reach an accumulator.
//
// Addressing: a Lane holds the uniform base pointers and 32-bit inner strides of one
// (batch, KV head) lane (kept in scalar registers), a thread's staging item has one
// precomputed 32-bit offset, and a tile adds a uniform offset -- so a load costs no
// per-tile address arithmetic.  Loads are issued unconditionally from valid addresses
// (loads behind branches are waited for one at a time on this GPU); full tiles use the
// affine fast path, partial tiles clamp token indices.
//
// Staging is split in two so the next tile's HBM loads overlap the current tile's MFMA
// work: load_*() issues the global loads of one tile into a per-thread register block,
// store_*() (after the barrier that frees the LDS) dequantizes and writes it.  A
// workgroup has NT = 512 threads (8 waves); every staging item is 16 payload bytes:
//   packed K   item = (key group gl, channel pair dp, 16-token half th): two 8-byte code
//              rows + the two channels' f16 scale and zero      -> 2*D items
//   packed V   item = (token pair tp, channel group cg, 16-channel half ch): two 8-byte
//              code rows + the two tokens' f16 scale and zero   -> 2*D items
//   16-bit K   item = (token, 8-channel chunk), 16 bytes        -> 8*D items
//   16-bit V   item = (token pair, 8-channel chunk), 2x16 bytes -> 4*D items
// The one tile that straddles the packed / 16-bit boundary of a prefix is staged by the
// generic synchronous path (stage_generic).
#pragma once

#include "ma_common.h"

namespace ma {

constexpr int TILE = 64;
constexpr int KGRP = 32;
constexpr int VGRP = 32;
constexpr int NT = 512;

template <int D>
struct TileLds {
    static constexpr int KS = D + 8;
    static constexpr int VS = TILE + 4;
    uint16_t k[TILE * KS];
    uint16_t vt[D * VS];
    uint64_t okmask;
};

struct PrefixDev {
    const uint8_t *kq;
    const uint16_t *ks, *kz;
    const uint8_t *vq;
    const uint16_t *vs, *vz;
    const void *kf, *vf;
    const uint8_t *mask;
    int64_t skq[4], sks[3], svq[4], svs[3], skf[3], svf[3];
    // the (b, h) strides of kq, ks (and kz), vq, vs (and vz), kf, vf as 32-bit values, set
    // when every lane's offset b * s[0] + h * s[1] fits in 31 bits (off32): the lane bases
    // then take 32-bit scalar multiplies instead of 64-bit ones in every wave
    int32_t lo32[6][2];
    int nq, nf, fdtype, off32;
};

inline PrefixDev prefix_dev(const ma_prefix *p, int B, int H) {
    PrefixDev a;
    a.kq = (const uint8_t *)p->kq;
    a.ks = (const uint16_t *)p->ks;
    a.kz = (const uint16_t *)p->kz;
    a.vq = (const uint8_t *)p->vq;
    a.vs = (const uint16_t *)p->vs;
    a.vz = (const uint16_t *)p->vz;
    a.kf = p->kf;
    a.vf = p->vf;
    a.mask = p->mask;
    for (int i = 0; i < 4; ++i) {
        a.skq[i] = p->skq[i];
        a.svq[i] = p->svq[i];
    }
    for (int i = 0; i < 3; ++i) {
        a.sks[i] = p->sks[i];
        a.svs[i] = p->svs[i];
        a.skf[i] = p->skf[i];
        a.svf[i] = p->svf[i];
    }
    a.nq = p->nq;
    a.nf = p->nf;
    a.fdtype = p->fdtype;
    const int64_t *ls[6] = {p->skq, p->sks, p->svq, p->svs, p->skf, p->svf};
    a.off32 = 1;
    for (int i = 0; i < 6; ++i) {
        const int64_t s0 = ls[i][0], s1 = ls[i][1];
        const bool fits = s0 >= 0 && s1 >= 0 && s0 <= INT32_MAX && s1 <= INT32_MAX &&
                          (int64_t)(B - 1) * s0 + (int64_t)(H - 1) * s1 <= INT32_MAX;
        a.off32 &= fits ? 1 : 0;
        a.lo32[i][0] = fits ? (int32_t)s0 : 0;
        a.lo32[i][1] = fits ? (int32_t)s1 : 0;
    }
    return a;
}

// One (batch, KV head) lane of a prefix: base pointers at token / group 0, inner strides.
struct Lane {
    const uint8_t *kq;        // + g*kq_g + d*kq_d (bytes)
    const uint16_t *ks, *kz;  // + g*ks_g + d
    const uint8_t *vq;        // + j*vq_n + c*vq_c (bytes)
    const uint16_t *vs, *vz;  // + j*vs_n + c
    const char *kf, *vf;      // 16/32-bit part, token j - nq: + (j-nq)*f_n elements
    const uint8_t *mask;      // + j, or null
    int kq_g, kq_d, ks_g, vq_n, vq_c, vs_n, kf_n, vf_n;
    int nq, ntot, fdtype, esz;  // esz: bytes per element of the 16/32-bit part
};

// LANE32: 1 -- the 32-bit lane offsets only (the caller has checked a.off32), 0 -- the
// 64-bit ones only, -1 -- chosen by a.off32 at run time.  A kernel compiled for one kind
// alone carries fewer scalar registers than one with both.
template <int LANE32 = -1>
__device__ __forceinline__ Lane make_lane(const PrefixDev &a, int b, int h, int bh) {
    Lane L;
    L.nq = a.nq;
    L.ntot = a.nq + a.nf;
    L.fdtype = a.fdtype;
    L.esz = a.fdtype == MA_F32 ? 4 : 2;
    if (LANE32 == 1 || (LANE32 < 0 && a.off32)) {
        const uint32_t okq = (uint32_t)(b * a.lo32[0][0] + h * a.lo32[0][1]);
        const uint32_t oks = (uint32_t)(b * a.lo32[1][0] + h * a.lo32[1][1]);
        const uint32_t ovq = (uint32_t)(b * a.lo32[2][0] + h * a.lo32[2][1]);
        const uint32_t ovs = (uint32_t)(b * a.lo32[3][0] + h * a.lo32[3][1]);
        const uint32_t okf = (uint32_t)(b * a.lo32[4][0] + h * a.lo32[4][1]);
        const uint32_t ovf = (uint32_t)(b * a.lo32[5][0] + h * a.lo32[5][1]);
        L.kq = a.kq + okq;
        L.ks = a.ks + oks;
        L.kz = a.kz + oks;
        L.vq = a.vq + ovq;
        L.vs = a.vs + ovs;
        L.vz = a.vz + ovs;
        L.kf = (const char *)a.kf + (uint64_t)okf * L.esz;
        L.vf = (const char *)a.vf + (uint64_t)ovf * L.esz;
    } else {
        L.kq = a.kq + b * a.skq[0] + h * a.skq[1];
        L.ks = a.ks + b * a.sks[0] + h * a.sks[1];
        L.kz = a.kz + b * a.sks[0] + h * a.sks[1];
        L.vq = a.vq + b * a.svq[0] + h * a.svq[1];
        L.vs = a.vs + b * a.svs[0] + h * a.svs[1];
        L.vz = a.vz + b * a.svs[0] + h * a.svs[1];
        L.kf = (const char *)a.kf + (b * a.skf[0] + h * a.skf[1]) * L.esz;
        L.vf = (const char *)a.vf + (b * a.svf[0] + h * a.svf[1]) * L.esz;
    }
    L.mask = a.mask ? a.mask + (int64_t)bh * L.ntot : nullptr;
    L.kq_g = (int)a.skq[2];
    L.kq_d = (int)a.skq[3];
    L.ks_g = (int)a.sks[2];
    L.vq_n = (int)a.svq[2];
    L.vq_c = (int)a.svq[3];
    L.vs_n = (int)a.svs[2];
    L.kf_n = (int)a.skf[2];
    L.vf_n = (int)a.svf[2];
    return L;
}

// A plain [B, H, n, D] 16/32-bit operand of one lane (the current block).
struct Dense {
    const char *base;
    int sn;  // elements per token
    int dtype, esz;
};

__device__ __forceinline__ Dense dense_lane(const void *ptr, const int64_t *s, int dtype, int b, int h) {
    Dense r;
    r.dtype = dtype;
    r.esz = dtype == MA_F32 ? 4 : 2;
    r.base = ptr ? (const char *)ptr + (b * s[0] + h * s[1]) * r.esz : nullptr;
    r.sn = (int)s[2];
    return r;
}

enum TileKind { TK_PACKED = 0, TK_DENSE = 1, TK_MIXED = 2 };

// kind of the prefix tile [n0, min(n0+64, end))
__device__ __forceinline__ int prefix_tile_kind(int nq, int n0, int end) {
    const int hi = min(n0 + TILE, end);
    if (hi <= nq) return TK_PACKED;
    if (n0 >= nq) return TK_DENSE;
    return TK_MIXED;
}

// Per-thread register block of one staged tile: NW payload words and flags (bit 0/1:
// token 0/1 of a V item live; bit 8: this wave-0 lane's token usable).
template <int NW>
struct PrefetchT {
    uint32_t w[NW];
    uint32_t flags;
};
using PfPacked = PrefetchT<6>;
using PfDense = PrefetchT<16>;

// 8 consecutive elements at byte address p of a 16/32-bit tensor, as bf16
__device__ __forceinline__ bf16x8_t load8_bf16(const char *p, int dtype) {
    if (dtype == MA_BF16) return *(const bf16x8_t *)p;
    return ma_load8_as_bf16(p, 0, dtype);
}

// Per-thread staging offsets, computed once per workgroup (bytes / elements).
struct ItemOffsets {
    uint32_t a, b;  // packed: code-row offset, scale offset; dense: K item 0 / 1 byte offsets
    uint32_t c;     // dense: V item byte offset (token 2tp, chunk)
};

template <int D>
__device__ __forceinline__ ItemOffsets packed_offsets(const Lane &L, int tid) {
    constexpr int KITEMS = 2 * D;
    ItemOffsets o{0u, 0u, 0u};
    if (tid < KITEMS) {
        const int dp = tid % (D / 2), th = (tid / (D / 2)) & 1, gl = tid / D;
        o.a = gl * L.kq_g + 2 * dp * L.kq_d + th * 8;
        o.b = gl * L.ks_g + 2 * dp;
    } else if (tid < 2 * KITEMS) {
        const int u = tid - KITEMS;
        const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
        o.a = 2 * tp * L.vq_n + cg * L.vq_c + ch * 8;
        o.b = 2 * tp * L.vs_n + cg;
    }
    return o;
}

template <int D>
__device__ __forceinline__ ItemOffsets dense_offsets(int sn_k, int sn_v, int esz, int tid) {
    constexpr int KITEMS = TILE * D / 8;
    ItemOffsets o{0u, 0u, 0u};
    {
        const int it = tid;
        const int t = it / (D / 8), chk = it % (D / 8);
        o.a = (t * sn_k + chk * 8) * esz;
    }
    {
        const int it = tid + NT;
        const int t = (it < KITEMS ? it : 0) / (D / 8), chk = it % (D / 8);
        o.b = (t * sn_k + chk * 8) * esz;
    }
    {
        const int tp = tid % (TILE / 2), chk = (tid / (TILE / 2)) % (D / 8);
        o.c = (2 * tp * sn_v + chk * 8) * esz;
    }
    return o;
}

__device__ __forceinline__ bool lane_live(const Lane &L, int j, int end) {
    bool ok = j < end;
    if (L.mask) ok = ok && L.mask[min(j, L.ntot - 1)] != 0;
    return ok;
}

// ---------------------------------------------------------------- packed int4 tiles
template <int D, bool WITH_V>
__device__ __forceinline__ void load_packed(PfPacked &pf, const Lane &L, const ItemOffsets &o, int n0, int end,
                                            int tid) {
    constexpr int KITEMS = 2 * D;
    pf.flags = 0;
    if (tid < TILE && lane_live(L, n0 + tid, end)) pf.flags |= 256u;
    const bool full = n0 + TILE <= end;
    if (tid < KITEMS) {
        const int gl = tid / D;
        const bool gok = full || n0 + gl * KGRP < end;
        // group past the end (partial tiles only): read group 0 of the lane, then zero it
        const int64_t gbase = gok ? (int64_t)(n0 / KGRP) * L.kq_g : -(int64_t)gl * L.kq_g;
        const int64_t sbase = gok ? (int64_t)(n0 / KGRP) * L.ks_g : -(int64_t)gl * L.ks_g;
        const uint8_t *r0 = L.kq + gbase + o.a;
        const uint2 x0 = *(const uint2 *)r0;
        const uint2 x1 = *(const uint2 *)(r0 + L.kq_d);
        const uint32_t sc = *(const uint32_t *)(L.ks + sbase + o.b), zp = *(const uint32_t *)(L.kz + sbase + o.b);
        pf.w[0] = gok ? x0.x : 0u;
        pf.w[1] = gok ? x0.y : 0u;
        pf.w[2] = gok ? x1.x : 0u;
        pf.w[3] = gok ? x1.y : 0u;
        pf.w[4] = gok ? sc : 0u;
        pf.w[5] = gok ? zp : 0u;
    } else if (WITH_V && tid < 2 * KITEMS) {
        const int u = tid - KITEMS;
        const int tp = u & 31;
        const int j = n0 + 2 * tp;
        const bool l0 = lane_live(L, j, end), l1 = lane_live(L, j + 1, end);
        pf.flags |= (l0 ? 1u : 0u) | (l1 ? 2u : 0u);
        uint2 x0, x1;
        uint32_t s0, s1, z0, z1;
        if (full) {  // affine addresses
            const uint8_t *p = L.vq + (int64_t)n0 * L.vq_n + o.a;
            x0 = *(const uint2 *)p;
            x1 = *(const uint2 *)(p + L.vq_n);
            const int64_t so = (int64_t)n0 * L.vs_n + o.b;
            s0 = L.vs[so];
            z0 = L.vz[so];
            s1 = L.vs[so + L.vs_n];
            z1 = L.vz[so + L.vs_n];
        } else {  // clamped token indices keep every load valid
            const int ch = (u >> 5) & 1, cg = u >> 6;
            const int j0 = min(j, L.nq - 1), j1 = min(j + 1, L.nq - 1);
            const uint8_t *p = L.vq + cg * L.vq_c + ch * 8;
            x0 = *(const uint2 *)(p + (int64_t)j0 * L.vq_n);
            x1 = *(const uint2 *)(p + (int64_t)j1 * L.vq_n);
            s0 = L.vs[(int64_t)j0 * L.vs_n + cg];
            z0 = L.vz[(int64_t)j0 * L.vs_n + cg];
            s1 = L.vs[(int64_t)j1 * L.vs_n + cg];
            z1 = L.vz[(int64_t)j1 * L.vs_n + cg];
        }
        pf.w[0] = l0 ? x0.x : 0u;
        pf.w[1] = l0 ? x0.y : 0u;
        pf.w[2] = l1 ? x1.x : 0u;
        pf.w[3] = l1 ? x1.y : 0u;
        pf.w[4] = (l0 ? s0 : 0u) | ((l1 ? s1 : 0u) << 16);
        pf.w[5] = (l0 ? z0 : 0u) | ((l1 ? z1 : 0u) << 16);
    }
}

template <int D, bool WITH_V>
__device__ __forceinline__ void store_packed(TileLds<D> &T, const PfPacked &pf, int tid) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    constexpr int KITEMS = 2 * D;
    if (tid < KITEMS) {
        const int dp = tid % (D / 2), th = (tid / (D / 2)) & 1, gl = tid / D;
        const float s0 = ma_f16_to_f32(pf.w[4] & 0xffff), s1 = ma_f16_to_f32(pf.w[4] >> 16);
        const float z0 = ma_f16_to_f32(pf.w[5] & 0xffff), z1 = ma_f16_to_f32(pf.w[5] >> 16);
        uint32_t *dst = (uint32_t *)&T.k[(gl * KGRP + th * 16) * KS + 2 * dp];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const uint32_t c0 = (pf.w[t >> 3] >> ((t & 7) * 4)) & 15u;
            const uint32_t c1 = (pf.w[2 + (t >> 3)] >> ((t & 7) * 4)) & 15u;
            dst[t * (KS / 2)] = ma_pack_bf16x2(ma_dq(c0, s0, z0), ma_dq(c1, s1, z1));
        }
    } else if (WITH_V && tid < 2 * KITEMS) {
        const int u = tid - KITEMS;
        const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
        const float s0 = ma_f16_to_f32(pf.w[4] & 0xffff), s1 = ma_f16_to_f32(pf.w[4] >> 16);
        const float z0 = ma_f16_to_f32(pf.w[5] & 0xffff), z1 = ma_f16_to_f32(pf.w[5] >> 16);
        uint32_t *dst = (uint32_t *)&T.vt[(cg * VGRP + ch * 16) * VS + 2 * tp];
        // dead tokens were loaded as zero codes with zero scale/zero: they stage 0.0
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const uint32_t c0 = (pf.w[c >> 3] >> ((c & 7) * 4)) & 15u;
            const uint32_t c1 = (pf.w[2 + (c >> 3)] >> ((c & 7) * 4)) & 15u;
            dst[c * (VS / 2)] = ma_pack_bf16x2(ma_dq(c0, s0, z0), ma_dq(c1, s1, z1));
        }
    }
}

// ---------------------------------------------------------------- 16/32-bit tiles
// Tokens [n0, n0+64) of `kbase`/`vbase` (byte pointers of token n0 - joff... see
// callers: the bases already point at the tile's first token), usable below `end`
// (absolute); `lane` (optional) supplies the liveness mask.
template <int D, bool WITH_V>
__device__ __forceinline__ void load_dense(PfDense &pf, const char *kbase, const char *vbase, int sn_k, int sn_v,
                                           int dtype, int esz, const ItemOffsets &o, const Lane *lane, int n0,
                                           int end, int tid) {
    constexpr int KITEMS = TILE * D / 8;      // (token, chunk)
    constexpr int VITEMS = TILE / 2 * D / 8;  // (token pair, chunk)
    constexpr int KR = (KITEMS + NT - 1) / NT;
    static_assert(KR <= 2 && VITEMS <= NT, "tile staging sized for D <= 128");
    pf.flags = 0;
    if (tid < TILE) {
        const int j = n0 + tid;
        const bool ok = lane ? lane_live(*lane, j, end) : j < end;
        if (ok) pf.flags |= 256u;
    }
    const bool full = n0 + TILE <= end;
#pragma unroll
    for (int r = 0; r < KR; ++r) {
        const int it = tid + r * NT;
        const int t = (it < KITEMS ? it : 0) / (D / 8), chk = it % (D / 8);
        bf16x8_t x;
        if (full) {
            x = load8_bf16(kbase + (r == 0 ? o.a : o.b), dtype);
        } else {
            const int tc = min(t, end - 1 - n0);  // clamped: the load is always valid
            x = load8_bf16(kbase + ((int64_t)tc * sn_k + chk * 8) * esz, dtype);
        }
        if (!(it < KITEMS && n0 + t < end)) x = bf16x8_t{};
        const uint4 u = __builtin_bit_cast(uint4, x);
        pf.w[4 * r + 0] = u.x;
        pf.w[4 * r + 1] = u.y;
        pf.w[4 * r + 2] = u.z;
        pf.w[4 * r + 3] = u.w;
    }
    if (!WITH_V) return;
    if (tid < VITEMS) {
        const int tp = tid % (TILE / 2), chk = tid / (TILE / 2);
        const int j = n0 + 2 * tp;
        const bool l0 = lane ? lane_live(*lane, j, end) : j < end;
        const bool l1 = lane ? lane_live(*lane, j + 1, end) : j + 1 < end;
        pf.flags |= (l0 ? 1u : 0u) | (l1 ? 2u : 0u);
        bf16x8_t x0, x1;
        if (full) {
            x0 = load8_bf16(vbase + o.c, dtype);
            x1 = load8_bf16(vbase + o.c + (int64_t)sn_v * esz, dtype);
        } else {
            const int t0 = min(2 * tp, end - 1 - n0), t1 = min(2 * tp + 1, end - 1 - n0);
            x0 = load8_bf16(vbase + ((int64_t)t0 * sn_v + chk * 8) * esz, dtype);
            x1 = load8_bf16(vbase + ((int64_t)t1 * sn_v + chk * 8) * esz, dtype);
        }
        if (!l0) x0 = bf16x8_t{};
        if (!l1) x1 = bf16x8_t{};
        const uint4 u0 = __builtin_bit_cast(uint4, x0), u1 = __builtin_bit_cast(uint4, x1);
        pf.w[8] = u0.x;
        pf.w[9] = u0.y;
        pf.w[10] = u0.z;
        pf.w[11] = u0.w;
        pf.w[12] = u1.x;
        pf.w[13] = u1.y;
        pf.w[14] = u1.z;
        pf.w[15] = u1.w;
    }
}

template <int D, bool WITH_V>
__device__ __forceinline__ void store_dense(TileLds<D> &T, const PfDense &pf, int tid) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    constexpr int KITEMS = TILE * D / 8;
    constexpr int VITEMS = TILE / 2 * D / 8;
#pragma unroll
    for (int r = 0; r < (KITEMS + NT - 1) / NT; ++r) {
        const int it = tid + r * NT;
        if (it < KITEMS) {
            const int t = it / (D / 8), chk = it % (D / 8);
            uint4 u = {pf.w[4 * r], pf.w[4 * r + 1], pf.w[4 * r + 2], pf.w[4 * r + 3]};
            *(uint4 *)&T.k[t * KS + chk * 8] = u;
        }
    }
    if (!WITH_V) return;
    if (tid < VITEMS) {
        const int tp = tid % (TILE / 2), chk = tid / (TILE / 2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t lo = (pf.w[8 + (e >> 1)] >> ((e & 1) * 16)) & 0xffffu;
            const uint32_t hi = (pf.w[12 + (e >> 1)] >> ((e & 1) * 16)) & 0xffffu;
            *(uint32_t *)&T.vt[(chk * 8 + e) * VS + 2 * tp] = lo | (hi << 16);
        }
    }
}

// okmask from the wave-0 flags (call before the barrier that publishes the tile)
template <class PF>
__device__ __forceinline__ void store_okmask(uint64_t &okmask, const PF &pf, int tid) {
    if (tid < TILE) {
        const uint64_t m = __ballot((pf.flags & 256u) != 0);
        if (tid == 0) okmask = m;
    }
}

// ---------------------------------------------------------------- generic path
// Synchronous element-wise staging of any prefix tile (packed groups, 16-bit groups, or
// both); used for the tile that straddles the packed / 16-bit boundary.
__device__ __forceinline__ float lane_key(const Lane &L, int j, int d) {
    if (j < L.nq) {
        const int g = j / KGRP, tt = j % KGRP;
        const uint32_t byte = L.kq[(int64_t)g * L.kq_g + (int64_t)d * L.kq_d + (tt >> 1)];
        const int64_t so = (int64_t)g * L.ks_g + d;
        return ma_dq((tt & 1) ? (byte >> 4) : (byte & 15u), ma_f16_to_f32(L.ks[so]), ma_f16_to_f32(L.kz[so]));
    }
    return ma_load_f(L.kf, (int64_t)(j - L.nq) * L.kf_n + d, L.fdtype);
}

__device__ __forceinline__ float lane_value(const Lane &L, int j, int d) {
    if (j < L.nq) {
        const int cg = d / VGRP, w = d % VGRP;
        const uint32_t byte = L.vq[(int64_t)j * L.vq_n + (int64_t)cg * L.vq_c + (w >> 1)];
        const int64_t so = (int64_t)j * L.vs_n + cg;
        return ma_dq((w & 1) ? (byte >> 4) : (byte & 15u), ma_f16_to_f32(L.vs[so]), ma_f16_to_f32(L.vz[so]));
    }
    return ma_load_f(L.vf, (int64_t)(j - L.nq) * L.vf_n + d, L.fdtype);
}

template <int D, bool WITH_V>
__device__ __forceinline__ void stage_generic(TileLds<D> &T, const Lane &L, int n0, int end, int tid) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    if (tid < TILE) {
        const uint64_t m = __ballot(lane_live(L, n0 + tid, end));
        if (tid == 0) T.okmask = m;
    }
    for (int it = tid; it < TILE * D; it += NT) {
        const int t = it / D, d = it % D;
        const int j = n0 + t;
        float kx = 0.f, vx = 0.f;
        if (j < end) {
            kx = lane_key(L, j, d);
            if (WITH_V && lane_live(L, j, end)) vx = lane_value(L, j, d);
        }
        T.k[t * KS + d] = ma_f32_to_bf16(kx);
        if (WITH_V) T.vt[d * VS + t] = ma_f32_to_bf16(vx);
    }
}

}  // namespace ma
