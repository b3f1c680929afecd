// LDS tile staging shared by the split-K attention and the score pass: 64 prefix
// tokens of one (batch, KV head) lane, dequantized (packed int4) or converted (16/32-bit)
// to bf16, laid out for the MFMA operand reads:
//   Ks[t][d]  (row stride KS = D + 8 bf16)  -> 16-byte A/B fragments along d
//   Vt[d][t]  (row stride VS = 64 + 4 bf16) -> 8-byte fragments along tokens
// Tokens outside the tile's range or dead (mask 0) are staged as zeros (values) and
// cleared in okmask (bit t = token t usable), so neither garbage nor NaN of an evicted
// slot can reach an accumulator.
#pragma once

#include "ma_common.h"

namespace ma {

constexpr int TILE = 64;
constexpr int KGRP = 32;
constexpr int VGRP = 32;

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
    int nq, nf, fdtype;
};

inline PrefixDev prefix_dev(const ma_prefix *p) {
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
    return a;
}

// Stage prefix tokens [n0, n0 + 64) of lane (b, h) into the tile; tokens >= end are
// invalid.  WITH_V = false skips V.  All threads of the block participate.
template <int D, bool WITH_V>
__device__ __forceinline__ void stage_prefix_tile(TileLds<D> &L, const PrefixDev &a, int b, int h, int bh, int n0,
                                                  int end, int tid, int nthreads) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    const int ntot = a.nq + a.nf;
    if (tid < TILE) {  // wave 0: one lane per token
        const int j = n0 + tid;
        bool ok = j < end;
        if (ok && a.mask) ok = a.mask[(int64_t)bh * ntot + j] != 0;
        const uint64_t m = __ballot(ok);
        if (tid == 0) L.okmask = m;
    }
    // ---- packed keys: item = (group in tile, channel pair)
    for (int it = tid; it < 2 * (D / 2); it += nthreads) {
        const int gl = it / (D / 2), dp = it % (D / 2);
        const int t0 = n0 + gl * KGRP;
        if (t0 >= a.nq || t0 >= end) continue;
        const int g = t0 / KGRP;
        const uint8_t *r0 = a.kq + b * a.skq[0] + h * a.skq[1] + (int64_t)g * a.skq[2] + (int64_t)(2 * dp) * a.skq[3];
        uint4 w0 = *(const uint4 *)r0;
        uint4 w1 = *(const uint4 *)(r0 + a.skq[3]);
        const int64_t so = b * a.sks[0] + h * a.sks[1] + (int64_t)g * a.sks[2] + 2 * dp;
        const uint32_t sc2 = *(const uint32_t *)(a.ks + so), zp2 = *(const uint32_t *)(a.kz + so);
        const float s0 = ma_f16_to_f32(sc2 & 0xffff), s1 = ma_f16_to_f32(sc2 >> 16);
        const float z0 = ma_f16_to_f32(zp2 & 0xffff), z1 = ma_f16_to_f32(zp2 >> 16);
        const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
        uint32_t *dst = (uint32_t *)&L.k[(gl * KGRP) * KS + 2 * dp];
#pragma unroll
        for (int t = 0; t < KGRP; ++t) {
            const uint32_t c0 = (a0[t >> 3] >> ((t & 7) * 4)) & 15u;
            const uint32_t c1 = (a1[t >> 3] >> ((t & 7) * 4)) & 15u;
            dst[t * (KS / 2)] = ma_pack_bf16x2(ma_dq(c0, s0, z0), ma_dq(c1, s1, z1));
        }
    }
    // ---- 16/32-bit keys: item = (token, 8-channel chunk)
    for (int it = tid; it < TILE * (D / 8); it += nthreads) {
        const int t = it / (D / 8), ch = it % (D / 8);
        const int j = n0 + t;
        if (j < a.nq) continue;
        bf16x8_t v = {};
        if (j < end) {
            const int jf = j - a.nq;
            v = ma_load8_as_bf16(a.kf, b * a.skf[0] + h * a.skf[1] + (int64_t)jf * a.skf[2] + ch * 8, a.fdtype);
        }
        *(bf16x8_t *)&L.k[t * KS + ch * 8] = v;
    }
    // zero key rows of a packed group that lies past `end`
    for (int it = tid; it < TILE * (D / 8); it += nthreads) {
        const int t = it / (D / 8), ch = it % (D / 8);
        const int j = n0 + t;
        const int t0 = n0 + (t / KGRP) * KGRP;
        if (j < a.nq && t0 >= end) *(bf16x8_t *)&L.k[t * KS + ch * 8] = bf16x8_t{};
    }
    if (!WITH_V) return;
    // ---- packed values: item = (token pair, channel group)
    for (int it = tid; it < (TILE / 2) * (D / VGRP); it += nthreads) {
        const int tp = it % (TILE / 2), cg = it / (TILE / 2);
        const int j = n0 + 2 * tp;
        if (j >= a.nq) continue;
        const bool ok0 = j < end, ok1 = j + 1 < end;
        uint32_t a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
        float s0 = 0.f, z0 = 0.f, s1 = 0.f, z1 = 0.f;
        const uint8_t *base = a.vq + b * a.svq[0] + h * a.svq[1] + (int64_t)cg * a.svq[3];
        const int64_t sbase = b * a.svs[0] + h * a.svs[1] + cg;
        if (ok0) {
            uint4 w = *(const uint4 *)(base + (int64_t)j * a.svq[2]);
            a0[0] = w.x; a0[1] = w.y; a0[2] = w.z; a0[3] = w.w;
            s0 = ma_f16_to_f32(a.vs[sbase + (int64_t)j * a.svs[2]]);
            z0 = ma_f16_to_f32(a.vz[sbase + (int64_t)j * a.svs[2]]);
        }
        if (ok1) {
            uint4 w = *(const uint4 *)(base + (int64_t)(j + 1) * a.svq[2]);
            a1[0] = w.x; a1[1] = w.y; a1[2] = w.z; a1[3] = w.w;
            s1 = ma_f16_to_f32(a.vs[sbase + (int64_t)(j + 1) * a.svs[2]]);
            z1 = ma_f16_to_f32(a.vz[sbase + (int64_t)(j + 1) * a.svs[2]]);
        }
        // dead slots stage zeros (their codes may be stale)
        const bool live0 = ok0 && (!a.mask || a.mask[(int64_t)bh * ntot + j]);
        const bool live1 = ok1 && (!a.mask || a.mask[(int64_t)bh * ntot + j + 1]);
        // rotate the channel order across the two half-waves to spread LDS banks
        const int rot = (tid & 32) ? 16 : 0;
#pragma unroll
        for (int cc = 0; cc < VGRP; ++cc) {
            const int c = (cc + rot) & (VGRP - 1);
            const uint32_t c0 = (a0[c >> 3] >> ((c & 7) * 4)) & 15u;
            const uint32_t c1 = (a1[c >> 3] >> ((c & 7) * 4)) & 15u;
            const float x0 = live0 ? ma_dq(c0, s0, z0) : 0.f;
            const float x1 = live1 ? ma_dq(c1, s1, z1) : 0.f;
            *(uint32_t *)&L.vt[(cg * VGRP + c) * VS + 2 * tp] = ma_pack_bf16x2(x0, x1);
        }
    }
    // ---- 16/32-bit values: item = (token pair, 8-channel chunk)
    for (int it = tid; it < (TILE / 2) * (D / 8); it += nthreads) {
        const int tp = it % (TILE / 2), ch = it / (TILE / 2);
        const int j = n0 + 2 * tp;
        if (j < a.nq) continue;
        bf16x8_t v0 = {}, v1 = {};
        const int64_t base = b * a.svf[0] + h * a.svf[1] + ch * 8;
        const bool live0 = j < end && (!a.mask || a.mask[(int64_t)bh * ntot + j]);
        const bool live1 = j + 1 < end && (!a.mask || a.mask[(int64_t)bh * ntot + j + 1]);
        if (live0) v0 = ma_load8_as_bf16(a.vf, base + (int64_t)(j - a.nq) * a.svf[2], a.fdtype);
        if (live1) v1 = ma_load8_as_bf16(a.vf, base + (int64_t)(j + 1 - a.nq) * a.svf[2], a.fdtype);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            bf16x2_t pr = {v0[e], v1[e]};
            *(bf16x2_t *)&L.vt[(ch * 8 + e) * VS + 2 * tp] = pr;
        }
    }
}

// Stage current-block tokens [n0, n0 + 64) (plain [B,H,Tc,D] tensors) into the tile.
template <int D>
__device__ __forceinline__ void stage_dense_tile(TileLds<D> &L, const ma_tensor4 &kc, const ma_tensor4 &vc, int b,
                                                 int h, int n0, int end, int tid, int nthreads) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    if (tid < TILE) {
        const uint64_t m = __ballot((n0 + tid) < end);
        if (tid == 0) L.okmask = m;
    }
    for (int it = tid; it < TILE * (D / 8); it += nthreads) {
        const int t = it / (D / 8), ch = it % (D / 8);
        const int j = n0 + t;
        bf16x8_t v = {};
        if (j < end) v = ma_load8_as_bf16(kc.ptr, b * kc.s[0] + h * kc.s[1] + (int64_t)j * kc.s[2] + ch * 8, kc.dtype);
        *(bf16x8_t *)&L.k[t * KS + ch * 8] = v;
    }
    for (int it = tid; it < (TILE / 2) * (D / 8); it += nthreads) {
        const int tp = it % (TILE / 2), ch = it / (TILE / 2);
        const int j = n0 + 2 * tp;
        bf16x8_t v0 = {}, v1 = {};
        const int64_t base = b * vc.s[0] + h * vc.s[1] + ch * 8;
        if (j < end) v0 = ma_load8_as_bf16(vc.ptr, base + (int64_t)j * vc.s[2], vc.dtype);
        if (j + 1 < end) v1 = ma_load8_as_bf16(vc.ptr, base + (int64_t)(j + 1) * vc.s[2], vc.dtype);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            bf16x2_t pr = {v0[e], v1[e]};
            *(bf16x2_t *)&L.vt[(ch * 8 + e) * VS + 2 * tp] = pr;
        }
    }
}

}  // namespace ma
