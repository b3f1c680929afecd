// LDS tile staging of the pipelined attention kernels: 64 tokens of one (batch, KV head)
// lane of a prefix, dequantized (packed int4) or converted (16/32-bit) to bf16 and laid
// out for the MFMA operand reads of v_mfma_f32_32x32x16_bf16:
//   K tile  Ks[t][d], row stride KS = D + 8 bf16 (68 or 36 dwords, 4 mod 32): a lane's
//           16-byte fragment K[t][8j..8j+7] -- 8 lanes of a ds_read_b128 phase hit 8
//           disjoint 4-bank groups.
//   V tile  Vt[d][c], row stride VS = 64 + 8 bf16 (36 dwords), token t stored at column
//           vcol(t): inside every 16-token chunk bits 2 and 3 of the token index are
//           swapped, which is the order in which the probabilities P^T come out of the
//           S^T accumulator (element i of a 32-token S^T half <-> token 8(i/4) + 4h + i%4
//           for lane half h), so lane half h reads its 8 k-slots as ONE 16-byte fragment.
// Dead or out-of-range tokens are staged as zero values (never NaN from stale slots);
// their keys are masked by the tile's live-token mask instead.
//
// Staging is split between "K lanes" and "V lanes" (KL each) so that K and V of a tile
// can be staged in different pipeline iterations: load_*() issues the global loads of one
// tile into a per-lane register block, store_*() dequantizes it into LDS.  Items:
//   packed K  (key group gl, channel pair dp, 16-token half th): 2 x 8 code bytes + the
//             two channels' f16 scale and zero                          -> 2*D items
//   packed V  (token pair tp, channel group cg, 16-channel half ch): 2 x 8 code bytes +
//             the two tokens' f16 scale and zero                        -> 2*D items
//   16-bit K  (token, 8-channel chunk): 16 bytes                         -> 8*D items
//   16-bit V  (token pair, 8-channel chunk): 2 x 16 bytes                -> 4*D items
#pragma once

#include "ma_tile.h"

namespace ma {

template <int D>
struct KTileL {
    static constexpr int KS = D + 8;
    uint16_t k[TILE * KS];
};

template <int D>
struct VTileL {
    static constexpr int VS = TILE + 8;
    uint16_t vt[D * VS];
};

// column of token t (0..63) inside a V^T row
__device__ __forceinline__ int vcol(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }

enum { ST_PACKED = 0, ST_DENSE = 1 };

// staging lanes per role
template <int KLANES, int D, int SRC>
struct StageShape {
    static constexpr int NK = SRC == ST_PACKED ? 2 * D : TILE * D / 8;        // K items per tile
    static constexpr int NV = SRC == ST_PACKED ? 2 * D : TILE / 2 * D / 8;    // V items per tile
    static constexpr int KPL = (NK + KLANES - 1) / KLANES;                   // items per K lane
    static constexpr int VPL = (NV + KLANES - 1) / KLANES;                   // items per V lane
    static constexpr int NWK = SRC == ST_PACKED ? 6 * KPL : 4 * KPL;
    static constexpr int NWV = 8 * VPL;
    static constexpr int NW = NWK > NWV ? NWK : NWV;
};

template <int NW>
struct StageRegs {
    uint32_t w[NW];
    uint32_t flags;   // K lanes: bit 8 = this lane's token (lane < 64) usable; V lanes: bit 2i/2i+1 = tokens live
};

// element t (0..7) of a code word split by nibble_bytes, as float
template <int T>
__device__ __forceinline__ float code_f32(uint32_t even, uint32_t odd) {
    return ma_ubyte_f32<T / 2>((T & 1) ? odd : even);
}
// the 8 dequantized elements of a code word, two code words (two channels or two tokens)
// at a time, packed as bf16 pairs: out[t] = (element t of w0, element t of w1)
__device__ __forceinline__ void dq8x2(uint32_t w0, uint32_t w1, float s0, float z0, float s1, float z1,
                                      uint32_t (&out)[8]) {
    uint32_t e0, o0, e1, o1;
    ma_nibble_bytes(w0, e0, o0);
    ma_nibble_bytes(w1, e1, o1);
    out[0] = ma_pack_bf16x2(__builtin_fmaf(code_f32<0>(e0, o0), s0, z0), __builtin_fmaf(code_f32<0>(e1, o1), s1, z1));
    out[1] = ma_pack_bf16x2(__builtin_fmaf(code_f32<1>(e0, o0), s0, z0), __builtin_fmaf(code_f32<1>(e1, o1), s1, z1));
    out[2] = ma_pack_bf16x2(__builtin_fmaf(code_f32<2>(e0, o0), s0, z0), __builtin_fmaf(code_f32<2>(e1, o1), s1, z1));
    out[3] = ma_pack_bf16x2(__builtin_fmaf(code_f32<3>(e0, o0), s0, z0), __builtin_fmaf(code_f32<3>(e1, o1), s1, z1));
    out[4] = ma_pack_bf16x2(__builtin_fmaf(code_f32<4>(e0, o0), s0, z0), __builtin_fmaf(code_f32<4>(e1, o1), s1, z1));
    out[5] = ma_pack_bf16x2(__builtin_fmaf(code_f32<5>(e0, o0), s0, z0), __builtin_fmaf(code_f32<5>(e1, o1), s1, z1));
    out[6] = ma_pack_bf16x2(__builtin_fmaf(code_f32<6>(e0, o0), s0, z0), __builtin_fmaf(code_f32<6>(e1, o1), s1, z1));
    out[7] = ma_pack_bf16x2(__builtin_fmaf(code_f32<7>(e0, o0), s0, z0), __builtin_fmaf(code_f32<7>(e1, o1), s1, z1));
}

// ------------------------------------------------------------------ packed K
// item u: gl = u / D, th = (u / (D/2)) & 1, dp = u % (D/2)
template <int D>
__device__ __forceinline__ void load_k_packed(uint32_t *w, const Lane &L, int u, int n0, int end) {
    const int dp = u % (D / 2), th = (u / (D / 2)) & 1, gl = u / D;
    const bool full = n0 + TILE <= end;
    const bool gok = full || n0 + gl * KGRP < end;
    const int g = gok ? n0 / KGRP + gl : 0;       // a group past the end reads group 0, then zeroes
    const uint8_t *r0 = L.kq + (int64_t)g * L.kq_g + (int64_t)(2 * dp) * L.kq_d + th * 8;
    const uint2 x0 = *(const uint2 *)r0;
    const uint2 x1 = *(const uint2 *)(r0 + L.kq_d);
    const int64_t so = (int64_t)g * L.ks_g + 2 * dp;
    const uint32_t sc = *(const uint32_t *)(L.ks + so), zp = *(const uint32_t *)(L.kz + so);
    w[0] = gok ? x0.x : 0u;
    w[1] = gok ? x0.y : 0u;
    w[2] = gok ? x1.x : 0u;
    w[3] = gok ? x1.y : 0u;
    w[4] = gok ? sc : 0u;
    w[5] = gok ? zp : 0u;
}

template <int D>
__device__ __forceinline__ void store_k_packed(uint16_t *Ks, const uint32_t *w, int u) {
    constexpr int KS = D + 8;
    const int dp = u % (D / 2), th = (u / (D / 2)) & 1, gl = u / D;
    const float s0 = ma_f16_to_f32(w[4] & 0xffff), s1 = ma_f16_to_f32(w[4] >> 16);
    const float z0 = ma_f16_to_f32(w[5] & 0xffff), z1 = ma_f16_to_f32(w[5] >> 16);
    uint32_t *dst = (uint32_t *)&Ks[(gl * KGRP + th * 16) * KS + 2 * dp];
#pragma unroll
    for (int q = 0; q < 2; ++q) {   // code word q: tokens 8q .. 8q+7 of the half
        uint32_t pk[8];
        dq8x2(w[q], w[2 + q], s0, z0, s1, z1, pk);
#pragma unroll
        for (int t = 0; t < 8; ++t) dst[(8 * q + t) * (KS / 2)] = pk[t];
    }
}

// Whole-tile fast path (a full 64-token tile of packed groups, no slot mask): an item's
// offsets from the tile's first key group are fixed per lane, so a tile moves only the
// wave-uniform base pointers (no per-tile 64-bit index arithmetic, clamps or liveness).
template <int D>
__device__ __forceinline__ uint2 k_item_offsets(const Lane &L, int u) {
    const int dp = u % (D / 2), th = (u / (D / 2)) & 1, gl = u / D;
    return uint2{(uint32_t)(gl * L.kq_g + 2 * dp * L.kq_d + th * 8), (uint32_t)(gl * L.ks_g + 2 * dp)};
}
// the words of load_k_packed for the tile whose first key group starts at kq / ks / kz
__device__ __forceinline__ void load_k_packed_fast(uint32_t *w, const uint8_t *kq, const uint16_t *ks,
                                                   const uint16_t *kz, int kq_d, uint2 o) {
    const uint2 x0 = *(const uint2 *)(kq + o.x);
    const uint2 x1 = *(const uint2 *)(kq + o.x + kq_d);
    w[0] = x0.x;
    w[1] = x0.y;
    w[2] = x1.x;
    w[3] = x1.y;
    w[4] = *(const uint32_t *)(ks + o.y);
    w[5] = *(const uint32_t *)(kz + o.y);
}

// ------------------------------------------------------------------ packed V
// item u: tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6; tokens 2tp, 2tp+1
template <int D>
__device__ __forceinline__ void load_v_packed(uint32_t *w, uint32_t &flags, const Lane &L, int u, int n0, int end) {
    const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
    const int j = n0 + 2 * tp;
    const bool l0 = lane_live(L, j, end), l1 = lane_live(L, j + 1, end);
    // clamped token indices keep every load valid on partial tiles
    const int j0 = min(j, L.nq - 1), j1 = min(j + 1, L.nq - 1);
    const uint8_t *p = L.vq + cg * L.vq_c + ch * 8;
    const uint2 x0 = *(const uint2 *)(p + (int64_t)j0 * L.vq_n);
    const uint2 x1 = *(const uint2 *)(p + (int64_t)j1 * L.vq_n);
    const uint32_t s0 = L.vs[(int64_t)j0 * L.vs_n + cg], z0 = L.vz[(int64_t)j0 * L.vs_n + cg];
    const uint32_t s1 = L.vs[(int64_t)j1 * L.vs_n + cg], z1 = L.vz[(int64_t)j1 * L.vs_n + cg];
    w[0] = l0 ? x0.x : 0u;
    w[1] = l0 ? x0.y : 0u;
    w[2] = l1 ? x1.x : 0u;
    w[3] = l1 ? x1.y : 0u;
    w[4] = l0 ? s0 : 0u;
    w[5] = l1 ? s1 : 0u;
    w[6] = l0 ? z0 : 0u;
    w[7] = l1 ? z1 : 0u;
    flags = (l0 ? 1u : 0u) | (l1 ? 2u : 0u);
}

// whole-tile fast path of load_v_packed (both tokens live)
template <int D>
__device__ __forceinline__ uint2 v_item_offsets(const Lane &L, int u) {
    const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
    return uint2{(uint32_t)(2 * tp * L.vq_n + cg * L.vq_c + ch * 8), (uint32_t)(2 * tp * L.vs_n + cg)};
}
// (every loaded value goes to a word of its own: combining the 16-bit scales here would
// make the wave wait for the loads where they are issued, a tile ahead of their use)
__device__ __forceinline__ void load_v_packed_fast(uint32_t *w, const uint8_t *vq, const uint16_t *vs,
                                                   const uint16_t *vz, int vq_n, int vs_n, uint2 o) {
    const uint2 x0 = *(const uint2 *)(vq + o.x);
    const uint2 x1 = *(const uint2 *)(vq + o.x + vq_n);
    w[0] = x0.x;
    w[1] = x0.y;
    w[2] = x1.x;
    w[3] = x1.y;
    w[4] = vs[o.y];
    w[5] = vs[o.y + vs_n];
    w[6] = vz[o.y];
    w[7] = vz[o.y + vs_n];
}

template <int D>
__device__ __forceinline__ void store_v_packed(uint16_t *Vt, const uint32_t *w, int u) {
    constexpr int VS = TILE + 8;
    const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
    const float s0 = ma_f16_to_f32((uint16_t)w[4]), s1 = ma_f16_to_f32((uint16_t)w[5]);
    const float z0 = ma_f16_to_f32((uint16_t)w[6]), z1 = ma_f16_to_f32((uint16_t)w[7]);
    uint32_t *dst = (uint32_t *)&Vt[(cg * VGRP + ch * 16) * VS + vcol(2 * tp)];
#pragma unroll
    for (int q = 0; q < 2; ++q) {   // code word q: channels 8q .. 8q+7 of the half
        uint32_t pk[8];
        dq8x2(w[q], w[2 + q], s0, z0, s1, z1, pk);
#pragma unroll
        for (int c = 0; c < 8; ++c) dst[(8 * q + c) * (VS / 2)] = pk[c];
    }
}

// ------------------------------------------------------------------ 16/32-bit K and V
// base: byte pointer of token 0 of the tile; sn: elements per token; tokens usable below
// `valid` (relative).  The loads keep bf16 and f16 words as stored (token indices clamped
// into the tile, so every load is valid); the conversion to bf16 and the zeroing of
// unusable or dead tokens happen when the words are staged, so the loads of a prefetched
// tile are not waited on where they are issued.  f32 sources are converted at load.
__device__ __forceinline__ uint4 load8_raw(const char *p, int dtype) {
    if (dtype == MA_F32) return __builtin_bit_cast(uint4, ma_load8_as_bf16(p, 0, MA_F32));
    return *(const uint4 *)p;
}
// the 8 elements of a raw item as bf16 pairs, zero when !ok
__device__ __forceinline__ uint4 stage8(uint4 w, int dtype, bool ok) {
    if (!ok) return uint4{0u, 0u, 0u, 0u};
    if (dtype == MA_F16) {   // f16 keys and values enter the MFMAs as bf16 (splitk.py:139, 152)
        const uint32_t x[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = ma_pack_bf16x2(ma_f16_to_f32(x[e] & 0xffff), ma_f16_to_f32(x[e] >> 16));
        return uint4{o[0], o[1], o[2], o[3]};
    }
    return w;
}

// item u of a K tile: token u / (D/8), 8 channels; returns whether the token is below `valid`
template <int D>
__device__ __forceinline__ bool load_k_dense(uint32_t *w, const char *base, int sn, int dtype, int esz, int u,
                                             int valid) {
    const int t = u / (D / 8), chk = u % (D / 8);
    const int tc = min(t, valid - 1);
    const uint4 q = load8_raw(base + ((int64_t)tc * sn + chk * 8) * esz, dtype);
    w[0] = q.x;
    w[1] = q.y;
    w[2] = q.z;
    w[3] = q.w;
    return t < valid;
}

template <int D>
__device__ __forceinline__ void store_k_dense(uint16_t *Ks, const uint32_t *w, int u, int dtype, bool ok) {
    constexpr int KS = D + 8;
    const int t = u / (D / 8), chk = u % (D / 8);
    *(uint4 *)&Ks[t * KS + chk * 8] = stage8(uint4{w[0], w[1], w[2], w[3]}, dtype, ok);
}

// item u of a V tile: tokens 2tp, 2tp+1 (tp = u % 32), 8 channels (chunk u / 32)
template <int D>
__device__ __forceinline__ void load_v_dense(uint32_t *w, const char *base, int sn, int dtype, int esz, int u,
                                             int valid) {
    const int tp = u % (TILE / 2), chk = u / (TILE / 2);
    const int t0 = min(2 * tp, valid - 1), t1 = min(2 * tp + 1, valid - 1);
    const uint4 a = load8_raw(base + ((int64_t)t0 * sn + chk * 8) * esz, dtype);
    const uint4 b = load8_raw(base + ((int64_t)t1 * sn + chk * 8) * esz, dtype);
    w[0] = a.x;
    w[1] = a.y;
    w[2] = a.z;
    w[3] = a.w;
    w[4] = b.x;
    w[5] = b.y;
    w[6] = b.z;
    w[7] = b.w;
}

// l0, l1: the two tokens are live (dead ones are staged as zeros)
template <int D>
__device__ __forceinline__ void store_v_dense(uint16_t *Vt, const uint32_t *w, int u, int dtype, bool l0, bool l1) {
    constexpr int VS = TILE + 8;
    const int tp = u % (TILE / 2), chk = u / (TILE / 2);
    const int col = vcol(2 * tp);
    const uint4 a = stage8(uint4{w[0], w[1], w[2], w[3]}, dtype, l0);
    const uint4 b = stage8(uint4{w[4], w[5], w[6], w[7]}, dtype, l1);
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t lo = (wa[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        const uint32_t hi = (wb[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        *(uint32_t *)&Vt[(chk * 8 + e) * VS + col] = lo | (hi << 16);
    }
}

// ------------------------------------------------------------------ element-wise staging
// Synchronous staging of any prefix tile (the one straddling the packed / 16-bit
// boundary, and 16-bit tail tiles of a packed prefix): lanes [0, nl) of the role.
template <int D>
__device__ __forceinline__ void stage_k_generic(uint16_t *Ks, const Lane &L, int n0, int end, int lane, int nl) {
    constexpr int KS = D + 8;
    for (int it = lane; it < TILE * D; it += nl) {
        const int t = it / D, d = it % D;
        const int j = n0 + t;
        Ks[t * KS + d] = ma_f32_to_bf16(j < end ? lane_key(L, j, d) : 0.f);
    }
}

template <int D>
__device__ __forceinline__ void stage_v_generic(uint16_t *Vt, const Lane &L, int n0, int end, int lane, int nl) {
    constexpr int VS = TILE + 8;
    for (int it = lane; it < TILE * D; it += nl) {
        const int t = it % TILE, d = it / TILE;
        const int j = n0 + t;
        Vt[d * VS + vcol(t)] = ma_f32_to_bf16(lane_live(L, j, end) ? lane_value(L, j, d) : 0.f);
    }
}

}  // namespace ma
