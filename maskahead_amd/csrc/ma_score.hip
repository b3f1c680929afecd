// Pass 2 of step 0 (the reference's prefix_scores, splitk.py:582-614, kernel 321-371):
// per prefix entry j of a KV head,
//   mass[j]  = (1/(G*T2)) * sum over the selection rows r of exp(s_rj - M_p[r]) / L_p[r]
//   score[j] = mass[j] * || v_j - centre ||          (value-aware ranking)
//
// score_kernel: workgroups of 1024 threads (16 waves, one per CU).  A "fast" workgroup
// takes a run of whole 64-token tiles of the launch's source kind (packed int4, or
// 16-bit) of one (batch, KV head) lane, software-pipelined with ONE barrier per tile and
// fixed wave roles:
//   * S waves 0 .. row_tiles-1: wave w owns selection rows 32w..32w+31, holds their Q
//     fragments and per-row constants c_r = M_p[r]*log2e + log2(L_p[r]) in registers,
//     and computes S = Q K^T of tile i with v_mfma_f32_32x32x16_bf16 (A = Q, B = K^T from
//     LDS; two independent 32-token accumulators): a lane holds ONE token and 16 rows, so
//     the sum over rows of exp2(s * scale*log2e - c_r) is 16 exp2 in registers plus one
//     exchange with lane ^ 32.  Per-(row tile, token) sums go to LDS.
//   * staging waves (the rest), tile i+1 during tile i: K items (8 tokens x 2 channels)
//     are dequantized into the other LDS K buffer; V items (one token x 16 channels) give
//     ||v - centre||^2 partials straight from registers, the D/16 items of a token
//     reduced by lane shuffles; then the loads of tile i+2 are issued, each from a
//     per-thread offset fixed for the whole run and a wave-uniform tile base.
//   * wave 15 (a staging wave) finishes tile i-1: sum over row tiles, live mask, mass and
//     score.
// "Tail" workgroups take one of the remaining tiles each (the tile that straddles a
// packed prefix's 16-bit residual, 16-bit tail tiles, a partial last tile, f32 prefixes)
// and stage it element-wise.  Both share a prologue that builds, once per workgroup, the
// selection-row tables in LDS (row of every selection row, its query offset and c_r, one
// load per row) and the value centre (mean of O_p over the selection rows, a fixed-order
// LDS reduction shared with ma_value_centre).
#include <atomic>

#include "ma_stage.h"

using namespace ma;

namespace {

constexpr int SNT = 1024;
constexpr int MAX_RT = 16;       // row tiles of 32 selection rows
constexpr int MAX_R2 = 32 * MAX_RT;
enum { SRC_PACKED = 0, SRC_DENSE = 1 };

struct ScoreArgs {
    ma_tensor4 q;
    PrefixDev pre;
    const int32_t *q_rows;   // NULL: the selection rows are block positions row0 .. row0 + T2 - 1
    int row0;
    const float *mp, *lp;
    const void *op;  // prefix-only output [B*H, R, D] (op_dtype): the value centre's source
    int op_dtype;
    float *mass, *score;
    int H, G, T, T2, R, R2, row_tiles, value;
    int vround;    // 0, or MA_BF16 / MA_F16: packed values rounded to that dtype for the distance
    int r2_total;  // selection rows of the whole call (the mean's divisor) when rows run in passes
    int accum;     // this pass adds its share to mass (passes after the first; mass only)
    int nfast;     // whole tiles of the source kind per lane: tiles [0, nfast)
    int per;       // tiles per fast workgroup
    int fast_wgs;  // fast workgroups per lane (blockIdx.x below it); then one tail tile each
    float sl2;
    // the read-set top-k's level-0 histogram of this pass's ranks (ma_topk_select_hist_ready):
    // 0 none, 1 the mass, 2 the score of every slot (dead slots -inf), counted into
    // hist[bh][key >> MA_TOPK_S0]
    int hist_rank;
    uint32_t *hist;
};

// ------------------------------------------------------------------ value centre
// centre[d] = (1/R2) * sum over rows r < R of cnt[r] * f32(op[bh, r, d]), cnt[r] = how many
// of the R2 selection rows are row r (the mean of O_p over the selection rows).  SNT
// threads: thread (slot s, chunk c) sums rows r = s, s + S, ... (ascending) of channels
// 8c..8c+7; the slots of a wave are then summed by lane exchanges (partners at xor CH, 2 CH,
// ...), and the NT / 64 wave sums in wave order -- one fixed order, shared by score_kernel
// and centre_kernel.
template <int D, int NT = SNT>
struct CentreSmem {
    static constexpr int CH = D / 8, S = NT / CH;
    float part[NT / 64][D];
};

// the slot sums acc[8] of this thread (slot tid / CH, chunk tid % CH) -> cen[0 .. D) in
// LDS (visible to the block on return; cs and cen may be any LDS)
template <int D, int NT>
__device__ __forceinline__ void centre_reduce(float (&acc)[8], CentreSmem<D, NT> &cs, float *cen, int r2) {
    constexpr int CH = D / 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = CH; o < 64; o *= 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o);
    }
    if (lane < CH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) cs.part[wave][lane * 8 + e] = acc[e];
    }
    __syncthreads();
    if (tid < D) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) t += cs.part[w][tid];
        cen[tid] = t / (float)r2;
    }
    __syncthreads();
}

// the row of selection row rr: (rr / T2) * T + clamp(q_rows[rr % T2], 0, T - 1)
__device__ __forceinline__ int sel_row(const int32_t *q_rows, int rr, int T2, int T, int *g_out, int *t_out) {
    const int g = rr / T2;
    const int t = min(max(q_rows[rr - g * T2], 0), T - 1);
    *g_out = g;
    *t_out = t;
    return g * T + t;
}

// ------------------------------------------------------------------ staging items
// Fast tiles are whole 64-token tiles of the launch's source kind.  Every item's global
// offsets are computed once per thread (32-bit, relative to the tile); per tile only the
// wave-uniform base pointers move, so the loads take a scalar base + vector offset.

// 8 nibbles of a word as floats, element i = bits 4i..4i+3 (byte masks + cvt_f32_ubyte)
__device__ __forceinline__ void nib8(uint32_t w, float *f) {
    uint32_t lo, hi;
    ma_nibble_bytes(w, lo, hi);
    f[0] = ma_ubyte_f32<0>(lo);
    f[1] = ma_ubyte_f32<0>(hi);
    f[2] = ma_ubyte_f32<1>(lo);
    f[3] = ma_ubyte_f32<1>(hi);
    f[4] = ma_ubyte_f32<2>(lo);
    f[5] = ma_ubyte_f32<2>(hi);
    f[6] = ma_ubyte_f32<3>(lo);
    f[7] = ma_ubyte_f32<3>(hi);
}

// K, packed: item u < 4D = (key group gl, 8-token quarter tq, channel pair dp), dp fastest
// (a wave's LDS writes hit 64 distinct banks).  Words: codes of channel 2dp and 2dp+1
// (8 tokens each), their f16 scales, their f16 zeros.
template <int D>
__device__ __forceinline__ uint2 kp_offsets(const Lane &L, int u) {
    const int dp = u % (D / 2), tq = (u / (D / 2)) & 3, gl = u / (2 * D);
    return uint2{(uint32_t)(gl * L.kq_g + 2 * dp * L.kq_d + tq * 4), (uint32_t)(gl * L.ks_g + 2 * dp)};
}

__device__ __forceinline__ void kp_load(uint32_t *w, const uint8_t *kq, const uint16_t *ks, const uint16_t *kz,
                                        int kq_d, uint2 o) {
    w[0] = *(const uint32_t *)(kq + o.x);
    w[1] = *(const uint32_t *)(kq + o.x + kq_d);
    w[2] = *(const uint32_t *)(ks + o.y);
    w[3] = *(const uint32_t *)(kz + o.y);
}

template <int D>
__device__ __forceinline__ void kp_store(uint16_t *Ks, const uint32_t *w, int u) {
    constexpr int KS = D + 8;
    const int dp = u % (D / 2), tq = (u / (D / 2)) & 3, gl = u / (2 * D);
    const float s0 = ma_f16_to_f32(w[2] & 0xffff), s1 = ma_f16_to_f32(w[2] >> 16);
    const float z0 = ma_f16_to_f32(w[3] & 0xffff), z1 = ma_f16_to_f32(w[3] >> 16);
    float c0[8], c1[8];
    nib8(w[0], c0);
    nib8(w[1], c1);
    uint32_t *dst = (uint32_t *)&Ks[(gl * KGRP + tq * 8) * KS + 2 * dp];
#pragma unroll
    for (int t = 0; t < 8; ++t)
        dst[t * (KS / 2)] = ma_pack_bf16x2(__builtin_fmaf(c0[t], s0, z0), __builtin_fmaf(c1[t], s1, z1));
}

// K, 16-bit: item u < 4D = (token t, 16-channel chunk); words: 32 raw bytes.
template <int D>
__device__ __forceinline__ uint32_t kd_offset(const Lane &L, int u) {
    const int t = u / (D / 16), chk = u % (D / 16);
    return (uint32_t)((t * L.kf_n + chk * 16) * 2);
}

__device__ __forceinline__ void d32_load(uint32_t *w, const char *base, uint32_t o) {
    const uint4 *p = (const uint4 *)(base + o);
    const uint4 a = p[0], b = p[1];
    w[0] = a.x;
    w[1] = a.y;
    w[2] = a.z;
    w[3] = a.w;
    w[4] = b.x;
    w[5] = b.y;
    w[6] = b.z;
    w[7] = b.w;
}

template <int D>
__device__ __forceinline__ void kd_store(uint16_t *Ks, const uint32_t *w, int u, int dtype) {
    constexpr int KS = D + 8;
    const int t = u / (D / 16), chk = u % (D / 16);
    uint4 *dst = (uint4 *)&Ks[t * KS + chk * 16];
    if (dtype == MA_BF16) {
        dst[0] = uint4{w[0], w[1], w[2], w[3]};
        dst[1] = uint4{w[4], w[5], w[6], w[7]};
    } else {  // f16 keys enter the dot as bf16 (splitk.py:139, 152)
        uint32_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            o[e] = ma_pack_bf16x2(ma_f16_to_f32(w[e] & 0xffff), ma_f16_to_f32(w[e] >> 16));
        dst[0] = uint4{o[0], o[1], o[2], o[3]};
        dst[1] = uint4{o[4], o[5], o[6], o[7]};
    }
}

// V, packed: item u < 4D = (token t, 16-channel half hq of a 32-channel group), hq fastest
// (the D/16 items of a token are adjacent lanes).  Words: 8 code bytes, f16 scale, f16 zero.
template <int D>
__device__ __forceinline__ uint2 vp_offsets(const Lane &L, int u) {
    const int t = u / (D / 16), hq = u % (D / 16), cg = hq >> 1, ch = hq & 1;
    return uint2{(uint32_t)(t * L.vq_n + cg * L.vq_c + ch * 8), (uint32_t)(t * L.vs_n + cg)};
}

// (scale and zero stay in words of their own until use: combining them here would make the
// wave wait for the loads where they are issued, one tile ahead)
__device__ __forceinline__ void vp_load(uint32_t *w, const uint8_t *vq, const uint16_t *vs, const uint16_t *vz,
                                        uint2 o) {
    const uint2 x = *(const uint2 *)(vq + o.x);
    w[0] = x.x;
    w[1] = x.y;
    w[2] = vs[o.y];
    w[3] = vz[o.y];
}

// squared distance of the item's 16 channels to the centre (cen16: those channels, LDS);
// VR: the values are first rounded to the dtype (MA_BF16 / MA_F16) of the reference's
// unpacked prefix, 0 = read as dequantized (f32)
template <int VR>
__device__ __forceinline__ float vp_dist(const uint32_t *w, const float *cen16) {
    const float s = ma_f16_to_f32((uint16_t)w[2]), z = ma_f16_to_f32((uint16_t)w[3]);
    float q[16];
    nib8(w[0], q);
    nib8(w[1], q + 8);
    float acc = 0.f;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        const f32x4_t cc = *(const f32x4_t *)&cen16[c4 * 4];
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
            float x0 = __builtin_fmaf(q[c4 * 4 + e], s, z), x1 = __builtin_fmaf(q[c4 * 4 + e + 1], s, z);
            if constexpr (VR == MA_BF16) {
                const uint32_t pk = ma_pack_bf16x2(x0, x1);
                x0 = __uint_as_float(pk << 16);
                x1 = __uint_as_float(pk & 0xffff0000u);
            } else if constexpr (VR == MA_F16) {
                x0 = ma_round_f16(x0);
                x1 = ma_round_f16(x1);
            }
            const float d0 = x0 - cc[e], d1 = x1 - cc[e + 1];
            acc = __builtin_fmaf(d0, d0, acc);
            acc = __builtin_fmaf(d1, d1, acc);
        }
    }
    return acc;
}

// V, 16-bit: item u < 4D = (token t, 16-channel chunk); words: 32 raw bytes.
template <int D>
__device__ __forceinline__ uint32_t vd_offset(const Lane &L, int u) {
    const int t = u / (D / 16), chk = u % (D / 16);
    return (uint32_t)((t * L.vf_n + chk * 16) * 2);
}

__device__ __forceinline__ float vd_dist(const uint32_t *w, const float *cen16, int dtype) {
    float acc = 0.f;
    const bool bf = dtype == MA_BF16;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        const f32x4_t cc = *(const f32x4_t *)&cen16[c4 * 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c4 * 4 + e;
            const uint32_t wd = w[c >> 1];
            // as stored (splitk.py:364-369)
            const float x = bf ? __uint_as_float((c & 1) ? (wd & 0xffff0000u) : (wd << 16))
                               : ma_f16_to_f32((uint16_t)(wd >> ((c & 1) * 16)));
            const float dl = x - cc[e];
            acc = __builtin_fmaf(dl, dl, acc);
        }
    }
    return acc;
}

// element-wise V distance of item u (any prefix kind; f32 prefixes keep f32 values)
template <int D>
__device__ __forceinline__ float vg_dist(const Lane &L, int u, int n0, int end, const float *cen16, int vround) {
    const int t = u / (D / 16), c0 = (u % (D / 16)) * 16;
    const int j = n0 + t;
    float acc = 0.f;
    if (j < end) {
#pragma unroll 2
        for (int c = 0; c < 16; ++c) {
            float x = lane_value(L, j, c0 + c);
            if (j < L.nq) x = vround == MA_BF16 ? ma_round_bf16(x) : vround == MA_F16 ? ma_round_f16(x) : x;
            const float dl = x - cen16[c];
            acc = __builtin_fmaf(dl, dl, acc);
        }
    }
    return acc;
}

// sum over the D/16 adjacent lanes of a token, into the token's first lane (DPP row moves)
template <int D>
__device__ __forceinline__ float token_sum(float v) {
    return ma_group_sum_first<D / 16>(v);
}

constexpr int MAX_R = 1024;   // query rows of a KV head (G * T)
// keys of KEY_TILES tiles are kept in LDS (two blocks, so one is counted into the level-0
// histogram while the next is written); a workgroup's keys are counted by all of its
// threads at once, once per block and after the last tile
constexpr int KEY_TILES = 64;

template <int D, int NT>
struct ScoreSmem {
    union {
        KTileL<D> kt[2];
        CentreSmem<D, NT> cs;
    } u;
    float red[2][2 * MAX_RT][TILE / 2];  // per (row tile, 32-token half) unit: its token sums
    float dist[3][TILE];
    float cen[D];
    float crow[MAX_R2];         // per selection row: M_p*log2e + log2(L_p), +inf when unused
    int rrow[MAX_R2];           // per selection row: its row in [0, R)
    int qoff[MAX_R2];           // per selection row: element offset of its query from (b, h*G, 0)
    int cnt[MAX_R];             // per row r < R: how many selection rows it is
    float rowc[MAX_R];          // per row r < R: M_p*log2e + log2(L_p), +inf when L_p = 0
    int qr[MAX_R2];             // q_rows (T2 <= MAX_R2 entries)
    union {
        uint4 qx[MAX_RT / 2][D / 16][64];   // (prologue) Q fragments of each row tile
        struct {
            uint32_t hist[MA_TOPK_H0];       // (tile loop) the workgroup's level-0 histogram
            uint32_t keys[2][KEY_TILES * TILE];
        } hk;
    } q;
};

// Every wave does both jobs, in lock step: S units (a 32-row tile x a 32-token half of a
// tile, or both halves) and staging items (thread t stages items t, t + NT, ...: K items
// [0, 4D), then V items [4D, 8D)).  HALVES: token halves per S unit.  NT = 1024 (one
// workgroup per CU, units of half a tile for up to 16 row tiles) or 512 (two workgroups per
// CU, so one's memory waits overlap the other's work; up to 8 row tiles, whole-tile units,
// every thread stages one K item and one V item).
template <int D, int SRC, int HALVES, int NT, bool HIST, bool LANE32>
__global__ void __launch_bounds__(NT) score_kernel(ScoreArgs a) {
    __shared__ ScoreSmem<D, NT> sm;
    constexpr int NWV = NT / 64;                       // waves
    constexpr int IPT = 8 * D > NT ? 8 * D / NT : 1;   // staging items per thread
    constexpr int KS = D + 8;
    constexpr int NKS = D / 16;
    constexpr int NIK = 4 * D;                         // K items per tile
    constexpr int TPI = D / 16;                        // V items (lanes) per token
    constexpr int NW = SRC == SRC_PACKED ? 4 : 8;      // staging words per item
    constexpr int CH = D / 8;                          // 8-channel chunks of a row

    const int h = blockIdx.y, b = blockIdx.z, bh = b * a.H + h;   // (no scalar division)
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;
    const bool value = a.value;
    const float sl2 = a.sl2;
    const int row_tiles = a.row_tiles;
    const int units = HALVES == 1 ? 2 * row_tiles : row_tiles;
    const bool s_wave = wave < units;
    const int rt = HALVES == 1 ? (wave >> 1) : wave;   // this S unit's row tile
    const int th0 = HALVES == 1 ? (wave & 1) : 0;      // and token half
    const int end = a.pre.nq + a.pre.nf;
    const int R = a.R, R2 = a.R2, T = a.T, T2 = a.T2;
    const bool fast = (int)blockIdx.x < a.fast_wgs;
    const int tile0 = fast ? blockIdx.x * a.per : a.nfast + (blockIdx.x - a.fast_wgs);
    const int ntiles = fast ? min(a.per, a.nfast - tile0) : 1;
    if (ntiles <= 0 || tile0 * TILE >= end) return;   // uniform over the workgroup

    // ---- fast staging state: this thread's item offsets inside a tile, once
    const int ni = value ? 2 * NIK : NIK;              // staging items per tile
    // Thread t stages item (t + j NT + rot) mod (IPT NT).  When the K and V items fill the
    // threads exactly, rot = NIK puts the V items (the dearer ones: dequantization plus the
    // distance) on waves 0 .. NWV/2 - 1, whose S units come first in each SIMD's MFMA
    // order, and the K items on the later waves, so that no wave has both the latest S
    // unit and a V item.
    const int rot = (value && 2 * NIK == IPT * NT) ? NIK : 0;
    auto item = [&](int j) { return (tid + j * NT + rot) % (IPT * NT); };
    uint32_t w[IPT][NW];
    uint2 off[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) off[j] = uint2{0u, 0u};
    const uint8_t *kq0 = nullptr, *vq0 = nullptr;
    const uint16_t *ks0 = nullptr, *kz0 = nullptr, *vs0 = nullptr, *vz0 = nullptr;
    const char *kf0 = nullptr, *vf0 = nullptr;
    int64_t kq_tile = 0, ks_tile = 0, vq_tile = 0, vs_tile = 0, kf_tile = 0, vf_tile = 0;
    int kq_d = 0;
    if (fast) {
        const Lane L = make_lane<LANE32 ? 1 : 0>(a.pre, b, h, bh);
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int u = item(j);
            if (u < NIK) off[j] = SRC == SRC_PACKED ? kp_offsets<D>(L, u) : uint2{kd_offset<D>(L, u), 0u};
            else if (u < ni)
                off[j] = SRC == SRC_PACKED ? vp_offsets<D>(L, u - NIK) : uint2{vd_offset<D>(L, u - NIK), 0u};
        }
        kq0 = L.kq;
        ks0 = L.ks;
        kz0 = L.kz;
        vq0 = L.vq;
        vs0 = L.vs;
        vz0 = L.vz;
        kf0 = L.kf;
        vf0 = L.vf;
        kq_d = L.kq_d;
        kq_tile = (int64_t)(TILE / KGRP) * L.kq_g;     // bytes per tile
        ks_tile = (int64_t)(TILE / KGRP) * L.ks_g;     // elements per tile
        vq_tile = (int64_t)TILE * L.vq_n;
        vs_tile = (int64_t)TILE * L.vs_n;
        kf_tile = (int64_t)TILE * L.kf_n * 2;
        vf_tile = (int64_t)TILE * L.vf_n * 2;
    }
    // this thread's item of tile i of the run into w
    auto load = [&](int i) {
        const int64_t ti = tile0 + i;   // whole tiles: packed tile ti starts at key group 2*ti
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int u = item(j);
            if (u < NIK) {
                if constexpr (SRC == SRC_PACKED)
                    kp_load(w[j], kq0 + ti * kq_tile, ks0 + ti * ks_tile, kz0 + ti * ks_tile, kq_d, off[j]);
                else d32_load(w[j], kf0 + ti * kf_tile, off[j].x);
            } else if (u < ni) {
                if constexpr (SRC == SRC_PACKED)
                    vp_load(w[j], vq0 + ti * vq_tile, vs0 + ti * vs_tile, vz0 + ti * vs_tile, off[j]);
                else d32_load(w[j], vf0 + ti * vf_tile, off[j].x);
            }
        }
    };

    // ---- prologue: the first tile's loads, q_rows and M_p / L_p of every row at once, then
    // the selection-row tables from LDS, then Q and the value centre
    if (fast) load(0);
    // in-order selection rows (the whole block, mode "all"): every table below is arithmetic,
    // so M_p / L_p, Q and the centre's rows are loaded in the first round trip
    const bool ident = a.q_rows == nullptr;
    if (!ident && tid < T2) sm.qr[tid] = a.q_rows[tid];
    // exp(s - M) / L == exp2(s*log2e - (M*log2e + log2 L)); rows without a live prefix
    // entry (L = 0) and padding rows contribute exactly 0.  Up to MAX_R rows per KV head the
    // constants of every row come in the same round trip as q_rows; beyond (long prefill
    // chunks, mass only) each selection row reads its own M_p / L_p below.
    const bool row_table = R <= MAX_R;
    auto row_const = [&](int r) {
        const float m = a.mp[(int64_t)bh * R + r], l = a.lp[(int64_t)bh * R + r];
        return l > 0.f ? __builtin_fmaf(m, MA_LOG2E, __log2f(l)) : __builtin_inff();
    };
    // selection row rr = g * T2 + i: block position t (clamped into the block), row g * T + t
    auto sel_pos = [&](int rr, int g) {
        return min(max(ident ? a.row0 + rr - g * T2 : sm.qr[rr - g * T2], 0), T - 1);
    };
    const int rt_pad = 32 * row_tiles;
    // Q of the unit's row tile: in-order rows need no table, so their loads are issued
    // here, before the tables below wait on M_p / L_p (one round trip for all of them)
    // With two S units per row tile (HALVES == 1: one per 32-token half) each loads half of
    // the row tile's fragments (k-steps th0 * NKS/2 ..) into qf[0 .. NKS/2) and the halves
    // are exchanged through LDS before the first tile (share_q).
    bf16x8_t qf[NKS];
    constexpr int QH = HALVES == 1 ? NKS / 2 : NKS;   // fragments loaded by this unit
    auto load_q = [&](int qo) {
        const int64_t qb = b * a.q.s[0] + (int64_t)h * a.G * a.q.s[1] + (qo < 0 ? 0 : qo);
        const int ks0 = HALVES == 1 ? th0 * QH : 0;
#pragma unroll
        for (int j = 0; j < QH; ++j) qf[j] = ma_load8_as_bf16(a.q.ptr, qb + (ks0 + j) * 16 + hf * 8, a.q.dtype);
    };
    if (s_wave && ident) {
        const int rr = rt * 32 + c32, g = rr / T2;
        load_q(rr < R2 ? g * (int)a.q.s[1] + sel_pos(rr, g) * (int)a.q.s[2] : -1);
    }
    // the value centre's first batch of O_p rows (rows osl, osl + CS, ... of channels
    // 8 och .. 8 och + 7), also in flight before the tables wait
    constexpr int CB = 4;
    constexpr int CS = NT / CH;
    const int osl = tid / CH, och = tid % CH;
    uint4 craw[CB], chi[CB];
    auto load_centre = [&](int r0) {
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int64_t off_o = ((int64_t)bh * R + min(r0 + j * CS, R - 1)) * D + och * 8;
            if (a.op_dtype == MA_F32) {
                craw[j] = *(const uint4 *)((const float *)a.op + off_o);
                chi[j] = *(const uint4 *)((const float *)a.op + off_o + 4);
            } else {
                craw[j] = *(const uint4 *)((const uint16_t *)a.op + off_o);
            }
        }
    };
    if (value && osl < R) load_centre(osl);
    if (ident) {
        for (int rr = tid; rr < rt_pad; rr += NT) {
            float c = __builtin_inff();
            int row = 0, qo = -1;
            if (rr < R2) {
                const int g = rr / T2, t = sel_pos(rr, g);
                row = g * T + t;
                qo = g * (int)a.q.s[1] + t * (int)a.q.s[2];
                c = row_const(row);
            }
            sm.crow[rr] = c;
            sm.rrow[rr] = row;
            sm.qoff[rr] = qo;
        }
    } else {
        if (row_table) {
            for (int r = tid; r < R; r += NT) sm.rowc[r] = row_const(r);
            for (int r = tid; r < MAX_R; r += NT) sm.cnt[r] = 0;
        }
        __syncthreads();
        for (int rr = tid; rr < rt_pad; rr += NT) {
            float c = __builtin_inff();
            int row = 0, qo = -1;
            if (rr < R2) {
                const int g = rr / T2, t = sel_pos(rr, g);
                row = g * T + t;
                qo = g * (int)a.q.s[1] + t * (int)a.q.s[2];
                if (row_table) {
                    atomicAdd(&sm.cnt[row], 1);
                    c = sm.rowc[row];
                } else {
                    c = row_const(row);
                }
            }
            sm.crow[rr] = c;
            sm.rrow[rr] = row;
            sm.qoff[rr] = qo;
        }
        __syncthreads();
    }
    if (s_wave && !ident) load_q(sm.qoff[rt * 32 + c32]);

    // value centre: centre[d] = (1/R2) * sum over rows r of cnt[r] * f32(O_p[r][d]), rows of
    // a slot in ascending order, then slots in groups of 8, then the groups
    if (value) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        // rows osl, osl + CS, ... of channels 8 och .. 8 och + 7, in batches of CB rows whose
        // loads are in flight together (the first batch was issued before the tables); a
        // row counts as often as it is a selection row (in order: every row once); rows past
        // R count 0 (their address is clamped)
        for (int r0 = osl; r0 < R; r0 += CB * CS) {
            if (r0 != osl) load_centre(r0);
            const uint4 *raw = craw, *hi = chi;
            float wgt[CB];
#pragma unroll
            for (int j = 0; j < CB; ++j) {
                const int r = r0 + j * CS;
                const int tpos = r % T - a.row0;
                wgt[j] = r >= R ? 0.f : ident ? (tpos >= 0 && tpos < T2 ? 1.f : 0.f) : (float)sm.cnt[r];
            }
            if (a.op_dtype == MA_F32) {
                // f32 rows: 8 channels in two 16-byte halves
#pragma unroll
                for (int j = 0; j < CB; ++j) {
                    const uint32_t wv[8] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w, hi[j].x, hi[j].y, hi[j].z, hi[j].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] += wgt[j] * __uint_as_float(wv[e]);
                }
            } else {
                const bool bf = a.op_dtype == MA_BF16;
#pragma unroll
                for (int j = 0; j < CB; ++j) {
                    const uint32_t wv[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint16_t hx = (uint16_t)(wv[e >> 1] >> ((e & 1) * 16));
                        acc[e] += wgt[j] * (bf ? ma_bf16_to_f32(hx) : ma_f16_to_f32(hx));
                    }
                }
            }
        }
        centre_reduce<D, NT>(acc, sm.u.cs, sm.cen, R2);
    }
    if (s_wave) {
        // padding rows of the last row tile: zero queries (applied only now, so that the Q
        // loads and the centre's loads are in flight together)
        const int rr = rt * 32 + c32;
        if (rr >= R2) {
#pragma unroll
            for (int j = 0; j < QH; ++j) qf[j] = bf16x8_t{};
        }
        if constexpr (HALVES == 1) {
#pragma unroll
            for (int j = 0; j < QH; ++j) sm.q.qx[rt][th0 * QH + j][lane] = __builtin_bit_cast(uint4, qf[j]);
        }
    }
    // after a barrier: the other unit's half of the row tile's fragments, in k-step order
    auto share_q = [&]() {
        if constexpr (HALVES == 1) {
            if (s_wave) {
                if (th0 == 0) {
#pragma unroll
                    for (int j = 0; j < QH; ++j) qf[QH + j] = __builtin_bit_cast(bf16x8_t, sm.q.qx[rt][QH + j][lane]);
                } else {
#pragma unroll
                    for (int j = 0; j < QH; ++j) qf[QH + j] = qf[j];
#pragma unroll
                    for (int j = 0; j < QH; ++j) qf[j] = __builtin_bit_cast(bf16x8_t, sm.q.qx[rt][j][lane]);
                }
            }
        }
    };

    // ---- S unit: tile in K buffer kb into the unit's token sums red[rb]
    auto s_tile = [&](int kb, int rb) {
        const uint16_t *Ks = sm.u.kt[kb].k;
#pragma unroll
        for (int hh = 0; hh < HALVES; ++hh) {
            const int th = HALVES == 1 ? th0 : hh;
            f32x16_t sv = f32x16_t{};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const bf16x8_t kf = *(const bf16x8_t *)&Ks[(th * 32 + c32) * KS + ks * 16 + hf * 8];
                sv = ma_mfma32(qf[ks], kf, sv);
            }
            float acc = 0.f;
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                // rows 8*i4 + 4*hf + 0..3 of the row tile
                const f32x4_t c4 = *(const f32x4_t *)&sm.crow[rt * 32 + i4 * 8 + hf * 4];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i4 * 4 + e], sl2, -c4[e]));
            }
            acc = ma_sum_xor32(acc);
            if (hf == 0) sm.red[rb][rt * 2 + th][c32] = acc;
        }
    };

    const float inv_r2 = 1.0f / (float)a.r2_total;
    const int hist_rank = HIST ? a.hist_rank : 0;   // HIST: 1 or 2
    auto finish = [&](int tile, int rb, int db) {
        const int j = tile * TILE + lane;
        uint32_t key = 0u;   // 0: past the end (counted nowhere)
        if (j < end) {
            float s = 0.f;
            const int th = lane >> 5, tl = lane & 31;
            // every row tile's sum read at once (the LDS reads of a loop would each wait on
            // the previous add); unused tiles add +0, in the same order
#pragma unroll
            for (int r = 0; r < (HALVES == 1 ? MAX_RT / 2 : MAX_RT); ++r) {
                const float x = sm.red[rb][r * 2 + th][tl];
                s += r < row_tiles ? x : 0.f;
            }
            bool live = true;
            const int64_t o = (int64_t)bh * end + j;
            if (a.pre.mask) live = a.pre.mask[o] != 0;
            const float m = live ? s * inv_r2 : 0.f;
            const float mf = a.accum ? a.mass[o] + m : m;   // the mass after this pass
            a.mass[o] = mf;
            float sc = 0.f;
            if (value) {
                sc = live ? m * __builtin_sqrtf(sm.dist[db][lane]) : 0.f;
                a.score[o] = sc;
            }
            // the key ma_topk_select gives this slot under the same mask
            if constexpr (HIST) key = ma_order_key(live ? (hist_rank == 2 ? sc : mf) : -__builtin_inff());
        }
        if constexpr (HIST) {
            const int r = tile - tile0;   // tile of the run
            sm.q.hk.keys[(r / KEY_TILES) & 1][(r % KEY_TILES) * TILE + lane] = key;
        }
    };
    // level-0 histogram: cleared (its LDS is the prologue's Q exchange buffer, free after
    // the first tile's barrier), keys of block kb counted (all threads, LDS atomics), and
    // the workgroup's nonzero bins added into the row's histogram
    auto zero_hist = [&]() {
        for (int i = tid; i < MA_TOPK_H0 / 4; i += NT) ((uint4 *)sm.q.hk.hist)[i] = make_uint4(0u, 0u, 0u, 0u);
    };
    auto count_keys = [&](int kb, int tiles) {
        const uint32_t *ks = sm.q.hk.keys[kb & 1];
        for (int e = tid; e < tiles * TILE; e += NT) {
            const uint32_t key = ks[e];
            if (key) atomicAdd(&sm.q.hk.hist[key >> MA_TOPK_S0], 1u);
        }
    };
    // after the last finish: the blocks not counted in the loop (block kb is counted at
    // iteration KEY_TILES (kb + 1) + 1 when the run has it), then the flush
    auto end_hist = [&]() {
        if (ntiles == 1) zero_hist();   // (no second iteration cleared it)
        __syncthreads();
        const int last = (ntiles - 1) / KEY_TILES;
        for (int kb = ntiles >= KEY_TILES + 2 ? (ntiles - 2) / KEY_TILES : 0; kb <= last; ++kb)
            count_keys(kb, min(KEY_TILES, ntiles - KEY_TILES * kb));
        __syncthreads();
        uint32_t *gh = a.hist + (int64_t)bh * MA_TOPK_H0;
        for (int i = tid; i < MA_TOPK_H0; i += NT) {
            const uint32_t x = sm.q.hk.hist[i];
            if (x) atomicAdd(&gh[i], x);
        }
    };

    if (!fast) {
        // ---- tail workgroup: one tile, staged element-wise by every thread
        const Lane L = make_lane<LANE32 ? 1 : 0>(a.pre, b, h, bh);
        const int n0 = tile0 * TILE;
        uint16_t *Ks = sm.u.kt[0].k;
#pragma unroll 1
        for (int it = tid; it < TILE * D; it += NT) {
            const int t = it / D, d = it % D;
            const int j = n0 + t;
            Ks[t * KS + d] = ma_f32_to_bf16(j < end ? lane_key(L, j, d) : 0.f);
        }
        if (value) {
            // V items (token, 16 channels), the D/16 lanes of a token adjacent
            for (int v0 = 0; v0 < NIK; v0 += NT) {
                const int v = v0 + tid;
                float dd = v < NIK ? vg_dist<D>(L, v, n0, end, &sm.cen[(v % TPI) * 16], a.vround) : 0.f;
                dd = token_sum<D>(dd);
                if (v < NIK && v % TPI == 0) sm.dist[0][v / TPI] = dd;
            }
        }
        __syncthreads();
        share_q();
        if (s_wave) s_tile(0, 0);
        __syncthreads();
        if (wave == NWV - 1) finish(tile0, 0, 0);
        if constexpr (HIST) end_hist();
        return;
    }

    // ---- fast workgroup: this thread's item of the tile in w into K buffer kb and
    // distance buffer db
    const int vround = a.vround;
    auto stage = [&](int kb, int db) {
        uint16_t *Ks = sm.u.kt[kb].k;
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int u = item(j);
            if (u < NIK) {
                if constexpr (SRC == SRC_PACKED) kp_store<D>(Ks, w[j], u);
                else kd_store<D>(Ks, w[j], u, a.pre.fdtype);
            } else if (value && u < NIK + NIK) {
                const float *cen16 = &sm.cen[((u - NIK) % TPI) * 16];
                float dd = 0.f;
                if constexpr (SRC == SRC_PACKED)
                    dd = vround == MA_BF16 ? vp_dist<MA_BF16>(w[j], cen16)
                                           : (vround == MA_F16 ? vp_dist<MA_F16>(w[j], cen16) : vp_dist<0>(w[j], cen16));
                else dd = vd_dist(w[j], cen16, a.pre.fdtype);
                dd = token_sum<D>(dd);
                if ((u - NIK) % TPI == 0) sm.dist[db][(u - NIK) / TPI] = dd;
            }
        }
    };

    stage(0, 0);
    if (ntiles > 1) load(1);
    __syncthreads();
    share_q();

    for (int i = 0; i < ntiles; ++i) {
        if constexpr (HIST) {
            if (i == 1) zero_hist();
            // key block kb complete (its last tile finished before the last barrier)
            if (i >= KEY_TILES + 1 && (i - 1) % KEY_TILES == 0) count_keys((i - 1) / KEY_TILES - 1, KEY_TILES);
        }
        if (s_wave) s_tile(i & 1, i & 1);
        // staging of tile i + 1, then the loads of tile i + 2
        if (i + 1 < ntiles) {
            stage((i + 1) & 1, (i + 1) % 3);
            if (i + 2 < ntiles) load(i + 2);
        }
        // tile i - 1 is complete in LDS since the last barrier
        if (wave == NWV - 1 && i > 0) finish(tile0 + i - 1, (i - 1) & 1, (i - 1) % 3);
        __syncthreads();
    }
    if (wave == NWV - 1) finish(tile0 + ntiles - 1, (ntiles - 1) & 1, (ntiles - 1) % 3);
    if constexpr (HIST) end_hist();
}

// ------------------------------------------------------------------ GQA-reduced VALU pass
// For at most SMALL_ROWS selection rows per KV head (a block position or two of a GQA
// group) a 32-row MFMA tile would be mostly padding and score_kernel's per-workgroup
// prologue (the value centre over every row of O_p, the row tables) would dominate.  Here
// every wave streams its own run of 32-token units (one key group each); the workgroup
// meets once, after a prologue that loads only the R2 selection rows' queries, their row
// constants and the centre (the mean of O_p over those rows, in row order, as the
// reference's index_select(...).mean(), splitk.py:598-601), while every wave's first unit
// is already in flight:
//   * staging: the unit's K is dequantized into the wave's LDS tile as bf16 [token][channel]
//     (the same items and stores as score_kernel's K buffer); the V items give the
//     squared distances to the centre straight from registers, one sum per token;
//   * scores: lane (token t, channel half hh) forms q_r . k_t over its D/2 channels with
//     v_dot2c_f32_bf16 for ROWS rows (R2 rounded up to 4, 8 or 16; the padding rows have
//     zero queries and row constant +inf, so they add exactly 0), queries broadcast from
//     LDS, adds the other half's sum (lane ^ 32) and sums exp2(s * scale*log2e - c_r);
//   * the next unit's loads are issued before the scores of this one.
constexpr int SMALL_ROWS = 16;
// the largest row count mode 0 sends here: none -- at config 2's prefix the padded MFMA
// pass measured as fast or faster (7 rows: 16.8 vs 17.4 us; 14 rows: 16.8 vs 21.9 us)
constexpr int AUTO_SMALL_ROWS = 0;
constexpr int SM_NT = 256;                   // threads per workgroup
constexpr int SM_WAVES = SM_NT / 64;
constexpr int UNIT = KGRP;                   // tokens per unit

template <int D>
struct SmallSmem {
    static constexpr int KS = D + 8;
    uint16_t k[SM_WAVES][UNIT * KS];     // each wave's unit: bf16 K [token][channel]
    float dist[SM_WAVES][UNIT];          // each wave's ||v - centre||^2 per token
    uint4 qv[SMALL_ROWS][D / 8];         // the selection rows' queries, 8 bf16 per entry (padding 0)
    float crow[SMALL_ROWS];              // per row: M_p*log2e + log2(L_p); +inf when L_p = 0 and for padding
    float cen[D];
};

// LDS written by some lanes of a wave, then read by others of the same wave: LDS executes a
// wave's accesses in order, so only the compiler must not move them across this point
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// KIND: 0 packed units, 1 16-bit units read with 16-byte loads, 2 element-wise (f32 or
// unaligned 16-bit prefixes; no registers staged)
template <int D>
struct SmallWords {
    static constexpr int NI = 2 * D / 64;   // K items and V items per lane and unit
    uint32_t k[NI][8], v[NI][8];
    uint2 ko[NI], vo[NI];
};

template <int D, int KIND>
__device__ __forceinline__ void small_offsets(const Lane &L, SmallWords<D> &W) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < SmallWords<D>::NI; ++i) {
        const int u = lane + 64 * i;
        if constexpr (KIND == 0) {
            W.ko[i] = kp_offsets<D>(L, u);
            W.vo[i] = vp_offsets<D>(L, u);
        } else if constexpr (KIND == 1) {
            W.ko[i] = uint2{kd_offset<D>(L, u), 0u};
            W.vo[i] = uint2{vd_offset<D>(L, u), 0u};
        }
    }
}

// unit uu's words of this lane; 16-bit units clamp tokens past the end (their results are
// not written)
template <int D, int KIND>
__device__ __forceinline__ void small_load(const Lane &L, SmallWords<D> &W, int uu, int end, bool value) {
    const int lane = threadIdx.x & 63;
    const int j0 = uu * UNIT;
    if constexpr (KIND == 0) {
        const int g = j0 / KGRP;
#pragma unroll
        for (int i = 0; i < SmallWords<D>::NI; ++i) {
            kp_load(W.k[i], L.kq + (int64_t)g * L.kq_g, L.ks + (int64_t)g * L.ks_g, L.kz + (int64_t)g * L.ks_g,
                    L.kq_d, W.ko[i]);
            if (value) vp_load(W.v[i], L.vq + (int64_t)j0 * L.vq_n, L.vs + (int64_t)j0 * L.vs_n,
                               L.vz + (int64_t)j0 * L.vs_n, W.vo[i]);
        }
    } else if constexpr (KIND == 1) {
        const int nv = min(UNIT, end - j0);   // tokens of the unit in the prefix
#pragma unroll
        for (int i = 0; i < SmallWords<D>::NI; ++i) {
            const int t = (lane + 64 * i) / (D / 16);
            const int shift = t < nv ? 0 : t - (nv - 1);   // clamp to the last token
            const int64_t jt = (int64_t)(j0 - L.nq) - shift;
            d32_load(W.k[i], L.kf + jt * L.kf_n * 2, W.ko[i].x);
            if (value) d32_load(W.v[i], L.vf + jt * L.vf_n * 2, W.vo[i].x);
        }
    }
}

// the units [u0, u1) of this wave (unit u0 already loaded when `loaded`)
template <int D, int KIND, int ROWS>
__device__ __forceinline__ void small_units(const ScoreArgs &a, SmallSmem<D> &sm, const Lane &L, SmallWords<D> &W,
                                            int bh, int wave, int u0, int u1, int end, bool loaded) {
    constexpr int KS = D + 8, NI = SmallWords<D>::NI;
    const int lane = threadIdx.x & 63;
    uint16_t *Ks = sm.k[wave];
    float *dist = sm.dist[wave];
    const bool value = a.value;
    const int vround = a.vround;
    const float inv_r2 = 1.0f / (float)a.r2_total, sl2 = a.sl2;
    if (!loaded) {
        small_offsets<D, KIND>(L, W);
        small_load<D, KIND>(L, W, u0, end, value);
    }
    for (int uu = u0; uu < u1; ++uu) {
        const int j0 = uu * UNIT;
        // ---- staging: K into the LDS tile, V distances per token
        if constexpr (KIND == 2) {
#pragma unroll 1
            for (int i = 0; i < NI; ++i) {
                const int u = lane + 64 * i, t = u / (D / 16), c0 = (u % (D / 16)) * 16;
                const int j = min(j0 + t, end - 1);
                uint32_t *dst = (uint32_t *)&Ks[t * KS + c0];
#pragma unroll 4
                for (int c = 0; c < 16; c += 2)
                    dst[c / 2] = ma_pack_bf16x2(lane_key(L, j, c0 + c), lane_key(L, j, c0 + c + 1));
                if (value) {
                    float dd = vg_dist<D>(L, u, j0, end, &sm.cen[c0], vround);
                    dd = token_sum<D>(dd);
                    if (u % (D / 16) == 0) dist[t] = dd;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int u = lane + 64 * i;
                if constexpr (KIND == 0) kp_store<D>(Ks, W.k[i], u);
                else kd_store<D>(Ks, W.k[i], u, L.fdtype);
                if (value) {
                    const float *cen16 = &sm.cen[(u % (D / 16)) * 16];
                    float dd;
                    if constexpr (KIND == 0)
                        dd = vround == MA_BF16 ? vp_dist<MA_BF16>(W.v[i], cen16)
                                               : (vround == MA_F16 ? vp_dist<MA_F16>(W.v[i], cen16) : vp_dist<0>(W.v[i], cen16));
                    else dd = vd_dist(W.v[i], cen16, L.fdtype);
                    dd = token_sum<D>(dd);
                    if (u % (D / 16) == 0) dist[u / (D / 16)] = dd;
                }
            }
            if (uu + 1 < u1) small_load<D, KIND>(L, W, uu + 1, end, value);
        }
        wave_lds_sync();
        // ---- scores: lane (token t, channel half hh)
        const int t = lane & 31, hh = lane >> 5;
        const uint4 *kr = (const uint4 *)&Ks[t * KS + hh * (D / 2)];
        float acc[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[r] = 0.f;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            const uint4 kw = kr[c];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const uint4 qw = sm.qv[r][hh * (D / 16) + c];
                float x = acc[r];
                x = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw.x), __builtin_bit_cast(bf16x2_t, kw.x), x, false);
                x = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw.y), __builtin_bit_cast(bf16x2_t, kw.y), x, false);
                x = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw.z), __builtin_bit_cast(bf16x2_t, kw.z), x, false);
                x = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw.w), __builtin_bit_cast(bf16x2_t, kw.w), x, false);
                acc[r] = x;
            }
        }
        float m = 0.f;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const float sv = ma_sum_xor32(acc[r]);   // both channel halves, the same in both lanes
            m += __builtin_amdgcn_exp2f(__builtin_fmaf(sv, sl2, -sm.crow[r]));
        }
        const int j = j0 + t;
        if (hh == 0 && j < end) {
            const int64_t o = (int64_t)bh * end + j;
            const bool live = !a.pre.mask || a.pre.mask[o] != 0;
            const float mm = live ? m * inv_r2 : 0.f;
            a.mass[o] = mm;
            if (value) a.score[o] = live ? mm * __builtin_sqrtf(dist[t]) : 0.f;
        }
        // the next unit's staging overwrites this unit's LDS after these reads (in order)
        wave_lds_sync();
    }
}

template <int D, int ROWS>
__global__ void __launch_bounds__(SM_NT) score_small_kernel(ScoreArgs a, int units, int dense_vec) {
    __shared__ SmallSmem<D> sm;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int end = a.pre.nq + a.pre.nf;
    const int R = a.R, R2 = a.R2, T = a.T, T2 = a.T2;
    const bool ident = a.q_rows == nullptr;
    // this wave's run of units: packed units [u0, pe) first, then the 16-bit tail [ts, u1)
    const int w = blockIdx.x * SM_WAVES + wave;
    const int u0 = w * a.per, u1 = min(units, u0 + a.per);
    const Lane L = make_lane(a.pre, b, h, bh);
    const int uq = L.nq / UNIT;
    const int pe = min(u1, uq), ts = max(u0, uq);
    const bool has_p = u0 < pe, has_t = ts < u1;
    // the first unit's loads go out before the prologue's
    SmallWords<D> W;
    if (has_p) {
        small_offsets<D, 0>(L, W);
        small_load<D, 0>(L, W, u0, end, a.value);
    } else if (has_t && dense_vec) {
        small_offsets<D, 1>(L, W);
        small_load<D, 1>(L, W, ts, end, a.value);
    }
    // ---- prologue: queries, row constants and the centre of the R2 <= ROWS rows
    // selection row rr = g * T2 + i: block position t (clamped into the block), row g * T + t
    auto sel = [&](int rr, int &g, int &t) {
        g = rr / T2;
        const int i = rr - g * T2;
        t = min(max(ident ? a.row0 + i : a.q_rows[i], 0), T - 1);
    };
    for (int e = tid; e < ROWS * (D / 8); e += SM_NT) {
        const int rr = e / (D / 8), c = e % (D / 8);
        int g, t;
        sel(rr < R2 ? rr : 0, g, t);
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
        const bf16x8_t x = ma_load8_as_bf16(a.q.ptr, qb + c * 8, a.q.dtype);
        sm.qv[rr][c] = rr < R2 ? __builtin_bit_cast(uint4, x) : uint4{0u, 0u, 0u, 0u};
    }
    if (tid < ROWS) {
        int g, t;
        sel(tid < R2 ? tid : 0, g, t);
        const float m = a.mp[(int64_t)bh * R + g * T + t], l = a.lp[(int64_t)bh * R + g * T + t];
        sm.crow[tid] = tid < R2 && l > 0.f ? __builtin_fmaf(m, MA_LOG2E, __log2f(l)) : __builtin_inff();
    }
    if (a.value && tid < D) {
        // all R2 loads in flight together (padding rows load row 0 and are not summed), then
        // the sum in row order
        float x[ROWS];
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) {
            int g, t;
            sel(rr < R2 ? rr : 0, g, t);
            const int64_t off = ((int64_t)bh * R + g * T + t) * D + tid;
            if (a.op_dtype == MA_F32) x[rr] = ((const float *)a.op)[off];
            else x[rr] = __uint_as_float((uint32_t)((const uint16_t *)a.op)[off]);   // raw bits, below
        }
        float c = 0.f;
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) {
            if (rr < R2) {
                const uint32_t bits = __float_as_uint(x[rr]);
                c += a.op_dtype == MA_F32 ? x[rr] : a.op_dtype == MA_BF16 ? ma_bf16_to_f32((uint16_t)bits)
                                                                           : ma_f16_to_f32((uint16_t)bits);
            }
        }
        sm.cen[tid] = c / (float)R2;
    }
    __syncthreads();
    if (has_p) small_units<D, 0, ROWS>(a, sm, L, W, bh, wave, u0, pe, end, true);
    if (has_t) {
        if (dense_vec) small_units<D, 1, ROWS>(a, sm, L, W, bh, wave, ts, u1, end, !has_p);
        else small_units<D, 2, ROWS>(a, sm, L, W, bh, wave, ts, u1, end, false);
    }
}

// the value centre of prefix_scores alone (same definition and order as score_kernel)
template <int D>
__global__ void __launch_bounds__(SNT) centre_kernel(const void *op, int op_dtype, int G, int T,
                                                     const int32_t *q_rows, int T2, float *centre) {
    using CS = CentreSmem<D>;
    constexpr int CH = D / 8;
    __shared__ CS cs;
    __shared__ int cnt[MAX_R];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const int R = G * T, R2 = G * T2;
    for (int r = tid; r < R; r += SNT) cnt[r] = 0;
    __syncthreads();
    for (int rr = tid; rr < R2; rr += SNT) {
        int g, t;
        atomicAdd(&cnt[sel_row(q_rows, rr, T2, T, &g, &t)], 1);
    }
    __syncthreads();
    const int osl = tid / CH, och = tid % CH;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    for (int r = osl; r < R; r += SNT / CH) {
        const int n = cnt[r];
        if (n > 0) {
            const int64_t off_o = ((int64_t)bh * R + r) * D + och * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] += (float)n * ma_load_f(op, off_o + e, op_dtype);
        }
    }
    __shared__ float cen[D];
    centre_reduce<D, SNT>(acc, cs, cen, R2);
    if (tid < D) centre[(int64_t)bh * D + tid] = cen[tid];
}

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

// 0: the VALU pass for at most AUTO_SMALL_ROWS selection rows (none), MFMA otherwise; 1:
// always MFMA; 2: always VALU (calls with more than SMALL_ROWS rows fail)
static std::atomic<int> g_score_path{0};

extern "C" int ma_prefix_scores_path(int mode) {
    if (mode < 0 || mode > 2) {
        ma_set_error("ma_prefix_scores_path: mode must be 0 (auto), 1 (MFMA) or 2 (VALU)");
        return -1;
    }
    return g_score_path.exchange(mode);
}

extern "C" int ma_value_centre(const void *op, int op_dtype, int B, int H, int G, int T, int D, const int32_t *q_rows,
                               int T2, float *centre, void *stream) {
    if (!op || !q_rows || !centre || B <= 0 || H <= 0 || G <= 0 || T <= 0 || T2 <= 0 || (D != 64 && D != 128)) {
        ma_set_error("ma_value_centre: bad arguments");
        return MA_EINVAL;
    }
    if (((uintptr_t)op & 15) != 0) {
        ma_set_error("ma_value_centre: op must be 16-byte aligned");
        return MA_EINVAL;
    }
    if (G * T2 > MAX_R2 || G * T > MAX_R) {
        ma_set_error("ma_value_centre: %d selection rows / %d rows per KV head exceed the built maximum %d / %d",
                     G * T2, G * T, MAX_R2, MAX_R);
        return MA_EUNSUPPORTED;
    }
    if (D == 128)
        hipLaunchKernelGGL(centre_kernel<128>, dim3(B * H), dim3(SNT), 0, (hipStream_t)stream, op, op_dtype, G, T,
                           q_rows, T2, centre);
    else
        hipLaunchKernelGGL(centre_kernel<64>, dim3(B * H), dim3(SNT), 0, (hipStream_t)stream, op, op_dtype, G, T,
                           q_rows, T2, centre);
    return ma_check_launch("ma_value_centre");
}

extern "C" int ma_topk_level0_into_state(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                         int64_t mask_stride, int rows, int n, void *state, void *stream);

static int prefix_scores(const char *who, ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                         const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                         int op_dtype, float scale, int value, int v_round, float *mass, float *score,
                         int hist_rank, void *topk_state, int64_t state_bytes, void *stream) {
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || T2 <= 0 || !q.ptr || (!q_rows && T2 > T) || !mp || !lp ||
        !mass || (value && (!score || !op))) {
        ma_set_error("%s: bad sizes or NULL pointer", who);
        return MA_EINVAL;
    }
    const int64_t m = q.dtype == MA_F32 ? 4 : 8;
    if (((uintptr_t)q.ptr & 15) || q.s[0] % m || q.s[1] % m || q.s[2] % m) {
        ma_set_error("%s: query must be 16-byte aligned with aligned row strides", who);
        return MA_EINVAL;
    }
    if (value && ((uintptr_t)op & 15)) {
        ma_set_error("%s: the prefix output O_p must be 16-byte aligned", who);
        return MA_EINVAL;
    }
    const int G = Hq / H, R = G * T, R2 = G * T2;
    if (value && ((R2 + 31) / 32 > MAX_RT || R > MAX_R)) {
        // the value score's centre is built in LDS over all rows of the KV head
        ma_set_error("%s: value-aware scores of %d selection rows / %d rows per KV head exceed the built maximum "
                     "%d / %d", who, R2, R, MAX_R2, MAX_R);
        return MA_EUNSUPPORTED;
    }
    if (G > MAX_R2) {
        ma_set_error("%s: %d query heads per KV head exceed the built maximum %d", who, G, MAX_R2);
        return MA_EUNSUPPORTED;
    }
    // mass only: the selection rows in passes of at most MAX_R2 rows (whole q_rows entries),
    // each adding its share of the mean to mass
    const int t2_pass = value ? T2 : (MAX_R2 / G < T2 ? MAX_R2 / G : T2);
    const int n = p->nq + p->nf;
    if (n == 0) return MA_OK;
    // 16-bit parts are read with 32-byte vector loads: every token row must stay aligned
    const bool dense_vec_ok = p->nf == 0 || (p->fdtype != MA_F32 && p->skf[2] % 16 == 0 && p->svf[2] % 16 == 0 &&
                                             ((uintptr_t)p->kf & 15) == 0 && ((uintptr_t)p->vf & 15) == 0 &&
                                             p->skf[0] % 16 == 0 && p->skf[1] % 16 == 0 && p->svf[0] % 16 == 0 &&
                                             p->svf[1] % 16 == 0);
    const int row_tiles_max = (G * t2_pass + 31) / 32;
    // one 1024-thread workgroup per CU: units of half a tile up to 8 row tiles, whole
    // tiles beyond.  (Two 512-thread workgroups per CU, NT = 512, measured 1.6x slower at
    // config 2: each workgroup loads its lane's Q and O_p rows in its prologue, so twice
    // the workgroups move twice those bytes.)
    const int halves = row_tiles_max <= 8 ? 1 : 2;
    const int wgs_per_cu = 1;
    const int tiles = (n + TILE - 1) / TILE;
    const bool packed = p->nq > 0;
    // whole tiles of the source kind go to the pipelined workgroups, the rest (a tile
    // straddling the packed / 16-bit boundary, 16-bit tail tiles, a partial last tile,
    // f32 or unaligned 16-bit prefixes) to one tail workgroup each
    int nfast = packed ? p->nq / TILE : n / TILE;
    if (!dense_vec_ok) nfast = 0;
    const int slots = wgs_per_cu * ma_num_cus();
    int per = nfast > 0 ? (nfast * B * H + slots - 1) / slots : 1;
    if (per < 1) per = 1;
    const int fast_wgs = nfast > 0 ? (nfast + per - 1) / per : 0;
    ScoreArgs sa{};
    sa.q = q;
    sa.pre = prefix_dev(p, B, H);
    sa.q_rows = q_rows;
    sa.mp = mp;
    sa.lp = lp;
    sa.op = op;
    sa.op_dtype = op_dtype;
    sa.mass = mass;
    sa.score = score;
    sa.H = H;
    sa.G = G;
    sa.T = T;
    sa.R = R;
    sa.r2_total = R2;
    sa.value = value;
    if (v_round != 0 && v_round != MA_BF16 && v_round != MA_F16) {
        ma_set_error("%s: v_round must be 0, MA_BF16 or MA_F16", who);
        return MA_EINVAL;
    }
    sa.vround = v_round;
    sa.sl2 = scale * MA_LOG2E;
    if (hist_rank) {
        if ((hist_rank != 1 && hist_rank != 2) || (hist_rank == 2 && !value) || !topk_state ||
            ((uintptr_t)topk_state & 255) || state_bytes < ma_topk_state_bytes(B * H)) {
            ma_set_error("%s: rank must be 1 (mass) or 2 (score, value-aware), and the top-k state %lld bytes "
                         "(256-byte aligned) for %d rows; got rank %d and %lld bytes", who,
                         (long long)ma_topk_state_bytes(B * H), B * H, hist_rank, (long long)state_bytes);
            return MA_EINVAL;
        }
    }
    sa.hist = (uint32_t *)topk_state;
    hipStream_t st = (hipStream_t)stream;
    // at most SMALL_ROWS selection rows: the GQA-reduced VALU pass, one pass over the rows
    const int path = g_score_path.load(std::memory_order_relaxed);
    if (path == 2 && R2 > SMALL_ROWS) {
        ma_set_error("%s: the VALU score pass takes at most %d selection rows per KV head, got %d", who, SMALL_ROWS,
                     R2);
        return MA_EUNSUPPORTED;
    }
    if (path == 2 || (path == 0 && R2 <= AUTO_SMALL_ROWS)) {
        const int units = (n + UNIT - 1) / UNIT;
        // about 8 waves per CU in all, each on a contiguous run of units
        const int waves_bh = max(1, min(units, 8 * ma_num_cus() / (B * H)));
        const int per = (units + waves_bh - 1) / waves_bh;
        const int waves = (units + per - 1) / per;
        sa.q_rows = q_rows;
        sa.row0 = 0;
        sa.T2 = T2;
        sa.R2 = R2;
        sa.row_tiles = 1;
        sa.accum = 0;
        sa.per = per;
        const dim3 g2((waves + SM_WAVES - 1) / SM_WAVES, B * H);
        const int dv = dense_vec_ok ? 1 : 0;
#define MA_SMALL(D_, R_) hipLaunchKernelGGL((score_small_kernel<D_, R_>), g2, dim3(SM_NT), 0, st, sa, units, dv)
        if (D == 128) {
            if (R2 <= 4) MA_SMALL(128, 4);
            else if (R2 <= 8) MA_SMALL(128, 8);
            else MA_SMALL(128, 16);
        } else {
            if (R2 <= 4) MA_SMALL(64, 4);
            else if (R2 <= 8) MA_SMALL(64, 8);
            else MA_SMALL(64, 16);
        }
#undef MA_SMALL
        rc = ma_check_launch(who);
        if (rc || !hist_rank) return rc;
        // this pass does not build the histogram in-kernel: the select's own level-0 launch
        return ma_topk_level0_into_state(hist_rank == 2 ? score : mass, n, p->mask, n, B * H, n, topk_state, stream);
    }
    sa.nfast = nfast;
    sa.per = per;
    sa.fast_wgs = fast_wgs;
    dim3 grid(fast_wgs + (tiles - nfast), H, B);
#define MA_SCORE(D_, S_, H_)                                                                          \
    do {                                                                                              \
        if (!sa.pre.off32) hipLaunchKernelGGL((score_kernel<D_, S_, H_, SNT, false, false>), grid, dim3(SNT), 0, st, sa); \
        else if (sa.hist_rank) hipLaunchKernelGGL((score_kernel<D_, S_, H_, SNT, true, true>), grid, dim3(SNT), 0, st, sa); \
        else hipLaunchKernelGGL((score_kernel<D_, S_, H_, SNT, false, true>), grid, dim3(SNT), 0, st, sa);                  \
    } while (0)
#define MA_SCORE_I(D_, S_)                        \
    do {                                          \
        if (halves == 1) MA_SCORE(D_, S_, 1);     \
        else MA_SCORE(D_, S_, 2);                 \
    } while (0)
    for (int t0 = 0; t0 < T2; t0 += t2_pass) {
        const int t2 = T2 - t0 < t2_pass ? T2 - t0 : t2_pass;
        sa.q_rows = q_rows ? q_rows + t0 : nullptr;
        sa.row0 = t0;
        sa.T2 = t2;
        sa.R2 = G * t2;
        sa.row_tiles = (G * t2 + 31) / 32;
        sa.accum = t0 > 0;
        sa.hist_rank = t0 + t2 >= T2 ? hist_rank : 0;   // the last pass sees the final mass
        if (D == 128) {
            if (packed) MA_SCORE_I(128, SRC_PACKED);
            else MA_SCORE_I(128, SRC_DENSE);
        } else {
            if (packed) MA_SCORE_I(64, SRC_PACKED);
            else MA_SCORE_I(64, SRC_DENSE);
        }
        const int rc2 = ma_check_launch(who);
        if (rc2) return rc2;
    }
#undef MA_SCORE_I
#undef MA_SCORE
    // lanes beyond 31-bit offsets run the kernel without the in-kernel histogram
    if (hist_rank && !sa.pre.off32)
        return ma_topk_level0_into_state(hist_rank == 2 ? score : mass, n, p->mask, n, B * H, n, topk_state, stream);
    return MA_OK;
}

extern "C" int ma_prefix_scores(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                                int op_dtype, float scale, int value, int v_round, float *mass, float *score,
                                void *stream) {
    return prefix_scores("ma_prefix_scores", q, B, Hq, T, D, p, H, q_rows, T2, mp, lp, op, op_dtype, scale, value,
                         v_round, mass, score, 0, nullptr, 0, stream);
}

extern "C" int ma_prefix_scores_hist(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                     const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                                     int op_dtype, float scale, int value, int v_round, float *mass, float *score,
                                     int rank, void *topk_state, int64_t state_bytes, void *stream) {
    if (rank != 1 && rank != 2) {
        ma_set_error("ma_prefix_scores_hist: rank must be 1 (mass) or 2 (score), got %d", rank);
        return MA_EINVAL;
    }
    return prefix_scores("ma_prefix_scores_hist", q, B, Hq, T, D, p, H, q_rows, T2, mp, lp, op, op_dtype, scale,
                         value, v_round, mass, score, rank, topk_state, state_bytes, stream);
}
