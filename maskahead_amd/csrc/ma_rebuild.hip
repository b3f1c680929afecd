// Packed-cache eviction rebuild: the plan of the session's lazy / full compaction
// (runtime/session.py:288-345) and PackedKVCache.rebuild (cache.py:236-335).
//
// After an eviction the live entries of every (layer, batch, KV head) lane are a
// scattered subset of the old slots.  The new storage of a lane is
//     [kept key groups | freshly quantized groups | tail groups] + bf16 stage
// where a kept group (one that still holds at least `need` live entries) is copied byte
// for byte with its dead slots, the survivors of sparser groups and the decided bf16
// entries are dequantized and quantized again into new groups of 32, and the entries
// still in the recent window stay in bf16.  Integer and byte work throughout; the
// requantization reproduces the reference's bf16-arithmetic quantizer (ma_quant.h).
//
// ma_rebuild_plan   one 1024-thread workgroup per lane: survivor counts per key group in
//                   LDS (16-bit counters), the kept groups in ascending order, then every
//                   live entry classified in (position, slot) order -- the order the lanes
//                   already hold after a keep-set selection, so the sort is skipped; lanes
//                   out of that order are sorted in LDS (bitonic, up to 16384 entries).
// ma_rebuild_packed one launch of 256-thread workgroups: one per lane fills the slot remap
//                   with -1, scatters the new slots into it in the reference's list order
//                   and rewrites the eviction state's slots through it; the others copy a
//                   kept group byte for byte, requantize a new group or gather 32 staged
//                   bf16 entries.  Old and new storage never alias.
#include "ma_common.h"
#include "ma_quant.h"

namespace {

constexpr int KG = 32;                    // key token group
constexpr int VG = 32;                    // value channel group
constexpr int PLAN_THREADS = 1024;
constexpr int PLAN_SORT_MAX = 16384;      // live entries of an out-of-order lane
constexpr int PLAN_GROUPS_MAX = 32768;    // key groups of the old quantized part
constexpr int RB_THREADS = 256;
constexpr int64_t SLOT_MASK = (1 << 24) - 1;

// ---------------------------------------------------------------- plan
struct PlanArgs {
    const int32_t *phys;
    int64_t sphys;
    const void *pos;
    int pos64;
    int64_t spos;
    int live, ql, ng, need, tail_groups, window;
    int64_t *gb, *enc, *stg;
    int64_t sgb, senc, sstg;
    int32_t *counts;
};

struct PlanSmem {
    union {
        uint32_t cnt[PLAN_GROUPS_MAX / 2];   // two 16-bit survivor counts per word
        int64_t key[PLAN_SORT_MAX];          // (pos << 24) + slot, sorted ascending
    } u;
    uint32_t kept[PLAN_GROUPS_MAX / 32];     // kept-group bitmask
    uint32_t wsum[PLAN_THREADS / 64];
    int unsorted;
};

// exclusive block prefix of x (1024 threads); total = the block's sum
__device__ __forceinline__ uint32_t block_exclusive(uint32_t x, uint32_t *wsum, uint32_t &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t inc = ma_wave_prefix_u32(x);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    uint32_t before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < PLAN_THREADS / 64; ++w) {
        const uint32_t s = wsum[w];
        before += w < wave ? s : 0u;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return before + inc - x;
}

__global__ void __launch_bounds__(PLAN_THREADS) rebuild_plan_kernel(PlanArgs a) {
    __shared__ PlanSmem S;
    const int lane = blockIdx.x, tid = threadIdx.x;
    const int32_t *phys = a.phys + lane * a.sphys;
    int64_t *gb = a.gb + lane * a.sgb;
    int64_t *enc = a.enc + lane * a.senc;
    int64_t *stg = a.stg + lane * a.sstg;
    auto pos_at = [&](int i) -> int64_t {
        return a.pos64 ? ((const int64_t *)a.pos)[lane * a.spos + i] : (int64_t)((const int32_t *)a.pos)[lane * a.spos + i];
    };
    auto key_at = [&](int i) -> int64_t { return pos_at(i) * (int64_t)(1 << 24) + phys[i]; };
    const int ng = a.ng, live = a.live;

    // survivors per old key group, and whether the lane is out of (position, slot) order
    for (int i = tid; i < (ng + 1) / 2; i += PLAN_THREADS) S.u.cnt[i] = 0;
    if (tid == 0) S.unsorted = 0;
    __syncthreads();
    int unsorted = 0;
    for (int i = tid; i < live; i += PLAN_THREADS) {
        const int p = phys[i];
        if (p >= 0 && p < a.ql) {
            const int g = p / KG;
            atomicAdd(&S.u.cnt[g >> 1], 1u << (16 * (g & 1)));
        }
        if (i + 1 < live && key_at(i) > key_at(i + 1)) unsorted = 1;
    }
    if (unsorted) S.unsorted = 1;   // every writer stores the same value
    __syncthreads();

    // kept groups: enough survivors and not one of the tail groups; ascending ids
    uint32_t nb = 0;
    for (int g0 = 0; g0 < ng; g0 += PLAN_THREADS) {
        const int g = g0 + tid;
        bool k = false;
        if (g < ng) {
            const int c = (int)((S.u.cnt[g >> 1] >> (16 * (g & 1))) & 0xffffu);
            k = c >= a.need && g < ng - a.tail_groups;
        }
        const uint64_t bal = __ballot(k);
        if ((tid & 63) == 0) {
            const int w0 = (g0 + (tid & ~63)) / 32;
            S.kept[w0] = (uint32_t)bal;
            S.kept[w0 + 1] = (uint32_t)(bal >> 32);
        }
        uint32_t tot;
        const uint32_t ex = block_exclusive(k ? 1u : 0u, S.wsum, tot);
        if (k) gb[nb + ex] = g;
        nb += tot;
    }
    for (int j = (int)nb + tid; j < ng; j += PLAN_THREADS) gb[j] = -1;
    __syncthreads();   // the bitmask is complete; the counters are dead (the sort reuses them)

    const bool sorted_in_lds = S.unsorted != 0;
    if (sorted_in_lds) {
        if (live > PLAN_SORT_MAX) {
            if (tid == 0) {
                a.counts[lane * 3 + 0] = -1;
                a.counts[lane * 3 + 1] = -1;
                a.counts[lane * 3 + 2] = -1;
            }
            return;   // the whole workgroup leaves together (uniform condition)
        }
        int P = 1;
        while (P < live) P <<= 1;
        for (int i = tid; i < P; i += PLAN_THREADS) S.u.key[i] = i < live ? key_at(i) : INT64_MAX;
        __syncthreads();
        for (int k = 2; k <= P; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int t = tid; t < P / 2; t += PLAN_THREADS) {
                    const int i = 2 * t - (t & (j - 1));   // lower index of the pair (bit j clear)
                    const int l = i + j;
                    const bool up = (i & k) == 0;
                    const int64_t x = S.u.key[i], y = S.u.key[l];
                    if ((x > y) == up) {
                        S.u.key[i] = y;
                        S.u.key[l] = x;
                    }
                }
                __syncthreads();
            }
        }
    }
    // entry e of the (position, slot) order: its raw slot and position
    auto entry = [&](int e, int &slot, int64_t &p) {
        if (sorted_in_lds) {
            const int64_t k = S.u.key[e];
            slot = (int)(k & SLOT_MASK);
            p = k >> 24;
        } else {
            slot = phys[e];
            p = pos_at(e);
        }
    };
    // recency threshold: the w-th largest position (the window stays bf16)
    const int w = a.window;
    int64_t thr = (int64_t)1 << 60;
    if (w > 0) {
        int s;
        entry(live - w, s, thr);
    }
    uint32_t ne = 0, ns = 0;
    for (int e0 = 0; e0 < live; e0 += PLAN_THREADS) {
        const int e = e0 + tid;
        bool is_enc = false, is_stg = false;
        int slot = 0;
        if (e < live) {
            int64_t p;
            entry(e, slot, p);
            const bool in_q = slot < a.ql;
            const bool kept = in_q && slot >= 0 && ((S.kept[(slot / KG) >> 5] >> ((slot / KG) & 31)) & 1u);
            is_stg = !in_q && p >= thr;
            is_enc = !kept && !is_stg;
        }
        uint32_t tot;
        const uint32_t ex = block_exclusive((is_enc ? 1u : 0u) | (is_stg ? 0x10000u : 0u), S.wsum, tot);
        const int64_t s64 = (int64_t)slot & SLOT_MASK;
        if (is_enc) enc[ne + (ex & 0xffffu)] = s64;
        if (is_stg) stg[ns + (ex >> 16)] = s64;
        ne += tot & 0xffffu;
        ns += tot >> 16;
    }
    for (int j = (int)ne + tid; j < live; j += PLAN_THREADS) enc[j] = -1;
    for (int j = (int)ns + tid; j < live; j += PLAN_THREADS) stg[j] = -1;
    if (tid == 0) {
        a.counts[lane * 3 + 0] = (int)nb;
        a.counts[lane * 3 + 1] = (int)ne;
        a.counts[lane * 3 + 2] = (int)ns;
    }
}

// ---------------------------------------------------------------- rebuild
// One lane's storage: payload and scale/zero of the quantized part, bf16 residual.
struct LaneStore {
    uint8_t *kq;
    uint16_t *ks, *kz;
    uint8_t *vq;
    uint16_t *vs, *vz;
    uint16_t *kr, *vr;
    int64_t kq_g, kq_d, ks_g, vq_n, vq_c, vs_n, kr_n, vr_n;
};

struct StoreDev {
    uint8_t *kq;
    uint16_t *ks, *kz;
    uint8_t *vq;
    uint16_t *vs, *vz;
    uint16_t *kr, *vr;
    int64_t skq[4], sks[3], svq[4], svs[3], skr[3], svr[3];
};

// DC 0: any layout, the strides inside a lane read from the descriptor.  DC 64 or 128: a
// store of that head_dim laid out as the cache allocates it (a key group's rows 16 B
// apart, its scales contiguous, value groups of 16 B, scales and residual rows dense),
// so every stride inside a lane is a compile-time constant (ma_rebuild_packed checks).
template <int DC>
__device__ __forceinline__ LaneStore lane_store(const StoreDev &s, int b, int h) {
    LaneStore L;
    L.kq = s.kq ? s.kq + b * s.skq[0] + h * s.skq[1] : nullptr;
    L.ks = s.ks ? s.ks + b * s.sks[0] + h * s.sks[1] : nullptr;
    L.kz = s.kz ? s.kz + b * s.sks[0] + h * s.sks[1] : nullptr;
    L.vq = s.vq ? s.vq + b * s.svq[0] + h * s.svq[1] : nullptr;
    L.vs = s.vs ? s.vs + b * s.svs[0] + h * s.svs[1] : nullptr;
    L.vz = s.vz ? s.vz + b * s.svs[0] + h * s.svs[1] : nullptr;
    L.kr = s.kr ? s.kr + b * s.skr[0] + h * s.skr[1] : nullptr;
    L.vr = s.vr ? s.vr + b * s.svr[0] + h * s.svr[1] : nullptr;
    if constexpr (DC > 0) {
        L.kq_g = DC * 16;
        L.kq_d = 16;
        L.ks_g = DC;
        L.vq_n = DC / 2;
        L.vq_c = 16;
        L.vs_n = DC / VG;
        L.kr_n = DC;
        L.vr_n = DC;
    } else {
        L.kq_g = s.skq[2];
        L.kq_d = s.skq[3];
        L.ks_g = s.sks[2];
        L.vq_n = s.svq[2];
        L.vq_c = s.svq[3];
        L.vs_n = s.svs[2];
        L.kr_n = s.skr[2];
        L.vr_n = s.svr[2];
    }
    return L;
}

struct RbArgs {
    StoreDev old, nw;
    int H, D, old_len, old_ql, old_ng;
    const int64_t *gb, *enc, *ga, *stg;
    int64_t sgb, senc, sga, sstg;
    int g1, m, g3, st, g2, lanes;
    int64_t *remap;
    int64_t sremap;
    int32_t *phys;
    int64_t sphys;
    int live;
    int32_t *status;
};

// Old entry `src` of a lane as bf16-rounded floats, channels d0 .. d0+7: the dequantized
// packed entry (reference.py:168-179, 259-268, then the bf16 cast of dequantize_layer)
// or the bf16 residual; an invalid slot (-1 padding, or out of range) is zeros.  DC > 0:
// the 8 key scales (and zeros) are one 16-byte load, the 8 code bytes constant offsets.
template <int DC>
__device__ __forceinline__ void old_entry8(const RbArgs &a, const LaneStore &o, int64_t src64, int d0, float *k8,
                                           float *v8) {
    if (src64 < 0 || src64 >= a.old_len) {
#pragma unroll
        for (int i = 0; i < 8; ++i) k8[i] = v8[i] = 0.f;
        return;
    }
    const int src = (int)src64;   // < old_len, an int
    if (src < a.old_ql) {
        const int g = src / KG, t = src % KG;
        const uint8_t *kb = o.kq + (int64_t)g * o.kq_g + (int64_t)d0 * o.kq_d + (t >> 1);
        const int64_t so = (int64_t)g * o.ks_g + d0;
        uint16_t sc[8], ze[8];
        if constexpr (DC > 0) {
            const uint4 sw = *(const uint4 *)(o.ks + so), zw = *(const uint4 *)(o.kz + so);
            const uint32_t s4[4] = {sw.x, sw.y, sw.z, sw.w}, z4[4] = {zw.x, zw.y, zw.z, zw.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[2 * i] = (uint16_t)(s4[i] & 0xffffu);
                sc[2 * i + 1] = (uint16_t)(s4[i] >> 16);
                ze[2 * i] = (uint16_t)(z4[i] & 0xffffu);
                ze[2 * i + 1] = (uint16_t)(z4[i] >> 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sc[i] = o.ks[so + i];
                ze[i] = o.kz[so + i];
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t byte = kb[(int64_t)i * o.kq_d];
            const uint32_t code = (t & 1) ? (byte >> 4) : (byte & 15u);
            k8[i] = ma_round_bf16(ma_dq(code, ma_f16_to_f32(sc[i]), ma_f16_to_f32(ze[i])));
        }
        const int c = d0 / VG;
        const uint8_t *vb = o.vq + (int64_t)src * o.vq_n + c * o.vq_c + (d0 % VG) / 2;
        const uint32_t w = *(const uint32_t *)vb;   // 4 bytes = channels d0 .. d0+7
        const int64_t vso = (int64_t)src * o.vs_n + c;
        const float vsc = ma_f16_to_f32(o.vs[vso]), vze = ma_f16_to_f32(o.vz[vso]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v8[i] = ma_round_bf16(ma_dq((w >> (4 * i)) & 15u, vsc, vze));
        return;
    }
    const int64_t r = src - a.old_ql;
    const uint4 kw = *(const uint4 *)(o.kr + r * o.kr_n + d0);
    const uint4 vw = *(const uint4 *)(o.vr + r * o.vr_n + d0);
    const uint32_t kk[4] = {kw.x, kw.y, kw.z, kw.w}, vv[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k8[2 * i] = ma_bf16_to_f32((uint16_t)(kk[i] & 0xffffu));
        k8[2 * i + 1] = ma_bf16_to_f32((uint16_t)(kk[i] >> 16));
        v8[2 * i] = ma_bf16_to_f32((uint16_t)(vv[i] & 0xffffu));
        v8[2 * i + 1] = ma_bf16_to_f32((uint16_t)(vv[i] >> 16));
    }
}

// slot list entry i of a lane (-1 past the list)
__device__ __forceinline__ int64_t list_at(const int64_t *p, int64_t stride, int lane, int n, int i) {
    return i < n ? p[lane * stride + i] : -1;
}

// One workgroup per lane, inside the data launch (it reads only the lists and the
// state's slots, never the storage): every old slot's remap set to -1, then remap[old
// slot] = new slot written in the reference's order (kept and tail groups, encoded,
// staged: a later list wins a slot named twice, the workgroup's barriers ordering its
// stores), then the eviction state's slots rewritten through it.  Each thread loads
// RM_BATCH list entries before it stores any, so a phase costs about one round trip.
// status bit 0: a list names a slot or group outside the old storage; bit 1: a live
// entry's slot maps to no new slot.
constexpr int RM_THREADS = RB_THREADS;
constexpr int RM_BATCH = 8;

__device__ void remap_lane(const RbArgs &a, int lane) {
    __shared__ int flags;
    const int tid = threadIdx.x;
    int64_t *rm = a.remap + lane * a.sremap;
    if (tid == 0) flags = 0;
    for (int i = tid; i < a.old_len; i += RM_THREADS) rm[i] = -1;
    __syncthreads();
    int bad = 0;
    // kept and tail groups: every slot of a copied group, dead ones included
    const int ngi = (a.g1 + a.g3) * KG;
    for (int u0 = 0; u0 < ngi; u0 += RM_THREADS * RM_BATCH) {
        int64_t g[RM_BATCH];
#pragma unroll
        for (int r = 0; r < RM_BATCH; ++r) {
            const int u = u0 + r * RM_THREADS + tid, j = u / KG;
            g[r] = u >= ngi ? -1 : j < a.g1 ? list_at(a.gb, a.sgb, lane, a.g1, j)
                                            : list_at(a.ga, a.sga, lane, a.g3, j - a.g1);
        }
#pragma unroll
        for (int r = 0; r < RM_BATCH; ++r) {
            const int u = u0 + r * RM_THREADS + tid, j = u / KG, t = u % KG;
            const int dst = j < a.g1 ? j : a.g1 + a.g2 + (j - a.g1);
            if (g[r] < -1 || g[r] >= a.old_ng) bad = 1;
            else if (u < ngi && g[r] >= 0) rm[g[r] * KG + t] = (int64_t)dst * KG + t;
        }
    }
    __syncthreads();
    auto scatter = [&](const int64_t *list, int64_t stride, int n, int64_t first) {
        for (int i0 = 0; i0 < n; i0 += RM_THREADS * RM_BATCH) {
            int64_t s[RM_BATCH];
#pragma unroll
            for (int r = 0; r < RM_BATCH; ++r) s[r] = list_at(list, stride, lane, n, i0 + r * RM_THREADS + tid);
#pragma unroll
            for (int r = 0; r < RM_BATCH; ++r) {
                if (s[r] < -1 || s[r] >= a.old_len) bad = 1;
                else if (s[r] >= 0) rm[s[r]] = first + i0 + r * RM_THREADS + tid;
            }
        }
    };
    scatter(a.enc, a.senc, a.m, (int64_t)a.g1 * KG);
    __syncthreads();
    scatter(a.stg, a.sstg, a.st, (int64_t)(a.g1 + a.g2 + a.g3) * KG);
    __syncthreads();
    int lost = 0;
    if (a.phys) {
        int32_t *ph = a.phys + lane * a.sphys;
        for (int i0 = 0; i0 < a.live; i0 += RM_THREADS * RM_BATCH) {
            int p[RM_BATCH];
            int64_t nw[RM_BATCH];
#pragma unroll
            for (int r = 0; r < RM_BATCH; ++r) {
                const int i = i0 + r * RM_THREADS + tid;
                p[r] = i < a.live ? ph[i] : -1;
            }
#pragma unroll
            for (int r = 0; r < RM_BATCH; ++r) nw[r] = (p[r] >= 0 && p[r] < a.old_len) ? rm[p[r]] : -1;
#pragma unroll
            for (int r = 0; r < RM_BATCH; ++r) {
                const int i = i0 + r * RM_THREADS + tid;
                if (i < a.live) {
                    if (nw[r] < 0) lost = 1;
                    ph[i] = (int32_t)nw[r];
                }
            }
        }
    }
    if (bad) atomicOr(&flags, 1);
    if (lost) atomicOr(&flags, 2);
    __syncthreads();
    if (tid == 0) a.status[lane] = flags;
}

// New group `dst` of a lane: old group `src` copied byte for byte (kept / tail groups;
// padding copies group 0, as the reference gathers clamped ids).
template <int DC>
__device__ void copy_group(const RbArgs &a, const LaneStore &o, const LaneStore &n, int64_t src, int dst) {
    const int tid = threadIdx.x, D = DC > 0 ? DC : a.D, ncg = D / VG;
    if (src < 0 || src >= a.old_ng) src = 0;
    for (int d = tid; d < D; d += RB_THREADS) {
        *(uint4 *)(n.kq + dst * n.kq_g + d * n.kq_d) = *(const uint4 *)(o.kq + src * o.kq_g + d * o.kq_d);
        n.ks[dst * n.ks_g + d] = o.ks[src * o.ks_g + d];
        n.kz[dst * n.ks_g + d] = o.kz[src * o.ks_g + d];
    }
    for (int u = tid; u < KG * ncg; u += RB_THREADS) {
        const int t = u / ncg, c = u % ncg;
        const int64_t so = src * KG + t, dn = (int64_t)dst * KG + t;
        *(uint4 *)(n.vq + dn * n.vq_n + c * n.vq_c) = *(const uint4 *)(o.vq + so * o.vq_n + c * o.vq_c);
        n.vs[dn * n.vs_n + c] = o.vs[so * o.vs_n + c];
        n.vz[dn * n.vs_n + c] = o.vz[so * o.vs_n + c];
    }
}

// New group g1 + j of a lane: the 32 old entries encode[32 j ..] (zeros past the list or
// for padding) dequantized to bf16 and quantized again in bf16 arithmetic
// (quantize_key_groups_into / quantize_values_into on the gathered bf16 rows).  Item (t,
// octet o) = channels 8o .. 8o+7 of entry t, one or two per thread.  A value group (32
// channels of one entry) is the items of 4 adjacent lanes: its range comes from two lane
// exchanges and each lane quantizes its 8 channels in registers.  Keys go through LDS
// (one column per channel) and are quantized by P = 256 / D adjacent lanes per channel,
// 32 / P tokens each, their ranges combined the same way.
template <int DC>
__device__ void encode_group(const RbArgs &a, const LaneStore &o, const LaneStore &n, int lane, int j) {
    __shared__ float xk[KG][129];   // head_dim <= 128 (+1: column reads across rows)
    const int tid = threadIdx.x, D = DC > 0 ? DC : a.D, oct = D / 8;
    const int g = a.g1 + j;
    for (int u = tid; u < KG * oct; u += RB_THREADS) {
        const int t = u / oct, oc = u % oct, d0 = oc * 8;
        const int64_t src = list_at(a.enc, a.senc, lane, a.m, j * KG + t);
        float k8[8], v8[8];
        old_entry8<DC>(a, o, src, d0, k8, v8);
#pragma unroll
        for (int i = 0; i < 8; ++i) xk[t][d0 + i] = k8[i];
        // the value group of channels 32 c .. 32 c + 31: lanes with octets 4c .. 4c + 3 (oct
        // is a multiple of 4 and divides 64, so they are adjacent lanes of one wave)
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            lo = fminf(lo, v8[i]);
            hi = fmaxf(hi, v8[i]);
        }
        lo = fminf(lo, __shfl_xor(lo, 1));
        hi = fmaxf(hi, __shfl_xor(hi, 1));
        lo = fminf(lo, __shfl_xor(lo, 2));
        hi = fmaxf(hi, __shfl_xor(hi, 2));
        const QuantGroup qp = quant_params(lo, hi, MA_BF16);
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= quant_code(v8[i], qp, MA_BF16) << (i * 4);
        const int c = d0 / VG, q = (d0 % VG) / 8;
        const int64_t tok = (int64_t)g * KG + t;
        *(uint32_t *)(n.vq + tok * n.vq_n + c * n.vq_c + q * 4) = w;
        if (q == 0) {
            const _Float16 s16 = (_Float16)qp.step, z16 = (_Float16)qp.lo;
            n.vs[tok * n.vs_n + c] = *(const uint16_t *)&s16;
            n.vz[tok * n.vs_n + c] = *(const uint16_t *)&z16;
        }
    }
    __syncthreads();
    // keys: channel d, tokens [part * TP, part * TP + TP)
    const int P = RB_THREADS / D, TP = KG / P;
    const int d = tid / P, part = tid % P, t0 = part * TP;
    float lo = INFINITY, hi = -INFINITY;
    for (int t = 0; t < TP; ++t) {
        lo = fminf(lo, xk[t0 + t][d]);
        hi = fmaxf(hi, xk[t0 + t][d]);
    }
    for (int m = 1; m < P; m <<= 1) {
        lo = fminf(lo, __shfl_xor(lo, m));
        hi = fmaxf(hi, __shfl_xor(hi, m));
    }
    const QuantGroup qp = quant_params(lo, hi, MA_BF16);
    uint32_t w[2] = {0, 0};
    for (int t = 0; t < TP; ++t) w[t >> 3] |= quant_code(xk[t0 + t][d], qp, MA_BF16) << ((t & 7) * 4);
    uint8_t *krow = n.kq + (int64_t)g * n.kq_g + d * n.kq_d + t0 / 2;
    if (TP == 16) *(uint2 *)krow = uint2{w[0], w[1]};
    else *(uint32_t *)krow = w[0];
    if (part == 0) {
        const _Float16 s16 = (_Float16)qp.step, z16 = (_Float16)qp.lo;
        n.ks[(int64_t)g * n.ks_g + d] = *(const uint16_t *)&s16;
        n.kz[(int64_t)g * n.ks_g + d] = *(const uint16_t *)&z16;
    }
}

// Staged entries 32 c .. 32 c + 31 of a lane: old entries as bf16 rows of the new
// residual (zeros for padding).
template <int DC>
__device__ void stage_chunk(const RbArgs &a, const LaneStore &o, const LaneStore &n, int lane, int c) {
    const int tid = threadIdx.x, oct = (DC > 0 ? DC : a.D) / 8;
    for (int u = tid; u < KG * oct; u += RB_THREADS) {
        const int t = c * KG + u / oct, d0 = (u % oct) * 8;
        if (t >= a.st) continue;
        const int64_t src = list_at(a.stg, a.sstg, lane, a.st, t);
        float k8[8], v8[8];
        old_entry8<DC>(a, o, src, d0, k8, v8);
        uint4 kw, vw;
        kw.x = ma_pack_bf16x2(k8[0], k8[1]);
        kw.y = ma_pack_bf16x2(k8[2], k8[3]);
        kw.z = ma_pack_bf16x2(k8[4], k8[5]);
        kw.w = ma_pack_bf16x2(k8[6], k8[7]);
        vw.x = ma_pack_bf16x2(v8[0], v8[1]);
        vw.y = ma_pack_bf16x2(v8[2], v8[3]);
        vw.z = ma_pack_bf16x2(v8[4], v8[5]);
        vw.w = ma_pack_bf16x2(v8[6], v8[7]);
        *(uint4 *)(n.kr + (int64_t)t * n.kr_n + d0) = kw;
        *(uint4 *)(n.vr + (int64_t)t * n.vr_n + d0) = vw;
    }
}

// grid: [remap: lanes] [copy: lanes x (g1 + g3)] [encode: lanes x g2] [stage: lanes x
// ceil(st/32)]: the remap workgroups first, so they run beside the requantization.

template <int DC>
__global__ void __launch_bounds__(RB_THREADS) rebuild_kernel(RbArgs a) {
    // 32-bit workgroup arithmetic: the host keeps the grid below 2^31 workgroups
    uint32_t idx = blockIdx.x;
    if (idx < (uint32_t)a.lanes) {
        remap_lane(a, (int)idx);
        return;
    }
    idx -= (uint32_t)a.lanes;
    const uint32_t ncopy = (uint32_t)(a.g1 + a.g3), g2 = (uint32_t)a.g2, nstc = (uint32_t)((a.st + KG - 1) / KG);
    int lane, kind, j;
    if (idx < (uint32_t)a.lanes * ncopy) {
        kind = 0;
        lane = (int)(idx / ncopy);
        j = (int)(idx % ncopy);
    } else if ((idx -= (uint32_t)a.lanes * ncopy) < (uint32_t)a.lanes * g2) {
        kind = 1;
        lane = (int)(idx / g2);
        j = (int)(idx % g2);
    } else {
        idx -= (uint32_t)a.lanes * g2;
        kind = 2;
        lane = (int)(idx / nstc);
        j = (int)(idx % nstc);
    }
    const int b = lane / a.H, h = lane % a.H;
    const LaneStore o = lane_store<DC>(a.old, b, h), n = lane_store<DC>(a.nw, b, h);
    if (kind == 0) {
        const int64_t src = j < a.g1 ? list_at(a.gb, a.sgb, lane, a.g1, j) : list_at(a.ga, a.sga, lane, a.g3, j - a.g1);
        copy_group<DC>(a, o, n, src, j < a.g1 ? j : a.g1 + a.g2 + (j - a.g1));
    } else if (kind == 1) {
        encode_group<DC>(a, o, n, lane, j);
    } else {
        stage_chunk<DC>(a, o, n, lane, j);
    }
}

StoreDev store_dev(const ma_prefix *p) {
    StoreDev s;
    s.kq = (uint8_t *)p->kq;
    s.ks = (uint16_t *)p->ks;
    s.kz = (uint16_t *)p->kz;
    s.vq = (uint8_t *)p->vq;
    s.vs = (uint16_t *)p->vs;
    s.vz = (uint16_t *)p->vz;
    s.kr = (uint16_t *)p->kf;
    s.vr = (uint16_t *)p->vf;
    for (int i = 0; i < 4; ++i) {
        s.skq[i] = p->skq[i];
        s.svq[i] = p->svq[i];
    }
    for (int i = 0; i < 3; ++i) {
        s.sks[i] = p->sks[i];
        s.svs[i] = p->svs[i];
        s.skr[i] = p->skf[i];
        s.svr[i] = p->svf[i];
    }
    return s;
}

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

extern "C" int ma_rebuild_plan(const int32_t *phys, int64_t phys_stride, const void *pos, int pos_is_i64,
                               int64_t pos_stride, int lanes, int live, int quantized_length, int need,
                               int tail_groups, int window, int64_t *groups_before, int64_t gb_stride,
                               int64_t *encode, int64_t enc_stride, int64_t *stage, int64_t stage_stride,
                               int32_t *counts, void *stream) {
    const char *who = "ma_rebuild_plan";
    if (lanes < 0 || live < 0 || quantized_length < 0 || quantized_length % KG || tail_groups < 0 || window < 0 ||
        window > live) {
        ma_set_error("%s: bad sizes (lanes=%d live=%d quantized_length=%d tail_groups=%d window=%d)", who, lanes,
                     live, quantized_length, tail_groups, window);
        return MA_EINVAL;
    }
    const int ng = quantized_length / KG > 1 ? quantized_length / KG : 1;
    if (ng > PLAN_GROUPS_MAX) {
        ma_set_error("%s: %d key groups exceed the %d this kernel counts", who, ng, PLAN_GROUPS_MAX);
        return MA_EUNSUPPORTED;
    }
    if (lanes == 0) return MA_OK;
    if (!groups_before || !counts || (live > 0 && (!phys || !pos || !encode || !stage))) {
        ma_set_error("%s: NULL pointer", who);
        return MA_EINVAL;
    }
    if (gb_stride < ng || (live > 0 && (enc_stride < live || stage_stride < live || phys_stride < live ||
                                        pos_stride < live))) {
        ma_set_error("%s: a lane stride is shorter than its row", who);
        return MA_EINVAL;
    }
    PlanArgs a;
    a.phys = phys;
    a.sphys = phys_stride;
    a.pos = pos;
    a.pos64 = pos_is_i64 ? 1 : 0;
    a.spos = pos_stride;
    a.live = live;
    a.ql = quantized_length;
    a.ng = ng;
    a.need = need;
    a.tail_groups = tail_groups;
    a.window = window;
    a.gb = groups_before;
    a.sgb = gb_stride;
    a.enc = encode;
    a.senc = enc_stride;
    a.stg = stage;
    a.sstg = stage_stride;
    a.counts = counts;
    hipLaunchKernelGGL(rebuild_plan_kernel, dim3(lanes), dim3(PLAN_THREADS), 0, (hipStream_t)stream, a);
    return ma_check_launch(who);
}

static int check_store(const ma_prefix *p, int D, int64_t ql, int64_t nres, const char *who, const char *which) {
    if (!p) {
        ma_set_error("%s: %s storage is NULL", who, which);
        return MA_EINVAL;
    }
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (p->nq != ql || p->nf != nres) {
        ma_set_error("%s: %s storage describes %d + %d entries, expected %lld + %lld", who, which, p->nq, p->nf,
                     (long long)ql, (long long)nres);
        return MA_EINVAL;
    }
    if (nres > 0) {
        if (p->fdtype != MA_BF16) {
            ma_set_error("%s: %s residual must be bf16", who, which);
            return MA_EUNSUPPORTED;
        }
        if ((((uintptr_t)p->kf | (uintptr_t)p->vf) & 15) || ((p->skf[0] | p->skf[1] | p->skf[2] | p->svf[0] |
                                                              p->svf[1] | p->svf[2]) & 7)) {
            ma_set_error("%s: %s residual rows must be 16-byte aligned", who, which);
            return MA_EINVAL;
        }
    }
    return MA_OK;
}

extern "C" int ma_rebuild_packed(const ma_prefix *old_store, int B, int H, int D, const ma_prefix *new_store,
                                 const int64_t *groups_before, int64_t gb_stride, int g1, const int64_t *encode,
                                 int64_t enc_stride, int m, const int64_t *groups_after, int64_t ga_stride, int g3,
                                 const int64_t *stage, int64_t stage_stride, int st, int64_t *remap,
                                 int64_t remap_stride, int32_t *phys, int64_t phys_stride, int live, int32_t *status,
                                 void *stream) {
    const char *who = "ma_rebuild_packed";
    if (B < 0 || H <= 0 || g1 < 0 || m < 0 || g3 < 0 || st < 0 || live < 0) {
        ma_set_error("%s: bad sizes (B=%d H=%d g1=%d m=%d g3=%d st=%d live=%d)", who, B, H, g1, m, g3, st, live);
        return MA_EINVAL;
    }
    if (!old_store) {
        ma_set_error("%s: old storage is NULL", who);
        return MA_EINVAL;
    }
    const int old_ql = old_store->nq, old_len = old_store->nq + old_store->nf;
    const int g2 = (m + KG - 1) / KG;
    int rc = check_store(old_store, D, old_ql, old_store->nf, who, "old");
    if (rc) return rc;
    rc = check_store(new_store, D, (int64_t)(g1 + g2 + g3) * KG, st, who, "new");
    if (rc) return rc;
    const int lanes = B * H;
    if (lanes == 0) return MA_OK;
    if ((g1 && !groups_before) || (m && !encode) || (g3 && !groups_after) || (st && !stage) || !status ||
        (old_len && !remap) || (live && !phys)) {
        ma_set_error("%s: NULL pointer", who);
        return MA_EINVAL;
    }
    // a list's lane stride is its row length or more, or 0 (one list for every lane)
    auto short_row = [](int64_t stride, int n) { return n && stride != 0 && stride < n; };
    if (short_row(gb_stride, g1) || short_row(enc_stride, m) || short_row(ga_stride, g3) ||
        short_row(stage_stride, st) || (old_len && remap_stride < old_len) || (live && phys_stride < live)) {
        ma_set_error("%s: a lane stride is shorter than its row", who);
        return MA_EINVAL;
    }
    if (phys && live > old_len) {
        ma_set_error("%s: %d live entries but only %d old slots", who, live, old_len);
        return MA_EINVAL;
    }
    RbArgs a;
    a.old = store_dev(old_store);
    a.nw = store_dev(new_store);
    a.H = H;
    a.D = D;
    a.old_len = old_len;
    a.old_ql = old_ql;
    a.old_ng = old_ql / KG;
    a.gb = groups_before;
    a.enc = encode;
    a.ga = groups_after;
    a.stg = stage;
    a.sgb = gb_stride;
    a.senc = enc_stride;
    a.sga = ga_stride;
    a.sstg = stage_stride;
    a.g1 = g1;
    a.m = m;
    a.g3 = g3;
    a.st = st;
    a.g2 = g2;
    a.lanes = lanes;
    a.remap = remap;
    a.sremap = remap_stride;
    a.phys = live ? phys : nullptr;
    a.sphys = phys_stride;
    a.live = live;
    a.status = status;
    if ((g1 + g3) && a.old_ng == 0) {
        ma_set_error("%s: key groups to copy but the old storage has none", who);
        return MA_EINVAL;
    }
    const int64_t blocks = (int64_t)lanes * (1 + g1 + g3 + g2 + (st + KG - 1) / KG);
    if (blocks > 0x7fffffff) {
        ma_set_error("%s: grid of %lld workgroups too large", who, (long long)blocks);
        return MA_EINVAL;
    }
    // the cache's own layout (both stores): the instantiation with constant inner strides
    auto dense = [D](const ma_prefix *p) {
        const bool al16 = !(((uintptr_t)p->ks | (uintptr_t)p->kz) & 15) && !((p->sks[0] | p->sks[1]) & 7);
        return al16 && p->skq[3] == 16 && p->skq[2] == (int64_t)D * 16 && p->sks[2] == D && p->svq[3] == 16 &&
               p->svq[2] == D / 2 && p->svs[2] == D / VG && p->skf[2] == D && p->svf[2] == D;
    };
    const int dc = (D == 64 || D == 128) && dense(old_store) && dense(new_store) ? D : 0;
    auto kern = dc == 128 ? rebuild_kernel<128> : dc == 64 ? rebuild_kernel<64> : rebuild_kernel<0>;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(RB_THREADS), 0, (hipStream_t)stream, a);
    return ma_check_launch(who);
}
