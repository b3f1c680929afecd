// Split-K (flash-decoding) attention over [prefix | current block] for every query row
// of a KV head's GQA group (the reference's splitk_attention, splitk.py:493-579).
//
// Pass 1 (splitk_fwd_kernel): one workgroup = one (batch, KV head) lane x one token range
// (a prefix split, or the current block) x up to 7 row tiles of 32 query rows; 8 waves of
// up to 256 VGPRs, software-pipelined over 64-token tiles with one barrier per tile:
//   waves 0..6   one row tile each.  S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = K rows
//                from LDS, B = Q^T held in registers), so a lane owns ONE query row and 16
//                tokens of each 32-token half; online softmax with a lazily raised
//                reference max; O^T = alpha * O^T + V^T P^T with P^T straight from the
//                softmax's registers (A = V^T from LDS).  The S^T MFMAs of tile i+1 are
//                issued interleaved with the exp2 work of tile i.
//   all waves    staging: threads 0..255 dequantize K items, 256..511 V items of tile i+2
//                into the third K / V buffer, then issue the loads of tile i+3.
// Pass 2 (splitk_combine_kernel): log-sum-exp merge of the partials into the output and
// the prefix-only statistics (M_p, L_p, O_p) of splitk.py:272-318.
#include <mutex>
#include <type_traits>

#include "ma_stage.h"

using namespace ma;

namespace {

constexpr int MAXS = 7;                     // row tiles (compute waves) per workgroup
// a row's running reference max is raised only when a tile's max exceeds it by more than
// 2^8 in exp2 units, so most tiles skip the accumulator rescale; p <= 2^8 stays exact
constexpr float LAZY_LOG2 = 8.0f;

struct FwdArgs {
    ma_tensor4 q;
    PrefixDev pre;
    ma_tensor4 kc, vc;
    int H, G, T, R, Tc, nsplit, split_n, causal, q_pos0, c_pos0, row_tiles, row_groups, BH;
    // this launch: splits [0, nsp) of its token range [tok_beg, tok_end) of every lane,
    // written to slots slot0 + split; with_cur: the current-block workgroups follow
    int nsp, slot0, tok_beg, tok_end, with_cur;
    float sl2;  // scale * log2(e)
    float scale;
    // partials of every (lane, slot, row), slot = split or nsplit (current block):
    // wm = row max (natural-log units), wl = sum of exp relative to it, wsc = scale and
    // wo = f16(O / scale), O = the slot's normalized output (wo * wsc); wo [..][R][D]
    float *wm, *wl, *wsc;
    _Float16 *wo;
};

// write a row tile's partials: per row the max in natural-log units, the sum of exp
// relative to it, and the normalized output O = acc / l as f16 on a per-row scale (the
// row's max |O|), so the partial is half the size of an f32 one and cannot overflow.  The
// wave's 32 x D tile of O goes through its own LDS region (16-byte granules, XOR-swizzled
// by row) so that every global store instruction writes whole rows, contiguously: the
// tile's rows are adjacent in wo.  Called by the whole wave; rows >= R are not written.
template <int D>
__device__ __forceinline__ void write_partial(const FwdArgs &a, const f32x16_t *acc, float m_ref, float m_true,
                                              float l, int bh, int slot, int rtile, int c32, int hf, int lane,
                                              uint4 *lds) {
    constexpr int NDT = D / 32;
    constexpr int NG = D / 8;       // 16-byte granules per row
    constexpr int RPI = 64 / NG;    // rows per store instruction
    typedef __attribute__((ext_vector_type(4))) _Float16 f16x4_t;
    const int row0 = rtile * 32;
    const int64_t prow0 = ((int64_t)bh * (a.nsplit + 1) + slot) * a.R + row0;
    const int nrows = min(32, a.R - row0);
    float mx = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(acc[dt][i]));
    mx = ma_max_xor32(mx);                       // the row's other half lives in lane ^ 32
    const float inv = mx > 0.f ? 1.0f / mx : 0.f;
    if (hf == 0 && c32 < nrows) {
        float f = 0.f;
        if (m_true != -INFINITY) f = __builtin_amdgcn_exp2f((m_ref - m_true) * a.sl2);
        a.wm[prow0 + c32] = m_true * a.scale;
        a.wl[prow0 + c32] = l * f;
        a.wsc[prow0 + c32] = l > 0.f ? mx / l : 0.f;    // O = acc / l = wo * wsc
    }
    // lane (c32, hf) holds columns dt * 32 + q4 * 8 + hf * 4 + (0..3) of row c32
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f16x4_t v = {(_Float16)(acc[dt][q4 * 4 + 0] * inv), (_Float16)(acc[dt][q4 * 4 + 1] * inv),
                               (_Float16)(acc[dt][q4 * 4 + 2] * inv), (_Float16)(acc[dt][q4 * 4 + 3] * inv)};
            const int g = (dt * 4 + q4) ^ (c32 % NG);
            *(f16x4_t *)((char *)&lds[c32 * NG + g] + hf * 8) = v;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint4 *dst = (uint4 *)(a.wo + prow0 * D);
    const int g = lane % NG;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
        const int r = i * RPI + lane / NG;
        const uint4 v = lds[r * NG + (g ^ (r % NG))];
        if (r < nrows) dst[r * NG + g] = v;
    }
}

// S wave: S^T = K Q^T for one 64-token tile (A = K rows from LDS, B = Q^T in registers).
// K fragments are loaded one k-step ahead of the MFMAs; the two token halves alternate,
// so consecutive MFMAs never wait on each other's accumulator.
template <int D>
__device__ __forceinline__ void s_qk(const uint16_t *K, const bf16x8_t *qf, int c32, int hf, f32x16_t *s) {
    constexpr int KS = D + 8;
    constexpr int NKS = D / 16;
    s[0] = f32x16_t{};
    s[1] = f32x16_t{};
    const uint16_t *k0 = &K[c32 * KS + hf * 8];
    const uint16_t *k1 = &K[(32 + c32) * KS + hf * 8];
    bf16x8_t ka0 = *(const bf16x8_t *)k0, ka1 = *(const bf16x8_t *)k1;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        bf16x8_t na0 = ka0, na1 = ka1;
        if (ks + 1 < NKS) {
            na0 = *(const bf16x8_t *)(k0 + (ks + 1) * 16);
            na1 = *(const bf16x8_t *)(k1 + (ks + 1) * 16);
        }
        s[0] = ma_mfma32(ka0, qf[ks], s[0]);
        s[1] = ma_mfma32(ka1, qf[ks], s[1]);
        ka0 = na0;
        ka1 = na1;
    }
}

// Workgroup index -> (segment, lane bh, row group, split).  Prefix splits first, the
// current-block workgroups last (they are short, so they fill in behind the splits).
struct Work {
    bool cur;
    int bh, rg, sp;
};

__device__ __forceinline__ Work decode_work(const FwdArgs &a) {
    Work w;
    int idx = blockIdx.x;
    const int npre = a.nsp * a.BH * a.row_groups;
    w.cur = idx >= npre;
    if (w.cur) idx -= npre;
    w.rg = idx % a.row_groups;
    idx /= a.row_groups;
    w.bh = idx % a.BH;
    w.sp = w.cur ? 0 : idx / a.BH;
    return w;
}

// Token source of one workgroup of the 16-bit kernel: the 16-bit part of a prefix, or
// the current block.  Token j of the workgroup's range lives at k + (j - tok0) * sk.
struct DSrc {
    const char *k, *v;
    int sk, sv, dtype, esz, tok0;
    const uint8_t *mask;  // liveness by absolute token index, or null
};

// ---------------------------------------------------------------- pass 1
// Every compute wave does S, softmax and PV of its own row tile (P never leaves its
// registers); staging is spread over all 8 waves.  After the loop the K / V buffers hold
// each wave's O tile for the partial write.
constexpr int NTH = 512;
constexpr int KLANES = NTH / 2;

constexpr int NBUF = 3;   // K / V buffers: S of tile i+1 is issued while tile i is finished

template <int D>
struct FwdSmem {
    union {
        struct {
            KTileL<D> kt[NBUF];
            VTileL<D> vt[NBUF];
        } t;
        uint4 o[MAXS][4 * D];   // 32 x D f16 per row tile (write_partial)
    } u;
    uint64_t kmask[NBUF];
};

// s_softmax with the probabilities kept in registers: pb[c] = P^T chunk c (16 tokens) in
// the register order of the PV B operand; returns whether the reference max was raised,
// in which case the accumulator must first be scaled by alpha (the lane's row's factor).
template <int D>
__device__ __forceinline__ bool s_softmax_r(f32x16_t *s, uint64_t okm, float &m_ref, float &m_true, float &l,
                                            int hf, bool need_mask, int lim, float sl2, bf16x8_t *pb,
                                            float &alpha) {
    if (need_mask) {
        const uint64_t okh = okm >> (hf * 4);
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tk = t2 * 32 + (i >> 2) * 8 + (i & 3);
                const bool ok = ((okh >> tk) & 1) && tk < lim;
                s[t2][i] = ok ? s[t2][i] : -INFINITY;
            }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[t2][i]);
    mt = ma_max_xor32(mt);
    m_true = fmaxf(m_true, mt);
    const bool need = (mt - m_ref) * sl2 > LAZY_LOG2;   // false for NaN (both -inf)
    bool resc = false;
    alpha = 1.0f;
    if (__any(need)) {
        const float m_new = need ? mt : m_ref;
        alpha = (m_new == m_ref) ? 1.0f : __builtin_amdgcn_exp2f((m_ref - m_new) * sl2);
        l *= alpha;
        m_ref = m_new;
        resc = true;
    }
    const float off = (m_ref == -INFINITY) ? 0.f : -m_ref * sl2;
    float ls = 0.f;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t2][i], sl2, off));
            s[t2][i] = p;
            ls += p;
        }
    l += ma_sum_xor32(ls);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[c][j] = (__bf16)s[c >> 1][(c & 1) * 8 + j];
    return resc;
}

// The softmax of s_softmax_r in two parts, free of branches, so that the next tile's S^T
// MFMAs can be interleaved with its exp2 part.  Part 1: the tile max, the lazily raised
// reference max and the factor alpha (1 exactly where the reference stays, so l * alpha
// and acc * alpha leave those rows' bits unchanged); returns whether this lane's row
// raised it.
__device__ __forceinline__ bool sm_max(const f32x16_t *s, float &m_ref, float &m_true, float &l, float sl2,
                                       float &alpha, float &off) {
    float mt = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[t2][i]);
    mt = ma_max_xor32(mt);
    m_true = fmaxf(m_true, mt);
    const bool need = (mt - m_ref) * sl2 > LAZY_LOG2;   // false for NaN (both -inf)
    const float m_new = need ? mt : m_ref;
    alpha = (m_new == m_ref) ? 1.0f : __builtin_amdgcn_exp2f((m_ref - m_new) * sl2);
    l *= alpha;
    m_ref = m_new;
    off = (m_ref == -INFINITY) ? 0.f : -m_ref * sl2;
    return need;
}
// S^T of the next tile (s_qk's MFMAs, in s_qk's order) interleaved in issue order with
// the current tile's probabilities: after each MFMA the exp2 of the next few elements,
// so that this wave's VALU work runs while its MFMAs are in the matrix pipe.  The same
// arithmetic as s_qk followed by the exp2 part of s_softmax_r.
template <int D>
__device__ __forceinline__ void qk_exp(const uint16_t *K, const bf16x8_t *qf, int c32, int hf, f32x16_t *sn,
                                       f32x16_t *sc, float &l, float sl2, float off, bf16x8_t *pb) {
    constexpr int KS = D + 8;
    constexpr int NKS = D / 16;
    constexpr int EPM = 32 / (2 * NKS);   // probabilities per MFMA
    sn[0] = f32x16_t{};
    sn[1] = f32x16_t{};
    const uint16_t *k0 = &K[c32 * KS + hf * 8];
    const uint16_t *k1 = &K[(32 + c32) * KS + hf * 8];
    bf16x8_t ka0 = *(const bf16x8_t *)k0, ka1 = *(const bf16x8_t *)k1;
    float ls = 0.f;
    auto expo = [&](int e0) {
#pragma unroll
        for (int e = e0; e < e0 + EPM; ++e) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e >> 4][e & 15], sl2, off));
            sc[e >> 4][e & 15] = p;
            ls += p;
        }
    };
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        bf16x8_t na0 = ka0, na1 = ka1;
        if (ks + 1 < NKS) {
            na0 = *(const bf16x8_t *)(k0 + (ks + 1) * 16);
            na1 = *(const bf16x8_t *)(k1 + (ks + 1) * 16);
        }
        sn[0] = ma_mfma32(ka0, qf[ks], sn[0]);
        expo((2 * ks) * EPM);
        __builtin_amdgcn_sched_barrier(0);
        sn[1] = ma_mfma32(ka1, qf[ks], sn[1]);
        expo((2 * ks + 1) * EPM);
        __builtin_amdgcn_sched_barrier(0);
        ka0 = na0;
        ka1 = na1;
    }
    l += ma_sum_xor32(ls);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[c][j] = (__bf16)sc[c >> 1][(c & 1) * 8 + j];
}

// O^T += V^T P^T for one tile, P^T from registers: chunk by chunk (16 tokens), the D/32
// accumulators alternating
template <int D>
__device__ __forceinline__ void pv_regs(const uint16_t *Vt, const bf16x8_t *pb, f32x16_t *acc, int c32, int hf) {
    constexpr int VS = TILE + 8;
    constexpr int NDT = D / 32;
    const uint16_t *vrow = &Vt[c32 * VS + hf * 8];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            acc[dt] = ma_mfma32(*(const bf16x8_t *)&vrow[dt * 32 * VS + c * 16], pb[c], acc[dt]);
}

// The current block of one (lane, row group) for the packed kernel: its tiles staged
// synchronously by every thread from the 16-bit current K/V, then S^T, softmax
// (block-causal mask) and PV; the partial goes to slot nsplit.
template <int D>
__device__ __forceinline__ void cur_segment(const FwdArgs &a, const Work &wk, FwdSmem<D> &S) {
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;
    const int bh = wk.bh, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;
    const Dense kc = dense_lane(a.kc.ptr, a.kc.s, a.kc.dtype, b, h);
    const Dense vc = dense_lane(a.vc.ptr, a.vc.s, a.vc.dtype, b, h);
    const int Tc = a.Tc;
    const int nt = (Tc + TILE - 1) / TILE;
    const int nS = min(MAXS, a.row_tiles - wk.rg * MAXS);
    const bool is_s = wave < nS;
    const int rtile = wk.rg * MAXS + wave;
    const int row = rtile * 32 + c32;
    const bool row_ok = row < a.R;
    const int qpos = a.q_pos0 + (row_ok ? row % a.T : 0);
    const bool causal = a.causal > 0;
    bf16x8_t qf[NKS];
    if (is_s) {
        const int g = row_ok ? row / a.T : 0, t = row_ok ? row % a.T : 0;
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = ma_load8_as_bf16(a.q.ptr, qb + ks * 16 + hf * 8, a.q.dtype);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = row_ok ? qf[ks] : bf16x8_t{};
    }
    float m_ref = -INFINITY, m_true = -INFINITY, l = 0.f;
    f32x16_t acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x16_t{};
    for (int i = 0; i < nt; ++i) {
        const int n0 = i * TILE;
        const int valid = Tc - n0;
        uint32_t w[8];
        const char *kb = kc.base + (int64_t)n0 * kc.sn * kc.esz;
        for (int u = tid; u < TILE * D / 8; u += NTH) {
            const bool ok = load_k_dense<D>(w, kb, kc.sn, kc.dtype, kc.esz, u, valid);
            store_k_dense<D>(S.u.t.kt[0].k, w, u, kc.dtype, ok);
        }
        const char *vb = vc.base + (int64_t)n0 * vc.sn * vc.esz;
        for (int u = tid; u < TILE / 2 * D / 8; u += NTH) {
            const int tp = u % (TILE / 2);
            load_v_dense<D>(w, vb, vc.sn, vc.dtype, vc.esz, u, valid);
            store_v_dense<D>(S.u.t.vt[0].vt, w, u, vc.dtype, 2 * tp < valid, 2 * tp + 1 < valid);
        }
        if (wave == 0) {
            const uint64_t m = __ballot(lane < valid);
            if (lane == 0) S.kmask[0] = m;
        }
        __syncthreads();  // tile staged
        if (is_s) {
            f32x16_t sv[2];
            s_qk<D>(S.u.t.kt[0].k, qf, c32, hf, sv);
            const int lim = causal ? (qpos / a.causal + 1) * a.causal - a.c_pos0 - n0 - hf * 4 : TILE;
            bf16x8_t pb[4];
            float alpha;
            if (s_softmax_r<D>(sv, S.kmask[0], m_ref, m_true, l, hf, true, lim, a.sl2, pb, alpha)) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
            }
            pv_regs<D>(S.u.t.vt[0].vt, pb, acc, c32, hf);
        }
        __syncthreads();  // buffers free
    }
    if (is_s) write_partial<D>(a, acc, m_ref, m_true, l, bh, a.nsplit, rtile, c32, hf, lane, &S.u.o[wave][0]);
}

// FULL (packed only): no slot mask and every split a run of whole 64-token tiles (the host
// checks nq % 64 == 0), so only the whole-tile staging path is built
template <int D, int SRC, bool FULL>
__global__ void __launch_bounds__(NTH) splitk_fwd_kernel(FwdArgs a) {
    __shared__ FwdSmem<D> S;
    using Shape = StageShape<KLANES, D, SRC == 0 ? ST_PACKED : ST_DENSE>;
    constexpr int NKS = D / 16;
    constexpr int NDT = D / 32;

    const Work wk = decode_work(a);
    if constexpr (SRC == 0) {
        if (wk.cur) {
            cur_segment<D>(a, wk, S);
            return;
        }
    }
    const int bh = wk.bh, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;

    const Lane L = make_lane(a.pre, b, h, bh);
    int n_beg, n_end;
    if (wk.cur) {
        n_beg = 0;
        n_end = a.Tc;
    } else {
        n_beg = a.tok_beg + wk.sp * a.split_n;
        n_end = min(n_beg + a.split_n, a.tok_end);
        if (n_end < n_beg) n_end = n_beg;
    }
    const int nt = (n_end - n_beg + TILE - 1) / TILE;
    const int slot = wk.cur ? a.nsplit : a.slot0 + wk.sp;
    DSrc ds;
    if constexpr (SRC != 0) {
        if (wk.cur) {
            const Dense kc = dense_lane(a.kc.ptr, a.kc.s, a.kc.dtype, b, h);
            const Dense vc = dense_lane(a.vc.ptr, a.vc.s, a.vc.dtype, b, h);
            ds = DSrc{kc.base, vc.base, kc.sn, vc.sn, kc.dtype, kc.esz, 0, nullptr};
        } else {
            ds = DSrc{L.kf, L.vf, L.kf_n, L.vf_n, L.fdtype, L.esz, L.nq, L.mask};
        }
        if constexpr (SRC == 2) {
            // every 16-bit operand of the launch is bf16: the staging's dtype choices fold
            ds.dtype = MA_BF16;
            ds.esz = 2;
        }
    }

    const int nS = min(MAXS, a.row_tiles - wk.rg * MAXS);
    const bool is_s = wave < nS;
    const int rtile = wk.rg * MAXS + wave;
    const int row = rtile * 32 + c32;
    const bool row_ok = row < a.R;
    const bool is_k = tid < KLANES;
    const int kl = tid, vl = tid - KLANES;

    auto tile_n0 = [&](int i) { return n_beg + i * TILE; };
    auto live = [&](int j) {
        if constexpr (SRC == 0) {
            return lane_live(L, j, n_end);
        } else {
            bool ok = j < n_end;
            if (ds.mask) ok = ok && ds.mask[min(j, L.ntot - 1)] != 0;
            return ok;
        }
    };

    StageRegs<Shape::NW> pr;
    pr.flags = 0;
    uint2 item_off = uint2{0u, 0u};
    if constexpr (SRC == 0) {
        if (is_k && kl < Shape::NK) item_off = k_item_offsets<D>(L, kl);
        else if (!is_k && vl < Shape::NV) item_off = v_item_offsets<D>(L, vl);
    }
    const bool fast_tiles = SRC == 0 && (FULL || !L.mask);
    // all-bf16 dense source without a slot mask: the byte offset of this thread's first
    // item from a whole tile's first token, computed once (a whole tile then costs one base
    // address per operand and no bounds checks).  Item r of a K lane is KLANES / (D / 8) * r
    // tokens further, item r of a V lane 8 r channels further (its second token one row
    // on): wave-uniform steps.  32-bit while 64 rows span < 2 GiB.
    uint32_t doff = 0u;
    bool dense_fast = false;
    if constexpr (SRC == 2) {
        static_assert(KLANES % (D / 8) == 0 && KLANES % (TILE / 2) == 0, "item steps are whole rows / chunks");
        const int64_t sn = is_k ? ds.sk : ds.sv;
        dense_fast = !ds.mask && sn >= 0 && sn * 2 * TILE < (int64_t)0x7fffffff;
        const int t = is_k ? kl / (D / 8) : 2 * (vl % (TILE / 2));
        const int chk = is_k ? kl % (D / 8) : vl / (TILE / 2);
        doff = (uint32_t)(((int64_t)t * sn + chk * 8) * 2);
    }
    auto load_k = [&](int i) {
        const int n0 = tile_n0(i);
        if constexpr (SRC == 0) {
            if (FULL || (fast_tiles && n0 + TILE <= n_end)) {
                pr.flags = kl < TILE ? 256u : 0u;
                if (kl < Shape::NK) {
                    const int64_t g0 = n0 / KGRP;
                    load_k_packed_fast(pr.w, L.kq + g0 * L.kq_g, L.ks + g0 * L.ks_g, L.kz + g0 * L.ks_g, L.kq_d,
                                       item_off);
                }
                return;
            }
        }
        pr.flags = (kl < TILE && live(n0 + kl)) ? 256u : 0u;
        if constexpr (SRC == 0) {
            if constexpr (!FULL) {
                if (kl < Shape::NK) load_k_packed<D>(pr.w, L, kl, n0, n_end);
            }
        } else {
            const char *base = ds.k + (int64_t)(n0 - ds.tok0) * ds.sk * ds.esz;
            if constexpr (SRC == 2) {
                if (dense_fast && n0 + TILE <= n_end) {
                    const int64_t kstep = (int64_t)(KLANES / (D / 8)) * ds.sk * 2;
#pragma unroll
                    for (int r = 0; r < Shape::KPL; ++r) {
                        if (kl + r * KLANES < Shape::NK) {
                            const uint4 q = *(const uint4 *)(base + r * kstep + doff);
                            pr.w[4 * r] = q.x;
                            pr.w[4 * r + 1] = q.y;
                            pr.w[4 * r + 2] = q.z;
                            pr.w[4 * r + 3] = q.w;
                        }
                    }
                    pr.flags |= (1u << Shape::KPL) - 1u;
                    return;
                }
            }
#pragma unroll
            for (int r = 0; r < Shape::KPL; ++r) {
                const int u = kl + r * KLANES;
                if (u < Shape::NK && load_k_dense<D>(&pr.w[4 * r], base, ds.sk, ds.dtype, ds.esz, u, n_end - n0))
                    pr.flags |= 1u << r;
            }
        }
    };
    auto store_k = [&](uint16_t *Ks, uint64_t &km) {
        if constexpr (SRC == 0) {
            if (kl < Shape::NK) store_k_packed<D>(Ks, pr.w, kl);
        } else {
#pragma unroll
            for (int r = 0; r < Shape::KPL; ++r) {
                const int u = kl + r * KLANES;
                if (u < Shape::NK) store_k_dense<D>(Ks, &pr.w[4 * r], u, ds.dtype, (pr.flags >> r) & 1u);
            }
        }
        if (kl < TILE) {
            const uint64_t m = __ballot((pr.flags & 256u) != 0);
            if (kl == 0) km = m;
        }
    };
    auto load_v = [&](int i) {
        const int n0 = tile_n0(i);
        if constexpr (SRC == 0) {
            if (FULL || (fast_tiles && n0 + TILE <= n_end)) {
                if (vl < Shape::NV) {
                    load_v_packed_fast(pr.w, L.vq + (int64_t)n0 * L.vq_n, L.vs + (int64_t)n0 * L.vs_n,
                                       L.vz + (int64_t)n0 * L.vs_n, L.vq_n, L.vs_n, item_off);
                    pr.flags = 3u;
                }
                return;
            }
            if constexpr (!FULL) {
                if (vl < Shape::NV) load_v_packed<D>(pr.w, pr.flags, L, vl, n0, n_end);
            }
        } else {
            const char *base = ds.v + (int64_t)(n0 - ds.tok0) * ds.sv * ds.esz;
            if constexpr (SRC == 2) {
                if (dense_fast && n0 + TILE <= n_end) {
#pragma unroll
                    for (int r = 0; r < Shape::VPL; ++r) {
                        if (vl + r * KLANES < Shape::NV) {
                            const char *pa = base + r * (KLANES / (TILE / 2)) * 16 + doff;
                            const uint4 qa = *(const uint4 *)pa;
                            const uint4 qb = *(const uint4 *)(pa + ds.sv * 2);
                            pr.w[8 * r] = qa.x;
                            pr.w[8 * r + 1] = qa.y;
                            pr.w[8 * r + 2] = qa.z;
                            pr.w[8 * r + 3] = qa.w;
                            pr.w[8 * r + 4] = qb.x;
                            pr.w[8 * r + 5] = qb.y;
                            pr.w[8 * r + 6] = qb.z;
                            pr.w[8 * r + 7] = qb.w;
                        }
                    }
                    pr.flags = (1u << (2 * Shape::VPL)) - 1u;
                    return;
                }
            }
            pr.flags = 0u;
#pragma unroll
            for (int r = 0; r < Shape::VPL; ++r) {
                const int u = vl + r * KLANES;
                if (u < Shape::NV) {
                    const int tp = u % (TILE / 2);
                    load_v_dense<D>(&pr.w[8 * r], base, ds.sv, ds.dtype, ds.esz, u, n_end - n0);
                    pr.flags |= (live(n0 + 2 * tp) ? 1u : 0u) << (2 * r);
                    pr.flags |= (live(n0 + 2 * tp + 1) ? 1u : 0u) << (2 * r + 1);
                }
            }
        }
    };
    auto store_v = [&](uint16_t *Vt) {
        if constexpr (SRC == 0) {
            if (vl < Shape::NV) store_v_packed<D>(Vt, pr.w, vl);
        } else {
#pragma unroll
            for (int r = 0; r < Shape::VPL; ++r) {
                const int u = vl + r * KLANES;
                if (u < Shape::NV)
                    store_v_dense<D>(Vt, &pr.w[8 * r], u, ds.dtype, (pr.flags >> (2 * r)) & 1u,
                                     (pr.flags >> (2 * r + 1)) & 1u);
            }
        }
    };
    auto load_tile = [&](int i) {
        if (is_k) load_k(i);
        else load_v(i);
    };
    // the buffer's byte offset is made opaque to the compiler, so that the row addresses of
    // a store are immediate offsets from one register instead of per-buffer constants held
    // across the loop (the third buffer lies beyond the 16-bit immediate range)
    auto store_tile = [&](int buf) {
        if (is_k) {
            int off = buf * (int)sizeof(KTileL<D>);
            asm volatile("" : "+v"(off));
            store_k((uint16_t *)((char *)S.u.t.kt[0].k + off), S.kmask[buf]);
        } else {
            int off = buf * (int)sizeof(VTileL<D>);
            asm volatile("" : "+v"(off));
            store_v((uint16_t *)((char *)S.u.t.vt[0].vt + off));
        }
    };

    const int qpos = a.q_pos0 + (row_ok ? row % a.T : 0);
    const bool causal = wk.cur && a.causal > 0;

    // prologue: tiles 0 and 1 staged, tile 2's loads in flight; Q of the row tile
    if (nt > 0) load_tile(0);
    bf16x8_t qf[NKS];
    if (is_s) {
        const int g = row_ok ? row / a.T : 0, t = row_ok ? row % a.T : 0;
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = ma_load8_as_bf16(a.q.ptr, qb + ks * 16 + hf * 8, a.q.dtype);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = row_ok ? qf[ks] : bf16x8_t{};
    }
    if (nt > 0) store_tile(0);
    if (nt > 1) {
        load_tile(1);
        store_tile(1);
    }
    if (nt > 2) load_tile(2);
    __syncthreads();

    float m_ref = -INFINITY, m_true = -INFINITY, l = 0.f;
    f32x16_t acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x16_t{};
    // Iteration it: S^T of tile it+1 is issued first (its MFMAs run while this wave does the
    // softmax of tile it, whose S^T the previous iteration issued), then PV of tile it, then
    // tile it+2 is staged into the buffer tiles it-1 used (both read before the last two
    // barriers) and the loads of tile it+3 are issued.
    f32x16_t sa[2], sb[2];
    if (is_s && nt > 0) s_qk<D>(S.u.t.kt[0].k, qf, c32, hf, sa);
    auto step = [&](int it, f32x16_t *sc, f32x16_t *sn) {
        const int cb = it % NBUF;
        const uint64_t mc = S.kmask[cb];
        if (is_s) {
            if constexpr (!FULL) {
                const int n0 = tile_n0(it);
                const int lim = causal ? (qpos / a.causal + 1) * a.causal - a.c_pos0 - n0 - hf * 4 : TILE;
                if (causal || mc != ~0ull) {
                    const uint64_t okh = mc >> (hf * 4);
#pragma unroll
                    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int tk = t2 * 32 + (i >> 2) * 8 + (i & 3);
                            const bool ok = ((okh >> tk) & 1) && tk < lim;
                            sc[t2][i] = ok ? sc[t2][i] : -INFINITY;
                        }
                }
            }
            float alpha, off;
            const bool resc = __any(sm_max(sc, m_ref, m_true, l, a.sl2, alpha, off));
            // S^T of tile it+1 (issued on the last tile too: that buffer holds an earlier
            // tile, whose result is never used), its 16 MFMAs interleaved with the exp2 part
            bf16x8_t pb[4];
            qk_exp<D>(S.u.t.kt[(it + 1) % NBUF].k, qf, c32, hf, sn, sc, l, a.sl2, off, pb);
            if (resc) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
            }
            pv_regs<D>(S.u.t.vt[cb].vt, pb, acc, c32, hf);
        }
        if (it + 2 < nt) {
            store_tile((it + 2) % NBUF);
            if (it + 3 < nt) load_tile(it + 3);
        }
        __syncthreads();
    };
    int it = 0;
    for (; it + 2 <= nt; it += 2) {
        step(it, sa, sb);
        step(it + 1, sb, sa);
    }
    if (it < nt) step(it, sa, sb);
    // every wave is past its last read of the K / V buffers: they take the O tiles
    if (is_s) write_partial<D>(a, acc, m_ref, m_true, l, bh, slot, rtile, c32, hf, lane, &S.u.o[wave][0]);
}

// Pass 2: grid (R, B*H), 128 threads = 8 split lanes x 16 channel octets.  Split lane
// sl sums splits sl, sl+8, ... in order with weights l_s * exp(m_s - M); its loads for 8
// splits (statistics and O) are issued together, the first batch before the maximum M over
// the prefix splits is known.  The 8 lanes' sums are added in lane order through LDS, so
// the result does not depend on timing.  Then the current block's partial joins.
constexpr int CMB_SL = 8;

template <int D>
__global__ void __launch_bounds__(128) splitk_combine_kernel(FwdArgs a, ma_tensor4 out, float *mp_out, float *lp_out,
                                                             void *op_out) {
    constexpr int OCT = D / 8;
    typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
    __shared__ float red[CMB_SL][D];
    __shared__ float lred[CMB_SL];
    __shared__ float smax[128 / 64];
    // workgroup id -> (row, lane) lane-fastest, as pass 1 numbers its workgroups, so a
    // lane's rows are merged on the XCDs whose L2 took that lane's partials
    const int BH = gridDim.x / a.R;
    const int row = blockIdx.x / BH, bh = blockIdx.x % BH, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int R = a.R, nsplit = a.nsplit;
    const int64_t base = (int64_t)bh * (nsplit + 1) * R + row;
    const int sl = tid / OCT, oc = tid % OCT;
    const bool lane_ok = sl < CMB_SL;
    // one batch: splits i0 + u*8, u < 8, of this split lane
    f16x8_t o[8];
    float bm[8], bl[8], bs[8];
    auto load_batch = [&](int i0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * CMB_SL;
            bm[u] = -INFINITY;
            bl[u] = 0.f;
            bs[u] = 0.f;
            o[u] = f16x8_t{};
            if (lane_ok && i < nsplit) {
                const int64_t pr = base + (int64_t)i * R;
                bm[u] = a.wm[pr];
                bl[u] = a.wl[pr];
                bs[u] = a.wsc[pr];
                o[u] = *(const f16x8_t *)&a.wo[pr * D + oc * 8];
            }
        }
    };
    load_batch(sl);
    // the current block's partial (slot nsplit), needed after the reduction
    const int64_t pc = base + (int64_t)nsplit * R;
    float mc = -INFINITY, lc = 0.f, oc_raw = 0.f, sc_c = 0.f;
    if (tid < D) {
        mc = a.wm[pc];
        lc = a.wl[pc];
        oc_raw = (float)a.wo[pc * D + tid];
        sc_c = a.wsc[pc];
    }
    // M = max over the prefix splits
    float m = -INFINITY;
    for (int sp = tid; sp < nsplit; sp += 128) m = fmaxf(m, a.wm[base + (int64_t)sp * R]);
    m = ma_wave_max(m);
    if ((tid & 63) == 0) smax[tid >> 6] = m;
    __syncthreads();
    const float M = fmaxf(smax[0], smax[1]);
    const float msafe = M == -INFINITY ? 0.f : M;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    for (int i0 = sl; lane_ok && i0 < nsplit;) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * CMB_SL;
            const float w = bl[u] * expf(bm[u] - msafe);
            if (i < nsplit && w != 0.f) {   // an empty split (weight 0) adds nothing
                const float ws = w * bs[u];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(ws, (float)o[u][e], acc[e]);
                lsum += w;
            }
        }
        i0 += 8 * CMB_SL;
        if (i0 < nsplit) load_batch(i0);
    }
    if (lane_ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[sl][oc * 8 + e] = acc[e];
        if (oc == 0) lred[sl] = lsum;
    }
    __syncthreads();
    if (tid >= D) return;
    const int d = tid;
    float op = 0.f, lp = 0.f;
#pragma unroll
    for (int k = 0; k < CMB_SL; ++k) {
        op += red[k][d];
        lp += lred[k];
    }
    // current block (slot nsplit)
    const float oc_d = lc > 0.f ? oc_raw * sc_c : 0.f;
    const float mm = fmaxf(M, mc);
    const float ms = (mm == -INFINITY) ? 0.f : mm;
    const float ea = expf(M - ms), eb = expf(mc - ms);
    const float den = lp * ea + lc * eb;
    const float inv = 1.0f / (den > 0.f ? den : 1.0f);
    const int g = row / a.T, t = row % a.T;
    const int64_t ob = b * out.s[0] + (int64_t)(h * a.G + g) * out.s[1] + (int64_t)t * out.s[2] + d;
    ma_store_f(out.ptr, ob, out.dtype, (op * ea + lc * oc_d * eb) * inv);
    if (mp_out) {
        if (d == 0) {
            mp_out[(int64_t)bh * R + row] = M;
            lp_out[(int64_t)bh * R + row] = lp;
        }
        ma_store_f(op_out, ((int64_t)bh * R + row) * D + d, out.dtype, op * (1.0f / (lp > 0.f ? lp : 1.0f)));
    }
}

// Tokens per split: about one workgroup per CU (a workgroup's 256 VGPRs per lane and
// 108 KB of LDS fill a CU), with
// one CU per (lane, row group) left for the current block's workgroups, so every
// workgroup of the launch runs in the first dispatch wave; at least one 64-token tile.
// Short prefixes (a sub-step's 2 048 selected entries) thus spread over many CUs: each
// workgroup's cost is mostly fixed latency, so more, shorter splits finish sooner
// (22.1 -> 17.9 us per sub-step at 4 KV heads x 2 048 entries, measured).
int choose_split(int n, int BH, int row_groups, int split_tokens) {
    if (split_tokens > 0) return split_tokens;
    const int units = BH * row_groups;
    int per = ma_num_cus() / units - 1;
    if (per < 1) per = 1;
    int sn = (n + per - 1) / per;
    sn = ((sn + TILE - 1) / TILE) * TILE;
    if (sn < TILE) sn = TILE;
    return sn;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

// Slots of the partials: ceil(nq / sn) packed splits, ceil(nf / sn) 16-bit splits, then
// the current block.
static int slot_count(int nq, int nf, int sn) { return (nq + sn - 1) / sn + (nf + sn - 1) / sn; }

static int row_groups_of(int Hq, int H, int T) {
    const int row_tiles = ((Hq / H) * T + 31) / 32;
    return (row_tiles + MAXS - 1) / MAXS;
}

extern "C" int64_t ma_splitk_workspace_bytes(int B, int H, int Hq, int T, int D, int nq, int nf,
                                             int split_tokens) {
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || D <= 0 || nq < 0 || nf < 0) return -1;
    const int R = (Hq / H) * T;
    const int sn = choose_split(nq + nf, B * H, row_groups_of(Hq, H, T), split_tokens);
    const int nsplit = slot_count(nq, nf, sn);
    const int64_t rows = (int64_t)B * H * (nsplit + 1) * R;
    return rows * 4 * 3 + rows * D * 2 + 256;
}

namespace {

struct Plan {
    FwdArgs fa;
    int row_groups, D, B;
};

int make_plan(Plan &pl, const char *who, ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
              ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale,
              int split_tokens, void *workspace, int64_t workspace_bytes) {
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || Tc < 0 || !q.ptr || !workspace) {
        ma_set_error("%s: bad sizes (B=%d H=%d Hq=%d T=%d Tc=%d) or NULL pointer", who, B, H, Hq, T, Tc);
        return MA_EINVAL;
    }
    if (split_tokens < 0 || split_tokens % TILE) {
        ma_set_error("%s: split_tokens %d must be a multiple of %d", who, split_tokens, TILE);
        return MA_EINVAL;
    }
    if (Tc > 0 && (!kc.ptr || !vc.ptr)) {
        ma_set_error("%s: current block pointers missing", who);
        return MA_EINVAL;
    }
    // 16-byte fragment loads: bases and row strides of the 16-bit operands must allow them
    auto vec_ok = [](const void *ptr, const int64_t *s, int dt) {
        if (!ptr) return true;
        int64_t m = dt == MA_F32 ? 4 : 8;
        return aligned16(ptr) && s[0] % m == 0 && s[1] % m == 0 && s[2] % m == 0;
    };
    if (!vec_ok(q.ptr, q.s, q.dtype) || !vec_ok(Tc ? kc.ptr : nullptr, kc.s, kc.dtype) ||
        !vec_ok(Tc ? vc.ptr : nullptr, vc.s, vc.dtype) || !vec_ok(p->nf ? p->kf : nullptr, p->skf, p->fdtype) ||
        !vec_ok(p->nf ? p->vf : nullptr, p->svf, p->fdtype)) {
        ma_set_error("%s: operands must be 16-byte aligned with strides that keep rows aligned", who);
        return MA_EINVAL;
    }
    const int G = Hq / H;
    const int R = G * T;
    const int row_tiles = (R + 31) / 32;
    const int row_groups = (row_tiles + MAXS - 1) / MAXS;
    const int n = p->nq + p->nf;
    const int sn = choose_split(n, B * H, row_groups, split_tokens);
    const int nsplit = slot_count(p->nq, p->nf, sn);
    const int64_t need = ma_splitk_workspace_bytes(B, H, Hq, T, D, p->nq, p->nf, sn);
    if (workspace_bytes < need) {
        ma_set_error("%s: workspace %lld bytes < %lld needed", who, (long long)workspace_bytes, (long long)need);
        return MA_EWORKSPACE;
    }
    const int64_t rows = (int64_t)B * H * (nsplit + 1) * R;
    float *wm = (float *)workspace;
    float *wl = wm + rows;
    float *wsc = wl + rows;
    _Float16 *wo = (_Float16 *)(((uintptr_t)(wsc + rows) + 15) & ~(uintptr_t)15);
    FwdArgs &fa = pl.fa;
    fa.q = q;
    fa.pre = prefix_dev(p, B, H);
    fa.kc = kc;
    fa.vc = vc;
    fa.H = H;
    fa.G = G;
    fa.T = T;
    fa.R = R;
    fa.Tc = Tc;
    fa.nsplit = nsplit;
    fa.split_n = sn;
    fa.causal = causal_block;
    fa.q_pos0 = q_pos0;
    fa.c_pos0 = c_pos0;
    fa.row_tiles = row_tiles;
    fa.row_groups = row_groups;
    fa.BH = B * H;
    fa.scale = scale;
    fa.sl2 = scale * MA_LOG2E;
    fa.wm = wm;
    fa.wl = wl;
    fa.wsc = wsc;
    fa.wo = wo;
    pl.row_groups = row_groups;
    pl.D = D;
    pl.B = B;
    return MA_OK;
}

template <int D>
int launch_partial_d(const Plan &pl, hipStream_t st) {
    // packed part [0, nq) and 16-bit part [nq, n) in a launch each; the current block is
    // attended in the merge
    FwdArgs fa = pl.fa;
    const int nq = fa.pre.nq, nf = fa.pre.nf, sn = fa.split_n;
    const int units = pl.B * fa.H * pl.row_groups;
    const int nsq = (nq + sn - 1) / sn, nsf = (nf + sn - 1) / sn;
    // the current block's workgroups (last in the grid) ride with the packed launch when
    // there is no 16-bit part, else with the 16-bit one
    const bool cur_in_packed = nsq > 0 && nsf == 0;
    if (nsq) {
        fa.nsp = nsq;
        fa.slot0 = 0;
        fa.tok_beg = 0;
        fa.tok_end = nq;
        fa.with_cur = cur_in_packed;
        // whole tiles everywhere: no slot mask, a packed part of whole tiles (every split is)
        const bool full = !fa.pre.mask && nq % TILE == 0;
        if (full)
            hipLaunchKernelGGL((splitk_fwd_kernel<D, 0, true>), dim3((nsq + fa.with_cur) * units), dim3(NTH), 0, st,
                               fa);
        else
            hipLaunchKernelGGL((splitk_fwd_kernel<D, 0, false>), dim3((nsq + fa.with_cur) * units), dim3(NTH), 0,
                               st, fa);
    }
    if (!cur_in_packed) {
        fa.nsp = nsf;
        fa.slot0 = nsq;
        fa.tok_beg = nq;
        fa.tok_end = nq + nf;
        fa.with_cur = 1;
        const bool bf = (nf == 0 || fa.pre.fdtype == MA_BF16) &&
                        (fa.Tc == 0 || (fa.kc.dtype == MA_BF16 && fa.vc.dtype == MA_BF16));
        if (bf)
            hipLaunchKernelGGL((splitk_fwd_kernel<D, 2, false>), dim3((nsf + 1) * units), dim3(NTH), 0, st, fa);
        else
            hipLaunchKernelGGL((splitk_fwd_kernel<D, 1, false>), dim3((nsf + 1) * units), dim3(NTH), 0, st, fa);
    }
    return ma_check_launch("ma_splitk_partial");
}

int launch_partial(const Plan &pl, hipStream_t st) {
    return pl.D == 128 ? launch_partial_d<128>(pl, st) : launch_partial_d<64>(pl, st);
}

int launch_merge(const Plan &pl, ma_tensor4 out, float *mp, float *lp, void *op, hipStream_t st) {
    if (!out.ptr) {
        ma_set_error("ma_splitk_merge: output is NULL");
        return MA_EINVAL;
    }
    if ((mp || lp || op) && !(mp && lp && op)) {
        ma_set_error("ma_splitk_merge: mp, lp and op go together");
        return MA_EINVAL;
    }
    const FwdArgs &fa = pl.fa;
    const dim3 cgrid(fa.R * pl.B * fa.H);
    if (pl.D == 128)
        hipLaunchKernelGGL(splitk_combine_kernel<128>, cgrid, dim3(128), 0, st, fa, out, mp, lp, op);
    else
        hipLaunchKernelGGL(splitk_combine_kernel<64>, cgrid, dim3(128), 0, st, fa, out, mp, lp, op);
    return ma_check_launch("ma_splitk_merge");
}

}  // namespace

extern "C" int ma_splitk_partial(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                                 ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale,
                                 int split_tokens, void *workspace, int64_t workspace_bytes, void *stream) {
    Plan pl;
    int rc = make_plan(pl, "ma_splitk_partial", q, B, Hq, T, D, p, H, kc, vc, Tc, causal_block, q_pos0, c_pos0, scale,
                       split_tokens, workspace, workspace_bytes);
    if (rc) return rc;
    return launch_partial(pl, (hipStream_t)stream);
}

extern "C" int ma_splitk_merge(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                               ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale,
                               ma_tensor4 out, float *mp, float *lp, void *op, int split_tokens, void *workspace,
                               int64_t workspace_bytes, void *stream) {
    Plan pl;
    int rc = make_plan(pl, "ma_splitk_merge", q, B, Hq, T, D, p, H, kc, vc, Tc, causal_block, q_pos0, c_pos0, scale,
                       split_tokens, workspace, workspace_bytes);
    if (rc) return rc;
    return launch_merge(pl, out, mp, lp, op, (hipStream_t)stream);
}

extern "C" int ma_splitk_attention(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                   ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0,
                                   float scale, ma_tensor4 out, float *mp, float *lp, void *op, int split_tokens,
                                   void *workspace, int64_t workspace_bytes, void *stream) {
    Plan pl;
    int rc = make_plan(pl, "ma_splitk_attention", q, B, Hq, T, D, p, H, kc, vc, Tc, causal_block, q_pos0, c_pos0,
                       scale, split_tokens, workspace, workspace_bytes);
    if (rc) return rc;
    rc = launch_partial(pl, (hipStream_t)stream);
    if (rc) return rc;
    return launch_merge(pl, out, mp, lp, op, (hipStream_t)stream);
}

// ---------------------------------------------------------------- no-allocation variant
// ma_splitk_attention with its split partials in a library-owned device array instead of a
// caller workspace, for callers that cannot allocate (code under HIP graph capture, tight
// serving loops).  The array is a file-scope __device__ symbol: each device the library
// runs on holds its own copy, at its own address, until the process ends.  Its device
// address is looked up once per device with hipGetSymbolAddress (the symbol's name in host
// code is only a host-side stand-in, never a device pointer) and that address is what the
// kernels receive.  Nothing in the partials needs clearing: pass 1 writes every slot the
// merge reads.  Calls that overlap in time on one device share the array and race.
namespace {

constexpr int64_t NOALLOC_SCRATCH_BYTES = 32ll << 20;
__device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// the device address of `scratch` on the current device (looked up on the first call)
int scratch_address(void **out, const char *who) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        ma_set_error("%s: no current device (%s)", who, e != hipSuccess ? hipGetErrorString(e) : "out of range");
        return MA_EHIP;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            ma_set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                         hipGetErrorString(e));
            return MA_EHIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MA_OK;
}

}  // namespace

extern "C" int64_t ma_splitk_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int ma_splitk_attention_noalloc(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                           ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0,
                                           int c_pos0, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
                                           int split_tokens, void *stream) {
    const char *who = "ma_splitk_attention_noalloc";
    const int64_t need = p ? ma_splitk_workspace_bytes(B, H, Hq, T, D, p->nq, p->nf, split_tokens) : -1;
    if (need < 0) {
        ma_set_error("%s: bad geometry (B=%d H=%d Hq=%d T=%d D=%d)", who, B, H, Hq, T, D);
        return MA_EINVAL;
    }
    if (need > NOALLOC_SCRATCH_BYTES) {
        ma_set_error("%s: this call needs %lld bytes of split partials, above the library's fixed %lld-byte "
                     "scratch; use ma_splitk_attention with a workspace",
                     who, (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
        return MA_EWORKSPACE;
    }
    void *ws = nullptr;
    int rc = scratch_address(&ws, who);
    if (rc) return rc;
    Plan pl;
    rc = make_plan(pl, who, q, B, Hq, T, D, p, H, kc, vc, Tc, causal_block, q_pos0, c_pos0, scale, split_tokens, ws,
                   NOALLOC_SCRATCH_BYTES);
    if (rc) return rc;
    rc = launch_partial(pl, (hipStream_t)stream);
    if (rc) return rc;
    return launch_merge(pl, out, mp, lp, op, (hipStream_t)stream);
}
