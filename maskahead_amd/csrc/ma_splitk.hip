// Split-K (flash-decoding) attention over [prefix | current block] for every query row
// of a KV head's GQA group (the reference's splitk_attention, splitk.py:493-579).
//
// Pass 1 (splitk_fwd_kernel): grid (nsplit + 1, B*H, row groups).  Workgroup = one
// prefix split (or, for blockIdx.x == nsplit, the current block) x up to 8 row tiles of
// 32 query rows, one wave per row tile.  Per 64-token tile the workgroup stages K as
// Ks[t][d] and V as Vt[d][t] (bf16, dequantized in the load path for packed caches) in
// LDS; each wave then computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = K rows,
// B = Q^T held in registers), so every lane owns ONE query row and a strip of 16 tokens
// per 32-token sub-tile: the row max needs one cross-half exchange, no shuffle trees.
// The exponentiated S^T registers are the B operand of O^T += V^T P^T directly (the
// token order of the MFMA's K index is permuted consistently on both operands), and the
// O^T accumulator keeps the lane's row too, so the online-softmax rescale is per lane.
// Pass 2 (splitk_combine_kernel): log-sum-exp merge of the partials into the output and
// the prefix-only statistics (M_p, L_p, O_p) of splitk.py:272-318.
#include <type_traits>

#include "ma_tile.h"

using namespace ma;

namespace {

constexpr int MAX_WAVES = NT / 64;
// a row's running reference max is raised only when a tile's max exceeds it by more than
// 2^8 in exp2 units, so most tiles skip the accumulator rescale; p <= 2^8 stays exact
constexpr float LAZY_LOG2 = 8.0f;

struct FwdArgs {
    ma_tensor4 q;
    PrefixDev pre;
    ma_tensor4 kc, vc;
    int H, G, T, R, Tc, nsplit, split_n, causal, q_pos0, c_pos0, row_tiles;
    float sl2;  // scale * log2(e)
    float scale;
    float *wm, *wl, *wacc;  // partials [B*H][nsplit+1][R] and [..][R][D]
};

// Online-softmax state of one query row (the lane's column of S^T); l and acc are
// relative to m_ref, m_true is the exact running max (raw logit units).
template <int D>
struct RowState {
    float m_ref, m_true, l;
    f32x16_t acc[D / 32];
};

template <int D>
__device__ __forceinline__ void row_reset(RowState<D> &st) {
    st.m_ref = -INFINITY;
    st.m_true = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] = f32x16_t{};
}

// One 64-token tile for a wave's 32 rows: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <int D>
__device__ __forceinline__ void attend_tile(const TileLds<D> &L, const bf16x8_t *qf, RowState<D> &st, int c32, int hf,
                                            bool need_mask, int lim, float sl2) {
    constexpr int KS = TileLds<D>::KS, VS = TileLds<D>::VS;
    constexpr int NKS = D / 16, NDT = D / 32;
    f32x16_t s[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
        s[t2] = f32x16_t{};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const bf16x8_t ka = *(const bf16x8_t *)&L.k[(t2 * 32 + c32) * KS + ks * 16 + hf * 8];
            s[t2] = ma_mfma32(ka, qf[ks], s[t2]);
        }
    }
    // element i of s[t2] <-> token t2*32 + (i/4)*8 + hf*4 + i%4
    if (need_mask) {
        const uint64_t okm = L.okmask >> (hf * 4);
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tk = t2 * 32 + (i >> 2) * 8 + (i & 3);
                const bool ok = ((okm >> tk) & 1) && tk < lim;
                s[t2][i] = ok ? s[t2][i] : -INFINITY;
            }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[t2][i]);
    mt = ma_max_xor32(mt);
    st.m_true = fmaxf(st.m_true, mt);
    const bool need = (mt - st.m_ref) * sl2 > LAZY_LOG2;   // false for NaN (both -inf)
    if (__any(need)) {
        const float m_new = need ? mt : st.m_ref;
        const float alpha = (m_new == st.m_ref) ? 1.0f : __builtin_amdgcn_exp2f((st.m_ref - m_new) * sl2);
        st.l *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) st.acc[dt] *= alpha;
        st.m_ref = m_new;
    }
    const float off = (st.m_ref == -INFINITY) ? 0.f : -st.m_ref * sl2;
    float ls = 0.f;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t2][i], sl2, off));
            s[t2][i] = p;
            ls += p;
        }
    st.l += ma_sum_xor32(ls);
    // P^T chunks (B operand): chunk c = 16 tokens, lane holds s[c/2][8*(c%2) .. +7]
    bf16x8_t pb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[c][j] = (__bf16)s[c >> 1][(c & 1) * 8 + j];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        const uint16_t *vrow = &L.vt[(dt * 32 + c32) * VS];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bf16x4_t lo = *(const bf16x4_t *)&vrow[c * 16 + hf * 4];
            const bf16x4_t hi = *(const bf16x4_t *)&vrow[c * 16 + 8 + hf * 4];
            const bf16x8_t va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            st.acc[dt] = ma_mfma32(va, pb[c], st.acc[dt]);
        }
    }
}

// write a row's partial (max in natural-log units, l and acc relative to the exact max)
template <int D>
__device__ __forceinline__ void write_partial(const FwdArgs &a, const RowState<D> &st, int bh, int slot, int row,
                                              int hf) {
    constexpr int NDT = D / 32;
    const int64_t prow = ((int64_t)bh * (a.nsplit + 1) + slot) * a.R + row;
    float f = 0.f;
    if (st.m_true != -INFINITY) f = __builtin_amdgcn_exp2f((st.m_ref - st.m_true) * a.sl2);
    if (hf == 0) {
        a.wm[prow] = st.m_true * a.scale;
        a.wl[prow] = st.l * f;
    }
    float *dst = a.wacc + prow * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4_t v = {st.acc[dt][q4 * 4 + 0] * f, st.acc[dt][q4 * 4 + 1] * f, st.acc[dt][q4 * 4 + 2] * f,
                               st.acc[dt][q4 * 4 + 3] * f};
            *(f32x4_t *)&dst[dt * 32 + q4 * 8 + hf * 4] = v;
        }
}

enum { SRC_PACKED = 0, SRC_DENSE = 1 };

// grid (max(nsplit,1), B*H, row groups), NT threads.  Split sp covers prefix tokens
// [sp*split_n, (sp+1)*split_n); split 0 also attends the current block afterwards and
// writes it as partial slot nsplit.  The prefix tiles of the source kind SRC run through
// the register prefetch (the next tile's loads are in flight while the current one is
// computed); with a packed prefix, its 16-bit residual tail and the current block are
// staged synchronously (a few tiles per call).
template <int D, int SRC>
__global__ void __launch_bounds__(NT) splitk_fwd_kernel(FwdArgs a) {
    __shared__ TileLds<D> T;
    constexpr int NKS = D / 16;

    const int sp = blockIdx.x, bh = blockIdx.y;
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;
    const int rtile = blockIdx.z * MAX_WAVES + wave;
    const int row = rtile * 32 + c32;
    const bool wave_active = rtile < a.row_tiles;
    const bool row_ok = row < a.R;
    const int g = row_ok ? row / a.T : 0, t = row_ok ? row % a.T : 0;

    bf16x8_t qf[NKS];
    {
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = ma_load8_as_bf16(a.q.ptr, qb + ks * 16 + hf * 8, a.q.dtype);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = row_ok ? qf[ks] : bf16x8_t{};
    }

    const Lane L = make_lane(a.pre, b, h, bh);
    const Dense kc = dense_lane(a.kc.ptr, a.kc.s, a.kc.dtype, b, h);
    const Dense vc = dense_lane(a.vc.ptr, a.vc.s, a.vc.dtype, b, h);
    const int nq = L.nq, ntot = L.ntot, Tc = a.Tc;
    const int pstart = sp * a.split_n;
    const int pend = min(pstart + a.split_n, ntot);
    const int n_pt = pstart < pend ? (pend - pstart + TILE - 1) / TILE : 0;
    const bool with_cur = sp == 0;
    const int n_ct = with_cur ? (Tc + TILE - 1) / TILE : 0;
    const int total = n_pt + n_ct;
    const int qpos = a.q_pos0 + t;
    const int causal = a.causal, c_pos0 = a.c_pos0;
    const float sl2 = a.sl2;

    const ItemOffsets off = SRC == SRC_PACKED ? packed_offsets<D>(L, tid) : dense_offsets<D>(L.kf_n, L.vf_n, L.esz, tid);
    const ItemOffsets coff = dense_offsets<D>(kc.sn, vc.sn, kc.esz, tid);

    auto tile_n0 = [&](int i) { return i < n_pt ? pstart + i * TILE : (i - n_pt) * TILE; };
    // does tile i go through the prefetch block?
    auto prefetched = [&](int i) {
        if (i >= n_pt) return SRC == SRC_DENSE;
        return prefix_tile_kind(nq, tile_n0(i), pend) == (SRC == SRC_PACKED ? TK_PACKED : TK_DENSE);
    };
    using PF = typename std::conditional<SRC == SRC_PACKED, PfPacked, PfDense>::type;
    auto load = [&](int i, PF &pf) {
        const int n0 = tile_n0(i);
        if constexpr (SRC == SRC_PACKED) {
            load_packed<D, true>(pf, L, off, n0, pend, tid);
        } else {
            if (i < n_pt) {
                const int64_t tb = (int64_t)(n0 - nq);
                load_dense<D, true>(pf, L.kf + tb * L.kf_n * L.esz, L.vf + tb * L.vf_n * L.esz, L.kf_n, L.vf_n,
                                    L.fdtype, L.esz, off, &L, n0, pend, tid);
            } else {
                load_dense<D, true>(pf, kc.base + (int64_t)n0 * kc.sn * kc.esz, vc.base + (int64_t)n0 * vc.sn * vc.esz,
                                    kc.sn, vc.sn, kc.dtype, kc.esz, coff, nullptr, n0, Tc, tid);
            }
        }
    };

    RowState<D> st;
    row_reset(st);
    PF pf;
    if (total > 0 && prefetched(0)) load(0, pf);
    for (int i = 0; i < total; ++i) {
        const bool cur = i >= n_pt;
        const int n0 = tile_n0(i);
        const int end = cur ? Tc : pend;
        __syncthreads();
        if (prefetched(i)) {
            if constexpr (SRC == SRC_PACKED) store_packed<D, true>(T, pf, tid);
            else store_dense<D, true>(T, pf, tid);
            store_okmask(T.okmask, pf, tid);
        } else if (cur) {
            PfDense tmp;
            load_dense<D, true>(tmp, kc.base + (int64_t)n0 * kc.sn * kc.esz, vc.base + (int64_t)n0 * vc.sn * vc.esz,
                                kc.sn, vc.sn, kc.dtype, kc.esz, coff, nullptr, n0, Tc, tid);
            store_dense<D, true>(T, tmp, tid);
            store_okmask(T.okmask, tmp, tid);
        } else {
            stage_generic<D, true>(T, L, n0, end, tid);
        }
        __syncthreads();
        if (i + 1 < total && prefetched(i + 1)) load(i + 1, pf);
        if (wave_active) {
            const bool cz = cur && causal > 0;
            const int lim = cz ? (qpos / causal + 1) * causal - c_pos0 - n0 - hf * 4 : TILE;
            const bool need_mask = cz || T.okmask != ~0ull;
            attend_tile<D>(T, qf, st, c32, hf, need_mask, lim, sl2);
        }
        if (i == n_pt - 1) {  // prefix segment done
            if (wave_active && row_ok) write_partial<D>(a, st, bh, sp, row, hf);
            row_reset(st);
        }
    }
    if (with_cur && wave_active && row_ok) write_partial<D>(a, st, bh, a.nsplit, row, hf);
}

// grid (ceil(R / rows_per_block), B*H), 256 threads; D/4 threads per row, 4 channels
// each.  First the exact maxima over the splits, then every split's weight is known and
// the loads of different splits are independent.
template <int D>
__global__ void __launch_bounds__(256) splitk_combine_kernel(const float *wm, const float *wl, const float *wacc,
                                                             int H, int G, int T, int R, int nsplit, ma_tensor4 out,
                                                             float *mp_out, float *lp_out, void *op_out) {
    constexpr int TPR = D / 4;
    constexpr int RPB = 256 / TPR;
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int row = blockIdx.x * RPB + threadIdx.x / TPR;
    const int d0 = (threadIdx.x % TPR) * 4;
    if (row >= R) return;
    const int64_t base = (int64_t)bh * (nsplit + 1) * R + row;
    float mp = -INFINITY;
#pragma unroll 16
    for (int sp = 0; sp < nsplit; ++sp) mp = fmaxf(mp, wm[base + (int64_t)sp * R]);
    const float msafe_p = (mp == -INFINITY) ? 0.f : mp;
    float lp = 0.f;
    f32x4_t op = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int sp = 0; sp < nsplit; ++sp) {
        const int64_t pr = base + (int64_t)sp * R;
        const float w = expf(wm[pr] - msafe_p);
        lp += wl[pr] * w;
        op += *(const f32x4_t *)&wacc[pr * D + d0] * w;
    }
    const int64_t pc = base + (int64_t)nsplit * R;
    const float mc = wm[pc], lc = wl[pc];
    const f32x4_t ac = *(const f32x4_t *)&wacc[pc * D + d0];
    const float m = fmaxf(mp, mc);
    const float msafe = (m == -INFINITY) ? 0.f : m;
    const float ea = expf(mp - msafe), eb = expf(mc - msafe);
    const float den = lp * ea + lc * eb;
    const float inv = 1.0f / (den > 0.f ? den : 1.0f);
    const int g = row / T, t = row % T;
    const int64_t ob = b * out.s[0] + (int64_t)(h * G + g) * out.s[1] + (int64_t)t * out.s[2] + d0;
#pragma unroll
    for (int e = 0; e < 4; ++e) ma_store_f(out.ptr, ob + e, out.dtype, (op[e] * ea + ac[e] * eb) * inv);
    if (mp_out) {
        if (d0 == 0) {
            mp_out[(int64_t)bh * R + row] = mp;
            lp_out[(int64_t)bh * R + row] = lp;
        }
        const float il = 1.0f / (lp > 0.f ? lp : 1.0f);
        const int64_t oo = ((int64_t)bh * R + row) * D + d0;
#pragma unroll
        for (int e = 0; e < 4; ++e) ma_store_f(op_out, oo + e, out.dtype, op[e] * il);
    }
}

int choose_split(int n, int BH, int row_groups, int split_tokens) {
    if (split_tokens > 0) return split_tokens;
    // aim at ~one workgroup per CU for the prefix splits; never below one tile
    int target = ma_num_cus();
    int per = target / (BH * row_groups);
    if (per < 1) per = 1;
    int sn = (n + per - 1) / per;
    sn = ((sn + TILE - 1) / TILE) * TILE;
    if (sn < 256) sn = 256;
    return sn;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

extern "C" int64_t ma_splitk_workspace_bytes(int B, int H, int Hq, int T, int D, int n, int split_tokens) {
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || D <= 0 || n < 0) return -1;
    const int R = (Hq / H) * T;
    const int row_tiles = (R + 31) / 32;
    const int row_groups = (row_tiles + MAX_WAVES - 1) / MAX_WAVES;
    const int sn = choose_split(n, B * H, row_groups, split_tokens);
    const int nsplit = n ? (n + sn - 1) / sn : 0;
    const int64_t rows = (int64_t)B * H * (nsplit + 1) * R;
    return rows * 4 * 2 + rows * D * 4 + 256;
}

namespace {

struct Plan {
    FwdArgs fa;
    int waves, row_groups, D, B;
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
    const int row_groups = (row_tiles + MAX_WAVES - 1) / MAX_WAVES;
    const int n = p->nq + p->nf;
    const int sn = choose_split(n, B * H, row_groups, split_tokens);
    const int nsplit = n ? (n + sn - 1) / sn : 0;
    const int64_t need = ma_splitk_workspace_bytes(B, H, Hq, T, D, n, sn);
    if (workspace_bytes < need) {
        ma_set_error("%s: workspace %lld bytes < %lld needed", who, (long long)workspace_bytes, (long long)need);
        return MA_EWORKSPACE;
    }
    const int64_t rows = (int64_t)B * H * (nsplit + 1) * R;
    float *wm = (float *)workspace;
    float *wl = wm + rows;
    float *wacc = (float *)(((uintptr_t)(wl + rows) + 15) & ~(uintptr_t)15);
    FwdArgs &fa = pl.fa;
    fa.q = q;
    fa.pre = prefix_dev(p);
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
    fa.scale = scale;
    fa.sl2 = scale * MA_LOG2E;
    fa.wm = wm;
    fa.wl = wl;
    fa.wacc = wacc;
    pl.waves = row_tiles < MAX_WAVES ? row_tiles : MAX_WAVES;
    pl.row_groups = row_groups;
    pl.D = D;
    pl.B = B;
    return MA_OK;
}

int launch_partial(const Plan &pl, hipStream_t st) {
    dim3 grid(pl.fa.nsplit > 0 ? pl.fa.nsplit : 1, pl.B * pl.fa.H, pl.row_groups);
    const bool packed = pl.fa.pre.nq > 0;
    if (pl.D == 128) {
        if (packed) hipLaunchKernelGGL((splitk_fwd_kernel<128, SRC_PACKED>), grid, dim3(NT), 0, st, pl.fa);
        else hipLaunchKernelGGL((splitk_fwd_kernel<128, SRC_DENSE>), grid, dim3(NT), 0, st, pl.fa);
    } else {
        if (packed) hipLaunchKernelGGL((splitk_fwd_kernel<64, SRC_PACKED>), grid, dim3(NT), 0, st, pl.fa);
        else hipLaunchKernelGGL((splitk_fwd_kernel<64, SRC_DENSE>), grid, dim3(NT), 0, st, pl.fa);
    }
    return ma_check_launch("ma_splitk_partial");
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
    const int rpb = 256 / (pl.D / 4);
    dim3 cgrid((fa.R + rpb - 1) / rpb, pl.B * fa.H);
    if (pl.D == 128)
        hipLaunchKernelGGL(splitk_combine_kernel<128>, cgrid, dim3(256), 0, st, fa.wm, fa.wl, fa.wacc, fa.H, fa.G,
                           fa.T, fa.R, fa.nsplit, out, mp, lp, op);
    else
        hipLaunchKernelGGL(splitk_combine_kernel<64>, cgrid, dim3(256), 0, st, fa.wm, fa.wl, fa.wacc, fa.H, fa.G,
                           fa.T, fa.R, fa.nsplit, out, mp, lp, op);
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

extern "C" int ma_splitk_merge(int B, int Hq, int T, int D, int H, int n, int split_tokens, ma_tensor4 out,
                               float *mp, float *lp, void *op, void *workspace, int64_t workspace_bytes,
                               void *stream) {
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || n < 0 || (D != 64 && D != 128) || !workspace ||
        split_tokens < 0 || split_tokens % TILE) {
        ma_set_error("ma_splitk_merge: bad sizes");
        return MA_EINVAL;
    }
    const int64_t need = ma_splitk_workspace_bytes(B, H, Hq, T, D, n, split_tokens);
    if (workspace_bytes < need) {
        ma_set_error("ma_splitk_merge: workspace %lld bytes < %lld needed", (long long)workspace_bytes,
                     (long long)need);
        return MA_EWORKSPACE;
    }
    Plan pl;
    const int G = Hq / H, R = G * T;
    const int row_tiles = (R + 31) / 32;
    const int row_groups = (row_tiles + MAX_WAVES - 1) / MAX_WAVES;
    const int sn = choose_split(n, B * H, row_groups, split_tokens);
    const int nsplit = n ? (n + sn - 1) / sn : 0;
    const int64_t rows = (int64_t)B * H * (nsplit + 1) * R;
    pl.fa.wm = (float *)workspace;
    pl.fa.wl = pl.fa.wm + rows;
    pl.fa.wacc = (float *)(((uintptr_t)(pl.fa.wl + rows) + 15) & ~(uintptr_t)15);
    pl.fa.H = H;
    pl.fa.G = G;
    pl.fa.T = T;
    pl.fa.R = R;
    pl.fa.nsplit = nsplit;
    pl.D = D;
    pl.B = B;
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
