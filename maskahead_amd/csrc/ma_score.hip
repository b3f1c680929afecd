// Pass 2 of step 0 (the reference's prefix_scores, splitk.py:582-614, kernel 321-371):
// per prefix entry j of a KV head,
//   mass[j]  = (1/(G*T2)) * sum over the selection rows r of exp(s_rj - M_p[r]) / L_p[r]
//   score[j] = mass[j] * || v_j - centre ||          (value-aware ranking)
// Workgroup = a run of 64-token tiles of one (batch, KV head) lane; up to 8 waves, each
// owning one or two 32-row tiles of the selection rows with their Q fragments held in
// registers.  Per tile the keys are staged (dequantized) in LDS as Ks[t][d] and each wave
// computes S = Q K^T with v_mfma_f32_32x32x16_bf16 (A = Q, B = K^T), so a lane holds ONE
// token and 16 rows: the sum over rows is in-register plus one cross-half exchange, then
// one LDS reduction over waves.  The value distance reads V once per entry, dequantized
// (and rounded to bf16 when the reference would read its unpacked bf16 prefix).
#include <type_traits>

#include "ma_tile.h"

using namespace ma;

namespace {

constexpr int MAX_WAVES = NT / 64;
enum { SRC_PACKED = 0, SRC_DENSE = 1 };

// centre[b,h,:] = mean over rows g*T + q_rows[t2] of f32(op): NTH threads as D channels
// x (NTH/D) row slices, each slice summing its rows in order, then the slices in order --
// one fixed summation order, shared by the score kernel's prologue and ma_value_centre.
template <int D, int NTH>
__device__ __forceinline__ float centre_partial(const void *op, int op_dtype, int bh, int G, int T,
                                                const int32_t *q_rows, int T2, int tid) {
    constexpr int SL = NTH / D;
    const int d = tid % D, sl = tid / D;
    const int R = G * T, R2 = G * T2;
    float s = 0.f;
    // one loop per dtype: no branch around the loads, which can then all be in flight
    if (op_dtype == MA_F32) {
        const float *o = (const float *)op;
#pragma unroll 8
        for (int rr = sl; rr < R2; rr += SL) {
            const int row = (rr / T2) * T + min(max(q_rows[rr % T2], 0), T - 1);
            s += o[((int64_t)bh * R + row) * D + d];
        }
    } else {
        const uint16_t *o = (const uint16_t *)op;
        const bool bf = op_dtype == MA_BF16;
#pragma unroll 8
        for (int rr = sl; rr < R2; rr += SL) {
            const int row = (rr / T2) * T + min(max(q_rows[rr % T2], 0), T - 1);
            const uint16_t x = o[((int64_t)bh * R + row) * D + d];
            s += bf ? ma_bf16_to_f32(x) : ma_f16_to_f32(x);
        }
    }
    return s;
}

template <int D, int NTH>
__device__ __forceinline__ float centre_combine(const float *part, int d, int R2) {
    float t = 0.f;
    for (int k = 0; k < NTH / D; ++k) t += part[k * D + d];
    return t / (float)R2;
}

struct ScoreArgs {
    ma_tensor4 q;
    PrefixDev pre;
    const int32_t *q_rows;
    const float *mp, *lp;
    const void *op;  // prefix-only output [B*H, R, D] (op_dtype): the value centre's source
    int op_dtype;
    float *mass, *score;
    int H, G, T, T2, R, R2, row_tiles, tiles_per_wg, value, vround;
    float sl2;
};

// distance partials of a packed V item: tokens 2tp, 2tp+1, channels cg*32 + ch*16 + 0..15
template <int D>
__device__ __forceinline__ void dist_packed(float (*dpart)[D / 16], const PfPacked &pf, const float *cen, int u,
                                            bool vround) {
    const int tp = u & 31, ch = (u >> 5) & 1, cg = u >> 6;
    const float s0 = ma_f16_to_f32(pf.w[4] & 0xffff), s1 = ma_f16_to_f32(pf.w[4] >> 16);
    const float z0 = ma_f16_to_f32(pf.w[5] & 0xffff), z1 = ma_f16_to_f32(pf.w[5] >> 16);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        float x0 = ma_dq((pf.w[c >> 3] >> ((c & 7) * 4)) & 15u, s0, z0);
        float x1 = ma_dq((pf.w[2 + (c >> 3)] >> ((c & 7) * 4)) & 15u, s1, z1);
        if (vround) {
            x0 = ma_round_bf16(x0);
            x1 = ma_round_bf16(x1);
        }
        const float cc = cen[cg * VGRP + ch * 16 + c];
        a0 = __builtin_fmaf(x0 - cc, x0 - cc, a0);
        a1 = __builtin_fmaf(x1 - cc, x1 - cc, a1);
    }
    dpart[2 * tp][cg * 2 + ch] = a0;
    dpart[2 * tp + 1][cg * 2 + ch] = a1;
}

// distance partials of a 16-bit V item: tokens 2tp, 2tp+1, channels chk*8 + 0..7
// (the loader already rounded them to bf16, which is what a 16-bit prefix holds)
template <int D>
__device__ __forceinline__ void dist_dense(float (*dpart)[D / 16], const PfDense &pf, const float *cen, int tid) {
    const int tp = tid % (TILE / 2), chk = tid / (TILE / 2);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x0 = ma_bf16_to_f32((pf.w[8 + (e >> 1)] >> ((e & 1) * 16)) & 0xffffu);
        const float x1 = ma_bf16_to_f32((pf.w[12 + (e >> 1)] >> ((e & 1) * 16)) & 0xffffu);
        const float cc = cen[chk * 8 + e];
        a0 = __builtin_fmaf(x0 - cc, x0 - cc, a0);
        a1 = __builtin_fmaf(x1 - cc, x1 - cc, a1);
    }
    // D/8 chunks fold pairwise into D/16 partial slots
    atomicAdd(&dpart[2 * tp][chk >> 1], a0);
    atomicAdd(&dpart[2 * tp + 1][chk >> 1], a1);
}

// Workgroup = `tiles_per_wg` consecutive 64-token tiles of one (batch, KV head) lane;
// NT threads.  Tiles of the source kind SRC go through the register prefetch; the tile
// straddling a packed prefix's 16-bit tail is staged synchronously.  The V items of the
// prefetch feed the value distance directly (no V tile in LDS).
template <int D, int RPW, int SRC>
__global__ void __launch_bounds__(NT) score_kernel(ScoreArgs a) {
    __shared__ TileLds<D> T;
    __shared__ float red[MAX_WAVES][TILE];
    __shared__ float cen[D];
    __shared__ float dpart[TILE][D / 16];
    constexpr int KS = TileLds<D>::KS;
    constexpr int NKS = D / 16;
    constexpr int NDP = D / 16;

    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;
    const bool value = a.value, vround = a.vround;
    const float sl2 = a.sl2;

    if (value) {
        // centre = mean of O_p over the selection rows, in one fixed order per workgroup
        float *part = &red[0][0];
        part[tid] = centre_partial<D, NT>(a.op, a.op_dtype, bh, a.G, a.T, a.q_rows, a.T2, tid);
        __syncthreads();
        if (tid < D) cen[tid] = centre_combine<D, NT>(part, tid, a.G * a.T2);
        __syncthreads();
    }
    for (int it = tid; it < MAX_WAVES * TILE; it += NT) red[it / TILE][it % TILE] = 0.f;

    // Q fragments (A operand) and per-row statistics of this wave's row tiles
    bf16x8_t qf[RPW][NKS];
    float ml2[RPW][16], il[RPW][16];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        // all loads from clamped, valid indices and issued unconditionally; padding rows
        // then select zeros (they contribute exp2(s*0 - 0) * 0 = 0)
        const int rt = wave + r * MAX_WAVES;
        const int rr = rt * 32 + c32;
        const bool ok = rt < a.row_tiles && rr < a.R2;
        const int rrc = ok ? rr : 0;
        const int g = rrc / a.T2;
        const int t = min(max(a.q_rows[rrc % a.T2], 0), a.T - 1);  // rows outside the block are clamped
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[r][ks] = ma_load8_as_bf16(a.q.ptr, qb + ks * 16 + hf * 8, a.q.dtype);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[r][ks] = ok ? qf[r][ks] : bf16x8_t{};
        int qr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int ri = rt * 32 + (i >> 2) * 8 + hf * 4 + (i & 3);
            qr[i] = a.q_rows[(ri < a.R2 ? ri : 0) % a.T2];
        }
        float mpv[16], lpv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int ri = rt * 32 + (i >> 2) * 8 + hf * 4 + (i & 3);
            const int ric = ri < a.R2 ? ri : 0;
            const int rf = (ric / a.T2) * a.T + min(max(qr[i], 0), a.T - 1);
            mpv[i] = a.mp[(int64_t)bh * a.R + rf];
            lpv[i] = a.lp[(int64_t)bh * a.R + rf];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int ri = rt * 32 + (i >> 2) * 8 + hf * 4 + (i & 3);
            const bool rok = rt < a.row_tiles && ri < a.R2;
            ml2[r][i] = rok ? mpv[i] * MA_LOG2E : 0.f;
            il[r][i] = rok ? 1.0f / (lpv[i] > 0.f ? lpv[i] : 1.0f) : 0.f;
        }
    }
    const float inv_r2 = 1.0f / (float)a.R2;
    const int row_tiles = a.row_tiles;
    float *mass_out = a.mass + (int64_t)bh * (a.pre.nq + a.pre.nf);
    float *score_out = a.score ? a.score + (int64_t)bh * (a.pre.nq + a.pre.nf) : nullptr;

    const Lane L = make_lane(a.pre, b, h, bh);
    const int nq = L.nq, ntot = L.ntot;
    const ItemOffsets off = SRC == SRC_PACKED ? packed_offsets<D>(L, tid) : dense_offsets<D>(L.kf_n, L.vf_n, L.esz, tid);
    const int tile0 = blockIdx.x * a.tiles_per_wg;
    const int ntiles = min(a.tiles_per_wg, (ntot + TILE - 1) / TILE - tile0);
    using PF = typename std::conditional<SRC == SRC_PACKED, PfPacked, PfDense>::type;
    auto prefetched = [&](int i) {
        return prefix_tile_kind(nq, (tile0 + i) * TILE, ntot) == (SRC == SRC_PACKED ? TK_PACKED : TK_DENSE);
    };
    auto load = [&](int i, PF &pf) {
        const int n0 = (tile0 + i) * TILE;
        if constexpr (SRC == SRC_PACKED) {
            load_packed<D, true>(pf, L, off, n0, ntot, tid);
        } else {
            const int64_t tb = (int64_t)(n0 - nq);
            load_dense<D, true>(pf, L.kf + tb * L.kf_n * L.esz, L.vf + tb * L.vf_n * L.esz, L.kf_n, L.vf_n, L.fdtype,
                                L.esz, off, &L, n0, ntot, tid);
        }
    };
    // an f32 prefix keeps f32 values for the distance (splitk.py:364-369 reads them as
    // stored); the 16-bit loader rounds to bf16, so such tiles take the exact path
    const bool exact_v = SRC == SRC_DENSE && L.fdtype == MA_F32;
    auto dist_generic = [&](int n0) {
        for (int it = tid; it < TILE * NDP; it += NT) {
            const int tl = it / NDP, c0 = (it % NDP) * 16;
            const int j = n0 + tl;
            float ss = 0.f;
            if (j < ntot) {
                for (int c = 0; c < 16; ++c) {
                    float x = lane_value(L, j, c0 + c);
                    if (vround) x = ma_round_bf16(x);
                    const float dl = x - cen[c0 + c];
                    ss = __builtin_fmaf(dl, dl, ss);
                }
            }
            dpart[tl][it % NDP] = ss;
        }
    };

    PF pf;
    if (ntiles > 0 && prefetched(0)) load(0, pf);
    for (int i = 0; i < ntiles; ++i) {
        const int n0 = (tile0 + i) * TILE;
        const bool pre_i = prefetched(i);
        __syncthreads();
        if (pre_i) {
            if constexpr (SRC == SRC_PACKED) {
                store_packed<D, false>(T, pf, tid);
                if (value && tid >= 2 * D && tid < 4 * D) dist_packed<D>(dpart, pf, cen, tid - 2 * D, vround);
            } else {
                if (value && !exact_v)
                    for (int it = tid; it < TILE * NDP; it += NT) dpart[it / NDP][it % NDP] = 0.f;
                store_dense<D, false>(T, pf, tid);
            }
            store_okmask(T.okmask, pf, tid);
        } else {
            stage_generic<D, false>(T, L, n0, ntot, tid);
        }
        if (value && (!pre_i || exact_v)) dist_generic(n0);
        __syncthreads();
        if constexpr (SRC == SRC_DENSE) {
            // 16-bit V items fold into the zeroed partial slots after the barrier
            if (value && !exact_v && pre_i && tid < TILE / 2 * D / 8) dist_dense<D>(dpart, pf, cen, tid);
        }
        if (i + 1 < ntiles && prefetched(i + 1)) load(i + 1, pf);

        float part[2] = {0.f, 0.f};  // this lane's token in each 32-token sub-tile
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (wave + r * MAX_WAVES >= row_tiles) break;
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
                f32x16_t sv = f32x16_t{};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const bf16x8_t kb = *(const bf16x8_t *)&T.k[(t2 * 32 + c32) * KS + ks * 16 + hf * 8];
                    sv = ma_mfma32(qf[r][ks], kb, sv);
                }
                float acc = 0.f;
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    acc = __builtin_fmaf(__builtin_amdgcn_exp2f(__builtin_fmaf(sv[e], sl2, -ml2[r][e])), il[r][e], acc);
                part[t2] += acc;
            }
        }
        part[0] = ma_sum_xor32(part[0]);
        part[1] = ma_sum_xor32(part[1]);
        if (hf == 0) {
            red[wave][c32] = part[0];
            red[wave][32 + c32] = part[1];
        }
        __syncthreads();
        if (tid < TILE) {
            const int j = n0 + tid;
            if (j < ntot) {
                const bool live = (T.okmask >> tid) & 1;
                float sm = 0.f;
#pragma unroll
                for (int w = 0; w < MAX_WAVES; ++w) sm += red[w][tid];
                const float mass_j = live ? sm * inv_r2 : 0.f;
                mass_out[j] = mass_j;
                if (value) {
                    float ss = 0.f;
#pragma unroll
                    for (int c = 0; c < NDP; ++c) ss += dpart[tid][c];
                    score_out[j] = live ? mass_j * sqrtf(ss) : 0.f;
                }
            }
        }
    }
}

template <int D>
__global__ void __launch_bounds__(NT) centre_kernel(const void *op, int op_dtype, int G, int T,
                                                    const int32_t *q_rows, int T2, float *centre) {
    __shared__ float part[NT];
    const int bh = blockIdx.x, tid = threadIdx.x;
    part[tid] = centre_partial<D, NT>(op, op_dtype, bh, G, T, q_rows, T2, tid);
    __syncthreads();
    if (tid < D) centre[(int64_t)bh * D + tid] = centre_combine<D, NT>(part, tid, G * T2);
}

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

extern "C" int ma_value_centre(const void *op, int op_dtype, int B, int H, int G, int T, int D, const int32_t *q_rows,
                               int T2, float *centre, void *stream) {
    if (!op || !q_rows || !centre || B <= 0 || H <= 0 || G <= 0 || T <= 0 || T2 <= 0 || (D != 64 && D != 128)) {
        ma_set_error("ma_value_centre: bad arguments");
        return MA_EINVAL;
    }
    if (D == 128)
        hipLaunchKernelGGL(centre_kernel<128>, dim3(B * H), dim3(NT), 0, (hipStream_t)stream, op, op_dtype, G, T,
                           q_rows, T2, centre);
    else
        hipLaunchKernelGGL(centre_kernel<64>, dim3(B * H), dim3(NT), 0, (hipStream_t)stream, op, op_dtype, G, T,
                           q_rows, T2, centre);
    return ma_check_launch("ma_value_centre");
}

extern "C" int ma_prefix_scores(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                                int op_dtype, float scale, int value, int v_round_bf16, float *mass, float *score, void *stream) {
    const char *who = "ma_prefix_scores";
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || T2 <= 0 || !q.ptr || !q_rows || !mp || !lp || !mass ||
        (value && (!score || !op))) {
        ma_set_error("%s: bad sizes or NULL pointer", who);
        return MA_EINVAL;
    }
    const int64_t m = q.dtype == MA_F32 ? 4 : 8;
    if (((uintptr_t)q.ptr & 15) || q.s[0] % m || q.s[1] % m || q.s[2] % m) {
        ma_set_error("%s: query must be 16-byte aligned with aligned row strides", who);
        return MA_EINVAL;
    }
    const int G = Hq / H, R = G * T, R2 = G * T2;
    const int row_tiles = (R2 + 31) / 32;
    if (row_tiles > 2 * MAX_WAVES) {
        ma_set_error("%s: %d selection rows per KV head exceed the built maximum %d", who, R2, 64 * MAX_WAVES);
        return MA_EUNSUPPORTED;
    }
    const int n = p->nq + p->nf;
    if (n == 0) return MA_OK;
    const int rpw = (row_tiles + MAX_WAVES - 1) / MAX_WAVES;
    const int tiles = (n + TILE - 1) / TILE;
    int per = (tiles * B * H + ma_num_cus() - 1) / ma_num_cus();
    if (per < 1) per = 1;
    ScoreArgs sa;
    sa.q = q;
    sa.pre = prefix_dev(p);
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
    sa.T2 = T2;
    sa.R = R;
    sa.R2 = R2;
    sa.row_tiles = row_tiles;
    sa.tiles_per_wg = per;
    sa.value = value;
    sa.vround = v_round_bf16;
    sa.sl2 = scale * MA_LOG2E;
    dim3 grid((tiles + per - 1) / per, B * H);
    dim3 block(NT);
    hipStream_t st = (hipStream_t)stream;
    const bool packed = p->nq > 0;
#define MA_SCORE(D_, R_, S_) hipLaunchKernelGGL((score_kernel<D_, R_, S_>), grid, block, 0, st, sa)
    if (D == 128) {
        if (rpw == 1) { if (packed) MA_SCORE(128, 1, SRC_PACKED); else MA_SCORE(128, 1, SRC_DENSE); }
        else { if (packed) MA_SCORE(128, 2, SRC_PACKED); else MA_SCORE(128, 2, SRC_DENSE); }
    } else {
        if (rpw == 1) { if (packed) MA_SCORE(64, 1, SRC_PACKED); else MA_SCORE(64, 1, SRC_DENSE); }
        else { if (packed) MA_SCORE(64, 2, SRC_PACKED); else MA_SCORE(64, 2, SRC_DENSE); }
    }
#undef MA_SCORE
    return ma_check_launch(who);
}
