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
#include "ma_tile.h"

using namespace ma;

namespace {

constexpr int MAX_WAVES = 8;

struct ScoreArgs {
    ma_tensor4 q;
    PrefixDev pre;
    const int32_t *q_rows;
    const float *mp, *lp, *centre;
    float *mass, *score;
    int H, G, T, T2, R, R2, row_tiles, tiles_per_wg, value, vround;
    float sl2;
};

template <int D, int RPW>
__global__ void __launch_bounds__(MAX_WAVES * 64) score_kernel(ScoreArgs a) {
    __shared__ TileLds<D> L;
    __shared__ float red[MAX_WAVES][TILE];
    __shared__ float cen[D];
    __shared__ float dpart[TILE][D / VGRP];
    constexpr int KS = TileLds<D>::KS;
    constexpr int NKS = D / 16;
    constexpr int NCG = D / VGRP;

    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, nthreads = blockDim.x, nwaves = nthreads >> 6;
    const int wave = tid >> 6, lane = tid & 63, c32 = lane & 31, hf = lane >> 5;
    const int ntot = a.pre.nq + a.pre.nf;

    if (a.value)
        for (int d = tid; d < D; d += nthreads) cen[d] = a.centre[(int64_t)bh * D + d];

    // Q fragments (A operand) and per-row softmax statistics of this wave's row tiles
    bf16x8_t qf[RPW][NKS];
    float ml2[RPW][16], il[RPW][16];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int rt = wave + r * nwaves;
        const int rr = rt * 32 + c32;
        const bool ok = rt < a.row_tiles && rr < a.R2;
        const int g = ok ? rr / a.T2 : 0;
        const int t = ok ? min(max(a.q_rows[rr % a.T2], 0), a.T - 1) : 0;  // rows outside the block are clamped
        const int64_t qb = b * a.q.s[0] + (int64_t)(h * a.G + g) * a.q.s[1] + (int64_t)t * a.q.s[2];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
            qf[r][ks] = ok ? ma_load8_as_bf16(a.q.ptr, qb + ks * 16 + hf * 8, a.q.dtype) : bf16x8_t{};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int ri = rt * 32 + (i >> 2) * 8 + hf * 4 + (i & 3);
            float m = 0.f, inv = 0.f;  // padding rows contribute exp2(s*0 - 0) * 0 = 0
            if (rt < a.row_tiles && ri < a.R2) {
                const int rf = (ri / a.T2) * a.T + min(max(a.q_rows[ri % a.T2], 0), a.T - 1);
                const float mpv = a.mp[(int64_t)bh * a.R + rf], lpv = a.lp[(int64_t)bh * a.R + rf];
                m = mpv * MA_LOG2E;
                inv = 1.0f / (lpv > 0.f ? lpv : 1.0f);
            }
            ml2[r][i] = m;
            il[r][i] = inv;
        }
    }
    const float inv_r2 = 1.0f / (float)a.R2;

    const int tile0 = blockIdx.x * a.tiles_per_wg;
    for (int tt = 0; tt < a.tiles_per_wg; ++tt) {
        const int n0 = (tile0 + tt) * TILE;
        if (n0 >= ntot) break;
        __syncthreads();
        stage_prefix_tile<D, false>(L, a.pre, b, h, bh, n0, ntot, tid, nthreads);
        __syncthreads();

        float part[2] = {0.f, 0.f};  // this lane's token in each 32-token sub-tile
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (wave + r * nwaves >= a.row_tiles) break;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                f32x16_t s = f32x16_t{};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    bf16x8_t kb = *(const bf16x8_t *)&L.k[(st * 32 + c32) * KS + ks * 16 + hf * 8];
                    s = ma_mfma32(qf[r][ks], kb, s);
                }
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    acc += exp2f(__builtin_fmaf(s[i], a.sl2, -ml2[r][i])) * il[r][i];
                part[st] += acc;
            }
        }
        part[0] = ma_sum_xor32(part[0]);
        part[1] = ma_sum_xor32(part[1]);
        if (hf == 0) {
            red[wave][c32] = part[0];
            red[wave][32 + c32] = part[1];
        }
        __syncthreads();
        // one thread per token: sum over waves, mask, store mass; keep it for the score
        float mass_j = 0.f;
        const int j = n0 + tid;
        const bool live = tid < TILE && j < ntot && ((L.okmask >> tid) & 1);
        if (tid < TILE && j < ntot) {
            float s = 0.f;
            for (int w = 0; w < nwaves; ++w) s += red[w][tid];
            mass_j = live ? s * inv_r2 : 0.f;
            a.mass[(int64_t)bh * ntot + j] = mass_j;
        }
        if (!a.value) continue;
        // value distance: item = (token, channel group)
        for (int it = tid; it < TILE * NCG; it += nthreads) {
            const int tl = it / NCG, cg = it % NCG;
            const int jj = n0 + tl;
            float ss = 0.f;
            if (jj < ntot) {
                if (jj < a.pre.nq) {
                    const uint8_t *src = a.pre.vq + b * a.pre.svq[0] + h * a.pre.svq[1] + (int64_t)jj * a.pre.svq[2] +
                                         (int64_t)cg * a.pre.svq[3];
                    const uint4 w = *(const uint4 *)src;
                    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
                    const int64_t so = b * a.pre.svs[0] + h * a.pre.svs[1] + (int64_t)jj * a.pre.svs[2] + cg;
                    const float sc = ma_f16_to_f32(a.pre.vs[so]), zp = ma_f16_to_f32(a.pre.vz[so]);
#pragma unroll
                    for (int c = 0; c < VGRP; ++c) {
                        float x = ma_dq((wv[c >> 3] >> ((c & 7) * 4)) & 15u, sc, zp);
                        if (a.vround) x = ma_round_bf16(x);
                        const float dlt = x - cen[cg * VGRP + c];
                        ss = __builtin_fmaf(dlt, dlt, ss);
                    }
                } else {
                    const int64_t vb = b * a.pre.svf[0] + h * a.pre.svf[1] + (int64_t)(jj - a.pre.nq) * a.pre.svf[2] +
                                       cg * VGRP;
#pragma unroll
                    for (int c = 0; c < VGRP; ++c) {
                        float x = ma_load_f(a.pre.vf, vb + c, a.pre.fdtype);
                        if (a.vround) x = ma_round_bf16(x);
                        const float dlt = x - cen[cg * VGRP + c];
                        ss = __builtin_fmaf(dlt, dlt, ss);
                    }
                }
            }
            dpart[tl][cg] = ss;
        }
        __syncthreads();
        if (tid < TILE && j < ntot) {
            float ss = 0.f;
#pragma unroll
            for (int cg = 0; cg < NCG; ++cg) ss += dpart[tid][cg];
            a.score[(int64_t)bh * ntot + j] = live ? mass_j * sqrtf(ss) : 0.f;
        }
    }
}

// centre[b,h,:] = mean over rows g*T + q_rows[t2] of f32(op); grid B*H, D threads.
__global__ void centre_kernel(const void *op, int op_dtype, int G, int T, int D, const int32_t *q_rows, int T2,
                              float *centre) {
    const int bh = blockIdx.x, d = threadIdx.x;
    if (d >= D) return;
    const int R = G * T;
    float s = 0.f;
    for (int g = 0; g < G; ++g)
        for (int t2 = 0; t2 < T2; ++t2)
            s += ma_load_f(op, ((int64_t)bh * R + g * T + min(max(q_rows[t2], 0), T - 1)) * D + d, op_dtype);
    centre[(int64_t)bh * D + d] = s / (float)(G * T2);
}

}  // namespace

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

extern "C" int ma_value_centre(const void *op, int op_dtype, int B, int H, int G, int T, int D, const int32_t *q_rows,
                               int T2, float *centre, void *stream) {
    if (!op || !q_rows || !centre || B <= 0 || H <= 0 || G <= 0 || T <= 0 || T2 <= 0 || D <= 0 || D > 1024) {
        ma_set_error("ma_value_centre: bad arguments");
        return MA_EINVAL;
    }
    hipLaunchKernelGGL(centre_kernel, dim3(B * H), dim3(D), 0, (hipStream_t)stream, op, op_dtype, G, T, D, q_rows, T2,
                       centre);
    return ma_check_launch("ma_value_centre");
}

extern "C" int ma_prefix_scores(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                const int32_t *q_rows, int T2, const float *mp, const float *lp, const float *centre,
                                float scale, int value, int v_round_bf16, float *mass, float *score, void *stream) {
    const char *who = "ma_prefix_scores";
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (B <= 0 || H <= 0 || Hq <= 0 || Hq % H || T <= 0 || T2 <= 0 || !q.ptr || !q_rows || !mp || !lp || !mass ||
        (value && (!score || !centre))) {
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
    const int waves = row_tiles < MAX_WAVES ? row_tiles : MAX_WAVES;
    const int rpw = (row_tiles + waves - 1) / waves;
    const int tiles = (n + TILE - 1) / TILE;
    int per = (tiles * B * H + ma_num_cus() - 1) / ma_num_cus();
    if (per < 1) per = 1;
    ScoreArgs sa;
    sa.q = q;
    sa.pre = prefix_dev(p);
    sa.q_rows = q_rows;
    sa.mp = mp;
    sa.lp = lp;
    sa.centre = centre;
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
    dim3 block(waves * 64);
    hipStream_t st = (hipStream_t)stream;
    if (D == 128) {
        if (rpw == 1) hipLaunchKernelGGL((score_kernel<128, 1>), grid, block, 0, st, sa);
        else hipLaunchKernelGGL((score_kernel<128, 2>), grid, block, 0, st, sa);
    } else {
        if (rpw == 1) hipLaunchKernelGGL((score_kernel<64, 1>), grid, block, 0, st, sa);
        else hipLaunchKernelGGL((score_kernel<64, 2>), grid, block, 0, st, sa);
    }
    return ma_check_launch(who);
}
