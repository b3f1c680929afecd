// One step 0 of a sparse layer from a single host call: the six launches of split-K
// attention (pass 1, merge), the score pass building the read-set top-k's first level, the
// select's boundary and emit kernels, and the gather -- what the reference session's
// _fast_step0 (session.py:1403-1454) runs as four Python-level ops.  Composition only: each
// stage is the library's own entry point, enqueued in order on one stream, so the results
// are those of calling them one by one.
#include "ma_common.h"

namespace {

constexpr int64_t ALIGN = 256;

int64_t align_up(int64_t x) { return (x + ALIGN - 1) / ALIGN * ALIGN; }

}  // namespace

extern "C" int64_t ma_step0_workspace_bytes(int B, int H, int Hq, int T, int D, int nq, int nf) {
    const int64_t sk = ma_splitk_workspace_bytes(B, H, Hq, T, D, nq, nf, 0);
    if (sk < 0 || B <= 0 || H <= 0 || nq + nf <= 0) return -1;
    const int64_t tk = ma_topk_workspace_bytes(B * H, nq + nf);
    if (tk <= 0) return -1;
    return align_up(sk) + align_up(tk);
}

extern "C" int ma_step0(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                        ma_tensor4 vc, int Tc, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
                        const int32_t *q_rows, int T2, int value, int rank, int v_round, float *mass, float *score,
                        int k, int64_t *idx, ma_tensor4 k_out, ma_tensor4 v_out, void *topk_state,
                        int64_t state_bytes, void *workspace, int64_t workspace_bytes, void *stream) {
    const char *who = "ma_step0";
    if (!p || !mp || !lp || !op || !mass || !idx || (value && !score)) {
        ma_set_error("%s: NULL statistics, score or index output", who);
        return MA_EINVAL;
    }
    if (rank != 1 && !(rank == 2 && value)) {
        ma_set_error("%s: rank must be 1 (mass) or 2 (score, with value = 1), got %d", who, rank);
        return MA_EINVAL;
    }
    const int n = p->nq + p->nf;
    if (n <= 0 || k <= 0 || k > n) {
        ma_set_error("%s: read budget k=%d outside [1, n=%d]", who, k, n);
        return MA_EINVAL;
    }
    const int64_t sk = ma_splitk_workspace_bytes(B, H, Hq, T, D, p->nq, p->nf, 0);
    const int64_t need = ma_step0_workspace_bytes(B, H, Hq, T, D, p->nq, p->nf);
    if (sk < 0 || need < 0) {
        ma_set_error("%s: bad geometry (B=%d H=%d Hq=%d T=%d D=%d n=%d)", who, B, H, Hq, T, D, n);
        return MA_EINVAL;
    }
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % ALIGN)) {
        ma_set_error("%s: workspace of %lld bytes (256-byte aligned) needed, got %lld", who, (long long)need,
                     (long long)workspace_bytes);
        return MA_EWORKSPACE;
    }
    char *ws = (char *)workspace;
    const int64_t sk_al = align_up(sk);
    int rc = ma_splitk_attention(q, B, Hq, T, D, p, H, kc, vc, Tc, 0, 0, 0, scale, out, mp, lp, op, 0, ws, sk, stream);
    if (rc) return rc;
    float *rk = rank == 2 ? score : mass;
    rc = ma_prefix_scores_hist(q, B, Hq, T, D, p, H, q_rows, T2, mp, lp, op, out.dtype, scale, value, v_round, mass,
                               value ? score : nullptr, rank, topk_state, state_bytes, stream);
    if (rc) return rc;
    rc = ma_topk_select_hist_ready(rk, n, p->mask, p->mask ? n : 0, B * H, n, k, idx, k, nullptr, topk_state,
                                   state_bytes, ws + sk_al, workspace_bytes - sk_al, stream);
    if (rc) return rc;
    if (!k_out.ptr && !v_out.ptr) return MA_OK;
    const int64_t sidx[2] = {(int64_t)H * k, k};
    return ma_gather_kv(p, B, H, D, idx, sidx, k, k_out, v_out, stream);
}
