/* maskahead_hip.h -- C ABI of the MI355X (gfx950) KV read/keep path.
 *
 * One shared library, maskahead_amd/libmaskahead_hip.so, hand-written HIP kernels for
 * the per-layer read/keep path of MaskAhead (brain-lab-research/MaskAhead).  The
 * reference binds these operations from Python (src/maskahead/kernels/splitk.py,
 * kernels/ops.py, runtime/session.py, eviction.py, cache.py); each entry point below
 * names the reference interface it replaces.  The Python package maskahead_amd binds
 * them with ctypes.
 *
 * Conventions
 *   - Every entry point enqueues work on `stream` (a hipStream_t passed as void*; NULL =
 *     the null stream) and returns at once: no host synchronisation, no allocation.
 *     Outputs and workspaces are owned by the caller.
 *   - Return value: MA_OK (0) or a negative MA_E* code; ma_last_error() then holds a
 *     message (per host thread).
 *   - Strides are in elements of the tensor's own dtype; the innermost dimension of
 *     every tensor must be contiguous (stride 1) unless stated otherwise.
 *   - f16 / bf16 tensors are passed as raw 16-bit storage.
 */
#ifndef MASKAHEAD_HIP_H
#define MASKAHEAD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ma_status {
    MA_OK = 0,
    MA_EINVAL = -1,       /* bad shape, stride or argument: Python raises ValueError          */
    MA_EUNSUPPORTED = -2, /* valid but not built (bit width, group, head_dim): KernelUnavailable */
    MA_EHIP = -3,         /* HIP runtime error at launch: RuntimeError                        */
    MA_EWORKSPACE = -4    /* workspace too small: ValueError                                  */
};

enum ma_dtype { MA_F32 = 0, MA_F16 = 1, MA_BF16 = 2 };

/* The prefix a kernel reads (splitk.py:408-462, Prefix): tokens [0, nq) from the packed
 * cache, tokens [nq, nq + nf) from a 16-bit (or f32) tensor -- the bf16 residual tail
 * of a packed cache, or the whole prefix of a 16-bit cache.  Layouts (cache.py:142-189):
 *   kq [B,H,G_n,D,KG*kbits/8] u8 (strides b,h,g,d; packed bytes contiguous)
 *   ks,kz [B,H,G_n,D] f16 (strides b,h,g; d contiguous)  -- kz shares ks' strides
 *   vq [B,H,n,D/VG,VG*vbits/8] u8 (strides b,h,n,c)
 *   vs,vz [B,H,n,D/VG] f16 (strides b,h,n; groups contiguous)
 *   kf,vf [B,H,nf,D] (strides b,h,n), dtype fdtype
 *   mask  [B,H,nq+nf] u8 contiguous, 0 = dead slot (never attended), or NULL. */
typedef struct ma_prefix {
    const void *kq;
    const void *ks;
    const void *kz;
    const void *vq;
    const void *vs;
    const void *vz;
    const void *kf;
    const void *vf;
    const uint8_t *mask;
    int64_t skq[4];
    int64_t sks[3];
    int64_t svq[4];
    int64_t svs[3];
    int64_t skf[3];
    int64_t svf[3];
    int32_t nq, nf;
    int32_t kbits, vbits;   /* 4 (packed) -- only consulted when nq > 0 */
    int32_t kgroup, vgroup; /* key token group, value channel group: 32 */
    int32_t fdtype;         /* ma_dtype of kf / vf */
    int32_t reserved;
} ma_prefix;

/* A dense [B, H, T, D]-style operand: pointer, dtype, strides b, h, t (d contiguous). */
typedef struct ma_tensor4 {
    void *ptr;
    int32_t dtype;
    int32_t reserved;
    int64_t s[3];
} ma_tensor4;

const char *ma_last_error(void);
int ma_version(void);

/* a3. dequantize_prefix (splitk.py:465-480; codec reference.py:48-55, 168-179, 259-268):
 * the whole prefix as [B,H,n,D] K and V in out dtype (bf16 or f32), n = nq + nf.
 * Bit-exact: x = f32(code)*f32(scale) + f32(zero), rounded to nearest even. */
int ma_dequant_prefix(const ma_prefix *p, int B, int H, int D, ma_tensor4 k_out, ma_tensor4 v_out,
                      void *stream);

/* a4 + a5. splitk_attention (splitk.py:493-579): softmax over [prefix | current] for all
 * R = (Hq/H)*T rows of every KV head.  Pass 1 writes per-split partials (max, sum, acc)
 * into `workspace`, pass 2 merges them (log-sum-exp) into `out` [B,Hq,T,D] and, when mp
 * is not NULL, the prefix-only statistics mp, lp f32 [B,H,R] (contiguous) and op
 * [B,H,R,D] (contiguous, dtype of out).  causal_block > 0: current key j is visible to
 * query t only if (c_pos0+j)/causal_block <= (q_pos0+t)/causal_block.
 * split_tokens: prefix tokens per split (multiple of 64; 0 = library default). */
int64_t ma_splitk_workspace_bytes(int B, int H, int Hq, int T, int D, int n, int split_tokens);
/* The two passes of ma_splitk_attention as separate launches (same arguments and
 * workspace): ma_splitk_partial writes the per-split partials (_sk_fwd, splitk.py:116-190),
 * ma_splitk_merge merges them (_sk_combine, splitk.py:272-318); n = prefix length. */
int ma_splitk_partial(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                      ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale,
                      int split_tokens, void *workspace, int64_t workspace_bytes, void *stream);
int ma_splitk_merge(int B, int Hq, int T, int D, int H, int n, int split_tokens, ma_tensor4 out, float *mp,
                    float *lp, void *op, void *workspace, int64_t workspace_bytes, void *stream);
int ma_splitk_attention(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                        ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0,
                        int c_pos0, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
                        int split_tokens, void *workspace, int64_t workspace_bytes, void *stream);

/* a6 (centre). The value centre of prefix_scores (splitk.py:599-601):
 * centre[b,h,:] = mean over g < G, t in q_rows of f32(op[b,h,g*T+t,:]); op dtype op_dtype. */
int ma_value_centre(const void *op, int op_dtype, int B, int H, int G, int T, int D,
                    const int32_t *q_rows, int T2, float *centre, void *stream);

/* a6. prefix_scores (splitk.py:582-614, kernel 321-371): per prefix entry j,
 * mass[j] = mean over the G*T2 selection rows of exp(s_rj - mp[r]) / lp[r] (0 on dead
 * slots) and, when value != 0, score[j] = mass[j] * ||v_j - centre|| (0 on dead slots).
 * v_round_bf16: the distance reads V rounded to bf16 (the reference reads its unpacked
 * bf16 prefix when it has one, splitk.py:513-516, 592).  mass/score [B,H,n] contiguous. */
int ma_prefix_scores(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                     const int32_t *q_rows, int T2, const float *mp, const float *lp,
                     const float *centre, float scale, int value, int v_round_bf16, float *mass,
                     float *score, void *stream);

/* a9. read-set top-k (session.py:1429-1438, reference.py:369-393): for each of `rows`
 * rows, the k largest of rank[row, 0..n) -- dead slots (mask 0) rank -inf, ties go to
 * the smaller index, -0.0 equals +0.0 and NaN ranks above +inf -- written as ascending
 * int64 indices to idx[row*idx_stride + i]; values (optional) gets rank at those indices.
 * rank row stride rank_stride, mask (optional) row stride mask_stride. */
int ma_topk_select(const float *rank, int64_t rank_stride, const uint8_t *mask, int64_t mask_stride,
                   int rows, int n, int k, int64_t *idx, int64_t idx_stride, float *values,
                   void *stream);

/* a11. gather_packed_kv (ops.py:570-662, 835-855; oracle reference.py:396-400): the
 * entries idx[b,h,0..k) of the prefix, dequantized, into k_out / v_out [B,H,k,D]
 * (bf16 or f32).  idx int64 with strides sidx (b, h; i contiguous). */
int ma_gather_kv(const ma_prefix *p, int B, int H, int D, const int64_t *idx, const int64_t sidx[2],
                 int k, ma_tensor4 k_out, ma_tensor4 v_out, void *stream);

/* f2. quantize_key_groups_into / quantize_values_into (ops.py:665-758; rule
 * reference.py:58-90, 182-213): 4-bit asymmetric quantization with the arithmetic of
 * the source dtype (f32, f16 or bf16, each op rounded to it), round half to even,
 * f16 scale / zero.  src [B,H,T,D] (strides s).  Keys: T multiple of KG, outputs
 * kq [B,H,T/KG,D,KG/2] (strides b,h,g,d), ks/kz [B,H,T/KG,D] (strides b,h,g).
 * Values: vq [B,H,T,D/VG,VG/2] (strides b,h,n,c), vs/vz [B,H,T,D/VG] (strides b,h,n). */
int ma_quantize_keys(ma_tensor4 src, int B, int H, int T, int D, int group, void *kq,
                     const int64_t skq[4], void *ks, void *kz, const int64_t sks[3], void *stream);
int ma_quantize_values(ma_tensor4 src, int B, int H, int T, int D, int group, void *vq,
                       const int64_t svq[4], void *vs, void *vz, const int64_t svs[3], void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MASKAHEAD_HIP_H */
