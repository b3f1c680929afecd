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

/* dequantize_prefix (splitk.py:465-480; codec reference.py:48-55, 168-179, 259-268):
 * the whole prefix as [B,H,n,D] K and V in out dtype (bf16, f16 or f32), n = nq + nf.
 * Bit-exact: x = f32(code)*f32(scale) + f32(zero), rounded to nearest even.  The split-K
 * and score entry points read a packed prefix with each value rounded to bf16 once, as
 * the reference's kernels do; the reference's host dispatch first unpacks a long packed
 * prefix to the query dtype (splitk.py:513-516), which for f16 queries rounds through
 * f16 as well: that caller passes this call's f16 copy as a 16-bit prefix instead. */
int ma_dequant_prefix(const ma_prefix *p, int B, int H, int D, ma_tensor4 k_out, ma_tensor4 v_out,
                      void *stream);

/* splitk_attention (splitk.py:493-579): softmax over [prefix | current] for all
 * R = (Hq/H)*T rows of every KV head.  Pass 1 writes per-split partials (max, sum and the
 * normalized output on a per-row f16 scale) into `workspace`, pass 2 merges them
 * (log-sum-exp) into `out` [B,Hq,T,D] and, when mp is not NULL, the prefix-only
 * statistics mp, lp f32 [B,H,R] (contiguous) and op [B,H,R,D] (contiguous, dtype of out).
 * causal_block > 0: current key j is visible to query t only if
 * (c_pos0+j)/causal_block <= (q_pos0+t)/causal_block.  split_tokens: prefix tokens per
 * split (multiple of 64; 0 = library default).  The workspace size depends on the packed
 * (nq) and 16-bit (nf) prefix lengths. */
int64_t ma_splitk_workspace_bytes(int B, int H, int Hq, int T, int D, int nq, int nf, int split_tokens);
/* The two passes of ma_splitk_attention as separate calls, with the same arguments and
 * workspace: ma_splitk_partial writes the per-split partials of the prefix (_sk_fwd,
 * splitk.py:116-190); ma_splitk_merge attends the current block and merges it with the
 * partials (the last split of _sk_fwd and _sk_combine, splitk.py:116-190, 272-318). */
int ma_splitk_partial(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                      ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale,
                      int split_tokens, void *workspace, int64_t workspace_bytes, void *stream);
int ma_splitk_merge(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
                    ma_tensor4 vc, int Tc, int causal_block, int q_pos0, int c_pos0, float scale, ma_tensor4 out,
                    float *mp, float *lp, void *op, int split_tokens, void *workspace, int64_t workspace_bytes,
                    void *stream);
int ma_splitk_attention(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                        ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0,
                        int c_pos0, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
                        int split_tokens, void *workspace, int64_t workspace_bytes, void *stream);

/* No counterpart in the reference: ma_splitk_attention for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as ma_splitk_attention, without the workspace: the split
 * partials live in a fixed library-owned device array of ma_splitk_noalloc_max_bytes()
 * bytes (32 MiB) per device, held until the process ends.  A call whose
 * ma_splitk_workspace_bytes() exceeds it returns MA_EWORKSPACE.  The call allocates
 * nothing; the first call on a device looks up that device's copy of the array.  All calls
 * on one device share the array, so calls that overlap in time on one device (two streams,
 * two host threads) race; order them on one stream. */
int64_t ma_splitk_noalloc_max_bytes(void);
int ma_splitk_attention_noalloc(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                                ma_tensor4 kc, ma_tensor4 vc, int Tc, int causal_block, int q_pos0,
                                int c_pos0, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
                                int split_tokens, void *stream);

/* The value centre of prefix_scores (splitk.py:599-601):
 * centre[b,h,:] = mean over g < G, t in q_rows of f32(op[b,h,g*T+t,:]); op dtype op_dtype. */
int ma_value_centre(const void *op, int op_dtype, int B, int H, int G, int T, int D,
                    const int32_t *q_rows, int T2, float *centre, void *stream);

/* prefix_scores (splitk.py:582-614, kernel 321-371): per prefix entry j,
 * mass[j] = mean over the G*T2 selection rows of exp(s_rj - mp[r]) / lp[r] (0 on dead
 * slots) and, when value != 0, score[j] = mass[j] * ||v_j - centre|| (0 on dead slots),
 * centre as ma_value_centre computes it from op (the prefix-only output of
 * ma_splitk_attention, [B,H,R,D] contiguous, dtype op_dtype; read only when value != 0).
 * q_rows: int32 [T2] block positions of the selection rows, or NULL for positions 0 .. T2-1
 * in order (T2 <= T; mode "all" is T2 = T).
 * v_round: 0, or MA_BF16 / MA_F16: the distance reads packed V rounded to that dtype (the
 * reference reads the prefix it unpacked to the query dtype when it has one,
 * splitk.py:513-516, 592).  mass/score [B,H,n] contiguous.  Mass-only calls take any number
 * of selection rows (run in passes of at most 512, each adding its share of the mean);
 * value-aware calls take at most 512 selection rows and 1 024 rows per KV head. */
int ma_prefix_scores(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                     const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                     int op_dtype, float scale, int value, int v_round, float *mass, float *score,
                     void *stream);

/* The score pass of ma_prefix_scores for few selection rows per KV head (the
 * reference serves every row count with BLOCK_M-row tl.dot tiles, splitk.py:321-371): a
 * GQA-reduced VALU pass for at most 16 rows (G*T2 <= 16) -- waves stream 32-token units
 * with no workgroup barrier, q . k by v_dot2c_f32_bf16 for every selection row, the value
 * centre from those rows of O_p only -- instead of 32-row MFMA tiles that are mostly
 * padding.  mode 0 (default) takes the MFMA pass for every row count (it measured as fast
 * or faster at config 2's prefix), 1 forces the MFMA pass, 2 the VALU pass (calls above 16
 * rows then fail); process-wide, for measurement and tests.  Returns the previous mode, or -1
 * for a bad mode.  No counterpart in the reference (Triton picks no variant). */
int ma_prefix_scores_path(int mode);

/* read-set top-k (session.py:1429-1438, reference.py:369-393): for each of `rows`
 * rows, the k largest of rank[row, 0..n) -- dead slots (mask 0) rank -inf, ties go to
 * the smaller index, -0.0 equals +0.0 and NaN ranks above +inf -- written as ascending
 * int64 indices to idx[row*idx_stride + i]; values (optional, [rows][k] contiguous) gets
 * rank at those indices.  rank row stride rank_stride, mask (optional) row stride
 * mask_stride.  Three launches over ceil(n / 1024) workgroups per row (n <= 4M).
 * state: ma_topk_state_bytes(rows) bytes (one 32 KB histogram block per row), 256-byte
 * aligned, zero-filled before its first use; every call leaves the
 * blocks of its rows zero again, so one state buffer of R blocks serves any number of
 * calls of up to R rows ordered on one stream (calls that overlap in time need their own).
 * workspace: ma_topk_workspace_bytes(rows, n) bytes of scratch, 256-byte aligned. */
int64_t ma_topk_state_bytes(int rows);
int64_t ma_topk_workspace_bytes(int rows, int n);
int ma_topk_select(const float *rank, int64_t rank_stride, const uint8_t *mask, int64_t mask_stride,
                   int rows, int n, int k, int64_t *idx, int64_t idx_stride, float *values,
                   void *state, int64_t state_bytes, void *workspace, int64_t workspace_bytes,
                   void *stream);

/* prefix_scores with the read-set top-k's first level built in.  No counterpart in the
 * reference (which runs its prefix-score op and then torch.topk, session.py:1418-1438):
 * ma_prefix_scores, and besides the outputs it builds the read-set top-k's first-level
 * histogram of rank 1 (the mass) or 2 (the score, value=1)
 * under the prefix's mask into `topk_state` (zero before, ma_topk_state_bytes(B*H) bytes,
 * 256-byte aligned).  The caller then runs ma_topk_select_hist_ready on that rank with the
 * prefix's mask and the same state, which skips the select's histogram launch and leaves
 * the state zero again: the pair returns what ma_prefix_scores + ma_topk_select return,
 * with one launch less. */
int ma_prefix_scores_hist(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H,
                          const int32_t *q_rows, int T2, const float *mp, const float *lp, const void *op,
                          int op_dtype, float scale, int value, int v_round, float *mass, float *score,
                          int rank, void *topk_state, int64_t state_bytes, void *stream);
int ma_topk_select_hist_ready(const float *rank, int64_t rank_stride, const uint8_t *mask,
                              int64_t mask_stride, int rows, int n, int k, int64_t *idx, int64_t idx_stride,
                              float *values, void *state, int64_t state_bytes, void *workspace,
                              int64_t workspace_bytes, void *stream);

/* Step 0 of a sparse layer in one call (the reference session's _fast_step0,
 * session.py:1403-1454, which runs splitk_attention(want_prefix=True), prefix_scores,
 * topk + sort and gather_packed_kv as four Python-level ops): enqueues, on `stream`,
 * ma_splitk_attention (outputs out, mp, lp, op; split_tokens auto, no causal mask),
 * ma_prefix_scores_hist (mass, and score when value = 1) with the read-set top-k's first
 * level of rank 1 (mass) or 2 (score, value = 1), ma_topk_select_hist_ready (k ascending
 * indices per (b, KV head) into idx [B, H, k] contiguous, dead slots of p->mask never
 * selected) and, when k_out / v_out are given, ma_gather_kv of those entries -- the
 * results of calling them one by one.  topk_state: as for ma_prefix_scores_hist (zero
 * before, left zero).  workspace: ma_step0_workspace_bytes() bytes, 256-byte aligned. */
int64_t ma_step0_workspace_bytes(int B, int H, int Hq, int T, int D, int nq, int nf);
int ma_step0(ma_tensor4 q, int B, int Hq, int T, int D, const ma_prefix *p, int H, ma_tensor4 kc,
             ma_tensor4 vc, int Tc, float scale, ma_tensor4 out, float *mp, float *lp, void *op,
             const int32_t *q_rows, int T2, int value, int rank, int v_round, float *mass, float *score, int k,
             int64_t *idx, ma_tensor4 k_out, ma_tensor4 v_out, void *topk_state, int64_t state_bytes,
             void *workspace, int64_t workspace_bytes, void *stream);

/* keep set of an eviction step (EvictionState.survivors, eviction.py:325-409, for the
 * score-ranked policies; capacity C = EvictionConfig.capacity, eviction.py:200-202): per
 * row (one (layer, batch, KV head) lane of n live entries), the W = min(window, C) newest
 * entries plus the top (C - W) of score among the others, where positions < sink_tokens
 * and pinned positions [pin_lo, pin_hi) rank +inf (NaN above +inf, ties to the smaller
 * index), written as C ascending live-axis indices to keep[row*keep_stride + i].
 * Positions (int32, or int64 when pos_is_i64) must increase strictly along each row --
 * the state keeps its live arrays in position order -- so index order is position order
 * and the newest W are the last W; status (optional, int32 [rows]) gets 1 for a row that
 * breaks this.  pin_lo_rows (optional, [rows]) overrides pin_lo per row.  n <= 4M.  The
 * selection runs as ma_topk_select's three launches, with the same state buffer
 * (ma_topk_state_bytes(rows)) and workspace (ma_topk_workspace_bytes(rows, n)). */
int ma_keep_select(const void *pos, int pos_is_i64, int64_t pos_stride, const float *score,
                   int64_t score_stride, int rows, int n, int capacity, int window, int64_t sink_tokens,
                   const int64_t *pin_lo_rows, int64_t pin_lo, int64_t pin_hi, int has_pin, int64_t *keep,
                   int64_t keep_stride, int32_t *status, void *state, int64_t state_bytes, void *workspace,
                   int64_t workspace_bytes, void *stream);

/* value_score (session.py:27-40): score[row, j] = a[row, j] * ||v_j - c||,
 * c = sum_j w_j v_j / max(sum_j w_j, 1e-12), rows = (b, h) of v [B,H,n,D] (strides b, h, n;
 * bf16, f16 or f32).  fp32_mode 0 (the reference default): w = bf16(a) and every step in
 * bf16 arithmetic as the reference's bf16 tensors compute it; fp32_mode 1: the f32 branch
 * (BITSIEVE_VSCORE_FP32).  a, score [rows, n] with row strides.  D <= 128, D % 8 == 0. */
int64_t ma_value_score_workspace_bytes(int rows, int n, int D);
int ma_value_score(const float *a, int64_t a_stride, ma_tensor4 v, int B, int H, int n, int D, int fp32_mode,
                   float *score, int64_t score_stride, void *workspace, int64_t workspace_bytes,
                   void *stream);
/* value score over a cache's live slots (the lookahead keep score of session.py:1995-2025:
 * value_score(a, live_values) with live_values = session.py:263-268): entry j of lane
 * (b, h) is slot slots[(b*H + h)*slot_stride + j] of the cache lane described by p, its
 * value dequantized (packed slots < p->nq) or read (16-bit rows) and rounded to vdtype
 * exactly as ma_gather_kv writes it; the scores equal ma_gather_kv + ma_value_score on
 * those rows, bit for bit, without the gathered [n, D] rows.  Slots outside the cache give
 * zero rows.  D 64 or 128; workspace ma_value_score_workspace_bytes(B*H, n, D). */
int ma_value_score_slots(const float *a, int64_t a_stride, const ma_prefix *p, const int32_t *slots,
                         int64_t slot_stride, int B, int H, int n, int D, int vdtype, int fp32_mode, float *score,
                         int64_t score_stride, void *workspace, int64_t workspace_bytes, void *stream);

/* compaction of survivors (PackedKVCache.compact, cache.py:342-367; compact_tokens,
 * cache.py:659-678; EvictionState.compact, eviction.py:411-418): for every lane (b, h) and
 * i < capacity, row i of each plane becomes the old row keep[b, h, i] -- in place, for any
 * keep (out-of-range entries give zero rows).  A plane p is a token-major tensor: base
 * bases[p] (element b=0, h=0, token 0), byte strides strides[3p..3p+2] (b, h, token) and
 * row_bytes[p] bytes per token (even).  keep int64 with strides skeep (b, h; entries
 * contiguous).  Up to 8 planes per call. */
int64_t ma_compact_workspace_bytes(int rows, int capacity, const int32_t *row_bytes, int nplanes);
int ma_compact_tokens(void *const *bases, const int64_t *strides, const int32_t *row_bytes, int nplanes, int B,
                      int H, int n, const int64_t *keep, const int64_t skeep[2], int capacity, void *workspace,
                      int64_t workspace_bytes, void *stream);

/* append of a finalized block into a 16-bit cache (PackedKVCache.stage_layer for
 * bf16 layouts, cache.py:423-547): dst[b, h, at + t, :] = src[b, h, t, :] for t < T,
 * converted to dst's dtype (round to nearest even). */
int ma_append_tokens(ma_tensor4 src, ma_tensor4 dst, int B, int H, int T, int D, int at, void *stream);

/* gather_packed_kv (ops.py:570-662, 835-855; oracle reference.py:396-400): the
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
/* PackedKVCache.stage_layer of a packed store (cache.py:423-548, with the plan of
 * begin_append, 385-421): over the token axis [k_res rows 0..old_res | k_new rows 0..T) (and the
 * same for V), the first `move` tokens (a multiple of 32) are quantized as
 * ma_quantize_keys / ma_quantize_values do into planes kq/ks/kz and vq/vs/vz whose first
 * group / row is where they go, and the remaining keep = old_res + T - move tokens are
 * written to the residual rows 0..keep (in place: its rows move down by `move`).  The
 * residual and the new tokens share one dtype (the quantizers' rule follows it), as the
 * reference's [residual | new.to(compute dtype)] tensor does.  Up to three launches,
 * no temporary. */
int ma_append_packed(ma_tensor4 k_res, ma_tensor4 v_res, int old_res, ma_tensor4 k_new, ma_tensor4 v_new, int B,
                     int H, int T, int D, int move, int keep, void *kq, const int64_t skq[4], void *ks, void *kz,
                     const int64_t sks[3], void *vq, const int64_t svq[4], void *vs, void *vz,
                     const int64_t svs[3], void *stream);

/* f1. packed eviction rebuild, plan half: the lists of the session's lazy / full
 * compaction (runtime/session.py:288-345, BitSieveSession._evict_to) for `lanes`
 * (layer, batch, KV head) lanes of `live` live entries each.  phys int32 (old slot of
 * each live entry, < 2^24) and pos (int32, or int64 if pos_is_i64) have lane strides
 * phys_stride / pos_stride.  A key group of the old quantized part [0, quantized_length)
 * is kept when it holds >= need live entries and is not one of its last tail_groups
 * groups (need > 32: none, the "full" mode); the window newest entries outside the
 * quantized part stay bf16; every other entry is re-encoded.  Outputs per lane, padded
 * with -1: groups_before [max(1, quantized_length/32)] kept group ids ascending,
 * encode [live] and stage [live] old slots in (position, slot) order; counts [lanes][3]
 * int32 = (kept groups, encoded, staged), all -1 for a lane out of (position, slot)
 * order with more than 16384 live entries (not built).  The caller pads the lists to
 * the largest count of any lane, as the reference does. */
int ma_rebuild_plan(const int32_t *phys, int64_t phys_stride, const void *pos, int pos_is_i64,
                    int64_t pos_stride, int lanes, int live, int quantized_length, int need, int tail_groups,
                    int window, int64_t *groups_before, int64_t gb_stride, int64_t *encode, int64_t enc_stride,
                    int64_t *stage, int64_t stage_stride, int32_t *counts, void *stream);

/* f1. packed eviction rebuild, data half: PackedKVCache.rebuild (cache.py:236-335) of the
 * B x H lanes of old_store into new_store (both as ma_prefix: nq = quantized length, kf/vf
 * = the bf16 residual of nf entries; new_store's pointers are written).  The new lane
 * is [groups_before | encode quantized into ceil(m/32) groups | groups_after] + stage as
 * the new residual: old key groups copied byte for byte (a -1 entry copies group 0),
 * old slots dequantized to bf16 and quantized again in bf16 arithmetic (-1 and the
 * padding of the last group: zeros), old slots kept as bf16 rows (-1: zeros).  Lists are
 * int64 [lanes][width] with lane strides (0: one list for every lane).  remap int64
 * [lanes][old length] (lane stride
 * remap_stride) = new slot of every old slot, -1 if dropped (a later list wins a slot
 * named twice: groups, then encode, then stage).  phys (optional, int32, lane stride
 * phys_stride, live entries) is rewritten through remap (EvictionState slots,
 * session.py:352-355).  status int32 [lanes]: bit 0 = a list entry outside the old
 * storage (ignored), bit 1 = a live entry with no new slot. */
int ma_rebuild_packed(const ma_prefix *old_store, int B, int H, int D, const ma_prefix *new_store,
                      const int64_t *groups_before, int64_t gb_stride, int g1, const int64_t *encode,
                      int64_t enc_stride, int m, const int64_t *groups_after, int64_t ga_stride, int g3,
                      const int64_t *stage, int64_t stage_stride, int st, int64_t *remap, int64_t remap_stride,
                      int32_t *phys, int64_t phys_stride, int live, int32_t *status, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MASKAHEAD_HIP_H */
