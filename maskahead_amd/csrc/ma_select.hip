// Per-row selection kernels with index-ascending tie-break:
//   * read set  (session.py:1429-1438): rank.masked_fill(dead, -inf).topk(k), indices sorted;
//   * keep set  (eviction.py:355-409, score-ranked policies): the W newest entries, plus the
//     top (C - W) of the score among the others where sinks and pinned positions rank
//     +inf, returned in position order.
//
// One workgroup (1024 threads) per row.  Element j = e*NT + tid lives in thread tid, slot
// e, as a monotone 32-bit key (larger float -> larger key, -0.0 == +0.0, NaN above +inf,
// padding 0 below every real key).  The k-th largest key T is found exactly by an LDS
// histogram radix select over three digits (11 + 11 + 10 bits): per digit one pass of LDS
// atomics over the keys that match the digits found so far, then a block-wide suffix
// scan of the bins.  An element is selected if key > T, or key == T and fewer than
// k - count(key > T) equal keys precede it in index order.  A block-wide exclusive scan of
// the selection flags in index order gives every selected element its output slot, so the
// output is ascending by construction -- no sort.
#include "ma_common.h"

namespace {

constexpr int NT = 1024;
constexpr int NW = NT / 64;
constexpr int NBINS = 2048;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

constexpr int NHC = 4;        // histogram copies (wave w counts into copy w % 4)
constexpr uint32_t KEY_NEG_INF = 0x007fffffu;   // ma_order_key(-inf); padding keys are 0

constexpr int CAND_MAX = 4096;   // keys of the boundary bin kept in LDS after the first digit

template <int VPT>
struct SelectSmem {
    uint32_t hist[NHC][NBINS];
    uint32_t cand[CAND_MAX];
    int ncand;
    int wsum[NW];
    uint32_t kred[2][NW];
    int found_digit, found_gt, found_cnt;
    int c_eq[VPT][NW], c_sel[VPT][NW];
    int p_eq[VPT + 1], p_sel[VPT + 1];
    int flag;
};

// Block-wide inclusive suffix sum of v over thread order (thread t gets sum over t' >= t).
template <int VPT>
__device__ __forceinline__ int block_suffix_incl(int v, SelectSmem<VPT> &S) {
    const int lane = lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_down(v, o);
        if (lane + o < 64) v += y;
    }
    if (lane == 0) S.wsum[wave] = v;   // lane 0 holds the wave total
    __syncthreads();
    int above = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) above += (w > wave) ? S.wsum[w] : 0;
    return v + above;
}

// The k-th largest of the block's keys (1 <= k <= number of keys).  Returns T and sets
// need = k - count(key > T), the number of keys equal to T that are selected.
// The digits adapt to the keys' range: above the highest bit in which the largest key and
// the smallest key above -inf differ, all those keys agree, so the first 11-bit digit
// starts there (scores that span a few binades then spread over many bins instead of
// piling into a few, which would serialize the LDS atomics).  Keys at -inf or below only
// matter when fewer than k keys are above -inf; then T is -inf.
template <int VPT>
__device__ uint32_t radix_kth(const uint32_t (&key)[VPT], int k, SelectSmem<VPT> &S, int &need, int &eq) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // range of the keys above -inf, and how many there are
    uint32_t kmax = 0u, kmin = 0xffffffffu;
    int nhi = 0;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool hi = key[e] > KEY_NEG_INF;
        kmax = max(kmax, key[e]);
        kmin = hi ? min(kmin, key[e]) : kmin;
        nhi += __popcll(__ballot(hi));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
    }
    if (lane == 0) {
        S.kred[0][wave] = kmax;
        S.kred[1][wave] = kmin;
        S.wsum[wave] = nhi;
    }
    __syncthreads();
    int tot_hi = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        kmax = max(kmax, S.kred[0][w]);
        kmin = min(kmin, S.kred[1][w]);
        tot_hi += S.wsum[w];
    }
    __syncthreads();  // kred / wsum are reused below
    if (tot_hi < k) {  // fewer than k keys above -inf: T = -inf
        need = k - tot_hi;
        eq = -1;        // not counted
        return KEY_NEG_INF;
    }
    const uint32_t diff = kmax ^ kmin;
    if (diff == 0u) {  // every key above -inf is equal
        need = k;
        eq = tot_hi;
        return kmax;
    }
    int hi = 31 - __builtin_clz(diff);            // highest bit that still varies
    uint32_t pmask = hi == 31 ? 0u : ~((2u << hi) - 1u);
    uint32_t prefix = kmax & pmask;
    int kk = k;
    bool listed = false;      // after the first digit: the boundary bin's keys are in S.cand
    int ncand = 0;
#pragma unroll 1
    while (hi >= 0) {
        const int w = hi + 1 < 11 ? hi + 1 : 11;
        const int shift = hi - w + 1;
        const int nb = 1 << w;
        for (int i = tid; i < NHC * NBINS; i += NT) (&S.hist[0][0])[i] = 0u;
        __syncthreads();
        uint32_t *hist = S.hist[wave % NHC];
        if (!listed) {
#pragma unroll
            for (int e = 0; e < VPT; ++e)
                if ((key[e] & pmask) == prefix) atomicAdd(&hist[(key[e] >> shift) & (uint32_t)(nb - 1)], 1u);
        } else {
            for (int i = tid; i < ncand; i += NT) {
                const uint32_t x = S.cand[i];
                if ((x & pmask) == prefix) atomicAdd(&hist[(x >> shift) & (uint32_t)(nb - 1)], 1u);
            }
        }
        __syncthreads();
        // thread t owns bins 2t (lower digit) and 2t+1
        const int b0 = 2 * tid;
        int c0 = 0, c1 = 0;
        if (b0 < nb) {
#pragma unroll
            for (int c = 0; c < NHC; ++c) {
                c0 += (int)S.hist[c][b0];
                c1 += (int)S.hist[c][b0 + 1];
            }
        }
        const int incl = block_suffix_incl<VPT>(c0 + c1, S);
        const int above = incl - c0 - c1;  // keys with a digit above both of my bins
        if (above < kk && above + c1 >= kk) {
            S.found_digit = b0 + 1;
            S.found_gt = above;
            S.found_cnt = c1;
        } else if (above + c1 < kk && above + c1 + c0 >= kk) {
            S.found_digit = b0;
            S.found_gt = above + c1;
            S.found_cnt = c0;
        }
        if (tid == 0) S.ncand = 0;
        __syncthreads();
        const uint32_t d = (uint32_t)S.found_digit;
        const int bin_cnt = S.found_cnt;
        kk -= S.found_gt;
        prefix |= d << shift;
        pmask |= (uint32_t)(nb - 1) << shift;
        hi = shift - 1;
        if (!listed && hi >= 0 && bin_cnt <= CAND_MAX) {
            // keep the boundary bin's keys in LDS; later digits read only those
#pragma unroll
            for (int e = 0; e < VPT; ++e)
                if ((key[e] & pmask) == prefix) S.cand[atomicAdd(&S.ncand, 1)] = key[e];
            __syncthreads();
            ncand = S.ncand;
            listed = true;
        }
        eq = bin_cnt;
        __syncthreads();  // found_* and wsum are rewritten by the next pass
    }
    need = kk;
    return prefix;
}

// Output slots of the selected keys (bit e of selbits: slot e of this thread) in index
// order: counts per (slot, wave), an exclusive scan over them, then each selected key's
// output slot = keys selected before it.
template <int VPT, class Emit>
__device__ __forceinline__ void select_emit(uint64_t selbits, SelectSmem<VPT> &S, Emit emit) {
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const uint64_t bs = __ballot((selbits >> e) & 1);
        if (lane == 0) S.c_sel[e][wave] = __popcll(bs);
    }
    __syncthreads();
    if (wave == 0) {
        int tot = 0;
        if (lane < VPT) {
            for (int w = 0; w < NW; ++w) {
                const int c = S.c_sel[lane][w];
                S.c_sel[lane][w] = tot;
                tot += c;
            }
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane < VPT) S.p_sel[lane] = incl - tot;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool sl = (selbits >> e) & 1;
        const uint64_t bs = __ballot(sl);
        if (sl) emit(e, S.p_sel[e] + S.c_sel[e][wave] + __popcll(bs & below));
    }
}

// Select key > T or (key == T and among the first `need` equal keys in index order), and
// give every selected element its rank in index order.  Writes slot (or -1) per slot e.
template <int VPT, class Emit>
__device__ void select_and_rank(const uint32_t (&key)[VPT], uint32_t thr, int need, int eq, SelectSmem<VPT> &S,
                                Emit emit) {
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const uint64_t below = (1ull << lane) - 1ull;
    if (eq == need) {
        // every key equal to T is selected: no tie ranking needed
        uint64_t selbits = 0;
#pragma unroll
        for (int e = 0; e < VPT; ++e) selbits |= (uint64_t)(key[e] >= thr) << e;
        select_emit<VPT>(selbits, S, emit);
        return;
    }
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const uint64_t be = __ballot(key[e] == thr);
        if (lane == 0) S.c_eq[e][wave] = __popcll(be);
    }
    __syncthreads();
    // wave 0, lane e: slot e's equal counts -> exclusive prefix over waves (in place) and,
    // by a wave scan, over slots
    if (wave == 0) {
        int tot = 0;
        if (lane < VPT) {
            for (int w = 0; w < NW; ++w) {
                const int c = S.c_eq[lane][w];
                S.c_eq[lane][w] = tot;
                tot += c;
            }
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane < VPT) S.p_eq[lane] = incl - tot;
    }
    __syncthreads();
    // tie rank of each equal key in index order
    uint64_t selbits = 0;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool is_eq = key[e] == thr;
        const int eb = S.p_eq[e] + S.c_eq[e][wave] + __popcll(__ballot(is_eq) & below);
        const bool sl = key[e] > thr || (is_eq && eb < need);
        selbits |= (uint64_t)sl << e;
    }
    select_emit<VPT>(selbits, S, emit);
}

// ---------------------------------------------------------------- read set
template <int VPT>
__global__ void __launch_bounds__(NT) topk_kernel(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                                  int64_t mask_stride, int n, int k, int64_t *idx,
                                                  int64_t idx_stride, float *values) {
    __shared__ SelectSmem<VPT> S;
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *rr = rank + (int64_t)row * rank_stride;
    const uint8_t *mr = mask ? mask + (int64_t)row * mask_stride : nullptr;
    uint32_t key[VPT];
    // branchless loads from clamped indices, 16 slots at a time in flight
#pragma unroll
    for (int e0 = 0; e0 < VPT; e0 += 16) {
        constexpr int CH = VPT < 16 ? VPT : 16;
        float v[CH];
        uint8_t mb[CH];
#pragma unroll
        for (int e = 0; e < CH; ++e) v[e] = rr[min((e0 + e) * NT + tid, n - 1)];
#pragma unroll
        for (int e = 0; e < CH; ++e) mb[e] = mr ? mr[min((e0 + e) * NT + tid, n - 1)] : (uint8_t)1;
#pragma unroll
        for (int e = 0; e < CH; ++e)
            key[e0 + e] = (e0 + e) * NT + tid < n ? ma_order_key(mb[e] ? v[e] : -INFINITY) : 0u;
    }
    int need, eq;
    const uint32_t thr = radix_kth<VPT>(key, k, S, need, eq);
    int64_t *out = idx + (int64_t)row * idx_stride;
    float *vout = values ? values + (int64_t)row * k : nullptr;
    select_and_rank<VPT>(key, thr, need, eq, S, [&](int e, int slot) {
        if (slot < k) {
            const int j = e * NT + tid;
            out[slot] = j;
            if (vout) vout[slot] = (mr && !mr[j]) ? -INFINITY : rr[j];
        }
    });
}

// ---------------------------------------------------------------- keep set
// Row = one (layer, batch, KV head) lane with n live entries whose positions increase
// strictly along the live axis (the eviction state's invariant: survivors are stored in
// position order and new entries are appended with larger positions).  Then the W newest
// entries are the last W, the contest runs over the first m = n - W entries, and index
// order is position order.  A row whose positions do not increase gets status 1.
template <int VPT, typename PosT>
__global__ void __launch_bounds__(NT) keep_kernel(const PosT *pos, int64_t pos_stride, const float *score,
                                                  int64_t score_stride, int n, int capacity, int window,
                                                  int64_t sink_tokens, const int64_t *pin_lo_rows, int64_t pin_lo,
                                                  int64_t pin_hi, int has_pin, int64_t *keep, int64_t keep_stride,
                                                  int32_t *status) {
    __shared__ SelectSmem<VPT> S;
    const int row = blockIdx.x, tid = threadIdx.x;
    const PosT *pr = pos + (int64_t)row * pos_stride;
    const float *sr = score + (int64_t)row * score_stride;
    const int w = min(window, capacity);
    const int m = n - w;         // contestants
    const int rest = capacity - w;
    const int64_t plo = pin_lo_rows ? pin_lo_rows[row] : pin_lo;
    if (tid == 0) S.flag = 0;
    __syncthreads();
    uint32_t key[VPT];
    bool bad = false;
#pragma unroll
    for (int e0 = 0; e0 < VPT; e0 += 8) {
        constexpr int CH = VPT < 8 ? VPT : 8;
        PosT p[CH], pn[CH];
        float v[CH];
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int jc = min((e0 + e) * NT + tid, n - 1);
            p[e] = pr[jc];
            pn[e] = pr[min(jc + 1, n - 1)];
            v[e] = sr[jc];
        }
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int j = (e0 + e) * NT + tid;
            bad |= (j + 1 < n) && !(p[e] < pn[e]);
            float x = v[e];
            if ((int64_t)p[e] < sink_tokens) x = INFINITY;
            if (has_pin && (int64_t)p[e] >= plo && (int64_t)p[e] < pin_hi) x = INFINITY;
            key[e0 + e] = j < m ? ma_order_key(x) : 0u;
        }
    }
    if (bad) S.flag = 1;   // benign race: every writer stores 1
    __syncthreads();
    if (tid == 0 && status) status[row] = S.flag;
    int64_t *out = keep + (int64_t)row * keep_stride;
    if (rest > 0) {
        int need, eq;
        const uint32_t thr = radix_kth<VPT>(key, rest, S, need, eq);
        select_and_rank<VPT>(key, thr, need, eq, S, [&](int e, int slot) {
            if (slot < rest) out[slot] = e * NT + tid;
        });
    }
    for (int i = tid; i < w; i += NT) out[rest + i] = m + i;
}

int vpt_for(int n) {
    const int v = (n + NT - 1) / NT;
    if (v <= 4) return 4;
    if (v <= 8) return 8;
    if (v <= 16) return 16;
    if (v <= 32) return 32;
    if (v <= 64) return 64;
    return 0;
}

}  // namespace

extern "C" int ma_topk_select(const float *rank, int64_t rank_stride, const uint8_t *mask, int64_t mask_stride,
                              int rows, int n, int k, int64_t *idx, int64_t idx_stride, float *values, void *stream) {
    if (!rank || !idx || rows < 0 || n < 0 || k < 0 || k > n || idx_stride < k || rank_stride < n ||
        (mask && mask_stride < n)) {
        ma_set_error("ma_topk_select: bad arguments (rows=%d n=%d k=%d)", rows, n, k);
        return MA_EINVAL;
    }
    if (rows == 0 || k == 0) return MA_OK;
    hipStream_t st = (hipStream_t)stream;
    const int vpt = vpt_for(n);
#define MA_TOPK(V)                                                                                                \
    hipLaunchKernelGGL(topk_kernel<V>, dim3(rows), dim3(NT), 0, st, rank, rank_stride, mask, mask_stride, n, k, idx, \
                       idx_stride, values)
    switch (vpt) {
        case 4: MA_TOPK(4); break;
        case 8: MA_TOPK(8); break;
        case 16: MA_TOPK(16); break;
        case 32: MA_TOPK(32); break;
        case 64: MA_TOPK(64); break;
        default:
            ma_set_error("ma_topk_select: n=%d exceeds the built maximum %d", n, 64 * NT);
            return MA_EUNSUPPORTED;
    }
#undef MA_TOPK
    return ma_check_launch("ma_topk_select");
}

extern "C" int ma_keep_select(const void *pos, int pos_is_i64, int64_t pos_stride, const float *score,
                              int64_t score_stride, int rows, int n, int capacity, int window, int64_t sink_tokens,
                              const int64_t *pin_lo_rows, int64_t pin_lo, int64_t pin_hi, int has_pin, int64_t *keep,
                              int64_t keep_stride, int32_t *status, void *stream) {
    if (!pos || !score || !keep || rows < 0 || n < 0 || capacity < 0 || capacity > n || window < 0 ||
        keep_stride < capacity || pos_stride < n || score_stride < n) {
        ma_set_error("ma_keep_select: bad arguments (rows=%d n=%d capacity=%d window=%d)", rows, n, capacity,
                     window);
        return MA_EINVAL;
    }
    if (rows == 0 || capacity == 0) return MA_OK;
    hipStream_t st = (hipStream_t)stream;
    const int vpt = vpt_for(n);
#define MA_KEEP(V)                                                                                                  \
    do {                                                                                                            \
        if (pos_is_i64)                                                                                             \
            hipLaunchKernelGGL((keep_kernel<V, int64_t>), dim3(rows), dim3(NT), 0, st, (const int64_t *)pos,         \
                               pos_stride, score, score_stride, n, capacity, window, sink_tokens, pin_lo_rows, pin_lo, \
                               pin_hi, has_pin, keep, keep_stride, status);                                          \
        else                                                                                                        \
            hipLaunchKernelGGL((keep_kernel<V, int32_t>), dim3(rows), dim3(NT), 0, st, (const int32_t *)pos,         \
                               pos_stride, score, score_stride, n, capacity, window, sink_tokens, pin_lo_rows, pin_lo, \
                               pin_hi, has_pin, keep, keep_stride, status);                                          \
    } while (0)
    switch (vpt) {
        case 4: MA_KEEP(4); break;
        case 8: MA_KEEP(8); break;
        case 16: MA_KEEP(16); break;
        case 32: MA_KEEP(32); break;
        case 64: MA_KEEP(64); break;
        default:
            ma_set_error("ma_keep_select: n=%d exceeds the built maximum %d", n, 64 * NT);
            return MA_EUNSUPPORTED;
    }
#undef MA_KEEP
    return ma_check_launch("ma_keep_select");
}
