// Per-row top-k selection with index-ascending tie-break (the read set of
// session.py:1429-1438: rank.masked_fill(dead, -inf).topk(k) followed by an ascending
// sort of the indices).
//
// One workgroup (1024 threads) per row; thread i owns the VPT consecutive entries
// [i*VPT, (i+1)*VPT) as monotone 32-bit keys in registers.  The k-th largest key T is
// found exactly by a most-significant-bit-first bisection (32 block-wide counts of
// key >= candidate).  An entry is selected if key > T, or key == T and fewer than
// k - count(key > T) equal keys precede it in index order; a block-wide exclusive scan
// of the selection flags, taken in index order, then gives every selected entry its
// output slot -- the output is ascending by construction, no sort.
#include "ma_common.h"

namespace {

constexpr int NT = 1024;
constexpr int NW = NT / 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// One workgroup per row.  Element j = e*NT + tid belongs to thread tid (slot e), so every
// load is coalesced and, within a slot, index order is thread order.  Counting uses wave
// ballots (a popcount per wave, no shuffles); the k-th largest key T is found by a
// most-significant-bit-first bisection, one barrier per bit (double-buffered counts).
// Output slot of a selected element = selected elements in earlier slots + in earlier
// waves of its slot + lanes below it in its wave: ascending indices, no sort.
template <int VPT>
__global__ void __launch_bounds__(NT) topk_kernel(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                                  int64_t mask_stride, int n, int k, int64_t *idx,
                                                  int64_t idx_stride, float *values) {
    __shared__ int cnt2[2][NW];
    __shared__ int c_gt[VPT][NW], c_eq[VPT][NW], c_sel[VPT][NW];
    __shared__ int p_eq[VPT + 1], p_sel[VPT + 1];
    static_assert(VPT <= 64, "one wave scans the slots");
    const int row = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
    const float *rr = rank + (int64_t)row * rank_stride;
    const uint8_t *mr = mask ? mask + (int64_t)row * mask_stride : nullptr;
    uint32_t key[VPT];
    // branchless loads from clamped indices, so all VPT loads are in flight at once
    float v[VPT];
#pragma unroll
    for (int e = 0; e < VPT; ++e) v[e] = rr[min(e * NT + tid, n - 1)];
    uint32_t live = 0xffffffffu;
    if (mr) {
        uint8_t mb[VPT];
#pragma unroll
        for (int e = 0; e < VPT; ++e) mb[e] = mr[min(e * NT + tid, n - 1)];
#pragma unroll
        for (int e = 0; e < VPT; ++e) v[e] = mb[e] ? v[e] : -INFINITY;
    }
    (void)live;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const int j = e * NT + tid;
        key[e] = j < n ? ma_order_key(v[e]) : 0u;  // 0: below every real key (-inf maps to 0x007fffff)
    }
    uint32_t thr = 0u;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = thr | (1u << bit);
        int c = 0;
#pragma unroll
        for (int e = 0; e < VPT; ++e) c += __popcll(__ballot(key[e] >= cand));
        if (lane == 0) cnt2[bit & 1][wave] = c;
        __syncthreads();
        int tot = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) tot += cnt2[bit & 1][w];
        if (tot >= k) thr = cand;
    }
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const uint64_t bg = __ballot(key[e] > thr);
        const uint64_t be = __ballot(key[e] == thr);
        if (lane == 0) {
            c_gt[e][wave] = __popcll(bg);
            c_eq[e][wave] = __popcll(be);
        }
    }
    __syncthreads();
    // wave 0, lane e: slot e's counts -> exclusive prefix over waves (in place) and, by a
    // wave scan, over slots; the gt total gives the number of equal keys still needed
    if (wave == 0) {
        int eq_tot = 0, gt_tot = 0;
        if (lane < VPT) {
            for (int w = 0; w < NW; ++w) {
                const int c = c_eq[lane][w];
                c_eq[lane][w] = eq_tot;
                eq_tot += c;
                gt_tot += c_gt[lane][w];
            }
        }
        int incl = eq_tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        gt_tot = ma_wave_sum_i(gt_tot);
        if (lane < VPT) p_eq[lane] = incl - eq_tot;
        if (lane == 0) p_eq[VPT] = k - gt_tot;  // equal keys still needed
    }
    __syncthreads();
    const int need = p_eq[VPT];
    uint64_t selbits = 0;  // bit e: this thread's slot-e element is selected
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool is_eq = key[e] == thr;
        const int eb = p_eq[e] + c_eq[e][wave] + __popcll(__ballot(is_eq) & below);
        const bool sl = key[e] > thr || (is_eq && eb < need);
        selbits |= (uint64_t)sl << e;
        const uint64_t bs = __ballot(sl);
        if (lane == 0) c_sel[e][wave] = __popcll(bs);
    }
    __syncthreads();
    if (wave == 0) {
        int tot = 0;
        if (lane < VPT) {
            for (int w = 0; w < NW; ++w) {
                const int c = c_sel[lane][w];
                c_sel[lane][w] = tot;
                tot += c;
            }
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane < VPT) p_sel[lane] = incl - tot;
    }
    __syncthreads();
    int64_t *out = idx + (int64_t)row * idx_stride;
    float *vout = values ? values + (int64_t)row * k : nullptr;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool sl = (selbits >> e) & 1;
        const uint64_t bs = __ballot(sl);
        const int slot = p_sel[e] + c_sel[e][wave] + __popcll(bs & below);
        if (sl && slot < k) {
            const int j = e * NT + tid;
            out[slot] = j;
            if (vout) vout[slot] = v[e];
        }
    }
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
    const int vpt = (n + NT - 1) / NT;
#define MA_TOPK(V)                                                                                                \
    hipLaunchKernelGGL(topk_kernel<V>, dim3(rows), dim3(NT), 0, st, rank, rank_stride, mask, mask_stride, n, k, idx, \
                       idx_stride, values)
    if (vpt <= 4) MA_TOPK(4);
    else if (vpt <= 8) MA_TOPK(8);
    else if (vpt <= 16) MA_TOPK(16);
    else if (vpt <= 32) MA_TOPK(32);
    else if (vpt <= 64) MA_TOPK(64);
    else {
        ma_set_error("ma_topk_select: n=%d exceeds the built maximum %d", n, 64 * NT);
        return MA_EUNSUPPORTED;
    }
#undef MA_TOPK
    return ma_check_launch("ma_topk_select");
}
