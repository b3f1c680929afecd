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

__device__ __forceinline__ int block_sum(int v, int *sh) {
    v = ma_wave_sum_i(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    int s = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += sh[w];
    return s;
}

// exclusive prefix sum over threads in index order; *total gets the block total
__device__ __forceinline__ int block_exclusive_scan(int v, int *sh, int *total) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    __syncthreads();
    if (lane == 63) sh[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int x = sh[w];
        if (w < wave) before += x;
        all += x;
    }
    *total = all;
    return before + incl - v;
}

template <int VPT>
__global__ void __launch_bounds__(NT) topk_kernel(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                                  int64_t mask_stride, int n, int k, int64_t *idx,
                                                  int64_t idx_stride, float *values) {
    __shared__ int sh[NW];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *rr = rank + (int64_t)row * rank_stride;
    const uint8_t *mr = mask ? mask + (int64_t)row * mask_stride : nullptr;
    const int base = tid * VPT;
    uint32_t key[VPT];
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const int j = base + e;
        uint32_t kk = 0u;  // below every real key (-inf maps to 0x007fffff)
        if (j < n) kk = ma_order_key((mr && !mr[j]) ? -INFINITY : rr[j]);
        key[e] = kk;
    }
    uint32_t thr = 0u;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = thr | (1u << bit);
        int c = 0;
#pragma unroll
        for (int e = 0; e < VPT; ++e) c += key[e] >= cand;
        if (block_sum(c, sh) >= k) thr = cand;
    }
    int gt = 0, eq = 0;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        gt += key[e] > thr;
        eq += key[e] == thr;
    }
    const int n_gt = block_sum(gt, sh);
    int eq_total;
    const int eq_start = block_exclusive_scan(eq, sh, &eq_total);
    const int need = k - n_gt;
    int nsel = 0, eq_before = eq_start;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool is_eq = key[e] == thr;
        nsel += (key[e] > thr) || (is_eq && eq_before < need);
        eq_before += is_eq;
    }
    int sel_total;
    int slot = block_exclusive_scan(nsel, sh, &sel_total);
    // second walk: same decisions, now writing
    eq_before = eq_start;
    int64_t *out = idx + (int64_t)row * idx_stride;
    float *vout = values ? values + (int64_t)row * k : nullptr;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool is_eq = key[e] == thr;
        const bool sel = (key[e] > thr) || (is_eq && eq_before < need);
        eq_before += is_eq;
        if (sel && slot < k) {
            const int j = base + e;
            out[slot] = j;
            if (vout) vout[slot] = (mr && !mr[j]) ? -INFINITY : rr[j];
            ++slot;
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
