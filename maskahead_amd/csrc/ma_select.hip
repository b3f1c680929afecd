// Keep-set selection with index-ascending tie-break (eviction.py:355-409, score-ranked
// policies): the W newest entries, plus the top (C - W) of the score among the others
// where sinks and pinned positions rank +inf, returned in position order.
//
// One workgroup (1024 threads) per row.  Thread t owns VPT/4 runs of 4 consecutive
// elements, run q covering j = 4*(q*NT + t) + c (so a wave's 16-byte loads are one
// contiguous 1 KB), held as monotone 32-bit keys (larger float -> larger key,
// -0.0 == +0.0, NaN above +inf, padding 0 below every real key).
// The k-th largest key T is found exactly by an LDS-histogram radix select whose 11-bit
// digits start at the highest bit that varies among the keys above -inf; after the first
// digit the keys of the boundary bin are kept in an LDS candidate list (appended with
// one atomic per wave).  An element is selected if key > T, or key == T and fewer than
// k - count(key > T) equal keys precede it in index order.  The output slot of a selected
// element is one block-wide exclusive scan of per-(thread, run) counts plus its rank
// inside the run: the output is ascending by
// construction -- no sort.  (Index order is run-major: run q of every thread, then run
// q + 1; the scans carry one count per run.)
#include "ma_common.h"

namespace {

constexpr int NT = 1024;
constexpr int NW = NT / 64;
constexpr int NBINS = 2048;
constexpr int NHC = 4;        // histogram copies (wave w counts into copy w % 4)
constexpr uint32_t KEY_NEG_INF = 0x007fffffu;   // ma_order_key(-inf); padding keys are 0
constexpr int CAND_MAX = 4096;   // keys of the boundary bin kept in LDS after the first digit

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

struct SelectSmem {
    uint32_t hist[NHC][NBINS];
    uint32_t cand[CAND_MAX];
    int ncand;
    int wsum[NW];
    uint32_t kred[2][NW];
    int found_digit, found_gt, found_cnt;
    int flag;
    int rsum[16][NW];
};

// Block-wide inclusive suffix sum of v over thread order (thread t gets sum over t' >= t).
__device__ __forceinline__ int block_suffix_incl(int v, SelectSmem &S) {
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const uint32_t pre = ma_wave_prefix_u32((uint32_t)v);          // lanes 0..lane
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)pre, 63);
    if (lane == 0) S.wsum[wave] = (int)tot;
    __syncthreads();
    int above = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) above += (w > wave) ? S.wsum[w] : 0;
    __syncthreads();   // wsum is reused
    return (int)(tot - pre) + v + above;
}

// Exclusive prefix of per-(run, thread) counts c[q] in index order (run-major, then
// thread): all NR runs are scanned at once, two runs per 32-bit word (a run holds at most
// 4 * NT = 4096 elements, so 16-bit halves never carry), one barrier pair.
template <int NR>
__device__ __forceinline__ void block_prefix_runs(int (&c)[NR], SelectSmem &S) {
    constexpr int NP = (NR + 1) / 2;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    uint32_t incl[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q)
        incl[q] = (uint32_t)c[2 * q] | (2 * q + 1 < NR ? (uint32_t)c[2 * q + 1] << 16 : 0u);
#pragma unroll
    for (int q = 0; q < NP; ++q) incl[q] = ma_wave_prefix_u32(incl[q]);
    if (lane == 63) {
#pragma unroll
        for (int q = 0; q < NP; ++q) S.rsum[q][wave] = (int)incl[q];
    }
    __syncthreads();
    int base = 0;   // counts of all earlier runs
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        uint32_t before = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const uint32_t x = (uint32_t)S.rsum[q][w];
            before += (w < wave) ? x : 0u;
            tot += x;
        }
        const uint32_t ex = before + incl[q];   // inclusive, both halves
        const int lo = (int)(ex & 0xffffu) - c[2 * q], tlo = (int)(tot & 0xffffu);
        c[2 * q] = base + lo;
        base += tlo;
        if (2 * q + 1 < NR) {
            const int hi = (int)(ex >> 16) - c[2 * q + 1], thi = (int)(tot >> 16);
            c[2 * q + 1] = base + hi;
            base += thi;
        }
    }
    __syncthreads();   // rsum is reused
}

// The k-th largest of the block's keys (1 <= k <= number of keys).  Returns T and sets
// need = k - count(key > T), the number of keys equal to T that are selected, and eq =
// count(key == T) (-1 when T is -inf and eq was not counted).
template <int VPT>
__device__ uint32_t radix_kth(const uint32_t (&key)[VPT], int k, SelectSmem &S, int &need, int &eq) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // range of the keys above -inf, and how many there are
    uint32_t kmax = 0u, kmin = 0xffffffffu;
    int nhi = 0;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const bool hi = key[e] > KEY_NEG_INF;
        kmax = max(kmax, key[e]);
        kmin = hi ? min(kmin, key[e]) : kmin;
        nhi += hi ? 1 : 0;
    }
    kmax = ma_wave_max_u32(kmax);
    kmin = ~ma_wave_max_u32(~kmin);
    nhi = (int)ma_wave_sum_u32((uint32_t)nhi);
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
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll 1
    while (hi >= 0) {
        const int w = hi + 1 < 11 ? hi + 1 : 11;
        const int shift = hi - w + 1;
        const int nb = 1 << w;
        for (int i = tid; i < NHC * NBINS; i += NT) (&S.hist[0][0])[i] = 0u;
        if (tid == 0) S.ncand = 0;
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
        const int incl = block_suffix_incl(c0 + c1, S);
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
        __syncthreads();
        const uint32_t d = (uint32_t)S.found_digit;
        const int bin_cnt = S.found_cnt;
        kk -= S.found_gt;
        prefix |= d << shift;
        pmask |= (uint32_t)(nb - 1) << shift;
        hi = shift - 1;
        if (!listed && hi >= 0 && bin_cnt <= CAND_MAX) {
            // keep the boundary bin's keys in LDS (one atomic per wave and slot); later
            // digits read only those
#pragma unroll
            for (int e = 0; e < VPT; ++e) {
                const bool in = (key[e] & pmask) == prefix;
                const uint64_t m = __ballot(in);
                if (m) {
                    int base = 0;
                    if (lane == 0) base = atomicAdd(&S.ncand, __popcll(m));
                    base = __builtin_amdgcn_readfirstlane(base);
                    if (in) S.cand[base + __popcll(m & below)] = key[e];
                }
            }
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

// Select key > T or (key == T and among the first `need` equal keys in index order), then
// emit(key, j, slot) for every selected element (its key, index j) with its output slot
// in index order.
template <int VPT, class Emit>
__device__ void select_emit(const uint32_t (&key)[VPT], uint32_t thr, int need, int eq, SelectSmem &S, Emit emit) {
    constexpr int NR = VPT / 4;
    const int tid = threadIdx.x;
    uint64_t selbits = 0;
    if (eq == need) {
        // every key equal to T is selected: no tie ranking needed
#pragma unroll
        for (int e = 0; e < VPT; ++e) selbits |= (uint64_t)(key[e] >= thr) << e;
    } else {
        int eb[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) {
            eb[q] = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) eb[q] += key[4 * q + c] == thr ? 1 : 0;
        }
        block_prefix_runs<NR>(eb, S);   // equal keys before each run
#pragma unroll
        for (int q = 0; q < NR; ++q) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = 4 * q + c;
                const bool is_eq = key[e] == thr;
                const bool sl = key[e] > thr || (is_eq && eb[q] < need);
                eb[q] += is_eq ? 1 : 0;
                selbits |= (uint64_t)sl << e;
            }
        }
    }
    int slot[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) slot[q] = __popcll((selbits >> (4 * q)) & 15ull);
    block_prefix_runs<NR>(slot, S);
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = 4 * q + c;
            if ((selbits >> e) & 1) {
                emit(key[e], 4 * (q * NT + tid) + c, slot[q]);
                ++slot[q];
            }
        }
    }
}

// float of a key (inverse of ma_order_key; -0.0 and NaN payloads come back canonical)
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// The VPT elements of this thread (runs of 4, run q at 4*(q*NT + t)) as floats: 16-byte
// loads when the row is aligned, clamped scalar loads otherwise.
template <int VPT>
__device__ __forceinline__ void load_runs(float (&v)[VPT], const float *row, int n, bool vec) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < VPT / 4; ++q) {
        const int j0 = 4 * (q * NT + tid);
        if (vec && j0 + 4 <= n) {
            const f32x4_t x = *(const f32x4_t *)(row + j0);
            v[4 * q] = x[0];
            v[4 * q + 1] = x[1];
            v[4 * q + 2] = x[2];
            v[4 * q + 3] = x[3];
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * q + c] = row[min(j0 + c, n - 1)];
        }
    }
}

__device__ __forceinline__ int elem_index(int e) { return 4 * ((e >> 2) * NT + (int)threadIdx.x) + (e & 3); }

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
                                                  int32_t *status, int vec) {
    __shared__ SelectSmem S;
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
    for (int q = 0; q < VPT / 4; ++q) {
        // run q: elements j0 .. j0+3, and the element before it for the order check
        const int j0 = 4 * (q * NT + tid);
        float v[4];
        if (vec && j0 + 4 <= n) {
            const f32x4_t x = *(const f32x4_t *)(sr + j0);
            v[0] = x[0];
            v[1] = x[1];
            v[2] = x[2];
            v[3] = x[3];
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = sr[min(j0 + c, n - 1)];
        }
        PosT p[5];
        p[0] = pr[min(max(j0 - 1, 0), n - 1)];
#pragma unroll
        for (int c = 0; c < 4; ++c) p[c + 1] = pr[min(j0 + c, n - 1)];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int j = j0 + c;
            bad |= (j > 0 && j < n) && !(p[c] < p[c + 1]);
            float x = v[c];
            if ((int64_t)p[c + 1] < sink_tokens) x = INFINITY;
            if (has_pin && (int64_t)p[c + 1] >= plo && (int64_t)p[c + 1] < pin_hi) x = INFINITY;
            key[4 * q + c] = j < m ? ma_order_key(x) : 0u;
        }
    }
    if (bad) S.flag = 1;   // benign race: every writer stores 1
    __syncthreads();
    if (tid == 0 && status) status[row] = S.flag;
    int64_t *out = keep + (int64_t)row * keep_stride;
    if (rest > 0) {
        int need, eq;
        const uint32_t thr = radix_kth<VPT>(key, rest, S, need, eq);
        select_emit<VPT>(key, thr, need, eq, S, [&](uint32_t, int j, int slot) {
            if (slot < rest) out[slot] = j;
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
    const int vec = ((uintptr_t)score & 15) == 0 && score_stride % 4 == 0;
#define MA_KEEP(V)                                                                                                  \
    do {                                                                                                            \
        if (pos_is_i64)                                                                                             \
            hipLaunchKernelGGL((keep_kernel<V, int64_t>), dim3(rows), dim3(NT), 0, st, (const int64_t *)pos,         \
                               pos_stride, score, score_stride, n, capacity, window, sink_tokens, pin_lo_rows, pin_lo, \
                               pin_hi, has_pin, keep, keep_stride, status, vec);                                     \
        else                                                                                                        \
            hipLaunchKernelGGL((keep_kernel<V, int32_t>), dim3(rows), dim3(NT), 0, st, (const int32_t *)pos,         \
                               pos_stride, score, score_stride, n, capacity, window, sink_tokens, pin_lo_rows, pin_lo, \
                               pin_hi, has_pin, keep, keep_stride, status, vec);                                     \
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
