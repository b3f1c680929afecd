// Per-row selection over many workgroups per row, ties at the k-th value going to the
// smaller index:
//   * read set (session.py:1429-1438, reference.py:369-393):
//     rank.masked_fill(dead, -inf).topk(k) with its indices sorted;
//   * keep set (EvictionState.survivors, eviction.py:325-409, score-ranked policies): the
//     W = min(window, C) newest entries plus the top (C - W) of the score among the others,
//     positions < sink_tokens and pinned positions ranking +inf, in position order.  The
//     state keeps a lane's live entries in position order, so the newest W are the last W,
//     the contest runs over the first m = n - W entries as a top-(C - W), and index order
//     is position order; a row whose positions do not increase strictly gets status 1.
//
// A row is cut into C chunks of CS = 256 * VPT elements; workgroup (c, row) owns chunk c
// in all three kernels, so a chunk is re-read from the L2 of the XCD that read it first.
// Elements are monotone 32-bit keys (larger float -> larger key, -0.0 == +0.0, NaN above
// +inf, dead slots -inf); the k-th largest key T is found digit by digit, 13 + 11 + 8 bits:
//   1. hist:     every chunk adds its 13-bit histogram into the row's global histogram
//                (skipped when the score pass has built it: ma_topk_select_hist_ready).
//   2. boundary: every workgroup reads the row's histogram and finds the bin d0 holding
//                the k-th key and how many keys of that bin are still to take (krem);
//                it counts its chunk's keys above bin d0 and writes the keys of bin d0 to
//                the chunk's candidate slots, in index order.
//   3. emit:     every workgroup reads the row's candidates (typically about 1% of the
//                row; for rows of at most SPEC_C chunks a fixed number of slots of every
//                chunk, loaded before the counts are known, when none overflows) and
//                finds the remaining 19 bits of T (two LDS histograms), the
//                number `need` of keys equal to T that are selected (the first `need` in
//                index order) and, from all chunks' counts, its own output base and how
//                many of its T-equal keys it takes; then it writes its selected indices,
//                ascending, to idx[base ..]: a block scan in index order, staged in LDS,
//                then contiguous stores.  It also clears its share of the row's histogram.
// Kernel boundaries are the only synchronisation: no workgroup waits for, or hands a
// result to, another inside a kernel (on this chip a device-scope fence or a returning
// atomic costs microseconds).  The small row-wide decisions (d0; T, need and the chunk
// bases) are recomputed by every workgroup of the row from the same data.
// Row r's histogram is block r of a state buffer that must be zero before its first use;
// each call clears its rows' blocks again, so a state buffer of R blocks serves every
// later call of up to R rows.  Chunk records and candidates go to a scratch workspace.
#include "ma_common.h"

namespace {

constexpr int TB = 256;                 // threads per workgroup
constexpr int TW = TB / 64;             // waves per workgroup
constexpr int D0_BITS = 13, D1_BITS = 11, D2_BITS = 8;
constexpr int S0 = 32 - D0_BITS;        // shift of the level-0 digit (19)
constexpr int S1 = S0 - D1_BITS;        // shift of the level-1 digit (8)
constexpr int H0 = 1 << D0_BITS;        // 8192 level-0 bins
constexpr int H1 = 1 << D1_BITS;        // 2048 level-1 bins
constexpr int H2 = 1 << D2_BITS;        // 256 level-2 bins
constexpr int MAX_CHUNKS = 1024;        // per row (4 chunks per thread in the chunk scans)
constexpr int NCR = 8;                  // candidates per thread kept in registers by the emit kernel
constexpr int SPEC_C = 64;              // read-set rows of up to this many chunks read their candidate
constexpr int SPEC_N = 8 * TB;          // slots speculatively (SPEC_N / C per chunk, see the emit kernel)
constexpr int NCL = 8192;               // candidates per row kept in LDS beyond that (a boundary bin
                                        // of a value-aware keep contest at 64k entries holds a few
                                        // thousand); more are re-read from the workspace
static_assert(D0_BITS + D1_BITS + D2_BITS == 32, "digits cover the key");
static_assert(D0_BITS == MA_TOPK_D0_BITS && H0 == MA_TOPK_H0 && S0 == MA_TOPK_S0,
              "the score pass builds level 0 with these digits");

// one row's block of the state buffer
struct alignas(256) RowState {
    uint32_t hist[H0];   // zero between calls
};
struct ChunkInfo {
    uint32_t gt;      // keys of the chunk above bin d0; bit 31: positions out of order (keep)
    uint32_t ncand;   // keys of the chunk in bin d0 (its candidates)
    uint32_t d0;      // the row's boundary bin and
    uint32_t krem;    // how many of its keys are selected
};

struct TopkArgs {
    const float *rank;
    int64_t rank_stride;
    const uint8_t *mask;
    int64_t mask_stride;
    int n, k, C, vec;
    int64_t *idx;
    int64_t idx_stride;
    float *values;
    RowState *state;     // [rows]
    ChunkInfo *chunk;    // [rows][C]
    uint32_t *cand;      // [rows][C][CS]: the candidates' keys per chunk (in index order)
    // keep set: positions (int32 or int64) and the sink / pin rules; keys of entries j >= m
    // (the W newest) are 0, so they never contest and are appended after the selection
    const void *pos;
    int pos_i64, m, w, has_pin;
    int64_t pos_stride, sink, pin_lo, pin_hi;
    const int64_t *pin_lo_rows;
    int32_t *status;
};

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Element e of this thread in chunk c: run q = e / 4 of 4 consecutive elements at
// c*CS + 4*(q*TB + t), so a wave's 16-byte loads are contiguous.  Index order inside the
// chunk is run-major.
template <int VPT>
__device__ __forceinline__ int chunk_index(int c, int e) {
    return c * (TB * VPT) + 4 * ((e >> 2) * TB + (int)threadIdx.x) + (e & 3);
}

__device__ __forceinline__ int64_t pos_at(const TopkArgs &a, int64_t off) {
    return a.pos_i64 ? ((const int64_t *)a.pos)[off] : (int64_t)((const int32_t *)a.pos)[off];
}

// keys of this thread's elements; 0 (below every real key) past the end of the row.  KEEP:
// the keep-set keys (sinks and pinned positions +inf, entries j >= m 0) and, in *bad, the
// order check of the thread's elements against their predecessors.
template <int VPT, bool KEEP>
__device__ __forceinline__ void chunk_keys(const TopkArgs &a, int row, int c, uint32_t (&key)[VPT],
                                           bool *bad = nullptr) {
    const float *rr = a.rank + (int64_t)row * a.rank_stride;
    const uint8_t *mr = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    int64_t plo = 0, prow = 0;
    if constexpr (KEEP) {
        plo = a.pin_lo_rows ? a.pin_lo_rows[row] : a.pin_lo;
        prow = (int64_t)row * a.pos_stride;
    }
#pragma unroll
    for (int q = 0; q < VPT / 4; ++q) {
        const int j0 = chunk_index<VPT>(c, 4 * q);
        float v[4];
        if (a.vec && j0 + 4 <= a.n) {
            const f32x4_t x = *(const f32x4_t *)(rr + j0);
            v[0] = x[0];
            v[1] = x[1];
            v[2] = x[2];
            v[3] = x[3];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = j0 + i < a.n ? rr[j0 + i] : 0.f;
        }
        if constexpr (KEEP) {
            int64_t p[5];   // the run's positions and its predecessor's (clamped indices)
            p[0] = pos_at(a, prow + min(max(j0 - 1, 0), a.n - 1));
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i + 1] = pos_at(a, prow + min(j0 + i, a.n - 1));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = j0 + i;
                if (bad) *bad |= (j > 0 && j < a.n) && !(p[i] < p[i + 1]);
                float x = v[i];
                if (p[i + 1] < a.sink) x = INFINITY;
                if (a.has_pin && p[i + 1] >= plo && p[i + 1] < a.pin_hi) x = INFINITY;
                key[4 * q + i] = j < a.m ? ma_order_key(x) : 0u;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = j0 + i;
                const bool live = !mr || (j < a.n && mr[j] != 0);
                key[4 * q + i] = j < a.n ? ma_order_key(live ? v[i] : -INFINITY) : 0u;
            }
        }
    }
}

// float of a key (inverse of ma_order_key; -0.0 and NaN payloads come back canonical)
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Exclusive prefix, in index order (run-major), of per-(run, thread) counts c[q]; returns
// the block total.  wsum: LDS [NR * TW].
template <int NR>
__device__ __forceinline__ uint32_t block_prefix_runs(uint32_t (&c)[NR], uint32_t *wsum) {
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    uint32_t incl[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) incl[q] = ma_wave_prefix_u32(c[q]);
    if (lane == 63) {
#pragma unroll
        for (int q = 0; q < NR; ++q) wsum[q * TW + wave] = incl[q];
    }
    __syncthreads();
    uint32_t base = 0;
#pragma unroll
    for (int q = 0; q < NR; ++q) {
        uint32_t before = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < TW; ++w) {
            const uint32_t x = wsum[q * TW + w];
            before += w < wave ? x : 0u;
            tot += x;
        }
        c[q] = base + before + incl[q] - c[q];
        base += tot;
    }
    __syncthreads();   // wsum is reused
    return base;
}

// Thread t holds the counts of bins [t*PB, (t+1)*PB).  Finds the bin d with
// count(bins above d) < kk <= count(bins >= d) and stores d and count(bins above d) in
// found[0], found[1] (LDS), visible to the whole block on return.  Requires
// 1 <= kk <= total.
template <int PB>
__device__ __forceinline__ void find_digit(const uint32_t (&h)[PB], uint32_t kk, uint32_t *wsum, uint32_t *found) {
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    uint32_t s = 0;
#pragma unroll
    for (int b = 0; b < PB; ++b) s += h[b];
    const uint32_t incl = ma_wave_prefix_u32(s);
    if (lane == 63) wsum[wave] = incl;
    if (tid == 0) {   // defined result should kk exceed the total
        found[0] = 0u;
        found[1] = 0u;
    }
    __syncthreads();
    uint32_t before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < TW; ++w) {
        const uint32_t x = wsum[w];
        before += w < wave ? x : 0u;
        tot += x;
    }
    uint32_t above = tot - (before + incl);   // keys in the bins of threads > t
#pragma unroll
    for (int b = PB - 1; b >= 0; --b) {
        if (above < kk && above + h[b] >= kk) {
            found[0] = (uint32_t)(tid * PB + b);
            found[1] = above;
        }
        above += h[b];
    }
    __syncthreads();
}

// Level-0 histogram of the chunk added into the row's histogram.
template <int VPT, bool KEEP>
__global__ void __launch_bounds__(TB) topk_hist_kernel(TopkArgs a) {
    __shared__ uint32_t h[H0];
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    for (int i = tid; i < H0 / 4; i += TB) ((uint4 *)h)[i] = make_uint4(0u, 0u, 0u, 0u);
    uint32_t key[VPT];
    chunk_keys<VPT, KEEP>(a, row, c, key);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < VPT; ++e)
        if (key[e]) atomicAdd(&h[key[e] >> S0], 1u);
    __syncthreads();
    uint32_t *gh = a.state[row].hist;
    for (int i = tid; i < H0; i += TB) {
        const uint32_t x = h[i];
        if (x) atomicAdd(&gh[i], x);
    }
}

// d0 / krem from the row's histogram; the chunk's count above bin d0 and its candidates.
template <int VPT, bool KEEP>
__global__ void __launch_bounds__(TB) topk_boundary_kernel(TopkArgs a) {
    constexpr int CS = TB * VPT, PB = H0 / TB;
    __shared__ uint32_t wsum[TW], found[2];
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    // thread t: bins [32t, 32t + 32), loaded together with the chunk's keys
    uint32_t cnt[PB];
    const uint4 *g4 = (const uint4 *)(a.state[row].hist + tid * PB);
#pragma unroll
    for (int i = 0; i < PB / 4; ++i) {
        const uint4 x = g4[i];
        cnt[4 * i] = x.x;
        cnt[4 * i + 1] = x.y;
        cnt[4 * i + 2] = x.z;
        cnt[4 * i + 3] = x.w;
    }
    uint32_t key[VPT];
    bool bad = false;
    chunk_keys<VPT, KEEP>(a, row, c, key, &bad);
    find_digit<PB>(cnt, (uint32_t)a.k, wsum, found);
    const uint32_t d0 = found[0], krem = (uint32_t)a.k - found[1];
    uint32_t packed[1] = {0u};   // low 16 bits: keys above bin d0; high: keys in bin d0
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        const uint32_t d = key[e] >> S0;
        packed[0] += key[e] && d > d0 ? 1u : 0u;
        packed[0] += key[e] && d == d0 ? 0x10000u : 0u;
    }
    const uint32_t total = block_prefix_runs<1>(packed, wsum);
    uint32_t *L = a.cand + ((int64_t)row * a.C + c) * CS;
    uint32_t pos = packed[0] >> 16;
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
        if (key[e] && (key[e] >> S0) == d0) {
            L[pos] = key[e];
            ++pos;
        }
    }
    const bool chunk_bad = KEEP && __syncthreads_or(bad);
    if (tid == 0) {
        ChunkInfo ci;
        ci.gt = (total & 0xffffu) | (chunk_bad ? 0x80000000u : 0u);
        ci.ncand = total >> 16;
        ci.d0 = d0;
        ci.krem = krem;
        a.chunk[(int64_t)row * a.C + c] = ci;
    }
}

// One wave: the bin d of the LDS histogram h[0, 64 PB) with count(bins above d) < kk <=
// count(bins >= d), and that count of bins above d (d = above = 0 should kk exceed the
// total).  Lane l sums bins [l PB, (l + 1) PB); a lane scan finds the lane holding d, and a
// second one over that lane's PB bins, one per lane, the bin.  All 64 lanes must be active.
template <int PB>
__device__ __forceinline__ void wave_find_digit(const uint32_t *h, uint32_t kk, uint32_t &d, uint32_t &above) {
    static_assert(PB % 4 == 0 && PB <= 64, "bins per lane");
    const int ln = lane_id();
    uint32_t s = 0u;
#pragma unroll
    for (int q = 0; q < PB / 4; ++q) {
        const uint4 x = ((const uint4 *)h)[ln * (PB / 4) + q];
        s += (x.x + x.y) + (x.z + x.w);
    }
    uint32_t incl = ma_wave_prefix_u32(s);
    const uint32_t ab = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) - incl;   // bins of later lanes
    d = 0u;
    above = 0u;
    const uint64_t m = __ballot(ab < kk && ab + s >= kk);
    if (!m) return;
    const int L = __builtin_ctzll(m);
    const uint32_t abl = (uint32_t)__builtin_amdgcn_readlane((int)ab, L);
    const uint32_t x = ln < PB ? h[L * PB + ln] : 0u;
    incl = ma_wave_prefix_u32(x);
    const uint32_t ab2 = abl + (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) - incl;
    const uint64_t m2 = __ballot(ln < PB && ab2 < kk && ab2 + x >= kk);
    if (!m2) return;
    const int j = __builtin_ctzll(m2);
    d = (uint32_t)(L * PB + j);
    above = (uint32_t)__builtin_amdgcn_readlane((int)ab2, j);
}

struct EmitSmem {
    alignas(16) uint32_t hist[H1];
    uint32_t pre[MAX_CHUNKS + 1];   // candidates of the chunks before chunk c
    uint32_t acnt[MAX_CHUNKS];      // per chunk: candidates above T
    uint32_t ecnt[MAX_CHUNKS];      // per chunk: candidates equal to T
    uint32_t wsum[4 * TW], found[2];   // (block_prefix_runs<NR> uses NR * TW)
    uint32_t base, take, eq;        // this workgroup's chunk
    uint32_t thr;                   // T (slot-speculative path)
    alignas(16) uint32_t hist2[H2]; // level 2 (slot-speculative path; read as uint4)
    uint32_t ncn[SPEC_C], gtc[SPEC_C];   // per chunk: candidates, keys above bin d0 (same)
    alignas(16) uint32_t ckey[NCL]; // the row's candidates (key, chunk) when more than
    uint16_t cchk[NCL];             // fit in registers
};
static_assert(MAX_CHUNKS <= 65536, "chunk ids are 16-bit");

// T, need and the chunk's base from the row's candidates; the chunk's selected indices,
// ascending, to idx[base ..]; values optional.
template <int VPT, bool KEEP>
__global__ void __launch_bounds__(TB) topk_emit_kernel(TopkArgs a) {
    constexpr int NR = VPT / 4, CS = TB * VPT;
    __shared__ EmitSmem S;
    __shared__ uint32_t sj[CS], sk[CS];
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, C = a.C;
    const ChunkInfo *info = a.chunk + (int64_t)row * C;
    // chunk records of chunks [4t, 4t + 4) and the chunk's keys, loads in flight together
    uint32_t gt[4], nc[4];
    bool any_bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ch = 4 * tid + i;
        gt[i] = 0u;
        nc[i] = 0u;
        if (ch < C) {
            const ChunkInfo x = info[ch];
            any_bad |= (x.gt >> 31) != 0u;
            gt[i] = x.gt & 0x7fffffffu;
            nc[i] = x.ncand;
        }
    }
    const uint32_t d0 = info[0].d0, krem = info[0].krem;
    // read set, at most SPEC_C chunks: P = SPEC_N / C (rounded down to a power of two, at
    // most CS) slots
    // of every chunk's candidate list, slot e & (P - 1) of chunk e / P for e = tid + i TB,
    // loaded in this round trip before the counts are known (slots past a chunk's count are
    // ignored below); used when no chunk has more than P candidates
    const uint32_t *L = a.cand + (int64_t)row * C * CS;
    const bool spec_try = !KEEP && C <= SPEC_C;
    constexpr int CS_LOG = VPT == 4 ? 10 : 12;   // log2(CS): a chunk has CS slots
    static_assert((1 << CS_LOG) == CS, "chunk size");
    const int pl = spec_try ? min(31 - __builtin_clz((uint32_t)(SPEC_N / C)), CS_LOG) : 0, P = 1 << pl;
    uint32_t spk[SPEC_N / TB];
#pragma unroll
    for (int i = 0; i < SPEC_N / TB; ++i) {
        const int e = tid + i * TB;
        spk[i] = spec_try && (e >> pl) < C ? L[(int64_t)(e >> pl) * CS + (e & (P - 1))] : 0u;
    }
    uint32_t key[VPT];
    chunk_keys<VPT, KEEP>(a, row, c, key);
    if constexpr (KEEP) {
        // workgroup 0 of the row: the order flag of the row and the W newest entries after
        // the selected ones
        const bool row_bad = __syncthreads_or(any_bad);
        if (c == 0) {
            if (tid == 0 && a.status) a.status[row] = row_bad ? 1 : 0;
            int64_t *wout = a.idx + (int64_t)row * a.idx_stride + a.k;
            for (int i = tid; i < a.w; i += TB) wout[i] = (int64_t)(a.m + i);
        }
    }
    bool spec = false;
    if (spec_try) {
        for (int i = tid; i < H1 / 4; i += TB) ((uint4 *)S.hist)[i] = make_uint4(0u, 0u, 0u, 0u);
        for (int i = tid; i < H2; i += TB) S.hist2[i] = 0u;
        if (tid < SPEC_C) {
            S.acnt[tid] = 0u;
            S.ecnt[tid] = 0u;
        }
        bool over = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ch = 4 * tid + i;
            if (ch < C) {
                S.ncn[ch] = nc[i];
                S.gtc[ch] = gt[i];
                over |= nc[i] > (uint32_t)P;
            }
        }
        spec = !__syncthreads_or(over);
    }
    uint32_t thr = 0u;
    if (spec) {
        // every thread counts its valid slots (spk, 0 elsewhere: candidate keys are real
        // keys, never 0) into the LDS histograms, level by level; one wave finds each digit
        // by lane scans (its LDS operations complete in order) and, at the end, with lane =
        // chunk, the T-equal keys taken in chunk order and the output bases
#pragma unroll
        for (int i = 0; i < SPEC_N / TB; ++i) {
            const int e = tid + i * TB, ch = e >> pl;
            spk[i] = ch < C && (uint32_t)(e & (P - 1)) < S.ncn[ch] ? spk[i] : 0u;
            if (spk[i]) atomicAdd(&S.hist[(spk[i] >> S1) & (H1 - 1)], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t d1, a1;
            wave_find_digit<H1 / 64>(S.hist, krem, d1, a1);
            if (tid == 0) {
                S.found[0] = d1;
                S.found[1] = krem - a1;
            }
        }
        __syncthreads();
        const uint32_t d1 = S.found[0], kr = S.found[1];
#pragma unroll
        for (int i = 0; i < SPEC_N / TB; ++i)
            if (spk[i] && ((spk[i] >> S1) & (H1 - 1)) == d1) atomicAdd(&S.hist2[spk[i] & (H2 - 1)], 1u);
        __syncthreads();
        if (tid < 64) {
            uint32_t d2, a2;
            wave_find_digit<H2 / 64>(S.hist2, kr, d2, a2);
            if (tid == 0) {
                S.thr = (d0 << S0) | (d1 << S1) | d2;
                S.take = kr - a2;   // (here: how many keys equal to T the row takes)
            }
        }
        __syncthreads();
        const uint32_t t = S.thr, need = S.take;
#pragma unroll
        for (int i = 0; i < SPEC_N / TB; ++i) {
            const int ch = (tid + i * TB) >> pl;
            if (spk[i] && spk[i] > t) atomicAdd(&S.acnt[ch], 1u);
            else if (spk[i] && spk[i] == t) atomicAdd(&S.ecnt[ch], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            const int ln = tid;
            const uint32_t ac = ln < C ? S.acnt[ln] : 0u, ec = ln < C ? S.ecnt[ln] : 0u;
            const uint32_t ebefore = ma_wave_prefix_u32(ec) - ec;
            const uint32_t take = need > ebefore ? min(need - ebefore, ec) : 0u;
            const uint32_t sel = ln < C ? S.gtc[ln] + ac + take : 0u;
            const uint32_t sbefore = ma_wave_prefix_u32(sel) - sel;
            if (ln == c) {
                S.base = sbefore;
                S.take = take;
                S.eq = ec;
            }
        }
    } else {
    uint32_t run[1] = {nc[0] + nc[1] + nc[2] + nc[3]};
    const uint32_t NC = block_prefix_runs<1>(run, S.wsum);
    {
        uint32_t p = run[0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ch = 4 * tid + i;
            if (ch < C) S.pre[ch] = p;
            p += nc[i];
        }
    }
    if (tid == 0) S.pre[C] = NC;
    for (int i = tid; i < H1; i += TB) S.hist[i] = 0u;
    for (int i = tid; i < C; i += TB) {
        S.acnt[i] = 0u;
        S.ecnt[i] = 0u;
    }
    __syncthreads();
    // candidate g of the row: chunk ch with pre[ch] <= g < pre[ch + 1], slot g - pre[ch]
    auto locate = [&](uint32_t g) {
        int lo = 0, hi = C - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (S.pre[mid] <= g) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    const bool inreg = NC <= (uint32_t)(NCR * TB);
    const bool inlds = !inreg && NC <= (uint32_t)NCL;
    uint32_t ck[NCR], cc[NCR];
    if (inlds) {
        // batches of 8 candidates per thread, their loads in flight together
        for (uint32_t g0 = 0; g0 < NC; g0 += 8 * TB) {
            uint32_t kx[8];
            int chs[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t g = g0 + tid + i * TB;
                chs[i] = g < NC ? locate(g) : 0;
                kx[i] = g < NC ? L[(int64_t)chs[i] * CS + (g - S.pre[chs[i]])] : 0u;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t g = g0 + tid + i * TB;
                if (g < NC) {
                    S.ckey[g] = kx[i];
                    S.cchk[g] = (uint16_t)chs[i];
                }
            }
        }
        __syncthreads();
    }
    if (inreg) {
#pragma unroll
        for (int i = 0; i < NCR; ++i) {
            const uint32_t g = tid + i * TB;
            ck[i] = 0u;   // no candidate (candidate keys are real keys, never 0)
            cc[i] = 0u;
            if (g < NC) {
                const int ch = locate(g);
                ck[i] = L[(int64_t)ch * CS + (g - S.pre[ch])];
                cc[i] = (uint32_t)ch;
            }
        }
    }
    auto each = [&](auto f) {
        if (inreg) {
#pragma unroll
            for (int i = 0; i < NCR; ++i)
                if (ck[i]) f(ck[i], cc[i]);
        } else if (inlds) {
            for (uint32_t g = tid; g < NC; g += TB) f(S.ckey[g], (uint32_t)S.cchk[g]);
        } else {
            for (uint32_t g = tid; g < NC; g += TB) {
                const int ch = locate(g);
                f(L[(int64_t)ch * CS + (g - S.pre[ch])], (uint32_t)ch);
            }
        }
    };
    // level 1: bits [S1, S0) of the candidates
    each([&](uint32_t x, uint32_t) { atomicAdd(&S.hist[(x >> S1) & (H1 - 1)], 1u); });
    __syncthreads();
    uint32_t d1, kr = krem;
    {
        constexpr int PB = H1 / TB;
        uint32_t cnt[PB];
#pragma unroll
        for (int b = 0; b < PB; ++b) cnt[b] = S.hist[tid * PB + b];
        find_digit<PB>(cnt, kr, S.wsum, S.found);
        d1 = S.found[0];
        kr -= S.found[1];
    }
    // level 2: the low bits of the candidates whose level-1 digit is d1
    for (int i = tid; i < H2; i += TB) S.hist[i] = 0u;
    __syncthreads();
    each([&](uint32_t x, uint32_t) {
        if (((x >> S1) & (H1 - 1)) == d1) atomicAdd(&S.hist[x & (H2 - 1)], 1u);
    });
    __syncthreads();
    uint32_t need;
    {
        uint32_t cnt[1] = {S.hist[tid]};
        find_digit<1>(cnt, kr, S.wsum, S.found);
        thr = (d0 << S0) | (d1 << S1) | S.found[0];
        need = kr - S.found[1];
    }
    // per chunk: candidates above / equal to T
    each([&](uint32_t x, uint32_t ch) {
        if (x > thr) atomicAdd(&S.acnt[ch], 1u);
        else if (x == thr) atomicAdd(&S.ecnt[ch], 1u);
    });
    __syncthreads();
    // chunks [4t, 4t + 4): keys equal to T are taken in chunk order
    {
        uint32_t e[4], sel[4], ex[1] = {0u}, sx[1] = {0u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ch = 4 * tid + i;
            e[i] = ch < C ? S.ecnt[ch] : 0u;
            ex[0] += e[i];
        }
        block_prefix_runs<1>(ex, S.wsum);
        uint32_t ebefore = ex[0];
        uint32_t take[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ch = 4 * tid + i;
            take[i] = need > ebefore ? min(need - ebefore, e[i]) : 0u;
            ebefore += e[i];
            sel[i] = ch < C ? gt[i] + S.acnt[ch] + take[i] : 0u;
            sx[0] += sel[i];
        }
        block_prefix_runs<1>(sx, S.wsum);
        uint32_t base = sx[0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * tid + i == c) {
                S.base = base;
                S.take = take[i];
                S.eq = e[i];
            }
            base += sel[i];
        }
    }
    }
    // this workgroup's share of the row's histogram, cleared for the next call (the
    // boundary kernel, its only reader, has finished)
    for (int b = c * TB + tid; b < H0; b += C * TB) a.state[row].hist[b] = 0u;
    __syncthreads();
    if (spec) thr = S.thr;
    const uint32_t cbase = S.base, ctake = S.take, ceq = S.eq;
    uint32_t selbits = 0;
    if (ctake == 0u || ctake >= ceq) {
        // none or all of the chunk's keys equal to T (padding keys 0 lie below any T)
        const bool all_eq = ctake != 0u;
#pragma unroll
        for (int e = 0; e < VPT; ++e) selbits |= (uint32_t)(key[e] > thr || (all_eq && key[e] == thr)) << e;
    } else {
        // the first `take` keys equal to T in index order
        uint32_t eb[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) {
            eb[q] = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) eb[q] += key[4 * q + i] == thr ? 1u : 0u;
        }
        block_prefix_runs<NR>(eb, S.wsum);
#pragma unroll
        for (int q = 0; q < NR; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = 4 * q + i;
                const bool is_eq = key[e] == thr;
                selbits |= (uint32_t)(key[e] > thr || (is_eq && eb[q] < ctake)) << e;
                eb[q] += is_eq ? 1u : 0u;
            }
        }
    }
    uint32_t slot[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) slot[q] = __popc((selbits >> (4 * q)) & 15u);
    const uint32_t nsel = block_prefix_runs<NR>(slot, S.wsum);
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * q + i;
            if ((selbits >> e) & 1u) {
                sj[slot[q]] = (uint32_t)chunk_index<VPT>(c, e);
                sk[slot[q]] = key[e];
                ++slot[q];
            }
        }
    }
    __syncthreads();
    int64_t *out = a.idx + (int64_t)row * a.idx_stride + cbase;
    float *vout = a.values ? a.values + (int64_t)row * a.k + cbase : nullptr;
    const float *rr = a.rank + (int64_t)row * a.rank_stride;
    const uint8_t *mr = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    // (cbase + nsel <= k by construction; the bound keeps inconsistent inputs from
    // writing past the row)
    const uint32_t nout = cbase < (uint32_t)a.k ? min(nsel, (uint32_t)a.k - cbase) : 0u;
    for (uint32_t i = tid; i < nout; i += TB) {
        const uint32_t j = sj[i];
        out[i] = (int64_t)j;
        if (vout) {
            // the selected value from its key; a zero or NaN key re-reads the element so
            // that -0.0 and NaN payloads come back as stored
            float x = key_value(sk[i]);
            if (x == 0.f || x != x) x = (mr && !mr[j]) ? -INFINITY : rr[j];
            vout[i] = x;
        }
    }
}

int topk_vpt(int n) { return n <= TB * 4 * MAX_CHUNKS ? 4 : (n <= TB * 16 * MAX_CHUNKS ? 16 : 0); }

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

int64_t chunk_bytes(int rows, int n) {
    const int vpt = topk_vpt(n);
    return align256((int64_t)rows * ((n + TB * vpt - 1) / (TB * vpt)) * (int64_t)sizeof(ChunkInfo));
}

}  // namespace

extern "C" int64_t ma_topk_state_bytes(int rows) {
    return rows > 0 ? (int64_t)rows * (int64_t)sizeof(RowState) : 0;
}

extern "C" int64_t ma_topk_workspace_bytes(int rows, int n) {
    if (rows <= 0 || n <= 0 || !topk_vpt(n)) return 0;
    const int vpt = topk_vpt(n);
    const int64_t C = (n + TB * vpt - 1) / (TB * vpt);
    return chunk_bytes(rows, n) + align256((int64_t)rows * C * TB * vpt * (int64_t)sizeof(uint32_t));
}

namespace {

// shared argument checks and fill of both entry points (rank = the score row, k = the
// number to select); MA_OK with rows == 0 or k == 0 and no keep window means nothing to do
int topk_prepare(TopkArgs &a, int &vpt, const char *who, const float *rank, int64_t rank_stride, int rows, int n,
                 int k, int64_t *idx, int64_t idx_stride, void *state, int64_t state_bytes, void *workspace,
                 int64_t workspace_bytes) {
    vpt = topk_vpt(n);
    if (!vpt) {
        ma_set_error("%s: n=%d exceeds the built maximum %d", who, n, TB * 16 * MAX_CHUNKS);
        return MA_EUNSUPPORTED;
    }
    const int64_t need_state = ma_topk_state_bytes(rows), need_ws = ma_topk_workspace_bytes(rows, n);
    if (!state || state_bytes < need_state || ((uintptr_t)state & 255) || !workspace ||
        workspace_bytes < need_ws || ((uintptr_t)workspace & 255)) {
        ma_set_error("%s: state of %lld and workspace of %lld bytes (256-byte aligned) needed, got %lld and %lld",
                     who, (long long)need_state, (long long)need_ws, (long long)state_bytes,
                     (long long)workspace_bytes);
        return MA_EINVAL;
    }
    a = TopkArgs{};
    a.rank = rank;
    a.rank_stride = rank_stride;
    a.n = n;
    a.k = k;
    a.C = (n + TB * vpt - 1) / (TB * vpt);
    a.vec = ((uintptr_t)rank & 15) == 0 && rank_stride % 4 == 0;
    a.idx = idx;
    a.idx_stride = idx_stride;
    a.state = (RowState *)state;
    a.chunk = (ChunkInfo *)workspace;
    a.cand = (uint32_t *)((char *)workspace + chunk_bytes(rows, n));
    return MA_OK;
}

// hist_ready: the rows' level-0 histograms are already in the state (built by the score
// pass), so the histogram launch is skipped
template <bool KEEP>
int topk_launch(const TopkArgs &a, int rows, int vpt, hipStream_t st, const char *who, bool hist_ready = false) {
    const dim3 grid(a.C, rows);
    if (vpt == 4) {
        if (!hist_ready) hipLaunchKernelGGL((topk_hist_kernel<4, KEEP>), grid, dim3(TB), 0, st, a);
        hipLaunchKernelGGL((topk_boundary_kernel<4, KEEP>), grid, dim3(TB), 0, st, a);
        hipLaunchKernelGGL((topk_emit_kernel<4, KEEP>), grid, dim3(TB), 0, st, a);
    } else {
        if (!hist_ready) hipLaunchKernelGGL((topk_hist_kernel<16, KEEP>), grid, dim3(TB), 0, st, a);
        hipLaunchKernelGGL((topk_boundary_kernel<16, KEEP>), grid, dim3(TB), 0, st, a);
        hipLaunchKernelGGL((topk_emit_kernel<16, KEEP>), grid, dim3(TB), 0, st, a);
    }
    return ma_check_launch(who);
}

int topk_select(const char *who, bool hist_ready, const float *rank, int64_t rank_stride, const uint8_t *mask,
                int64_t mask_stride, int rows, int n, int k, int64_t *idx, int64_t idx_stride, float *values,
                void *state, int64_t state_bytes, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!rank || !idx || rows < 0 || n < 0 || k < 0 || k > n || idx_stride < k || rank_stride < n ||
        (mask && mask_stride < n) || rows > 65535) {
        ma_set_error("%s: bad arguments (rows=%d n=%d k=%d)", who, rows, n, k);
        return MA_EINVAL;
    }
    if (rows == 0 || k == 0) return MA_OK;
    TopkArgs a;
    int vpt = 0;
    const int rc = topk_prepare(a, vpt, who, rank, rank_stride, rows, n, k, idx, idx_stride, state, state_bytes,
                                workspace, workspace_bytes);
    if (rc) return rc;
    a.mask = mask;
    a.mask_stride = mask_stride;
    a.values = values;
    return topk_launch<false>(a, rows, vpt, (hipStream_t)stream, who, hist_ready);
}

}  // namespace

extern "C" int ma_topk_select(const float *rank, int64_t rank_stride, const uint8_t *mask, int64_t mask_stride,
                              int rows, int n, int k, int64_t *idx, int64_t idx_stride, float *values,
                              void *state, int64_t state_bytes, void *workspace, int64_t workspace_bytes,
                              void *stream) {
    return topk_select("ma_topk_select", false, rank, rank_stride, mask, mask_stride, rows, n, k, idx, idx_stride,
                       values, state, state_bytes, workspace, workspace_bytes, stream);
}

extern "C" int ma_topk_select_hist_ready(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                         int64_t mask_stride, int rows, int n, int k, int64_t *idx,
                                         int64_t idx_stride, float *values, void *state, int64_t state_bytes,
                                         void *workspace, int64_t workspace_bytes, void *stream) {
    return topk_select("ma_topk_select_hist_ready", true, rank, rank_stride, mask, mask_stride, rows, n, k, idx,
                       idx_stride, values, state, state_bytes, workspace, workspace_bytes, stream);
}

// The level-0 histograms alone, into a state (for the score passes that do not build them
// in-kernel); part of the library's internals, not of the C ABI header.
extern "C" int ma_topk_level0_into_state(const float *rank, int64_t rank_stride, const uint8_t *mask,
                                         int64_t mask_stride, int rows, int n, void *state, void *stream) {
    const int vpt = topk_vpt(n);
    if (!vpt || rows <= 0 || !state) return MA_EINVAL;
    TopkArgs a = TopkArgs{};
    a.rank = rank;
    a.rank_stride = rank_stride;
    a.mask = mask;
    a.mask_stride = mask_stride;
    a.n = n;
    a.C = (n + TB * vpt - 1) / (TB * vpt);
    a.vec = ((uintptr_t)rank & 15) == 0 && rank_stride % 4 == 0;
    a.state = (RowState *)state;
    const dim3 grid(a.C, rows);
    if (vpt == 4) hipLaunchKernelGGL((topk_hist_kernel<4, false>), grid, dim3(TB), 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL((topk_hist_kernel<16, false>), grid, dim3(TB), 0, (hipStream_t)stream, a);
    return ma_check_launch("ma_topk_level0_into_state");
}

extern "C" int ma_keep_select(const void *pos, int pos_is_i64, int64_t pos_stride, const float *score,
                              int64_t score_stride, int rows, int n, int capacity, int window, int64_t sink_tokens,
                              const int64_t *pin_lo_rows, int64_t pin_lo, int64_t pin_hi, int has_pin, int64_t *keep,
                              int64_t keep_stride, int32_t *status, void *state, int64_t state_bytes,
                              void *workspace, int64_t workspace_bytes, void *stream) {
    if (!pos || !score || !keep || rows < 0 || n < 0 || capacity < 0 || capacity > n || window < 0 ||
        keep_stride < capacity || pos_stride < n || score_stride < n || rows > 65535) {
        ma_set_error("ma_keep_select: bad arguments (rows=%d n=%d capacity=%d window=%d)", rows, n, capacity,
                     window);
        return MA_EINVAL;
    }
    if (rows == 0 || capacity == 0) return MA_OK;
    const int w = window < capacity ? window : capacity;
    TopkArgs a;
    int vpt = 0;
    const int rc = topk_prepare(a, vpt, "ma_keep_select", score, score_stride, rows, n, capacity - w, keep,
                                keep_stride, state, state_bytes, workspace, workspace_bytes);
    if (rc) return rc;
    a.pos = pos;
    a.pos_i64 = pos_is_i64 != 0;
    a.pos_stride = pos_stride;
    a.m = n - w;
    a.w = w;
    a.has_pin = has_pin != 0;
    a.sink = sink_tokens;
    a.pin_lo = pin_lo;
    a.pin_hi = pin_hi;
    a.pin_lo_rows = pin_lo_rows;
    a.status = status;
    return topk_launch<true>(a, rows, vpt, (hipStream_t)stream, "ma_keep_select");
}
