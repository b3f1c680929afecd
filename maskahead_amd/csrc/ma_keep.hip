// Keep path of an eviction step: the value-aware keep score, in-place compaction of the
// survivors and the append of a finalized block.
//
// value score (session.py:27-40): score_j = a_j * ||v_j - c||, c = sum_j w_j v_j / sum_j w_j.
//   Default (bf16) mode reproduces the reference's bf16 tensor arithmetic: w = bf16(a);
//   c = bf16(bf16(sum w v) / max(bf16(sum w), bf16(1e-12))); every v - c rounded to bf16;
//   the norm rounded to bf16; the product with a in f32.  The sums are accumulated in f64
//   (exact for these bf16 products up to the final rounding), and every rounding to bf16
//   goes through f32 first, which is how a float64 value becomes bfloat16 in torch.
//   fp32 mode (the reference's BITSIEVE_VSCORE_FP32 branch): the same formula in f32 on
//   the stored values, sums in f64.
//   Three launches: per-chunk partial sums (grid chunks x rows, chunks of 256 entries),
//   the centre per row, the per-entry distances and scores (grid chunks x rows).  Fixed
//   summation order: results are deterministic.
//   Slot form (ma_value_score_slots): v_j is the value of slot slots[row, j] of a cache
//   lane, dequantized and rounded to the compute dtype exactly as ma_gather_kv writes it
//   (the reference's live_values, session.py:263-268), read straight from the packed codes
//   or the 16-bit rows: the same scores as ma_gather_kv + ma_value_score, without writing
//   and re-reading the gathered [live, D] rows.
//
// compaction (cache.py:342-367 / 659-678, eviction.py:411-418): dst[i] = src[keep[i]] for
//   i < C, in place, for several token-major planes of one lane at once (bf16 K and V,
//   packed per-token codes and scales, eviction-state arrays).  Race-free for any keep:
//   launch 1 copies the sources that lie inside the destination range [0, C) (and move)
//   into a scratch buffer; launch 2 writes every destination from the scratch or, for
//   sources at index >= C, which no launch writes, directly from the cache.
//
// append (cache.py:385-566, bf16 layout): dst[b, h, at + t, :] = src[b, h, t, :].
#include <algorithm>

#include "ma_common.h"

namespace {

constexpr int VS_TOK = 16;   // tokens per step of a 256-thread value-score workgroup
constexpr int VS_NT = 256;
constexpr int VS_CHUNK = 256;   // tokens per workgroup: 16 steps, loaded VS_BATCH steps at a time
constexpr int VS_BATCH = 4;

// f64 -> bf16 the way torch converts a float64 tensor: to f32 (nearest even), then to bf16
// (nearest even).  The second rounding is done on the f32 bits with integer arithmetic so
// the two conversions cannot be merged into one direct f64 -> bf16 rounding, which differs
// whenever the f32 value lands exactly on a bf16 midpoint.
__device__ __forceinline__ float bf16_via_f32(double x) {
    uint32_t u = __float_as_uint((float)x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(u | 0x00400000u);  // NaN stays NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
}

struct VsArgs {
    const float *a;       // [rows, n] (row stride sa)
    const void *v;        // [B, H, n, D] (strides b, h, n in elements), dtype vdtype
    int64_t sa, sv0, sv1, sv2;
    int H, n, D, vdtype, fp32_mode, chunk;
    // slot form: entry j of row (b, h) is slot slots[row * sslot + j] of lane (b, h) of a
    // cache whose slots [0, nq) are packed (value codes vq [B, H, nq, D/32, 16] u8, scale /
    // zero vs, vz [B, H, nq, D/32] f16) and [nq, nq + nf) 16-bit rows vf (dtype fdtype);
    // values rounded to vdtype, as the gather writes them; slots outside [0, nq + nf) are 0
    const int32_t *slots;
    int64_t sslot;
    const uint8_t *vq;
    const uint16_t *vsc, *vzp;
    const void *vf;
    int64_t svq[4], svs[3], svf[3];
    int nq, nf, fdtype;
    double *part;         // [rows, nchunks, D + 1]
    float *centre;        // [rows, D]
    float *score;         // [rows, n] (row stride ss)
    int64_t ss;
    int nchunks;
};

__device__ __forceinline__ const char *vrow(const VsArgs &a, int row, int j) {
    const int b = row / a.H, h = row % a.H;
    const int esz = a.vdtype == MA_F32 ? 4 : 2;
    return (const char *)a.v + ((int64_t)b * a.sv0 + (int64_t)h * a.sv1 + (int64_t)j * a.sv2) * esz;
}

// 8 channels [c0, c0+8) of a value row as f32
__device__ __forceinline__ void load8(const char *p, int c0, int dtype, float (&x)[8]) {
    if (dtype == MA_F32) {
        const f32x4_t *q = (const f32x4_t *)((const float *)p + c0);
        const f32x4_t u = q[0], w = q[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = u[i];
            x[4 + i] = w[i];
        }
    } else {
        const uint4 u = *(const uint4 *)((const uint16_t *)p + c0);
        const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint16_t h = (uint16_t)(wv[i >> 1] >> ((i & 1) * 16));
            x[i] = dtype == MA_BF16 ? ma_bf16_to_f32(h) : ma_f16_to_f32(h);
        }
    }
}

__device__ __forceinline__ float round_to(float x, int dtype) {
    if (dtype == MA_BF16) return ma_round_bf16(x);
    if (dtype == MA_F16) return ma_round_f16(x);
    return x;
}

// 8 channels [c0, c0+8) of entry j of a row: a dense row, or (SLOTS) the value of the
// entry's cache slot as ma_gather_kv writes it in dtype vdtype
template <bool SLOTS>
__device__ __forceinline__ void entry8(const VsArgs &a, int row, int j, int c0, float (&x)[8]) {
    if constexpr (!SLOTS) {
        load8(vrow(a, row, j), c0, a.vdtype, x);
    } else {
        const int b = row / a.H, h = row % a.H;
        const int s = a.slots[(int64_t)row * a.sslot + j];
        if (s >= 0 && s < a.nq) {
            const int cg = c0 / 32;
            const uint32_t w = *(const uint32_t *)(a.vq + b * a.svq[0] + h * a.svq[1] + (int64_t)s * a.svq[2] +
                                                   cg * a.svq[3] + (c0 % 32) / 2);
            const int64_t so = b * a.svs[0] + h * a.svs[1] + (int64_t)s * a.svs[2] + cg;
            const float sc = ma_f16_to_f32(a.vsc[so]), ze = ma_f16_to_f32(a.vzp[so]);
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = round_to(ma_dq((w >> (4 * i)) & 15u, sc, ze), a.vdtype);
        } else if (s >= a.nq && s < a.nq + a.nf) {
            const char *p = (const char *)a.vf +
                            (b * a.svf[0] + h * a.svf[1] + (int64_t)(s - a.nq) * a.svf[2]) * (a.fdtype == MA_F32 ? 4 : 2);
            load8(p, c0, a.fdtype, x);
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = round_to(x[i], a.vdtype);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = 0.f;
        }
    }
}

// grid (nchunks, rows), 256 threads = 16 token lanes x 16 channel octets (D <= 128).
template <bool SLOTS>
__global__ void __launch_bounds__(VS_NT) vs_partial_kernel(VsArgs a) {
    __shared__ double red[VS_TOK][129];
    const int chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int tl = tid / 16, oc = tid % 16;
    const int c0 = oc * 8;
    const bool cok = c0 < a.D;
    const int j0 = chunk * a.chunk, j1 = min(j0 + a.chunk, a.n);
    const float *ar = a.a + (int64_t)row * a.sa;
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    double den = 0.0;
    // VS_BATCH steps' loads in flight together (tokens past the chunk load the chunk's first
    // token and weigh 0); the f64 sums of these products are exact, so the order of the
    // steps does not change the result
    for (int jb = j0; jb < j1; jb += VS_TOK * VS_BATCH) {
        float aw[VS_BATCH], x[VS_BATCH][8];
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int j = jb + u * VS_TOK + tl;
            const bool ok = j < j1;
            const int jl = ok ? j : j0;
            aw[u] = ok ? ar[jl] : 0.f;
            if (cok) entry8<SLOTS>(a, row, jl, c0, x[u]);
        }
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const double w = a.fp32_mode ? (double)aw[u] : (double)ma_round_bf16(aw[u]);
            if (cok) {
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[i] = __builtin_fma(w, (double)x[u][i], acc[i]);
            }
            den += w;
        }
    }
    if (cok)
#pragma unroll
        for (int i = 0; i < 8; ++i) red[tl][c0 + i] = acc[i];
    if (oc == 0) red[tl][128] = den;
    __syncthreads();
    double *out = a.part + ((int64_t)row * a.nchunks + chunk) * (a.D + 1);
    for (int c = tid; c <= a.D; c += VS_NT) {
        const int cc = c == a.D ? 128 : c;
        double s = 0.0;
#pragma unroll
        for (int t = 0; t < VS_TOK; ++t) s += red[t][cc];
        out[c] = s;
    }
}

// The all-bf16 form of the two passes (rows, 16-bit cache rows and vdtype bf16; bf16
// mode): the same arithmetic as vs_partial_kernel / vs_score_kernel with every load of a
// batch of VS_BATCH steps issued as straight-line code -- the slots (or rows) first, then
// the codes, scales and 16-bit rows they name, at clamped addresses, the choices made by
// selects afterwards -- so a thread has a batch's loads in flight together instead of
// waiting for them one branch at a time.  HASQ / HASF: the cache lane has packed slots /
// 16-bit rows (slot form; the dense form reads rows).
template <bool SLOTS, bool HASQ, bool HASF>
__device__ __forceinline__ void load_batch_bf(const VsArgs &a, int row, int jb, int j0, int j1, int tl, int c0,
                                              float (&x)[VS_BATCH][8], float (&aw)[VS_BATCH]) {
    const float *ar = a.a + (int64_t)row * a.sa;
    int jl[VS_BATCH];
#pragma unroll
    for (int u = 0; u < VS_BATCH; ++u) {
        const int j = jb + u * VS_TOK + tl;
        jl[u] = j < j1 ? j : j0;
        aw[u] = ar[jl[u]];
    }
    if constexpr (!SLOTS) {
        uint4 w[VS_BATCH];
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) w[u] = *(const uint4 *)((const uint16_t *)vrow(a, row, jl[u]) + c0);
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const uint32_t wv[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) x[u][i] = ma_bf16_to_f32((uint16_t)(wv[i >> 1] >> ((i & 1) * 16)));
        }
    } else {
        const int b = row / a.H, h = row % a.H;
        int sl[VS_BATCH];
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) sl[u] = a.slots[(int64_t)row * a.sslot + jl[u]];
        const int cg = c0 / 32;
        uint32_t w[VS_BATCH];
        uint16_t scb[VS_BATCH], zeb[VS_BATCH];
        uint4 r[VS_BATCH];
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int s = sl[u];
            if constexpr (HASQ) {
                const int sq = s >= 0 && s < a.nq ? s : 0;
                w[u] = *(const uint32_t *)(a.vq + b * a.svq[0] + h * a.svq[1] + (int64_t)sq * a.svq[2] +
                                           cg * a.svq[3] + (c0 % 32) / 2);
                const int64_t so = b * a.svs[0] + h * a.svs[1] + (int64_t)sq * a.svs[2] + cg;
                scb[u] = a.vsc[so];
                zeb[u] = a.vzp[so];
            }
            if constexpr (HASF) {
                const int sf = s >= a.nq && s < a.nq + a.nf ? s - a.nq : 0;
                r[u] = *(const uint4 *)((const uint16_t *)a.vf + b * a.svf[0] + h * a.svf[1] +
                                        (int64_t)sf * a.svf[2] + c0);
            }
        }
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int s = sl[u];
            const bool q = HASQ && s >= 0 && s < a.nq, f = HASF && s >= a.nq && s < a.nq + a.nf;
            float sc = 0.f, ze = 0.f;
            uint32_t wu = 0;
            uint32_t rv[4] = {0u, 0u, 0u, 0u};
            if constexpr (HASQ) {
                sc = ma_f16_to_f32(scb[u]);
                ze = ma_f16_to_f32(zeb[u]);
                wu = w[u];
            }
            if constexpr (HASF) {
                rv[0] = r[u].x;
                rv[1] = r[u].y;
                rv[2] = r[u].z;
                rv[3] = r[u].w;
            }
            // the choice made on bf16 pairs (channels 2 i2, 2 i2 + 1 in one word, as the 16-bit
            // rows hold them): one select and one mask per two values
            const uint32_t keep = (q || f) ? 0xffffffffu : 0u;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                uint32_t pw = rv[i2];
                if constexpr (HASQ) {
                    const uint32_t pq = ma_pack_bf16x2(ma_dq((wu >> (8 * i2)) & 15u, sc, ze),
                                                       ma_dq((wu >> (8 * i2 + 4)) & 15u, sc, ze));
                    pw = q ? pq : pw;
                }
                pw &= keep;
                x[u][2 * i2] = __uint_as_float(pw << 16);
                x[u][2 * i2 + 1] = __uint_as_float(pw & 0xffff0000u);
            }
        }
    }
}

template <bool SLOTS, bool HASQ, bool HASF>
__global__ void __launch_bounds__(VS_NT) vs_partial_bf_kernel(VsArgs a) {
    __shared__ double red[VS_TOK][129];
    const int chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int tl = tid / 16, oc = tid % 16;
    const bool cok = oc * 8 < a.D;
    const int c0 = cok ? oc * 8 : 0;        // lanes past D read channel 0 and are not written
    const int j0 = chunk * a.chunk, j1 = min(j0 + a.chunk, a.n);
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    double den = 0.0;
    for (int jb = j0; jb < j1; jb += VS_TOK * VS_BATCH) {
        float aw[VS_BATCH], x[VS_BATCH][8];
        load_batch_bf<SLOTS, HASQ, HASF>(a, row, jb, j0, j1, tl, c0, x, aw);
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const bool ok = jb + u * VS_TOK + tl < j1;
            const double w = ok ? (double)ma_round_bf16(aw[u]) : 0.0;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fma(w, (double)x[u][i], acc[i]);
            den += w;
        }
    }
    if (cok)
#pragma unroll
        for (int i = 0; i < 8; ++i) red[tl][c0 + i] = acc[i];
    if (oc == 0) red[tl][128] = den;
    __syncthreads();
    double *out = a.part + ((int64_t)row * a.nchunks + chunk) * (a.D + 1);
    for (int c = tid; c <= a.D; c += VS_NT) {
        const int cc = c == a.D ? 128 : c;
        double s = 0.0;
#pragma unroll
        for (int t = 0; t < VS_TOK; ++t) s += red[t][cc];
        out[c] = s;
    }
}

template <bool SLOTS, bool HASQ, bool HASF>
__global__ void __launch_bounds__(VS_NT) vs_score_bf_kernel(VsArgs a) {
    __shared__ float cen[128];
    const int chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    for (int d = tid; d < a.D; d += VS_NT) cen[d] = a.centre[(int64_t)row * a.D + d];
    __syncthreads();
    const int tl = tid / 16, oc = tid % 16;
    const bool cok = oc * 8 < a.D;
    const int c0 = cok ? oc * 8 : 0;
    const int j0 = chunk * a.chunk, j1 = min(j0 + a.chunk, a.n);
    float *sr = a.score + (int64_t)row * a.ss;
    float cc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cc[i] = cen[c0 + i];
    for (int jb0 = j0; jb0 < j1; jb0 += VS_TOK * VS_BATCH) {
        float x[VS_BATCH][8], aw[VS_BATCH];
        load_batch_bf<SLOTS, HASQ, HASF>(a, row, jb0, j0, j1, tl, c0, x, aw);
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int j = jb0 + u * VS_TOK + tl;
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float dl = ma_round_bf16(x[u][i] - cc[i]);
                ss = __builtin_fma((double)dl, (double)dl, ss);
            }
            if (!cok) ss = 0.0;
            // sum over the 16 lanes of this entry (lanes tl*16 .. tl*16+15 of the wave pair)
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
            if (j < j1 && oc == 0) sr[j] = aw[u] * bf16_via_f32(__builtin_sqrt(ss));
        }
    }
}

// grid rows, VC_NT threads: centre[row, d] from the chunk partials.  Thread (slot s,
// column d) sums the chunks s, s + VC_SLOTS, ... (VC_UNROLL loads in flight), then the
// slots are added in slot order: a fixed order, and in the bf16 mode every sum of the
// products is exact in f64, so no order changes a result there.
constexpr int VC_SLOTS = 8, VC_NT = 1024, VC_UNROLL = 8;
__global__ void __launch_bounds__(VC_NT) vs_centre_kernel(VsArgs a) {
    __shared__ double part[VC_SLOTS][129];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int slot = tid / 128, d = tid % 128;   // column D is the denominator
    const double *p = a.part + (int64_t)row * a.nchunks * (a.D + 1);
    if (d <= a.D) {
        double acc = 0.0;
#pragma unroll VC_UNROLL
        for (int c = slot; c < a.nchunks; c += VC_SLOTS) acc += p[(int64_t)c * (a.D + 1) + d];
        part[slot][d] = acc;
    }
    // with D == 128 the denominator column has no thread of its own: column 0's threads of
    // every slot sum it as well
    if (a.D == 128 && d == 0) {
        double acc = 0.0;
#pragma unroll VC_UNROLL
        for (int c = slot; c < a.nchunks; c += VC_SLOTS) acc += p[(int64_t)c * (a.D + 1) + 128];
        part[slot][128] = acc;
    }
    __syncthreads();
    if (tid >= a.D) return;
    double num = 0.0, den = 0.0;
#pragma unroll
    for (int s2 = 0; s2 < VC_SLOTS; ++s2) {
        num += part[s2][tid];
        den += part[s2][a.D];
    }
    float cen;
    if (a.fp32_mode) {
        const double dd = den > 1e-12 ? den : 1e-12;
        cen = (float)(num / dd);
    } else {
        const double nb = (double)bf16_via_f32(num);
        double db = (double)bf16_via_f32(den);
        const double lo = (double)bf16_via_f32(1e-12);
        if (!(db >= lo)) db = lo;   // torch.clamp_min on the bf16 sum
        cen = bf16_via_f32(nb / db);
    }
    a.centre[(int64_t)row * a.D + tid] = cen;
}

// grid (nchunks, rows), 256 threads: 16 lanes per entry (8 channels each), 16 entries per
// step.
template <bool SLOTS>
__global__ void __launch_bounds__(VS_NT) vs_score_kernel(VsArgs a) {
    __shared__ float cen[128];
    const int chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    for (int d = tid; d < a.D; d += VS_NT) cen[d] = a.centre[(int64_t)row * a.D + d];
    __syncthreads();
    const int tl = tid / 16, oc = tid % 16;
    const int c0 = oc * 8;
    const bool cok = c0 < a.D;
    const int j0 = chunk * a.chunk, j1 = min(j0 + a.chunk, a.n);
    const float *ar = a.a + (int64_t)row * a.sa;
    float *sr = a.score + (int64_t)row * a.ss;
    float cc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cc[i] = cok ? cen[c0 + i] : 0.f;
    for (int jb0 = j0; jb0 < j1; jb0 += VS_TOK * VS_BATCH) {
        // VS_BATCH steps' loads in flight together (tokens past the chunk are not written)
        float x[VS_BATCH][8], aw[VS_BATCH];
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int j = jb0 + u * VS_TOK + tl;
            const int jl = j < j1 ? j : j0;
            if (cok) entry8<SLOTS>(a, row, jl, c0, x[u]);
            aw[u] = ar[jl];
        }
#pragma unroll
        for (int u = 0; u < VS_BATCH; ++u) {
            const int j = jb0 + u * VS_TOK + tl;
            double ss = 0.0;
            if (cok) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float dl = x[u][i] - cc[i];          // exact difference rounded to f32
                    if (!a.fp32_mode) dl = ma_round_bf16(dl);
                    ss = __builtin_fma((double)dl, (double)dl, ss);
                }
            }
            // sum over the 16 lanes of this entry (lanes tl*16 .. tl*16+15 of the wave pair)
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
            if (j < j1 && oc == 0) {
                float nrm;
                if (a.fp32_mode) nrm = (float)__builtin_sqrt(ss);
                else nrm = bf16_via_f32(__builtin_sqrt(ss));
                sr[j] = aw[u] * nrm;
            }
        }
    }
}

// ---------------------------------------------------------------- compaction
struct Plane {
    char *base;          // element (b=0, h=0, token 0)
    int64_t sb, sh, sn;  // byte strides
    int32_t row_bytes, unit;
};

constexpr int MAX_PLANES = 8;

struct CompactArgs {
    Plane pl[MAX_PLANES];
    int nplanes, H, C, n;
    int lpe;              // threads per entry: the widest plane's copy units, a power of two <= 16
    const int64_t *keep;
    int64_t skb, skh;     // keep strides (elements), entries contiguous
    char *scratch;        // [rows][C][total_row_bytes]
    int64_t total_row_bytes;
    int32_t plane_off[MAX_PLANES];  // byte offset of plane p inside a scratch row
};

template <int U>
struct UnitT;
template <>
struct UnitT<16> { using T = uint4; };
template <>
struct UnitT<8> { using T = uint2; };
template <>
struct UnitT<4> { using T = uint32_t; };
template <>
struct UnitT<2> { using T = uint16_t; };

// copy `bytes` bytes from s to d in units of U (one thread per unit, `lanes` threads)
template <int U>
__device__ __forceinline__ void copy_units(char *d, const char *s, int bytes, int lane, int lanes, bool zero) {
    using T = typename UnitT<U>::T;
    for (int o = lane * U; o < bytes; o += lanes * U) {
        T v{};
        if (!zero) v = *(const T *)(s + o);
        *(T *)(d + o) = v;
    }
}

__device__ __forceinline__ void copy_bytes(char *d, const char *s, int bytes, int unit, int lane, int lanes,
                                           bool zero) {
    switch (unit) {
        case 16: copy_units<16>(d, s, bytes, lane, lanes, zero); break;
        case 8: copy_units<8>(d, s, bytes, lane, lanes, zero); break;
        case 4: copy_units<4>(d, s, bytes, lane, lanes, zero); break;
        default: copy_units<2>(d, s, bytes, lane, lanes, zero); break;
    }
}

// grid (ceil(C / (256 / lpe)), rows), 256 threads: 256 / lpe entries x lpe lanes.
// PHASE 0: sources inside [0, C) that move -> scratch.  PHASE 1: every destination.
template <int PHASE>
__global__ void __launch_bounds__(256) compact_kernel(CompactArgs a) {
    const int row = blockIdx.y, b = row / a.H, h = row % a.H;
    const int i = blockIdx.x * (256 / a.lpe) + threadIdx.x / a.lpe;
    const int lane = threadIdx.x % a.lpe;
    if (i >= a.C) return;
    const int64_t src = a.keep[(int64_t)b * a.skb + (int64_t)h * a.skh + i];
    const bool valid = src >= 0 && src < a.n;
    const bool inside = valid && src < a.C;
    if (valid && src == i) return;  // stays where it is
    char *srow = a.scratch + ((int64_t)row * a.C + i) * a.total_row_bytes;
    for (int p = 0; p < a.nplanes; ++p) {
        const Plane &P = a.pl[p];
        char *lane_base = P.base + b * P.sb + h * P.sh;
        if (PHASE == 0) {
            if (inside) copy_bytes(srow + a.plane_off[p], lane_base + src * P.sn, P.row_bytes, P.unit, lane, a.lpe,
                                   false);
        } else {
            const char *from = inside ? srow + a.plane_off[p] : lane_base + (valid ? src : 0) * P.sn;
            copy_bytes(lane_base + (int64_t)i * P.sn, from, P.row_bytes, P.unit, lane, a.lpe, !valid);
        }
    }
}

// ---------------------------------------------------------------- append
// grid (ceil(T*D/8 / 256), B*H): dst[b,h,at+t,:] = src[b,h,t,:] converted to dst dtype
__global__ void __launch_bounds__(256) append_kernel(ma_tensor4 src, ma_tensor4 dst, int H, int T, int D, int at) {
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int it = blockIdx.x * 256 + threadIdx.x;
    const int per = D / 8;
    if (it >= T * per) return;
    const int t = it / per, c0 = (it % per) * 8;
    const int64_t so = b * src.s[0] + h * src.s[1] + (int64_t)t * src.s[2] + c0;
    const int64_t d0 = b * dst.s[0] + h * dst.s[1] + (int64_t)(at + t) * dst.s[2] + c0;
    if (src.dtype == dst.dtype && dst.dtype != MA_F32) {
        *(uint4 *)((uint16_t *)dst.ptr + d0) = *(const uint4 *)((const uint16_t *)src.ptr + so);
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ma_store_f(dst.ptr, d0 + e, dst.dtype, ma_load_f(src.ptr, so + e, src.dtype));
}

}  // namespace

extern "C" int64_t ma_value_score_workspace_bytes(int rows, int n, int D) {
    if (rows <= 0 || n < 0 || D <= 0 || D > 128) return -1;
    const int nchunks = n ? (n + VS_CHUNK - 1) / VS_CHUNK : 1;
    return (int64_t)rows * nchunks * (D + 1) * 8 + (int64_t)rows * D * 4 + 256;
}

extern "C" int ma_value_score(const float *a, int64_t a_stride, ma_tensor4 v, int B, int H, int n, int D,
                              int fp32_mode, float *score, int64_t score_stride, void *workspace,
                              int64_t workspace_bytes, void *stream) {
    const char *who = "ma_value_score";
    if (!a || !v.ptr || !score || B <= 0 || H <= 0 || n < 0 || D <= 0 || D > 128 || D % 8 || a_stride < n ||
        score_stride < n || (v.dtype != MA_BF16 && v.dtype != MA_F16 && v.dtype != MA_F32)) {
        ma_set_error("%s: bad arguments (B=%d H=%d n=%d D=%d)", who, B, H, n, D);
        return MA_EINVAL;
    }
    const int64_t m = v.dtype == MA_F32 ? 4 : 8;
    if (((uintptr_t)v.ptr & 15) || v.s[0] % m || v.s[1] % m || v.s[2] % m) {
        ma_set_error("%s: values must be 16-byte aligned with aligned row strides", who);
        return MA_EINVAL;
    }
    const int rows = B * H;
    const int64_t need = ma_value_score_workspace_bytes(rows, n, D);
    if (!workspace || workspace_bytes < need) {
        ma_set_error("%s: workspace %lld bytes < %lld needed", who, (long long)workspace_bytes, (long long)need);
        return MA_EWORKSPACE;
    }
    if (n == 0) return MA_OK;
    VsArgs va;
    va.a = a;
    va.v = v.ptr;
    va.sa = a_stride;
    va.sv0 = v.s[0];
    va.sv1 = v.s[1];
    va.sv2 = v.s[2];
    va.H = H;
    va.n = n;
    va.D = D;
    va.vdtype = v.dtype;
    va.fp32_mode = fp32_mode;
    va.chunk = VS_CHUNK;
    va.nchunks = (n + va.chunk - 1) / va.chunk;
    va.part = (double *)(((uintptr_t)workspace + 15) & ~(uintptr_t)15);
    va.centre = (float *)(va.part + (int64_t)rows * va.nchunks * (D + 1));
    va.score = score;
    va.ss = score_stride;
    va.slots = nullptr;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(va.nchunks, rows);
    if (v.dtype == MA_BF16 && !fp32_mode) {
        hipLaunchKernelGGL((vs_partial_bf_kernel<false, false, false>), grid, dim3(VS_NT), 0, st, va);
        hipLaunchKernelGGL(vs_centre_kernel, dim3(rows), dim3(VC_NT), 0, st, va);
        hipLaunchKernelGGL((vs_score_bf_kernel<false, false, false>), grid, dim3(VS_NT), 0, st, va);
        return ma_check_launch(who);
    }
    hipLaunchKernelGGL(vs_partial_kernel<false>, grid, dim3(VS_NT), 0, st, va);
    hipLaunchKernelGGL(vs_centre_kernel, dim3(rows), dim3(VC_NT), 0, st, va);
    hipLaunchKernelGGL(vs_score_kernel<false>, grid, dim3(VS_NT), 0, st, va);
    return ma_check_launch(who);
}

int ma_validate_prefix(const ma_prefix *p, int D, const char *who);

extern "C" int ma_value_score_slots(const float *a, int64_t a_stride, const ma_prefix *p, const int32_t *slots,
                                    int64_t slot_stride, int B, int H, int n, int D, int vdtype, int fp32_mode,
                                    float *score, int64_t score_stride, void *workspace, int64_t workspace_bytes,
                                    void *stream) {
    const char *who = "ma_value_score_slots";
    int rc = ma_validate_prefix(p, D, who);
    if (rc) return rc;
    if (!a || !slots || !score || B <= 0 || H <= 0 || n < 0 || D <= 0 || D > 128 || D % 32 || a_stride < n ||
        score_stride < n || slot_stride < n || (vdtype != MA_BF16 && vdtype != MA_F16 && vdtype != MA_F32) ||
        (p->nq > 0 && (p->vbits != 4 || p->vgroup != 32))) {
        ma_set_error("%s: bad arguments (B=%d H=%d n=%d D=%d)", who, B, H, n, D);
        return MA_EINVAL;
    }
    if (p->nq > 0 && ((p->svq[0] | p->svq[1]) & 3)) {
        ma_set_error("%s: value code strides must be multiples of 4 bytes", who);
        return MA_EINVAL;
    }
    if (p->nf > 0 && (((uintptr_t)p->vf & 15) || p->svf[0] % 8 || p->svf[1] % 8 || p->svf[2] % 8)) {
        ma_set_error("%s: 16-bit rows must be 16-byte aligned with aligned row strides", who);
        return MA_EINVAL;
    }
    const int rows = B * H;
    const int64_t need = ma_value_score_workspace_bytes(rows, n, D);
    if (!workspace || workspace_bytes < need) {
        ma_set_error("%s: workspace %lld bytes < %lld needed", who, (long long)workspace_bytes, (long long)need);
        return MA_EWORKSPACE;
    }
    if (n == 0) return MA_OK;
    VsArgs va = VsArgs{};
    va.a = a;
    va.sa = a_stride;
    va.H = H;
    va.n = n;
    va.D = D;
    va.vdtype = vdtype;
    va.fp32_mode = fp32_mode;
    va.chunk = VS_CHUNK;
    va.nchunks = (n + va.chunk - 1) / va.chunk;
    va.part = (double *)(((uintptr_t)workspace + 15) & ~(uintptr_t)15);
    va.centre = (float *)(va.part + (int64_t)rows * va.nchunks * (D + 1));
    va.score = score;
    va.ss = score_stride;
    va.slots = slots;
    va.sslot = slot_stride;
    va.vq = (const uint8_t *)p->vq;
    va.vsc = (const uint16_t *)p->vs;
    va.vzp = (const uint16_t *)p->vz;
    va.vf = p->vf;
    for (int i = 0; i < 4; ++i) va.svq[i] = p->svq[i];
    for (int i = 0; i < 3; ++i) {
        va.svs[i] = p->svs[i];
        va.svf[i] = p->svf[i];
    }
    va.nq = p->nq;
    va.nf = p->nf;
    va.fdtype = p->fdtype;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(va.nchunks, rows);
    if (vdtype == MA_BF16 && !fp32_mode && (p->nf == 0 || p->fdtype == MA_BF16)) {
        // the all-bf16 passes, instantiated for packed slots, 16-bit rows or both
        auto both = [&](auto partial, auto score) {
            hipLaunchKernelGGL(partial, grid, dim3(VS_NT), 0, st, va);
            hipLaunchKernelGGL(vs_centre_kernel, dim3(rows), dim3(VC_NT), 0, st, va);
            hipLaunchKernelGGL(score, grid, dim3(VS_NT), 0, st, va);
        };
        if (p->nq > 0 && p->nf > 0) both(vs_partial_bf_kernel<true, true, true>, vs_score_bf_kernel<true, true, true>);
        else if (p->nq > 0) both(vs_partial_bf_kernel<true, true, false>, vs_score_bf_kernel<true, true, false>);
        else both(vs_partial_bf_kernel<true, false, true>, vs_score_bf_kernel<true, false, true>);
        return ma_check_launch(who);
    }
    hipLaunchKernelGGL(vs_partial_kernel<true>, grid, dim3(VS_NT), 0, st, va);
    hipLaunchKernelGGL(vs_centre_kernel, dim3(rows), dim3(VC_NT), 0, st, va);
    hipLaunchKernelGGL(vs_score_kernel<true>, grid, dim3(VS_NT), 0, st, va);
    return ma_check_launch(who);
}

extern "C" int64_t ma_compact_workspace_bytes(int rows, int capacity, const int32_t *row_bytes, int nplanes) {
    if (rows <= 0 || capacity < 0 || nplanes <= 0 || nplanes > MAX_PLANES || !row_bytes) return -1;
    int64_t tot = 0;
    for (int p = 0; p < nplanes; ++p) tot += ((int64_t)row_bytes[p] + 15) & ~(int64_t)15;
    return (int64_t)rows * capacity * tot + 256;
}

extern "C" int ma_compact_tokens(void *const *bases, const int64_t *strides, const int32_t *row_bytes, int nplanes,
                                 int B, int H, int n, const int64_t *keep, const int64_t skeep[2], int capacity,
                                 void *workspace, int64_t workspace_bytes, void *stream) {
    const char *who = "ma_compact_tokens";
    if (!bases || !strides || !row_bytes || nplanes <= 0 || nplanes > MAX_PLANES || B <= 0 || H <= 0 || n < 0 ||
        !keep || !skeep || capacity < 0 || capacity > n) {
        ma_set_error("%s: bad arguments (planes=%d B=%d H=%d n=%d C=%d)", who, nplanes, B, H, n, capacity);
        return MA_EINVAL;
    }
    CompactArgs ca;
    int64_t tot = 0;
    for (int p = 0; p < nplanes; ++p) {
        Plane &P = ca.pl[p];
        P.base = (char *)bases[p];
        P.sb = strides[3 * p + 0];
        P.sh = strides[3 * p + 1];
        P.sn = strides[3 * p + 2];
        P.row_bytes = row_bytes[p];
        if (!P.base || P.row_bytes <= 0 || P.row_bytes % 2) {
            ma_set_error("%s: plane %d: NULL base or odd row size %d", who, p, P.row_bytes);
            return MA_EINVAL;
        }
        const uint64_t al = (uint64_t)(uintptr_t)P.base | (uint64_t)P.sb | (uint64_t)P.sh | (uint64_t)P.sn |
                            (uint64_t)P.row_bytes;
        P.unit = (al % 16 == 0) ? 16 : (al % 8 == 0) ? 8 : (al % 4 == 0) ? 4 : 2;
        ca.plane_off[p] = (int32_t)tot;
        tot += ((int64_t)P.row_bytes + 15) & ~(int64_t)15;
    }
    int units = 1;
    for (int p = 0; p < nplanes; ++p)
        units = std::max(units, (int)((ca.pl[p].row_bytes + ca.pl[p].unit - 1) / ca.pl[p].unit));
    ca.lpe = 1;
    while (ca.lpe < 16 && ca.lpe < units) ca.lpe <<= 1;
    const int64_t need = (int64_t)B * H * capacity * tot + 256;
    if (!workspace || workspace_bytes < need) {
        ma_set_error("%s: workspace %lld bytes < %lld needed", who, (long long)workspace_bytes, (long long)need);
        return MA_EWORKSPACE;
    }
    if (capacity == 0) return MA_OK;
    ca.nplanes = nplanes;
    ca.H = H;
    ca.C = capacity;
    ca.n = n;
    ca.keep = keep;
    ca.skb = skeep[0];
    ca.skh = skeep[1];
    ca.scratch = (char *)(((uintptr_t)workspace + 15) & ~(uintptr_t)15);
    ca.total_row_bytes = tot;
    hipStream_t st = (hipStream_t)stream;
    const int per_block = 256 / ca.lpe;
    const dim3 grid((capacity + per_block - 1) / per_block, B * H);
    hipLaunchKernelGGL(compact_kernel<0>, grid, dim3(256), 0, st, ca);
    hipLaunchKernelGGL(compact_kernel<1>, grid, dim3(256), 0, st, ca);
    return ma_check_launch(who);
}

extern "C" int ma_append_tokens(ma_tensor4 src, ma_tensor4 dst, int B, int H, int T, int D, int at, void *stream) {
    const char *who = "ma_append_tokens";
    if (!src.ptr || !dst.ptr || B <= 0 || H <= 0 || T < 0 || D <= 0 || D % 8 || at < 0) {
        ma_set_error("%s: bad arguments", who);
        return MA_EINVAL;
    }
    auto al = [](const ma_tensor4 &t) {
        const int64_t m = t.dtype == MA_F32 ? 4 : 8;
        return ((uintptr_t)t.ptr & 15) == 0 && t.s[0] % m == 0 && t.s[1] % m == 0 && t.s[2] % m == 0;
    };
    if (!al(src) || !al(dst)) {
        ma_set_error("%s: tensors must be 16-byte aligned with aligned row strides", who);
        return MA_EINVAL;
    }
    if (T == 0) return MA_OK;
    const int items = T * (D / 8);
    hipLaunchKernelGGL(append_kernel, dim3((items + 255) / 256, B * H), dim3(256), 0, (hipStream_t)stream, src, dst,
                       H, T, D, at);
    return ma_check_launch(who);
}
