// Packed-KV codec kernels: whole-prefix dequant, gather of selected entries, and the
// 4-bit quantizers of the append path.  All integer/byte work, bit-exact against the
// reference's torch codec (reference.py:35-268).
#include "ma_common.h"
#include "ma_quant.h"

namespace {

constexpr int KG = 32;  // key token group (the only one shipped configs use)
constexpr int VG = 32;  // value channel group

struct PrefixArgs {
    const uint8_t *kq;
    const uint16_t *ks, *kz;
    const uint8_t *vq;
    const uint16_t *vs, *vz;
    const void *kf, *vf;
    int64_t skq[4], sks[3], svq[4], svs[3], skf[3], svf[3];
    int nq, nf, fdtype;
};

PrefixArgs make_args(const ma_prefix *p) {
    PrefixArgs a;
    a.kq = (const uint8_t *)p->kq;
    a.ks = (const uint16_t *)p->ks;
    a.kz = (const uint16_t *)p->kz;
    a.vq = (const uint8_t *)p->vq;
    a.vs = (const uint16_t *)p->vs;
    a.vz = (const uint16_t *)p->vz;
    a.kf = p->kf;
    a.vf = p->vf;
    for (int i = 0; i < 4; ++i) {
        a.skq[i] = p->skq[i];
        a.svq[i] = p->svq[i];
    }
    for (int i = 0; i < 3; ++i) {
        a.sks[i] = p->sks[i];
        a.svs[i] = p->svs[i];
        a.skf[i] = p->skf[i];
        a.svf[i] = p->svf[i];
    }
    a.nq = p->nq;
    a.nf = p->nf;
    a.fdtype = p->fdtype;
    return a;
}

// Dequantized key element (token j < nq, channel d) of lane (b, h).
__device__ __forceinline__ float key_elem(const PrefixArgs &a, int b, int h, int j, int d) {
    int g = j / KG, tt = j % KG;
    const uint8_t *row = a.kq + b * a.skq[0] + h * a.skq[1] + (int64_t)g * a.skq[2] + (int64_t)d * a.skq[3];
    uint32_t byte = row[tt >> 1];
    uint32_t code = (tt & 1) ? (byte >> 4) : (byte & 15u);
    int64_t so = b * a.sks[0] + h * a.sks[1] + (int64_t)g * a.sks[2] + d;
    return ma_dq(code, ma_f16_to_f32(a.ks[so]), ma_f16_to_f32(a.kz[so]));
}

// ---------------------------------------------------------------- dequant_prefix
// grid (ceil(n/64), B*H), 256 threads; one tile = 64 tokens x D channels of K and V.
__global__ void __launch_bounds__(256) dequant_prefix_kernel(PrefixArgs a, int H, int D, ma_tensor4 ko,
                                                             ma_tensor4 vo) {
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int n0 = blockIdx.x * 64;
    const int n = a.nq + a.nf;
    const int tid = threadIdx.x;
    const int ncg = D / VG;

    // keys, packed part: item = (group in tile, channel)
    for (int it = tid; it < 2 * D; it += 256) {
        int gl = it / D, d = it % D;
        int t0 = n0 + gl * KG;
        if (t0 >= a.nq) continue;
        int g = t0 / KG;
        const uint8_t *row = a.kq + b * a.skq[0] + h * a.skq[1] + (int64_t)g * a.skq[2] + (int64_t)d * a.skq[3];
        uint4 raw = *(const uint4 *)row;
        uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        int64_t so = b * a.sks[0] + h * a.sks[1] + (int64_t)g * a.sks[2] + d;
        float sc = ma_f16_to_f32(a.ks[so]), zp = ma_f16_to_f32(a.kz[so]);
        int64_t ob = b * ko.s[0] + h * ko.s[1] + d;
#pragma unroll
        for (int t = 0; t < KG; ++t) {
            uint32_t code = (w[t >> 3] >> ((t & 7) * 4)) & 15u;
            ma_store_f(ko.ptr, ob + (int64_t)(t0 + t) * ko.s[2], ko.dtype, ma_dq(code, sc, zp));
        }
    }
    // values, packed part: item = (token, channel group)
    for (int it = tid; it < 64 * ncg; it += 256) {
        int tl = it / ncg, cg = it % ncg;
        int j = n0 + tl;
        if (j >= a.nq) continue;
        const uint8_t *src = a.vq + b * a.svq[0] + h * a.svq[1] + (int64_t)j * a.svq[2] + (int64_t)cg * a.svq[3];
        uint4 raw = *(const uint4 *)src;
        uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        int64_t so = b * a.svs[0] + h * a.svs[1] + (int64_t)j * a.svs[2] + cg;
        float sc = ma_f16_to_f32(a.vs[so]), zp = ma_f16_to_f32(a.vz[so]);
        int64_t ob = b * vo.s[0] + h * vo.s[1] + (int64_t)j * vo.s[2] + cg * VG;
#pragma unroll
        for (int c = 0; c < VG; ++c) {
            uint32_t code = (w[c >> 3] >> ((c & 7) * 4)) & 15u;
            ma_store_f(vo.ptr, ob + c, vo.dtype, ma_dq(code, sc, zp));
        }
    }
    // 16-bit part (residual tail, or the whole prefix of a bf16 cache)
    for (int it = tid; it < 64 * D; it += 256) {
        int tl = it / D, d = it % D;
        int j = n0 + tl;
        if (j < a.nq || j >= n) continue;
        int jf = j - a.nq;
        float kx = ma_load_f(a.kf, b * a.skf[0] + h * a.skf[1] + (int64_t)jf * a.skf[2] + d, a.fdtype);
        float vx = ma_load_f(a.vf, b * a.svf[0] + h * a.svf[1] + (int64_t)jf * a.svf[2] + d, a.fdtype);
        ma_store_f(ko.ptr, b * ko.s[0] + h * ko.s[1] + (int64_t)j * ko.s[2] + d, ko.dtype, kx);
        ma_store_f(vo.ptr, b * vo.s[0] + h * vo.s[1] + (int64_t)j * vo.s[2] + d, vo.dtype, vx);
    }
}

// ---------------------------------------------------------------- gather
// grid (ceil(k / TPB_TOK), B*H), 256 threads; D/4 threads per selected entry, 4
// channels each.  Indices outside [0, n) produce zeros (never an out-of-bounds read).
// vec: the 4 key scales / zeros of a thread are one 8-byte load each and bf16 outputs are
// written 8 bytes at a time (the host checks the alignment this needs).
__global__ void __launch_bounds__(256) gather_kernel(PrefixArgs a, int H, int D, const int64_t *idx, int64_t sib,
                                                     int64_t sih, int k, ma_tensor4 ko, ma_tensor4 vo, int vec) {
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int tpt = D / 4;               // threads per token
    const int toks = 256 / tpt;
    const int i = blockIdx.x * toks + threadIdx.x / tpt;
    const int c0 = (threadIdx.x % tpt) * 4;
    if (i >= k) return;
    const int n = a.nq + a.nf;
    const int64_t j64 = idx[b * sib + h * sih + i];
    float kx[4] = {0.f, 0.f, 0.f, 0.f}, vx[4] = {0.f, 0.f, 0.f, 0.f};
    if (j64 >= 0 && j64 < n) {
        const int j = (int)j64;
        if (j < a.nq) {
            const int g = j / KG, tt = j % KG;
            const uint8_t *krow = a.kq + b * a.skq[0] + h * a.skq[1] + (int64_t)g * a.skq[2] + (int64_t)c0 * a.skq[3];
            uint32_t kb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) kb[e] = krow[(int64_t)e * a.skq[3] + (tt >> 1)];
            const int64_t so = b * a.sks[0] + h * a.sks[1] + (int64_t)g * a.sks[2] + c0;
            uint16_t ks[4], kz[4];
            if (vec) {
                const uint2 sv = *(const uint2 *)&a.ks[so], zv = *(const uint2 *)&a.kz[so];
                ks[0] = sv.x & 0xffffu; ks[1] = sv.x >> 16; ks[2] = sv.y & 0xffffu; ks[3] = sv.y >> 16;
                kz[0] = zv.x & 0xffffu; kz[1] = zv.x >> 16; kz[2] = zv.y & 0xffffu; kz[3] = zv.y >> 16;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ks[e] = a.ks[so + e];
                    kz[e] = a.kz[so + e];
                }
            }
            const int cg = c0 / VG, w = c0 % VG;
            const uint8_t *src = a.vq + b * a.svq[0] + h * a.svq[1] + (int64_t)j * a.svq[2] + (int64_t)cg * a.svq[3];
            const uint32_t two = (uint32_t)src[w >> 1] | ((uint32_t)src[(w >> 1) + 1] << 8);
            const int64_t vso = b * a.svs[0] + h * a.svs[1] + (int64_t)j * a.svs[2] + cg;
            const float vsc = ma_f16_to_f32(a.vs[vso]), vzp = ma_f16_to_f32(a.vz[vso]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t code = (tt & 1) ? (kb[e] >> 4) : (kb[e] & 15u);
                kx[e] = ma_dq(code, ma_f16_to_f32(ks[e]), ma_f16_to_f32(kz[e]));
                vx[e] = ma_dq((two >> (4 * e)) & 15u, vsc, vzp);
            }
        } else {
            const int jf = j - a.nq;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kx[e] = ma_load_f(a.kf, b * a.skf[0] + h * a.skf[1] + (int64_t)jf * a.skf[2] + c0 + e, a.fdtype);
                vx[e] = ma_load_f(a.vf, b * a.svf[0] + h * a.svf[1] + (int64_t)jf * a.svf[2] + c0 + e, a.fdtype);
            }
        }
    }
    const int64_t ok = b * ko.s[0] + h * ko.s[1] + (int64_t)i * ko.s[2] + c0;
    const int64_t ov = b * vo.s[0] + h * vo.s[1] + (int64_t)i * vo.s[2] + c0;
    if (vec && ko.dtype == MA_BF16 && vo.dtype == MA_BF16) {
        uint2 kw, vw;
        kw.x = (uint32_t)ma_f32_to_bf16(kx[0]) | ((uint32_t)ma_f32_to_bf16(kx[1]) << 16);
        kw.y = (uint32_t)ma_f32_to_bf16(kx[2]) | ((uint32_t)ma_f32_to_bf16(kx[3]) << 16);
        vw.x = (uint32_t)ma_f32_to_bf16(vx[0]) | ((uint32_t)ma_f32_to_bf16(vx[1]) << 16);
        vw.y = (uint32_t)ma_f32_to_bf16(vx[2]) | ((uint32_t)ma_f32_to_bf16(vx[3]) << 16);
        *(uint2 *)((uint16_t *)ko.ptr + ok) = kw;
        *(uint2 *)((uint16_t *)vo.ptr + ov) = vw;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ma_store_f(ko.ptr, ok + e, ko.dtype, kx[e]);
            ma_store_f(vo.ptr, ov + e, vo.dtype, vx[e]);
        }
    }
}

// ---------------------------------------------------------------- quantizers
// The source of a quantizer: token rows 0 .. na-1 from `a`, the rest from `b` (row i - na)
// -- [residual | new tokens] of an append without building that tensor; na = 0 reads `b`
// alone.  a and b have the same dtype.
struct TwoSrc {
    ma_tensor4 a, b;
    int na;
};

// DT: the dtype, a compile-time constant so that a thread's loads are straight-line code
// (all of them in flight at once) instead of one branch per element
template <int DT>
__device__ __forceinline__ float two_load(const TwoSrc &s, int b, int h, int i, int d) {
    const bool in_a = i < s.na;
    const char *base = (const char *)(in_a ? s.a.ptr : s.b.ptr);
    const int64_t sb = in_a ? s.a.s[0] : s.b.s[0], sh = in_a ? s.a.s[1] : s.b.s[1],
                  st = in_a ? s.a.s[2] : s.b.s[2];
    const int r = in_a ? i : i - s.na;
    return ma_load_f(base, b * sb + h * sh + (int64_t)r * st + d, DT);
}

// keys: grid (T/KG, B*H), D threads; thread = one channel of one token group.
template <int DT>
__global__ void quantize_keys_kernel(TwoSrc src, int H, int D, uint8_t *kq, int64_t q0, int64_t q1, int64_t q2,
                                     int64_t q3, _Float16 *ks, _Float16 *kz, int64_t s0, int64_t s1, int64_t s2) {
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int g = blockIdx.x;
    const int d = threadIdx.x;
    if (d >= D) return;
    float x[KG];
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int t = 0; t < KG; ++t) {
        x[t] = two_load<DT>(src, b, h, g * KG + t, d);
        lo = fminf(lo, x[t]);
        hi = fmaxf(hi, x[t]);
    }
    constexpr int dtype = DT;
    QuantGroup qp = quant_params(lo, hi, dtype);
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < KG; ++t) w[t >> 3] |= quant_code(x[t], qp, dtype) << ((t & 7) * 4);
    uint4 out = {w[0], w[1], w[2], w[3]};
    *(uint4 *)(kq + b * q0 + h * q1 + (int64_t)g * q2 + (int64_t)d * q3) = out;
    int64_t so = b * s0 + h * s1 + (int64_t)g * s2 + d;
    ks[so] = (_Float16)qp.step;
    kz[so] = (_Float16)qp.lo;
}

// values: one thread per (token, channel group); grid-stride over B*H*T*(D/VG) items.
template <int DT>
__global__ void __launch_bounds__(256) quantize_values_kernel(TwoSrc src, int BH, int H, int T, int D, uint8_t *vq,
                                                              int64_t q0, int64_t q1, int64_t q2, int64_t q3,
                                                              _Float16 *vs, _Float16 *vz, int64_t s0, int64_t s1,
                                                              int64_t s2) {
    const int ncg = D / VG;
    const int64_t total = (int64_t)BH * T * ncg;
    constexpr int dtype = DT;
    for (int64_t it = (int64_t)blockIdx.x * 256 + threadIdx.x; it < total; it += (int64_t)gridDim.x * 256) {
        int cg = (int)(it % ncg);
        int64_t rest = it / ncg;
        int j = (int)(rest % T);
        int bh = (int)(rest / T), b = bh / H, h = bh % H;
        float x[VG];
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int c = 0; c < VG; ++c) {
            x[c] = two_load<DT>(src, b, h, j, cg * VG + c);
            lo = fminf(lo, x[c]);
            hi = fmaxf(hi, x[c]);
        }
        QuantGroup qp = quant_params(lo, hi, dtype);
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < VG; ++c) w[c >> 3] |= quant_code(x[c], qp, dtype) << ((c & 7) * 4);
        uint4 out = {w[0], w[1], w[2], w[3]};
        *(uint4 *)(vq + b * q0 + h * q1 + (int64_t)j * q2 + (int64_t)cg * q3) = out;
        int64_t so = b * s0 + h * s1 + (int64_t)j * s2 + cg;
        vs[so] = (_Float16)qp.step;
        vz[so] = (_Float16)qp.lo;
    }
}

// The residual an append keeps: token rows [move, na + T) of [a | b] into a's rows
// [0, keep), for K (blockIdx.y 0) and V (1).  Rows of a move down by `move` in place, so
// one workgroup per lane copies them in chunks of CH rows, every chunk read whole before
// any of it is written: a chunk's destination rows lie below the source rows of every
// later chunk.  (move = 0 leaves a's rows where they are and appends b's.)
constexpr int RK_NT = 256;
template <int DT>
__global__ void __launch_bounds__(RK_NT) residual_keep_kernel(TwoSrc k, TwoSrc v, int H, int D, int move, int keep) {
    const TwoSrc &s = blockIdx.y ? v : k;
    const int bh = blockIdx.x, b = bh / H, h = bh % H;
    const int first = move == 0 ? s.na : 0;      // move = 0: a's rows stay, b's follow them
    const int per = RK_NT / D;                   // rows per pass of the workgroup
    const int r0 = threadIdx.x / D, d = threadIdx.x % D;
    constexpr int RPT = 32;                      // rows per thread per chunk (64 rows at D = 128)
    char *dst = (char *)s.a.ptr;
    for (int c0 = first; c0 < keep; c0 += per * RPT) {
        float x[RPT];
#pragma unroll
        for (int e = 0; e < RPT; ++e) {
            const int r = c0 + e * per + r0;
            x[e] = r < keep && r0 < per ? two_load<DT>(s, b, h, r + move, d) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < RPT; ++e) {
            const int r = c0 + e * per + r0;
            if (r < keep && r0 < per)
                ma_store_f(dst, b * s.a.s[0] + h * s.a.s[1] + (int64_t)r * s.a.s[2] + d, DT, x[e]);
        }
        __syncthreads();
    }
}

template <int DT>
void quant_keys_as(dim3 grid, int D, hipStream_t st, const TwoSrc &src, int H, void *kq, const int64_t *skq, void *ks,
                   void *kz, const int64_t *sks) {
    hipLaunchKernelGGL(quantize_keys_kernel<DT>, grid, dim3(D), 0, st, src, H, D, (uint8_t *)kq, skq[0], skq[1], skq[2],
                       skq[3], (_Float16 *)ks, (_Float16 *)kz, sks[0], sks[1], sks[2]);
}

void launch_quant_keys(int dtype, dim3 grid, int D, hipStream_t st, const TwoSrc &src, int H, void *kq,
                       const int64_t *skq, void *ks, void *kz, const int64_t *sks) {
    if (dtype == MA_BF16) quant_keys_as<MA_BF16>(grid, D, st, src, H, kq, skq, ks, kz, sks);
    else if (dtype == MA_F16) quant_keys_as<MA_F16>(grid, D, st, src, H, kq, skq, ks, kz, sks);
    else quant_keys_as<MA_F32>(grid, D, st, src, H, kq, skq, ks, kz, sks);
}

template <int DT>
void quant_values_as(int blocks, hipStream_t st, const TwoSrc &src, int BH, int H, int T, int D, void *vq,
                     const int64_t *svq, void *vs, void *vz, const int64_t *svs) {
    hipLaunchKernelGGL(quantize_values_kernel<DT>, dim3(blocks), dim3(256), 0, st, src, BH, H, T, D, (uint8_t *)vq,
                       svq[0], svq[1], svq[2], svq[3], (_Float16 *)vs, (_Float16 *)vz, svs[0], svs[1], svs[2]);
}

void launch_quant_values(int dtype, int blocks, hipStream_t st, const TwoSrc &src, int BH, int H, int T, int D,
                         void *vq, const int64_t *svq, void *vs, void *vz, const int64_t *svs) {
    if (dtype == MA_BF16) quant_values_as<MA_BF16>(blocks, st, src, BH, H, T, D, vq, svq, vs, vz, svs);
    else if (dtype == MA_F16) quant_values_as<MA_F16>(blocks, st, src, BH, H, T, D, vq, svq, vs, vz, svs);
    else quant_values_as<MA_F32>(blocks, st, src, BH, H, T, D, vq, svq, vs, vz, svs);
}

}  // namespace

// ---------------------------------------------------------------- validation helpers
int ma_validate_prefix(const ma_prefix *p, int D, const char *who) {
    if (!p) {
        ma_set_error("%s: prefix is NULL", who);
        return MA_EINVAL;
    }
    if (D != 64 && D != 128) {
        ma_set_error("%s: head_dim %d not built (64, 128)", who, D);
        return MA_EUNSUPPORTED;
    }
    if (p->nq < 0 || p->nf < 0) {
        ma_set_error("%s: negative prefix length", who);
        return MA_EINVAL;
    }
    if (p->nq > 0) {
        if (p->kbits != 4 || p->vbits != 4) {
            ma_set_error("%s: packed bit widths k=%d v=%d not built (4/4)", who, p->kbits, p->vbits);
            return MA_EUNSUPPORTED;
        }
        if (p->kgroup != KG || p->vgroup != VG) {
            ma_set_error("%s: groups k=%d v=%d not built (32/32)", who, p->kgroup, p->vgroup);
            return MA_EUNSUPPORTED;
        }
        if (p->nq % KG) {
            ma_set_error("%s: quantized length %d is not a multiple of %d", who, p->nq, KG);
            return MA_EINVAL;
        }
        if (!p->kq || !p->ks || !p->kz || !p->vq || !p->vs || !p->vz) {
            ma_set_error("%s: packed prefix pointers missing", who);
            return MA_EINVAL;
        }
        if ((((uintptr_t)p->kq | (uintptr_t)p->vq) & 15) || ((p->skq[2] | p->skq[3] | p->svq[2] | p->svq[3]) & 15)) {
            ma_set_error("%s: packed payload rows must be 16-byte aligned", who);
            return MA_EINVAL;
        }
        // key scale/zero are read as f16 pairs (two channels per 32-bit load)
        if ((((uintptr_t)p->ks | (uintptr_t)p->kz) & 3) || ((p->sks[0] | p->sks[1] | p->sks[2]) & 1)) {
            ma_set_error("%s: key scale/zero must be 4-byte aligned with even strides", who);
            return MA_EINVAL;
        }
    }
    if (p->nf > 0) {
        if (!p->kf || !p->vf) {
            ma_set_error("%s: 16-bit prefix pointers missing", who);
            return MA_EINVAL;
        }
        if (p->fdtype != MA_BF16 && p->fdtype != MA_F16 && p->fdtype != MA_F32) {
            ma_set_error("%s: bad prefix dtype %d", who, p->fdtype);
            return MA_EINVAL;
        }
    }
    return MA_OK;
}

static bool out_dtype_ok(int dt) { return dt == MA_BF16 || dt == MA_F32 || dt == MA_F16; }

extern "C" int ma_dequant_prefix(const ma_prefix *p, int B, int H, int D, ma_tensor4 k_out, ma_tensor4 v_out,
                                 void *stream) {
    int rc = ma_validate_prefix(p, D, "ma_dequant_prefix");
    if (rc) return rc;
    if (B <= 0 || H <= 0 || !k_out.ptr || !v_out.ptr || !out_dtype_ok(k_out.dtype) || !out_dtype_ok(v_out.dtype)) {
        ma_set_error("ma_dequant_prefix: bad sizes or outputs");
        return MA_EINVAL;
    }
    int n = p->nq + p->nf;
    if (n == 0) return MA_OK;
    dim3 grid((n + 63) / 64, B * H);
    hipLaunchKernelGGL(dequant_prefix_kernel, grid, dim3(256), 0, (hipStream_t)stream, make_args(p), H, D, k_out,
                       v_out);
    return ma_check_launch("ma_dequant_prefix");
}

extern "C" int ma_gather_kv(const ma_prefix *p, int B, int H, int D, const int64_t *idx, const int64_t sidx[2], int k,
                            ma_tensor4 k_out, ma_tensor4 v_out, void *stream) {
    int rc = ma_validate_prefix(p, D, "ma_gather_kv");
    if (rc) return rc;
    if (B <= 0 || H <= 0 || k < 0 || !idx || !sidx || !k_out.ptr || !v_out.ptr || !out_dtype_ok(k_out.dtype) ||
        !out_dtype_ok(v_out.dtype)) {
        ma_set_error("ma_gather_kv: bad sizes or outputs");
        return MA_EINVAL;
    }
    if (k == 0) return MA_OK;
    int toks = 256 / (D / 4);
    dim3 grid((k + toks - 1) / toks, B * H);
    // 8-byte scale / zero loads and output stores: 8-byte aligned bases, strides in whole
    // groups of 4 elements
    auto al8 = [](const void *ptr) { return ((uintptr_t)ptr & 7) == 0; };
    const int vec = al8(p->ks) && al8(p->kz) && p->sks[0] % 4 == 0 && p->sks[1] % 4 == 0 && p->sks[2] % 4 == 0 &&
                    al8(k_out.ptr) && al8(v_out.ptr) && k_out.s[0] % 4 == 0 && k_out.s[1] % 4 == 0 &&
                    k_out.s[2] % 4 == 0 && v_out.s[0] % 4 == 0 && v_out.s[1] % 4 == 0 && v_out.s[2] % 4 == 0;
    hipLaunchKernelGGL(gather_kernel, grid, dim3(256), 0, (hipStream_t)stream, make_args(p), H, D, idx, sidx[0],
                       sidx[1], k, k_out, v_out, vec);
    return ma_check_launch("ma_gather_kv");
}

extern "C" int ma_quantize_keys(ma_tensor4 src, int B, int H, int T, int D, int group, void *kq, const int64_t skq[4],
                                void *ks, void *kz, const int64_t sks[3], void *stream) {
    if (group != KG) {
        ma_set_error("ma_quantize_keys: token group %d not built (32)", group);
        return MA_EUNSUPPORTED;
    }
    if (B <= 0 || H <= 0 || T < 0 || T % KG || D <= 0 || D > 1024 || !src.ptr || !kq || !ks || !kz || !skq || !sks ||
        ((uintptr_t)kq & 15) || ((skq[2] | skq[3]) & 15) || !out_dtype_ok(src.dtype)) {
        ma_set_error("ma_quantize_keys: bad geometry (T %% 32, 16-byte aligned payload rows)");
        return MA_EINVAL;
    }
    if (T == 0) return MA_OK;
    dim3 grid(T / KG, B * H);
    const TwoSrc two{src, src, 0};
    launch_quant_keys(src.dtype, grid, D, (hipStream_t)stream, two, H, kq, skq, ks, kz, sks);
    return ma_check_launch("ma_quantize_keys");
}

extern "C" int ma_quantize_values(ma_tensor4 src, int B, int H, int T, int D, int group, void *vq,
                                  const int64_t svq[4], void *vs, void *vz, const int64_t svs[3], void *stream) {
    if (group != VG) {
        ma_set_error("ma_quantize_values: channel group %d not built (32)", group);
        return MA_EUNSUPPORTED;
    }
    if (B <= 0 || H <= 0 || T < 0 || D <= 0 || D % VG || !src.ptr || !vq || !vs || !vz || !svq || !svs ||
        ((uintptr_t)vq & 15) || ((svq[2] | svq[3]) & 15) || !out_dtype_ok(src.dtype)) {
        ma_set_error("ma_quantize_values: bad geometry (D %% 32, 16-byte aligned payload rows)");
        return MA_EINVAL;
    }
    if (T == 0) return MA_OK;
    int64_t items = (int64_t)B * H * T * (D / VG);
    int blocks = (int)((items + 255) / 256);
    if (blocks > 65535) blocks = 65535;
    const TwoSrc two{src, src, 0};
    launch_quant_values(src.dtype, blocks, (hipStream_t)stream, two, B * H, H, T, D, vq, svq, vs, vz, svs);
    return ma_check_launch("ma_quantize_values");
}

extern "C" int ma_append_packed(ma_tensor4 k_res, ma_tensor4 v_res, int old_res, ma_tensor4 k_new, ma_tensor4 v_new,
                                int B, int H, int T, int D, int move, int keep, void *kq, const int64_t skq[4],
                                void *ks, void *kz, const int64_t sks[3], void *vq, const int64_t svq[4], void *vs,
                                void *vz, const int64_t svs[3], void *stream) {
    const char *who = "ma_append_packed";
    if (B <= 0 || H <= 0 || T <= 0 || old_res < 0 || move < 0 || keep < 0 || move % KG || move + keep != old_res + T ||
        D <= 0 || D % VG || D > RK_NT || RK_NT % D || !k_new.ptr || !v_new.ptr ||
        ((old_res > 0 || keep > 0) && (!k_res.ptr || !v_res.ptr))) {
        ma_set_error("%s: bad geometry (move %% 32, move + keep = old_res + T, D | 256)", who);
        return MA_EINVAL;
    }
    if (k_new.dtype != v_new.dtype || !out_dtype_ok(k_new.dtype) ||
        ((old_res > 0 || keep > 0) && (k_res.dtype != k_new.dtype || v_res.dtype != k_new.dtype))) {
        ma_set_error("%s: the residual and the new tokens must share one 16-bit or f32 dtype", who);
        return MA_EINVAL;
    }
    const TwoSrc tk{k_res, k_new, old_res}, tv{v_res, v_new, old_res};
    if (move) {
        if (!kq || !ks || !kz || !skq || !sks || !vq || !vs || !vz || !svq || !svs || ((uintptr_t)kq & 15) ||
            ((uintptr_t)vq & 15) || ((skq[2] | skq[3] | svq[2] | svq[3]) & 15)) {
            ma_set_error("%s: packed planes missing or payload rows not 16-byte aligned", who);
            return MA_EINVAL;
        }
        launch_quant_keys(k_new.dtype, dim3(move / KG, B * H), D, (hipStream_t)stream, tk, H, kq, skq, ks, kz, sks);
        int rc = ma_check_launch(who);
        if (rc) return rc;
        const int64_t items = (int64_t)B * H * move * (D / VG);
        int blocks = (int)((items + 255) / 256);
        if (blocks > 65535) blocks = 65535;
        launch_quant_values(k_new.dtype, blocks, (hipStream_t)stream, tv, B * H, H, move, D, vq, svq, vs, vz, svs);
        rc = ma_check_launch(who);
        if (rc) return rc;
    }
    if (keep > (move ? 0 : old_res)) {
        const dim3 grid(B * H, 2);
        if (k_new.dtype == MA_BF16)
            hipLaunchKernelGGL(residual_keep_kernel<MA_BF16>, grid, dim3(RK_NT), 0, (hipStream_t)stream, tk, tv, H, D,
                               move, keep);
        else if (k_new.dtype == MA_F16)
            hipLaunchKernelGGL(residual_keep_kernel<MA_F16>, grid, dim3(RK_NT), 0, (hipStream_t)stream, tk, tv, H, D,
                               move, keep);
        else
            hipLaunchKernelGGL(residual_keep_kernel<MA_F32>, grid, dim3(RK_NT), 0, (hipStream_t)stream, tk, tv, H, D,
                               move, keep);
        return ma_check_launch(who);
    }
    return MA_OK;
}
