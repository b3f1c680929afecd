// Shared device helpers for the gfx950 kernels of libmaskahead_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "maskahead_hip.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

#define MA_WAVE 64

// ---- host-side error reporting (ma_runtime.cpp)
void ma_set_error(const char *fmt, ...);
int ma_check_launch(const char *what);
int ma_num_cus();

// ---- scalar conversions
__device__ __forceinline__ float ma_f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float ma_bf16_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}
// round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint16_t ma_f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t ma_pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float ma_round_bf16(float f) {
    return ma_bf16_to_f32(ma_f32_to_bf16(f));
}
__device__ __forceinline__ float ma_round_f16(float f) {
    return (float)(_Float16)f;
}

// load one element of a 16/32-bit float tensor as f32
__device__ __forceinline__ float ma_load_f(const void *base, int64_t off, int dtype) {
    if (dtype == MA_BF16) return ma_bf16_to_f32(((const uint16_t *)base)[off]);
    if (dtype == MA_F16) return ma_f16_to_f32(((const uint16_t *)base)[off]);
    return ((const float *)base)[off];
}
__device__ __forceinline__ void ma_store_f(void *base, int64_t off, int dtype, float v) {
    if (dtype == MA_BF16) ((uint16_t *)base)[off] = ma_f32_to_bf16(v);
    else if (dtype == MA_F16) ((_Float16 *)base)[off] = (_Float16)v;
    else ((float *)base)[off] = v;
}

// 8 consecutive elements of a float tensor, converted to bf16 (16-byte aligned for 16-bit
// dtypes when off is a multiple of 8)
__device__ __forceinline__ bf16x8_t ma_load8_as_bf16(const void *base, int64_t off, int dtype) {
    if (dtype == MA_BF16) {
        return *(const bf16x8_t *)((const uint16_t *)base + off);
    }
    bf16x8_t r;
    if (dtype == MA_F16) {
        typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
        f16x8_t h = *(const f16x8_t *)((const uint16_t *)base + off);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = (__bf16)(float)h[i];
    } else {
        const f32x4_t *p = (const f32x4_t *)((const float *)base + off);
        f32x4_t a = p[0], b = p[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r[i] = (__bf16)a[i];
            r[4 + i] = (__bf16)b[i];
        }
    }
    return r;
}

// x = f32(code) * f32(scale) + f32(zero); the product is exact, so fused or not the
// result carries one rounding -- bit-identical to the reference's two torch ops.
__device__ __forceinline__ float ma_dq(uint32_t code, float scale, float zero) {
    return __builtin_fmaf((float)code, scale, zero);
}

// ---- wave reductions (64 lanes)
__device__ __forceinline__ float ma_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float ma_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ int ma_wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Combine a lane's value with that of its partner lane l ^ 32 (v_permlane32_swap on
// gfx950 exchanges the upper half of one copy with the lower half of the other, so the
// two results hold {own, partner} in some order; max and + are symmetric, and IEEE
// addition is commutative, so both lanes of a pair get bit-identical results).
__device__ __forceinline__ float ma_max_xor32(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float ma_sum_xor32(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- DPP lane moves (GFX9 encodings): a lane reads lane i+n (row_shl) / i-n (row_shr)
// inside its 16-lane row, or lane 15 / 31 of the previous row (row_bcast); lanes whose
// source is outside the row read 0.  They go through the VALU, not the LDS crossbar that
// __shfl_* uses, so a wave scan costs a few cycles per step instead of an LDS round trip.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t ma_dpp(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xf, true);
}
enum { MA_DPP_SHL1 = 0x101, MA_DPP_SHL2 = 0x102, MA_DPP_SHL4 = 0x104, MA_DPP_SHL8 = 0x108,
       MA_DPP_SHR1 = 0x111, MA_DPP_SHR2 = 0x112, MA_DPP_SHR4 = 0x114, MA_DPP_SHR8 = 0x118,
       MA_DPP_BCAST15 = 0x142, MA_DPP_BCAST31 = 0x143 };

// inclusive prefix sum over the 64 lanes of the wave (lane i gets lanes 0..i); u32 wraps
__device__ __forceinline__ uint32_t ma_wave_prefix_u32(uint32_t x) {
    x += ma_dpp<MA_DPP_SHR1>(x);
    x += ma_dpp<MA_DPP_SHR2>(x);
    x += ma_dpp<MA_DPP_SHR4>(x);
    x += ma_dpp<MA_DPP_SHR8>(x);
    x += ma_dpp<MA_DPP_BCAST15, 0xa>(x);   // rows 1, 3 += last lane of rows 0, 2
    x += ma_dpp<MA_DPP_BCAST31, 0xc>(x);   // rows 2, 3 += lane 31
    return x;
}
// the same value in every lane: sum / max over the wave (u32)
__device__ __forceinline__ uint32_t ma_wave_sum_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_readlane((int)ma_wave_prefix_u32(x), 63);
}
__device__ __forceinline__ uint32_t ma_wave_max_u32(uint32_t x) {
    x = max(x, ma_dpp<MA_DPP_SHR1>(x));
    x = max(x, ma_dpp<MA_DPP_SHR2>(x));
    x = max(x, ma_dpp<MA_DPP_SHR4>(x));
    x = max(x, ma_dpp<MA_DPP_SHR8>(x));
    x = max(x, ma_dpp<MA_DPP_BCAST15, 0xa>(x));
    x = max(x, ma_dpp<MA_DPP_BCAST31, 0xc>(x));
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
// sum of lanes i .. i+N-1 into lane i, for lanes i that are multiples of N (N = 2, 4, 8,
// 16; groups do not cross a 16-lane row); ((x0 + x1) + (x2 + x3)) + ... order
template <int N>
__device__ __forceinline__ float ma_group_sum_first(float x) {
    if constexpr (N >= 2) x += __uint_as_float(ma_dpp<MA_DPP_SHL1>(__float_as_uint(x)));
    if constexpr (N >= 4) x += __uint_as_float(ma_dpp<MA_DPP_SHL2>(__float_as_uint(x)));
    if constexpr (N >= 8) x += __uint_as_float(ma_dpp<MA_DPP_SHL4>(__float_as_uint(x)));
    if constexpr (N >= 16) x += __uint_as_float(ma_dpp<MA_DPP_SHL8>(__float_as_uint(x)));
    return x;
}

__device__ __forceinline__ f32x16_t ma_mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The 8 nibbles of a code word (nibble i = code of element i) as bytes: even nibbles
// 0,2,4,6 in bytes 0..3 of `even`, odd nibbles 1,3,5,7 in bytes 0..3 of `odd`, so every
// code converts to float with one v_cvt_f32_ubyteN (no per-code bit-field extract; the
// compiler folds a plain shift-and-mask back into one, hence the explicit instruction).
__device__ __forceinline__ void ma_nibble_bytes(uint32_t w, uint32_t &even, uint32_t &odd) {
    even = w & 0x0f0f0f0fu;
    odd = (w >> 4) & 0x0f0f0f0fu;
}
template <int K>
__device__ __forceinline__ float ma_ubyte_f32(uint32_t x) {
    float r;
    if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
    else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
    else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
// ---- monotone float key for selection: larger float -> larger key; -0.0 == +0.0;
// NaN above +inf (torch.topk ranks NaN first)
__device__ __forceinline__ uint32_t ma_order_key(float f) {
    if (f != f) return 0xffffffffu;
    if (f == 0.0f) f = 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

#define MA_LOG2E 1.4426950408889634f

// ---- the read-set top-k's first digit (13 bits of the order key): shared by the select
// kernels and the score pass that can build this level's histogram
constexpr int MA_TOPK_D0_BITS = 13;
constexpr int MA_TOPK_H0 = 1 << MA_TOPK_D0_BITS;
constexpr int MA_TOPK_S0 = 32 - MA_TOPK_D0_BITS;
