// 4-bit quantizer arithmetic shared by the append quantizers (ma_codec.hip) and the
// eviction rebuild (ma_rebuild.hip): the reference's quantize_keys / quantize_values
// (reference.py:58-90, 182-213) evaluated as torch's CPU kernels do.
#pragma once
#include "ma_common.h"

namespace {

// Arithmetic "in the source dtype": every op computed in f32 and rounded to the source
// type, which is how torch's CPU kernels evaluate bf16/f16 tensors (reference.py:78-81).
__device__ __forceinline__ float rnd(float x, int dtype) {
    if (dtype == MA_BF16) return ma_round_bf16(x);
    if (dtype == MA_F16) return ma_round_f16(x);
    return x;
}

struct QuantGroup {
    float lo, step;
    float inv;  // RN(1 / step): the IEEE reciprocal, once per group
};

__device__ __forceinline__ QuantGroup quant_params(float lo, float hi, int dtype) {
    float step = rnd(rnd(hi - lo, dtype) / 15.0f, dtype);
    step = rnd(fmaxf(step, 1e-8f), dtype);
    return {lo, step, 1.0f / step};
}

// a / q.step rounded to f32 as the IEEE division rounds it.  For bf16 operands (a = x - lo
// rounded to bf16, step a bf16 value) the group's reciprocal and one Markstein correction
// give that quotient exactly -- checked for every pair of bf16 significands, the only
// thing the result depends on for normal operands -- in three operations instead of the
// division's ten.  An infinite a implies an infinite step (a <= hi - lo), and subnormal
// quotients map to code 0 either way, so the codes agree for every input.  Other dtypes
// divide.
__device__ __forceinline__ float quant_div(float a, QuantGroup q, int dtype) {
#pragma clang fp contract(off)
    if (dtype != MA_BF16) return a / q.step;
    const float q0 = a * q.inv;
    const float r = __builtin_fmaf(-q0, q.step, a);
    return __builtin_fmaf(r, q.inv, q0);
}

__device__ __forceinline__ uint32_t quant_code(float x, QuantGroup q, int dtype) {
    float r = rnd(quant_div(rnd(x - q.lo, dtype), q, dtype), dtype);
    float c = __builtin_rintf(r);  // half to even
    c = fminf(fmaxf(c, 0.0f), 15.0f);
    return (uint32_t)c;
}

}  // namespace
