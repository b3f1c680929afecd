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
};

__device__ __forceinline__ QuantGroup quant_params(float lo, float hi, int dtype) {
    float step = rnd(rnd(hi - lo, dtype) / 15.0f, dtype);
    step = rnd(fmaxf(step, 1e-8f), dtype);
    return {lo, step};
}

__device__ __forceinline__ uint32_t quant_code(float x, QuantGroup q, int dtype) {
    float r = rnd(rnd(x - q.lo, dtype) / q.step, dtype);
    float c = __builtin_rintf(r);  // half to even
    c = fminf(fmaxf(c, 0.0f), 15.0f);
    return (uint32_t)c;
}

}  // namespace
