// Activation functions of the dense layers and the edge MLPs (device side).
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace rune {

// Logistic function from the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32: about 1 ulp each), so sigmoid, tanh and SiLU cost a handful of
// instructions instead of libm's expf and an IEEE divide.  exp2 of a large
// argument gives inf and the reciprocal 0, so the tails saturate correctly.
__device__ inline float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}

__device__ inline float act_f(int a, float x) {
    if (a == RUNE_ACT_SILU) return x * sigmoid_fast(x);
    if (a == RUNE_ACT_TANH) return 2.0f * sigmoid_fast(2.0f * x) - 1.0f;
    if (a == RUNE_ACT_GELU) return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    if (a == kActSigmoid) return sigmoid_fast(x);
    return x;
}

__device__ inline float act_d(int a, float x) {
    if (a == RUNE_ACT_SILU) {
        float s = sigmoid_fast(x);
        return s * (1.0f + x * (1.0f - s));
    }
    if (a == RUNE_ACT_TANH) {
        float t = 2.0f * sigmoid_fast(2.0f * x) - 1.0f;
        return 1.0f - t * t;
    }
    if (a == RUNE_ACT_GELU)
        return 0.5f * (1.0f + erff(x * 0.70710678118654752f)) +
               x * expf(-0.5f * x * x) * 0.39894228040143268f;
    return 1.0f;
}

}  // namespace rune
