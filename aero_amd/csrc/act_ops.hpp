// Activation functions of the act·mul ops, shared by act.hip and the GEMV's
// fused gate/up epilogue so both compute the same values: SiLU g*sigmoid(g)
// (src/tensor.cpp:104-106,120-125), erf GELU with the Abramowitz & Stegun
// 7.1.26 erf (src/tensor.cpp:52-59,108-114), tanh-approximate GELU, identity,
// and the sigmoid of the attention output gate (src/attention_layer.cpp:
// 262-263: att * (1/(1+exp(-g))), the same product as sigmoid(g) * att).
#pragma once
#include "common.hpp"
#include "aero_hip.h"

#pragma clang fp contract(off)

namespace aero {

__device__ __forceinline__ float erf_as(float v) {
    const float s = copysignf(1.0f, v);
    const float a = fabsf(v);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t
                      - 0.284496736f) * t + 0.254829592f) * t;
    return s * (1.0f - p * expf(-a * a));
}

template <int KIND>
__device__ __forceinline__ float act(float v) {
    if constexpr (KIND == AERO_ACT_SILU) {
        return v * (1.0f / (1.0f + expf(-v)));

    } else if constexpr (KIND == AERO_ACT_GELU) {
        return 0.5f * v * (1.0f + erf_as(v * 0.7071067811865476f));
    } else if constexpr (KIND == AERO_ACT_SIGMOID) {
        return 1.0f / (1.0f + expf(-v));
    } else if constexpr (KIND == AERO_ACT_GELU_TANH) {
        return 0.5f * v *
               (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    } else {
        return v;
    }
}

}  // namespace aero
