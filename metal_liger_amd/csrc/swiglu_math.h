// SwiGLU element math (ops/fused_swiglu.py:26-50), shared by the streaming
// kernels (swiglu.hip) and the fused LoRA MLP backward (lora.hip) so that
// both produce the same bits: fp32, the reference's evaluation order, one
// rounding per operation (no contraction into FMAs).
#pragma once

#include "common.h"

namespace mla {

// sigmoid(x) = 1 / (1 + e^-x) with the hardware exp2 and reciprocal
// (each ~1 ulp); saturates correctly to 0 / 1 for large |x|.
__device__ __forceinline__ float sigmoid_f(float x) {
#pragma clang fp contract(off)
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// h = silu(g) u
__device__ __forceinline__ float swiglu_fwd_elem(float g, float u) {
#pragma clang fp contract(off)
  return (g * sigmoid_f(g)) * u;
}

// dg = dy u s (1 + g (1 - s)), du = dy silu(g), s = sigmoid(g)
__device__ __forceinline__ void swiglu_bwd_elem(float g, float u, float dy, float& dg, float& du) {
#pragma clang fp contract(off)
  const float s = sigmoid_f(g);
  du = dy * (g * s);
  dg = ((dy * u) * s) * (1.0f + g * (1.0f - s));
}

// swiglu_bwd_elem, and h = silu(g) u as swiglu_fwd_elem forms it (the same
// operations on the same sigmoid, so the same bits)
__device__ __forceinline__ void swiglu_bwd_fwd_elem(float g, float u, float dy, float& dg,
                                                    float& du, float& h) {
#pragma clang fp contract(off)
  const float s = sigmoid_f(g);
  const float gs = g * s;
  h = gs * u;
  du = dy * gs;
  dg = ((dy * u) * s) * (1.0f + g * (1.0f - s));
}

}  // namespace mla
