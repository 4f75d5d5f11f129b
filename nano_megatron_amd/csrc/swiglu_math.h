// The SwiGLU activation's fp32 math, shared by the SwiGLU kernels and the
// gate/up GEMM's fused epilogue (both must round identically).
#pragma once

#include "common.h"

namespace nmb {

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)) from the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32), against ~25 VALU instructions for expf plus an IEEE
// division, which made these kernels VALU-bound.  Relative error: the rounded
// argument t = -g log2 e contributes up to |t| ln2 fp32 ulps (2^t saturates
// to inf or 0 beyond |t| = 128), exp2, rcp and the final product a few more.
// Limits: g -> -inf: 2^+inf = inf, 1/inf = 0; g -> +inf: sigmoid 1; NaN
// propagates.
__device__ __forceinline__ float sigmoid_f(float g) {
  constexpr float kLog2e = 1.4426950408889634f;
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

// silu(g) = g sigmoid(g), rounded to T where the reference's F.silu output is
// rounded.  For bf16 the result equals that of the exact formula the reference
// evaluates in fp32 (g / (1 + exp(-g)), IEEE division, exp as this GPU's
// expf): the gate is a bf16 value wherever this runs, and over all 65,280
// finite bf16 gates the fast product rounds to the same bf16 value as the
// exact formula except at four, whose exact results (evaluated on the GPU)
// are selected here: g = 5.9375 (exact 5.92187452, just below the tie at
// 5.921875) and g = -87.5, -88, -88.5 (2^t near the top of the fp32 range,
// where the reciprocal loses the subnormal result).  The test suite repeats
// the enumeration against the exact formula.  (A branch to the exact formula
// near every bf16 tie -- within 64 fp32 ulps, ~0.2% of elements but ~12% of a
// wavefront's -- split the unrolled epilogues into one block per element and
// cost the gate/up GEMM 10%.)
template <typename T>
__device__ __forceinline__ float silu_t(float g, float sig) {
  float s = round_as<T>(mul_rn(g, sig));
  if constexpr (sizeof(T) == 2) {
    s = g == 5.9375f ? 5.90625f : s;
    s = g == -87.5f ? __uint_as_float(0x83950000u) : s;
    s = g == -88.0f ? __uint_as_float(0x83350000u) : s;
    s = g == -88.5f ? __uint_as_float(0x82DD0000u) : s;
  }
  return s;
}

// out = bf16-or-fp32 rounding of silu(g) * u (reference models/gpt/mlp.py:77:
// F.silu(gate) * up, each operation rounded to the tensor dtype)
template <typename T>
__device__ __forceinline__ float swiglu_t(float g, float u) {
  return mul_rn(silu_t<T>(g, sigmoid_f(g)), u);
}

// The backward of out = silu(g) * u for one element, given d = dL/dout
// (autograd of models/gpt/mlp.py:77): du = d * silu(g); dg = bf16(d * u) *
// sigmoid(g) (1 + g (1 - sigmoid(g))); o = silu(g) * u re-emitted for the
// down projection's weight gradient.  Shared by the SwiGLU backward kernel and
// the down projection's GEMM epilogue, which must agree bit for bit.
template <typename T>
__device__ __forceinline__ void swiglu_bwd_elem(float g, float u, float d, float& dg, float& du, float& o) {
  const float sig = sigmoid_f(g);
  const float s = silu_t<T>(g, sig);
  o = mul_rn(s, u);
  du = mul_rn(d, s);
  const float ds = round_as<T>(mul_rn(d, u));
  dg = ds * sig * (1.0f + g * (1.0f - sig));
}

}  // namespace nmb
