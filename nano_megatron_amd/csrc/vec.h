// 16-byte vector load/store helpers: 8 bf16 or 4 fp32 per access, converted
// to/from fp32 registers.
#pragma once

#include "common.h"

namespace nmb {

template <typename T> struct VecTraits { static constexpr int N = 16 / sizeof(T); };

template <typename T>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&out)[VecTraits<T>::N]) {
  uint4 raw = *reinterpret_cast<const uint4*>(p);
  T e[VecTraits<T>::N];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < VecTraits<T>::N; ++i) out[i] = to_f32(e[i]);
}

template <typename T>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&in)[VecTraits<T>::N]) {
  T e[VecTraits<T>::N];
#pragma unroll
  for (int i = 0; i < VecTraits<T>::N; ++i) e[i] = from_f32<T>(in[i]);
  uint4 raw;
  __builtin_memcpy(&raw, e, 16);
  *reinterpret_cast<uint4*>(p) = raw;
}

}  // namespace nmb
