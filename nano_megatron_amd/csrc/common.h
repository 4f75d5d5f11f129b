// Shared helpers for the nano_megatron_amd gfx950 kernels.
//
// Conventions of the C ABI (include/nmb.h):
//   * every entry point returns an int status (NMB_OK, NMB_EINVAL, NMB_EUNSUPPORTED,
//     NMB_EHIP) and never throws across the boundary;
//   * the message of the last failure on the calling thread is kept in a
//     thread-local buffer read by nmb_last_error();
//   * tensors are raw device pointers owned by the caller; the library allocates
//     no device memory (scratch is a caller-provided workspace);
//   * work is enqueued on the caller's hipStream_t and nothing synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/nmb.h"

namespace nmb {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Round-to-nearest-even conversions (clang lowers float->__bf16 to the
// hardware RNE convert on gfx950; NaN stays NaN).
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// Round a float through the storage type T and back (identity for fp32).
template <typename T> __device__ __forceinline__ float round_as(float x) {
  return to_f32(from_f32<T>(x));
}

// Products and sums without FMA contraction, so fp32 results reproduce the
// separately rounded tensor ops of the reference.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace nmb

#define NMB_REQUIRE(cond, ...)              \
  do {                                      \
    if (!(cond)) {                          \
      ::nmb::set_error(__VA_ARGS__);        \
      return NMB_EINVAL;                    \
    }                                       \
  } while (0)

#define NMB_REQUIRE_SUPPORTED(cond, ...)    \
  do {                                      \
    if (!(cond)) {                          \
      ::nmb::set_error(__VA_ARGS__);        \
      return NMB_EUNSUPPORTED;              \
    }                                       \
  } while (0)

// Check the launch that was just enqueued.
#define NMB_CHECK_LAUNCH(what)                                                    \
  do {                                                                            \
    hipError_t _e = hipGetLastError();                                            \
    if (_e != hipSuccess) {                                                       \
      ::nmb::set_error("%s: kernel launch failed: %s", what, hipGetErrorString(_e)); \
      return NMB_EHIP;                                                            \
    }                                                                             \
  } while (0)
