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

// n / d for n < 2^31 by a precomputed multiplier (round-up method of
// Granlund and Montgomery): s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  while ((uint64_t{1} << f.s) < d) ++f.s;
  f.m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << f.s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

// Products and sums without FMA contraction, so fp32 results reproduce the
// separately rounded tensor ops of the reference.  __fmul_rn / __fadd_rn are
// plain operators in this HIP header, which HIP's default -ffp-contract fuses
// (add_rn(c, mul_rn(a, b)) became one v_fmac); the pragma keeps each
// operation rounded on its own.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// Cross-lane exchanges without an LDS round trip (ds_bpermute costs a full LDS
// latency per step).  v_permlane32_swap a, b swaps the upper 32 lanes of a
// with the lower 32 lanes of b, so with a = b = v it leaves a = [v_lo, v_lo]
// and b = [v_hi, v_hi]; v_permlane16_swap does the same for the odd 16-lane
// rows of a and the even rows of b.  Written as inline asm: this compiler
// folds the builtin's second result into the first when both operands are the
// same value.  The s_nops give the VALU-to-permlane distances.
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// v + v of lane l ^ 16 (resp. l ^ 32), and the max of the two, in every lane
__device__ __forceinline__ float xor16_sum(float v) { float a = v, b = v; permlane16_swap(a, b); return a + b; }
__device__ __forceinline__ float xor32_sum(float v) { float a = v, b = v; permlane32_swap(a, b); return a + b; }
__device__ __forceinline__ float xor16_max(float v) { float a = v, b = v; permlane16_swap(a, b); return fmaxf(a, b); }
__device__ __forceinline__ float xor32_max(float v) { float a = v, b = v; permlane32_swap(a, b); return fmaxf(a, b); }

// DPP source of lane l within its 16-lane row: quad_perm [1,0,3,2] (l ^ 1),
// quad_perm [2,3,0,1] (l ^ 2), row_half_mirror (7 - l within 8), row_mirror
// (15 - l within 16)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, the same bits in every lane (each step adds two
// values that every lane of a group sees in some order, and IEEE addition is
// commutative): pairs, quads, half rows, rows by DPP; then rows by permlane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return xor32_sum(xor16_sum(v));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return xor32_max(xor16_max(v));
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
