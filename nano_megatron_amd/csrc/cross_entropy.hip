// Token cross entropy over one chunk of LM-head logits, for gfx950.
//
// Follows _VocabParallelCrossEntropy at TP=1 (reference
// tensor_parallel/cross_entropy.py:30-86): logits are converted to fp32,
// loss = log(sum(exp(z - max))) - (z_t - max), ignored targets give 0; the
// backward is (softmax - onehot) * grad, cast back to the logits dtype.
//
// The host drives this per token chunk of the tied LM-head GEMM output, so the
// full [tokens, vocab] logits never exist: the forward keeps only the fp32 lse
// per token, and the backward recomputes a chunk's logits and overwrites them
// in place with the gradient.  One 256-thread workgroup owns one row; the row
// (16 KiB at vocab 8192 in bf16) is read with 16-byte accesses, once into
// registers when its length is 256, 512, 1024 or 2048 vectors.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  v = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  v = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return v;
}

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32): a few fp32 ulps, for
// x <= 0 here (logits minus their maximum or the row's lse); the loss and the
// gradients are fp32 sums and bf16 roundings of these terms, not bit-exact
// reproductions of the reference's reduction order anyway.
__device__ __forceinline__ float fexp(float x) {
  constexpr float kLog2e = 1.4426950408889634f;
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename T>
__device__ __forceinline__ void unpack(const uint4& raw, float (&out)[VecTraits<T>::N]) {
  T e[VecTraits<T>::N];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < VecTraits<T>::N; ++i) out[i] = to_f32(e[i]);
}

// VPT > 0: the row is exactly 256 x VPT vectors, read once into registers
// (all loads in flight together); VPT = 0: any row length, two passes.
template <typename T, int VPT>
__global__ __launch_bounds__(256) void ce_fwd_kernel(const T* __restrict__ logits, int64_t ld,
                                                     const int64_t* __restrict__ targets,
                                                     int64_t vocab, int64_t ignore_index,
                                                     float* __restrict__ loss,
                                                     float* __restrict__ lse) {
  constexpr int V = VecTraits<T>::N;
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* z = logits + row * ld;
  float m = -__builtin_inff();
  float s = 0.f;
  if constexpr (VPT > 0) {
    uint4 raw[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) raw[j] = ld16(z + (j * 256 + threadIdx.x) * V);
    float v[VPT][V];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      unpack<T>(raw[j], v[j]);
#pragma unroll
      for (int k = 0; k < V; ++k) m = fmaxf(m, v[j][k]);
    }
    m = block_max(m, sh);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
      for (int k = 0; k < V; ++k) s += fexp(v[j][k] - m);
  } else {
    for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
      float v[V];
      load_vec<T>(z + c, v);
#pragma unroll
      for (int k = 0; k < V; ++k) m = fmaxf(m, v[k]);
    }
    m = block_max(m, sh);
    for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
      float v[V];
      load_vec<T>(z + c, v);
#pragma unroll
      for (int k = 0; k < V; ++k) s += fexp(v[k] - m);
    }
  }
  s = block_sum(s, sh);
  if (threadIdx.x == 0) {
    const int64_t t = targets[row];
    const float log_s = logf(s);
    lse[row] = m + log_s;
    if (t == ignore_index) {
      loss[row] = 0.f;
    } else if (t < 0 || t >= vocab) {
      loss[row] = __builtin_nanf("");  // host validates; poison instead of reading out of range
    } else {
      loss[row] = log_s - (to_f32(z[t]) - m);
    }
  }
}

// in place: z <- (softmax(z) - onehot(t)) * grad, or 0 for an ignored row
template <typename T, int VPT>
__global__ __launch_bounds__(256) void ce_bwd_kernel(T* __restrict__ logits, int64_t ld,
                                                     const int64_t* __restrict__ targets,
                                                     int64_t vocab, int64_t ignore_index,
                                                     const float* __restrict__ lse,
                                                     const float* __restrict__ grad) {
  constexpr int V = VecTraits<T>::N;
  const int64_t row = blockIdx.x;
  T* z = logits + row * ld;
  const int64_t t = targets[row];
  const bool ignored = t == ignore_index;
  const float l = lse[row];
  const float gr = grad[row];
  auto grad_of = [&](float (&v)[V], int64_t c) {
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float p = fexp(v[k] - l);
      if (c + k == t) p -= 1.0f;
      v[k] = ignored ? 0.f : p * gr;
    }
  };
  if constexpr (VPT > 0) {
    uint4 raw[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) raw[j] = ld16(z + (j * 256 + threadIdx.x) * V);
    float v[VPT][V];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      unpack<T>(raw[j], v[j]);
      grad_of(v[j], static_cast<int64_t>(j * 256 + threadIdx.x) * V);
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) store_vec<T>(z + (j * 256 + threadIdx.x) * V, v[j]);
  } else {
    for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
      float v[V];
      load_vec<T>(z + c, v);
      grad_of(v, c);
      store_vec<T>(z + c, v);
    }
  }
}

// launch with VPT = vocab / (256 V) when that is 1, 2, 4 or 8, else the loop form
template <typename T, template <typename, int> class K, typename... Args>
void launch_rows(int64_t rows, int64_t vocab, hipStream_t stream, Args... args) {
  constexpr int V = VecTraits<T>::N;
  const int64_t vpt = vocab % (256 * V) == 0 ? vocab / (256 * V) : 0;
  const dim3 grid(static_cast<unsigned>(rows));
  switch (vpt) {
    case 1: hipLaunchKernelGGL((K<T, 1>::fn), grid, dim3(256), 0, stream, args...); break;
    case 2: hipLaunchKernelGGL((K<T, 2>::fn), grid, dim3(256), 0, stream, args...); break;
    case 4: hipLaunchKernelGGL((K<T, 4>::fn), grid, dim3(256), 0, stream, args...); break;
    case 8: hipLaunchKernelGGL((K<T, 8>::fn), grid, dim3(256), 0, stream, args...); break;
    default: hipLaunchKernelGGL((K<T, 0>::fn), grid, dim3(256), 0, stream, args...); break;
  }
}

template <typename T, int VPT>
struct FwdK {
  static constexpr auto fn = ce_fwd_kernel<T, VPT>;
};
template <typename T, int VPT>
struct BwdK {
  static constexpr auto fn = ce_bwd_kernel<T, VPT>;
};

template <typename T>
int check(const void* logits, int64_t ld, const int64_t* targets, int64_t rows, int64_t vocab) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE(logits != nullptr && targets != nullptr, "cross_entropy: null tensor");
  NMB_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab, "cross_entropy: invalid shape");
  NMB_REQUIRE_SUPPORTED(vocab % V == 0 && ld % V == 0,
                        "cross_entropy: vocab and row stride must be multiples of %d", V);
  NMB_REQUIRE(aligned16(logits), "cross_entropy: logits must be 16-byte aligned");
  NMB_REQUIRE(rows <= 0x7fffffff, "cross_entropy: too many rows");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t rows,
                          int64_t vocab, int64_t ignore_index, float* loss, float* lse,
                          int dtype, hipStream_t stream) {
  NMB_REQUIRE(loss != nullptr && lse != nullptr, "ce_fwd: null output");
  if (dtype == NMB_BF16) {
    int st = nmb::check<nmb::bf16>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    nmb::launch_rows<nmb::bf16, nmb::FwdK>(rows, vocab, stream, static_cast<const nmb::bf16*>(logits),
                                           ld, targets, vocab, ignore_index, loss, lse);
  } else if (dtype == NMB_F32) {
    int st = nmb::check<float>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    nmb::launch_rows<float, nmb::FwdK>(rows, vocab, stream, static_cast<const float*>(logits), ld,
                                       targets, vocab, ignore_index, loss, lse);
  } else {
    NMB_REQUIRE_SUPPORTED(false, "ce_fwd: unsupported dtype code %d", dtype);
  }
  NMB_CHECK_LAUNCH("ce_fwd");
  return NMB_OK;
}

extern "C" int nmb_ce_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t rows,
                          int64_t vocab, int64_t ignore_index, const float* lse,
                          const float* grad, int dtype, hipStream_t stream) {
  NMB_REQUIRE(lse != nullptr && grad != nullptr, "ce_bwd: null input");
  if (dtype == NMB_BF16) {
    int st = nmb::check<nmb::bf16>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    nmb::launch_rows<nmb::bf16, nmb::BwdK>(rows, vocab, stream, static_cast<nmb::bf16*>(logits), ld,
                                           targets, vocab, ignore_index, lse, grad);
  } else if (dtype == NMB_F32) {
    int st = nmb::check<float>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    nmb::launch_rows<float, nmb::BwdK>(rows, vocab, stream, static_cast<float*>(logits), ld, targets,
                                       vocab, ignore_index, lse, grad);
  } else {
    NMB_REQUIRE_SUPPORTED(false, "ce_bwd: unsupported dtype code %d", dtype);
  }
  NMB_CHECK_LAUNCH("ce_bwd");
  return NMB_OK;
}
