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
// (16 KiB at vocab 8192 in bf16) is read with 16-byte accesses, the second
// pass hits the cache.
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

template <typename T>
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
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
    float v[V];
    load_vec<T>(z + c, v);
#pragma unroll
    for (int k = 0; k < V; ++k) m = fmaxf(m, v[k]);
  }
  m = block_max(m, sh);
  float s = 0.f;
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
    float v[V];
    load_vec<T>(z + c, v);
#pragma unroll
    for (int k = 0; k < V; ++k) s += expf(v[k] - m);
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

template <typename T>
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
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * V; c < vocab; c += 256 * V) {
    float v[V];
    load_vec<T>(z + c, v);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float p = expf(v[k] - l);
      if (c + k == t) p -= 1.0f;
      v[k] = ignored ? 0.f : p * gr;
    }
    store_vec<T>(z + c, v);
  }
}

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
    hipLaunchKernelGGL(nmb::ce_fwd_kernel<nmb::bf16>, dim3(static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, static_cast<const nmb::bf16*>(logits), ld, targets,
                       vocab, ignore_index, loss, lse);
  } else if (dtype == NMB_F32) {
    int st = nmb::check<float>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    hipLaunchKernelGGL(nmb::ce_fwd_kernel<float>, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                       stream, static_cast<const float*>(logits), ld, targets, vocab,
                       ignore_index, loss, lse);
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
    hipLaunchKernelGGL(nmb::ce_bwd_kernel<nmb::bf16>, dim3(static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, static_cast<nmb::bf16*>(logits), ld, targets, vocab,
                       ignore_index, lse, grad);
  } else if (dtype == NMB_F32) {
    int st = nmb::check<float>(logits, ld, targets, rows, vocab);
    if (st) return st;
    if (rows == 0) return NMB_OK;
    hipLaunchKernelGGL(nmb::ce_bwd_kernel<float>, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                       stream, static_cast<float*>(logits), ld, targets, vocab, ignore_index, lse,
                       grad);
  } else {
    NMB_REQUIRE_SUPPORTED(false, "ce_bwd: unsupported dtype code %d", dtype);
  }
  NMB_CHECK_LAUNCH("ce_bwd");
  return NMB_OK;
}
