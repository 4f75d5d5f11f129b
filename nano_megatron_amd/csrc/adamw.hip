// Fused fp32-master AdamW with global gradient-norm clipping for gfx950.
//
// Follows FlatShardZeROStrategy.clip_grad_norm + optimizer_step at DP=1
// (reference data_parallel/_zero.py:130-199):
//   norm = sqrt(sum g^2) over all parameters; coef = min(max_norm / (norm + 1e-6), 1)
//   g' = coef * g (fp32)
//   m = b1 m + (1 - b1) g';  v = b2 v + (1 - b2) g'^2
//   p = p * (1 - lr wd);  p -= (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps)
//   param = cast(p)
// The parameters are many tensors; their gradients and working copies are
// reached through device tables (pointers per tensor, element prefix sums),
// while the fp32 master / moments are flat arrays indexed by the same prefix
// sums.  The element range is cut into fixed chunks; each block owns one
// chunk, so every reduction has a fixed order (deterministic), and the clip
// coefficient stays on the device (no host synchronisation).
#include <math.h>

#include "common.h"

namespace nmb {
namespace {

constexpr int64_t kChunk = 32768;

// Index of the tensor holding flat element i: largest t with offsets[t] <= i.
__device__ __forceinline__ int find_tensor(const int64_t* __restrict__ offsets, int n, int64_t i) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// 8 consecutive elements as fp32 (16- or 32-byte aligned loads and stores).
__device__ __forceinline__ void load8(const bf16* p, float* o) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(v[e]);
}
__device__ __forceinline__ void load8(const float* p, float* o) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = a[e];
    o[4 + e] = b[e];
  }
}
__device__ __forceinline__ void store8(bf16* p, const float* v) {
  bf16x8 w;
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = static_cast<bf16>(v[e]);
  *reinterpret_cast<bf16x8*>(p) = w;
}
__device__ __forceinline__ void store8(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// The part [a, b) of segment [lo, hi) that runs 8 elements at a time: a and b
// multiples of 8 (the flat fp32 arrays are then 32-byte aligned) and the
// tensor's own pointers 16-byte aligned at a; the rest runs element by element.
template <typename T>
__device__ __forceinline__ void vector_span(const T* base, int64_t lo, int64_t hi, int64_t* a, int64_t* b) {
  int64_t va = (lo + 7) & ~int64_t{7};
  int64_t vb = hi & ~int64_t{7};
  if (vb < va || (reinterpret_cast<uintptr_t>(base + va) & 15) != 0) va = vb = hi;
  *a = va;
  *b = vb;
}

template <typename G>
__global__ __launch_bounds__(256) void sumsq_kernel(const uint64_t* __restrict__ grads,
                                                    const int64_t* __restrict__ offsets, int n,
                                                    int64_t total, float* __restrict__ partial) {
  __shared__ float sh[4];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t c1 = min(total, c0 + kChunk);
  float acc = 0.f;
  for (int t = find_tensor(offsets, n, c0); t < n && offsets[t] < c1; ++t) {
    const int64_t lo = max(c0, offsets[t]), hi = min(c1, offsets[t + 1]);
    const G* g = reinterpret_cast<const G*>(grads[t]) - offsets[t];
    int64_t a, b;
    vector_span(g, lo, hi, &a, &b);
    // four vectors per thread and iteration, loaded before any is summed (one
    // load in flight per thread left the kernel latency-bound); the sum runs
    // in the same order as one vector at a time
    int64_t i = a + 8 * threadIdx.x;
    for (; i + 3 * 8 * 256 < b; i += 4 * 8 * 256) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) load8(g + i + u * 8 * 256, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += v[u][e] * v[u][e];
    }
    for (; i < b; i += 8 * 256) {
      float v[8];
      load8(g + i, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += v[e] * v[e];
    }
    for (int64_t i = lo + threadIdx.x; i < a; i += 256) {
      const float v = to_f32(g[i]);
      acc += v * v;
    }
    for (int64_t i = b + threadIdx.x; i < hi; i += 256) {
      const float v = to_f32(g[i]);
      acc += v * v;
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// One block: norm and clip coefficient from the partial sums (fixed order).
__global__ __launch_bounds__(256) void clip_coef_kernel(const float* __restrict__ partial,
                                                        int nparts, float max_norm,
                                                        float* __restrict__ scalars) {
  __shared__ float sh[4];
  float acc = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 256) acc += partial[i];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float norm = sqrtf((sh[0] + sh[1]) + (sh[2] + sh[3]));
    float coef = 1.f;
    if (max_norm > 0.f) coef = fminf(max_norm / (norm + 1.0e-6f), 1.f);
    scalars[0] = norm;
    scalars[1] = coef;
  }
}

// fp32 scalars of the update, each formed in double on the host and rounded
// once (as torch rounds a Python float meeting an fp32 tensor)
struct AdamArgs {
  float b1, one_minus_b1, b2, one_minus_b2, decay, eps, sqrt_bc2, neg_step;
  int has_decay;
};

// The update's fp32 scalars from the reference's Python scalars
// (_zero.py:176-189), each formed in double and rounded once.
AdamArgs make_args(double lr, double beta1, double beta2, double eps, double weight_decay,
                   int64_t step) {
  const double bc1 = 1.0 - pow(beta1, static_cast<double>(step));
  const double bc2 = 1.0 - pow(beta2, static_cast<double>(step));
  AdamArgs a;
  a.b1 = static_cast<float>(beta1);
  a.one_minus_b1 = static_cast<float>(1.0 - beta1);
  a.b2 = static_cast<float>(beta2);
  a.one_minus_b2 = static_cast<float>(1.0 - beta2);
  a.has_decay = weight_decay != 0.0;
  a.decay = static_cast<float>(1.0 - lr * weight_decay);
  a.eps = static_cast<float>(eps);
  a.sqrt_bc2 = static_cast<float>(pow(bc2, 0.5));
  a.neg_step = static_cast<float>(-(lr / bc1));
  return a;
}

// One element of the update, the reference's tensor operations in their order
// (data_parallel/_zero.py:184-189), rounded as torch's kernels round them:
//   m.mul_(b1).add_(g, alpha=1-b1)       m = fma(1-b1, g, m*b1)  (add with alpha is a fused multiply-add)
//   v.mul_(b2).addcmul_(g, g, value=1-b2) v = fma((1-b2)*g, g, v*b2)  (self + value*t1*t2, last step fused)
//   w.mul_(1 - lr wd)
//   den = v.sqrt().div_(sqrt(bc2)).add_(eps)  (correctly rounded sqrt and division)
//   w.addcdiv_(m, den, value=-lr/bc1)     w = w + ((-lr/bc1)*m)/den  (self + value*t1/t2)
// Every other step is rounded on its own (no contraction).  Checked against
// the oracle, which runs these torch operations on the CPU: the moments match
// bit for bit; the master can differ by an ulp where torch's CPU square root is
// not correctly rounded.
__device__ __forceinline__ void adam_elem(float gv, float& m, float& v, float& w, const AdamArgs& a) {
  m = __builtin_fmaf(a.one_minus_b1, gv, mul_rn(m, a.b1));
  v = __builtin_fmaf(mul_rn(a.one_minus_b2, gv), gv, mul_rn(v, a.b2));
  if (a.has_decay) w = mul_rn(w, a.decay);
  // sqrtf is the correctly rounded square root (this HIP header maps
  // __fsqrt_rn to the approximate hardware one)
  const float den = add_rn(__fdiv_rn(sqrtf(v), a.sqrt_bc2), a.eps);
  w = add_rn(w, __fdiv_rn(mul_rn(a.neg_step, m), den));
}

template <typename P, typename G>
__global__ __launch_bounds__(256) void adamw_kernel(const uint64_t* __restrict__ params,
                                                    const uint64_t* __restrict__ grads,
                                                    const int64_t* __restrict__ offsets, int n,
                                                    int64_t total, float* __restrict__ master,
                                                    float* __restrict__ exp_avg,
                                                    float* __restrict__ exp_avg_sq,
                                                    const float* __restrict__ scalars,
                                                    AdamArgs a_arg,
                                                    const AdamArgs* __restrict__ a_dev) {
  // the scalars by value, or (a replayed graph) from device memory
  const AdamArgs a = a_dev != nullptr ? *a_dev : a_arg;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t c1 = min(total, c0 + kChunk);
  const float coef = scalars[1];
  for (int t = find_tensor(offsets, n, c0); t < n && offsets[t] < c1; ++t) {
    const int64_t lo = max(c0, offsets[t]), hi = min(c1, offsets[t + 1]);
    const G* g = reinterpret_cast<const G*>(grads[t]) - offsets[t];
    P* p = reinterpret_cast<P*>(params[t]) - offsets[t];
    int64_t va, vb;
    vector_span(g, lo, hi, &va, &vb);
    if ((reinterpret_cast<uintptr_t>(p + va) & 15) != 0) va = vb = hi;  // both tensors vector-aligned
    // two groups of 8 per thread and iteration, all loads before any store: a
    // wait after a store covers every outstanding load (loads and stores share
    // one counter), so one group per iteration leaves the loads idle half the
    // time.  A second group past vb re-reads the first and is not stored.
    for (int64_t i = va + 8 * threadIdx.x; i < vb; i += 16 * 256) {
      const bool two = i + 8 * 256 < vb;
      const int64_t j = two ? i + 8 * 256 : i;
      float gv[2][8], m[2][8], v[2][8], w[2][8];
      load8(g + i, gv[0]);
      load8(g + j, gv[1]);
      load8(exp_avg + i, m[0]);
      load8(exp_avg + j, m[1]);
      load8(exp_avg_sq + i, v[0]);
      load8(exp_avg_sq + j, v[1]);
      load8(master + i, w[0]);
      load8(master + j, w[1]);
      // keeps the scheduler from moving loads below the stores (it does, to
      // save registers, which brings back the shared-counter wait)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) adam_elem(mul_rn(gv[h][e], coef), m[h][e], v[h][e], w[h][e], a);
      store8(exp_avg + i, m[0]);
      store8(exp_avg_sq + i, v[0]);
      store8(master + i, w[0]);
      store8(p + i, w[0]);
      if (two) {
        store8(exp_avg + j, m[1]);
        store8(exp_avg_sq + j, v[1]);
        store8(master + j, w[1]);
        store8(p + j, w[1]);
      }
    }
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
      if (i >= va && i < vb) continue;  // done above
      float m = exp_avg[i], v = exp_avg_sq[i], w = master[i];
      adam_elem(mul_rn(to_f32(g[i]), coef), m, v, w, a);
      exp_avg[i] = m;
      exp_avg_sq[i] = v;
      master[i] = w;
      p[i] = from_f32<P>(w);
    }
  }
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_adamw_workspace_bytes(int64_t total_elements, size_t* bytes) {
  NMB_REQUIRE(bytes != nullptr && total_elements >= 0, "adamw_workspace_bytes: bad args");
  const int64_t nblocks = (total_elements + nmb::kChunk - 1) / nmb::kChunk;
  *bytes = static_cast<size_t>(nblocks + 4) * sizeof(float);
  return NMB_OK;
}

namespace nmb {
namespace {

int check_hyper(double lr, double beta1, double beta2, double eps, int64_t step) {
  NMB_REQUIRE(step >= 1, "adamw_step: step must be >= 1, got %lld", (long long)step);
  // lr 0 is a valid rate (a cosine schedule ends at min_lr, which may be 0):
  // the moments still advance and the weights stay
  NMB_REQUIRE(lr >= 0.0 && eps > 0.0 && beta1 >= 0.0 && beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0,
              "adamw_step: invalid hyper-parameters");
  return NMB_OK;
}

// sumsq, clip coefficient, update; the update's scalars are a_val, or *a_dev
// when a_dev is given
int step_impl(const uint64_t* params, const uint64_t* grads, const int64_t* offsets, int n_tensors,
              int64_t total_elements, float* master, float* exp_avg, float* exp_avg_sq,
              int param_dtype, int grad_dtype, const AdamArgs& a_val, const AdamArgs* a_dev,
              float max_norm, float* norm_out, void* workspace, size_t workspace_bytes,
              hipStream_t stream) {
  NMB_REQUIRE(params && grads && offsets && master && exp_avg && exp_avg_sq,
              "adamw_step: null argument");
  NMB_REQUIRE(n_tensors > 0 && total_elements > 0, "adamw_step: empty parameter set");
  const int64_t nblocks = (total_elements + kChunk - 1) / kChunk;
  NMB_REQUIRE(nblocks < (int64_t{1} << 30), "adamw_step: too many elements");
  const size_t need = static_cast<size_t>(nblocks + 4) * sizeof(float);
  NMB_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "adamw_step: workspace of %zu bytes is smaller than the %zu required",
              workspace_bytes, need);
  NMB_REQUIRE_SUPPORTED((param_dtype == NMB_BF16 && grad_dtype == NMB_BF16) ||
                            (param_dtype == NMB_F32 && grad_dtype == NMB_F32) ||
                            (param_dtype == NMB_BF16 && grad_dtype == NMB_F32),
                        "adamw_step: unsupported dtype pair %d/%d", param_dtype, grad_dtype);
  float* partial = static_cast<float*>(workspace);
  float* scalars = norm_out != nullptr ? norm_out : partial + nblocks;
  const unsigned grid = static_cast<unsigned>(nblocks);
  if (grad_dtype == NMB_BF16)
    hipLaunchKernelGGL(sumsq_kernel<bf16>, dim3(grid), dim3(256), 0, stream, grads, offsets,
                       n_tensors, total_elements, partial);
  else
    hipLaunchKernelGGL(sumsq_kernel<float>, dim3(grid), dim3(256), 0, stream, grads, offsets,
                       n_tensors, total_elements, partial);
  NMB_CHECK_LAUNCH("adamw_step(sumsq)");
  hipLaunchKernelGGL(clip_coef_kernel, dim3(1), dim3(256), 0, stream, partial,
                     static_cast<int>(nblocks), max_norm, scalars);
  NMB_CHECK_LAUNCH("adamw_step(clip)");
#define NMB_ADAM(P, G)                                                                        \
  hipLaunchKernelGGL((adamw_kernel<P, G>), dim3(grid), dim3(256), 0, stream, params, grads,   \
                     offsets, n_tensors, total_elements, master, exp_avg, exp_avg_sq, scalars, \
                     a_val, a_dev)
  if (param_dtype == NMB_BF16 && grad_dtype == NMB_BF16) NMB_ADAM(bf16, bf16);
  else if (param_dtype == NMB_F32) NMB_ADAM(float, float);
  else NMB_ADAM(bf16, float);
#undef NMB_ADAM
  NMB_CHECK_LAUNCH("adamw_step(update)");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_adamw_step(const uint64_t* params, const uint64_t* grads,
                              const int64_t* offsets, int n_tensors, int64_t total_elements,
                              float* master, float* exp_avg, float* exp_avg_sq, int param_dtype,
                              int grad_dtype, double lr, double beta1, double beta2, double eps,
                              double weight_decay, int64_t step, float max_norm, float* norm_out,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int st = nmb::check_hyper(lr, beta1, beta2, eps, step);
  if (st != NMB_OK) return st;
  return nmb::step_impl(params, grads, offsets, n_tensors, total_elements, master, exp_avg,
                        exp_avg_sq, param_dtype, grad_dtype,
                        nmb::make_args(lr, beta1, beta2, eps, weight_decay, step), nullptr,
                        max_norm, norm_out, workspace, workspace_bytes, stream);
}

extern "C" int nmb_adamw_hyper_bytes(size_t* bytes) {
  NMB_REQUIRE(bytes != nullptr, "adamw_hyper_bytes: null argument");
  *bytes = sizeof(nmb::AdamArgs);
  return NMB_OK;
}

extern "C" int nmb_adamw_hyper(double lr, double beta1, double beta2, double eps,
                               double weight_decay, int64_t step, void* record) {
  NMB_REQUIRE(record != nullptr, "adamw_hyper: null record");
  const int st = nmb::check_hyper(lr, beta1, beta2, eps, step);
  if (st != NMB_OK) return st;
  const nmb::AdamArgs a = nmb::make_args(lr, beta1, beta2, eps, weight_decay, step);
  __builtin_memcpy(record, &a, sizeof(a));
  return NMB_OK;
}

extern "C" int nmb_adamw_step_hyper(const uint64_t* params, const uint64_t* grads,
                                    const int64_t* offsets, int n_tensors, int64_t total_elements,
                                    float* master, float* exp_avg, float* exp_avg_sq,
                                    int param_dtype, int grad_dtype, const void* hyper,
                                    float max_norm, float* norm_out, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  NMB_REQUIRE(hyper != nullptr, "adamw_step_hyper: null hyper-parameter record");
  NMB_REQUIRE((reinterpret_cast<uintptr_t>(hyper) & 3) == 0,
              "adamw_step_hyper: the record must be 4-byte aligned");
  return nmb::step_impl(params, grads, offsets, n_tensors, total_elements, master, exp_avg,
                        exp_avg_sq, param_dtype, grad_dtype, nmb::AdamArgs{},
                        static_cast<const nmb::AdamArgs*>(hyper), max_norm, norm_out, workspace,
                        workspace_bytes, stream);
}
