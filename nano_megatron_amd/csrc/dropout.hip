// Dropout with an optional fused residual add, for gfx950.
//
// out = cast(residual + cast(keep(idx) ? x * scale : 0)), the rounding points of
// the reference's `residual + parallel_dropout(x, p, ...)` (models/gpt/layer.py:
// 114-137; nn/dropout.py:47-70 calls F.dropout, which rounds x * mask / (1 - p)
// to the tensor dtype before the add).  Without a residual it is the dropout
// alone, which is also its own backward: d x = dropout(d out) with the same
// seed.  keep(idx) is the counter-based mask of dropout_math.h over the
// flattened element index, so no mask is stored between forward, recompute
// and backward.  Pure HBM streaming: one 16-byte vector per lane, a SplitMix64
// evaluation per two elements.
#include <algorithm>

#include "common.h"
#include "dropout_math.h"
#include "vec.h"

namespace nmb {
namespace {

template <typename T>
__device__ __forceinline__ float dropout_elem(float x, float r, uint32_t bits, const DropoutParams& d) {
#pragma clang fp contract(off)
  const float y = round_as<T>(bits >= d.threshold ? x * d.scale : 0.f);
  return r + y;
}

// item t < nvec is vector t (V elements); item nvec + e is the scalar tail
// element nvec * V + e.  Items are walked grid-stride (the grid is capped at
// kMaxBlocks, so any n up to the entry point's limit launches).  out may alias
// x or res (each item reads its elements before it writes them), so the
// pointers are not restrict.
constexpr int64_t kMaxBlocks = 65536;

template <typename T>
__global__ __launch_bounds__(256) void dropout_add_kernel(const T* x, const T* res, T* out, int64_t nvec,
                                                          int64_t n, DropoutParams d) {
  constexpr int V = VecTraits<T>::N;
  const int64_t items = nvec + (n - nvec * V);
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < items;
       t += static_cast<int64_t>(gridDim.x) * 256) {
    if (t < nvec) {
      float xv[V], rv[V], ov[V];
      load_vec<T>(x + t * V, xv);
      if (res != nullptr) {
        load_vec<T>(res + t * V, rv);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) rv[e] = 0.f;
      }
      const uint64_t base = static_cast<uint64_t>(t) * V;  // even: element pairs share one draw
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        const uint64_t z = splitmix64(d.seed, (base + e) >> 1);
        ov[e] = dropout_elem<T>(xv[e], rv[e], static_cast<uint32_t>(z), d);
        ov[e + 1] = dropout_elem<T>(xv[e + 1], rv[e + 1], static_cast<uint32_t>(z >> 32), d);
      }
      store_vec<T>(out + t * V, ov);
    } else {
      const int64_t i = nvec * V + (t - nvec);
      const float r = res != nullptr ? to_f32(res[i]) : 0.f;
      out[i] = from_f32<T>(dropout_elem<T>(to_f32(x[i]), r, keep_bits(d.seed, static_cast<uint64_t>(i)), d));
    }
  }
}

template <typename T>
void launch(const void* x, const void* res, void* out, int64_t n, const DropoutParams& d, hipStream_t stream) {
  constexpr int V = VecTraits<T>::N;
  // the vector path needs 16-byte alignment of every operand; else all scalar
  const bool vec = aligned16(x) && aligned16(out) && (res == nullptr || aligned16(res));
  const int64_t nvec = vec ? n / V : 0;
  const int64_t threads = nvec + (n - nvec * V);
  const int64_t blocks = std::min<int64_t>((threads + 255) / 256, kMaxBlocks);
  hipLaunchKernelGGL((dropout_add_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<const T*>(x), static_cast<const T*>(res), static_cast<T*>(out), nvec, n, d);
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_dropout_add(const void* x, const void* residual, void* out, int64_t n, float p,
                               uint64_t seed, int dtype, hipStream_t stream) {
  NMB_REQUIRE_SUPPORTED(dtype == NMB_BF16 || dtype == NMB_F32, "dropout_add: unsupported dtype code %d", dtype);
  NMB_REQUIRE(n >= 0, "dropout_add: negative element count %lld", (long long)n);
  NMB_REQUIRE(p >= 0.f && p < 1.f, "dropout_add: p must be in [0, 1), got %g", static_cast<double>(p));
  if (n == 0) return NMB_OK;  // an empty tensor may have a null data pointer
  NMB_REQUIRE(x != nullptr && out != nullptr, "dropout_add: null tensor");
  NMB_REQUIRE_SUPPORTED(n < (int64_t{1} << 38), "dropout_add: more than 2^38 elements");
  const nmb::DropoutParams d = nmb::make_dropout(static_cast<double>(p), seed);
  if (dtype == NMB_BF16)
    nmb::launch<nmb::bf16>(x, residual, out, n, d, stream);
  else
    nmb::launch<float>(x, residual, out, n, d, stream);
  NMB_CHECK_LAUNCH("dropout_add");
  return NMB_OK;
}
