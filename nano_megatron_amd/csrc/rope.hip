// Rotary position embedding for gfx950.
//
// Follows RotaryEmbedding.forward / apply_rotary_pos_emb (reference
// nn/rotary.py:27-38, 52, 55-70): inv_freq = 1/theta^(2i/D) (fp32, computed
// by the host), f = pos * inv_freq, emb = cat(f, f), cos/sin rounded to the
// activation dtype, and
//   out = x * cos + rotate_half(x) * sin,   rotate_half(x) = cat(-x2, x1)
// with a rounding after each multiply and after the add (three tensor ops in
// the reference).  The backward is the same map with sin negated (rotation by
// -theta), since rotate_half^T = -rotate_half.
//
// One thread owns V consecutive pairs (i, i + D/2) of one (b, s, h) row, so
// the operation can run in place.  The cos/sin table is fp32 [n_pos, D/2]
// and stays in L2.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ cos_t,
                                                         float* __restrict__ sin_t,
                                                         const float* __restrict__ inv_freq,
                                                         int64_t n_pos, int64_t half) {
  const int64_t total = n_pos * half;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t p = i / half;
    const int64_t j = i - p * half;
    const float f = mul_rn(static_cast<float>(p), inv_freq[j]);
    cos_t[i] = cosf(f);
    sin_t[i] = sinf(f);
  }
}

struct RopeArgs {
  int64_t seq, heads, half, n_pos;
  int64_t xs_b, xs_s, xs_h, os_b, os_s, os_h;
  int64_t pos_bstride, pos_offset;
  int64_t total;  // rows * vecs_per_row
  int vecs_per_row;
  float sin_sign;
};

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t,
                                                   const int32_t* __restrict__ positions,
                                                   RopeArgs a) {
  constexpr int V = VecTraits<T>::N;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < a.total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = gid / a.vecs_per_row;
    const int i0 = static_cast<int>(gid - row * a.vecs_per_row) * V;
    const int64_t h = row % a.heads;
    const int64_t bs = row / a.heads;
    const int64_t s = bs % a.seq;
    const int64_t b = bs / a.seq;
    int64_t pos = positions != nullptr ? static_cast<int64_t>(positions[b * a.pos_bstride + s])
                                       : a.pos_offset + s;
    // An out-of-table position is a caller error; read a valid row and poison
    // the result rather than touch memory outside the table.
    const bool bad = pos < 0 || pos >= a.n_pos;
    if (bad) pos = 0;
    const T* xr = x + b * a.xs_b + s * a.xs_s + h * a.xs_h;
    T* orow = out + b * a.os_b + s * a.os_s + h * a.os_h;
    float x1[V], x2[V];
    load_vec<T>(xr + i0, x1);
    load_vec<T>(xr + a.half + i0, x2);
    const float* cr = cos_t + pos * a.half + i0;
    const float* sr = sin_t + pos * a.half + i0;
    float o1[V], o2[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float c = round_as<T>(cr[i]);
      const float sn = round_as<T>(sr[i]) * a.sin_sign;
      // first half:  x1*c + (-x2)*s ; second half: x2*c + x1*s
      o1[i] = round_as<T>(add_rn(round_as<T>(mul_rn(x1[i], c)), round_as<T>(mul_rn(-x2[i], sn))));
      o2[i] = round_as<T>(add_rn(round_as<T>(mul_rn(x2[i], c)), round_as<T>(mul_rn(x1[i], sn))));
      if (bad) o1[i] = o2[i] = __builtin_nanf("");
    }
    store_vec<T>(orow + i0, o1);
    store_vec<T>(orow + a.half + i0, o2);
  }
}

template <typename T>
int apply_impl(const void* x, void* out, const float* cos_t, const float* sin_t, int64_t n_pos,
               const int32_t* positions, int64_t pos_bstride, int64_t pos_offset, int64_t batch,
               int64_t seq, int64_t heads, int64_t head_dim, const int64_t* xs,
               const int64_t* os, int inverse, hipStream_t stream) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE(x != nullptr && out != nullptr && cos_t != nullptr && sin_t != nullptr &&
                  xs != nullptr && os != nullptr,
              "rope_apply: null argument");
  NMB_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0 && n_pos > 0, "rope_apply: invalid shape");
  NMB_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "RoPE head_dim must be even, got %lld",
              (long long)head_dim);
  const int64_t half = head_dim / 2;
  NMB_REQUIRE_SUPPORTED(half % V == 0, "rope_apply: head_dim/2 (%lld) must be a multiple of %d",
                        (long long)half, V);
  for (int i = 0; i < 3; ++i) {
    NMB_REQUIRE_SUPPORTED(xs[i] % V == 0 && os[i] % V == 0,
                          "rope_apply: strides must be multiples of %d elements", V);
  }
  NMB_REQUIRE(aligned16(x) && aligned16(out) && aligned16(cos_t) && aligned16(sin_t),
              "rope_apply: tensors must be 16-byte aligned");
  if (positions == nullptr) {
    NMB_REQUIRE(pos_offset >= 0 && pos_offset + seq <= n_pos,
                "rope_apply: positions [%lld, %lld) exceed the cos/sin table of %lld rows",
                (long long)pos_offset, (long long)(pos_offset + seq), (long long)n_pos);
  }
  RopeArgs a;
  a.seq = seq;
  a.heads = heads;
  a.half = half;
  a.n_pos = n_pos;
  a.xs_b = xs[0];
  a.xs_s = xs[1];
  a.xs_h = xs[2];
  a.os_b = os[0];
  a.os_s = os[1];
  a.os_h = os[2];
  a.pos_bstride = pos_bstride;
  a.pos_offset = pos_offset;
  a.vecs_per_row = static_cast<int>(half / V);
  a.total = batch * seq * heads * a.vecs_per_row;
  a.sin_sign = inverse ? -1.f : 1.f;
  if (a.total == 0) return NMB_OK;
  int64_t blocks = (a.total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((rope_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<const T*>(x), static_cast<T*>(out), cos_t, sin_t, positions, a);
  NMB_CHECK_LAUNCH("rope_apply");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_rope_table(float* cos_table, float* sin_table, const float* inv_freq,
                              int64_t n_pos, int64_t half, hipStream_t stream) {
  NMB_REQUIRE(cos_table != nullptr && sin_table != nullptr && inv_freq != nullptr,
              "rope_table: null argument");
  NMB_REQUIRE(n_pos > 0 && half > 0, "rope_table: invalid shape");
  int64_t blocks = (n_pos * half + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(nmb::rope_table_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, cos_table, sin_table, inv_freq, n_pos, half);
  NMB_CHECK_LAUNCH("rope_table");
  return NMB_OK;
}

extern "C" int nmb_rope_apply(const void* x, void* out, const float* cos_table,
                              const float* sin_table, int64_t n_pos, const int32_t* positions,
                              int64_t pos_batch_stride, int64_t pos_offset, int64_t batch,
                              int64_t seq, int64_t heads, int64_t head_dim,
                              const int64_t* x_strides, const int64_t* out_strides, int inverse,
                              int dtype, hipStream_t stream) {
  if (dtype == NMB_BF16)
    return nmb::apply_impl<nmb::bf16>(x, out, cos_table, sin_table, n_pos, positions,
                                      pos_batch_stride, pos_offset, batch, seq, heads, head_dim,
                                      x_strides, out_strides, inverse, stream);
  if (dtype == NMB_F32)
    return nmb::apply_impl<float>(x, out, cos_table, sin_table, n_pos, positions,
                                  pos_batch_stride, pos_offset, batch, seq, heads, head_dim,
                                  x_strides, out_strides, inverse, stream);
  NMB_REQUIRE_SUPPORTED(false, "rope_apply: unsupported dtype code %d", dtype);
}
