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
// the operation can run in place; the row comes from the thread index by
// multiply-high divisions, and both halves and both table rows are loaded
// before any is used.  The cos/sin table is fp32 [n_pos, D/2] and stays in L2.
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
  int64_t total;  // rows * vecs_per_row (< 2^31)
  int vecs_per_row;
  float sin_sign;
  FastDiv by_vecs, by_heads, by_seq;  // index divisions by vecs_per_row, heads, seq
};

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t,
                                                   const int32_t* __restrict__ positions,
                                                   RopeArgs a) {
  constexpr int V = VecTraits<T>::N;
  const uint32_t gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= static_cast<uint32_t>(a.total)) return;
  // gid = ((b seq + s) heads + h) vecs_per_row + v, by multiply-high divisions
  const uint32_t row = fast_div(gid, a.by_vecs);
  const int i0 = static_cast<int>(gid - row * a.by_vecs.d) * V;
  const uint32_t bs = fast_div(row, a.by_heads);
  const int64_t h = row - bs * a.by_heads.d;
  const uint32_t b32 = fast_div(bs, a.by_seq);
  const int64_t s = bs - b32 * a.by_seq.d, b = b32;
  const T* xr = x + b * a.xs_b + s * a.xs_s + h * a.xs_h;
  // x first (independent of the position), then the table rows
  const uint4 raw1 = *reinterpret_cast<const uint4*>(xr + i0);
  const uint4 raw2 = *reinterpret_cast<const uint4*>(xr + a.half + i0);
  int64_t pos = positions != nullptr ? static_cast<int64_t>(positions[b * a.pos_bstride + s])
                                     : a.pos_offset + s;
  // An out-of-table position is a caller error; read a valid row and poison
  // the result rather than touch memory outside the table.
  const bool bad = pos < 0 || pos >= a.n_pos;
  if (bad) pos = 0;
  float cv[V], sv[V];
#pragma unroll
  for (int k = 0; k < V; k += 4) {
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cos_t + pos * a.half + i0 + k);
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sin_t + pos * a.half + i0 + k);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cv[k + e] = c4[e];
      sv[k + e] = s4[e];
    }
  }
  T e1[V], e2[V];
  __builtin_memcpy(e1, &raw1, 16);
  __builtin_memcpy(e2, &raw2, 16);
  float o1[V], o2[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float x1 = to_f32(e1[i]), x2 = to_f32(e2[i]);
    const float c = round_as<T>(cv[i]);
    const float sn = round_as<T>(sv[i]) * a.sin_sign;
    // first half:  x1*c + (-x2)*s ; second half: x2*c + x1*s
    o1[i] = round_as<T>(add_rn(round_as<T>(mul_rn(x1, c)), round_as<T>(mul_rn(-x2, sn))));
    o2[i] = round_as<T>(add_rn(round_as<T>(mul_rn(x2, c)), round_as<T>(mul_rn(x1, sn))));
    if (bad) o1[i] = o2[i] = __builtin_nanf("");
  }
  T* orow = out + b * a.os_b + s * a.os_s + h * a.os_h;
  store_vec<T>(orow + i0, o1);
  store_vec<T>(orow + a.half + i0, o2);
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
  NMB_REQUIRE_SUPPORTED(a.total < (int64_t{1} << 31) - 256,
                        "rope_apply: more than 2^31 vectors of %d elements", V);
  a.by_vecs = make_fastdiv(static_cast<uint32_t>(a.vecs_per_row));
  a.by_heads = make_fastdiv(static_cast<uint32_t>(heads));
  a.by_seq = make_fastdiv(static_cast<uint32_t>(seq));
  const int64_t blocks = (a.total + 255) / 256;  // one vector per thread
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
