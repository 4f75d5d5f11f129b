// SwiGLU forward and fused recompute-backward for gfx950.
//
// Follows GPTMLP.forward's `F.silu(gate) * up` (reference models/gpt/mlp.py:77)
// with the reference's rounding points: s = cast(silu(gate)) computed in fp32,
// out = cast(s * up).  The backward is the autograd of that expression:
//   d_up = cast(d_out * s);  ds = cast(d_out * up);
//   d_gate = cast(ds * sigmoid(g) * (1 + g * (1 - sigmoid(g))))
// and it re-emits `out` for the down-projection weight gradient, so the
// forward never has to keep it.  Pure HBM streaming with 16-byte accesses.
// d_gate uses the fast sigmoid below (a few fp32 ulps before its bf16
// rounding); the activation itself rounds exactly as the exact formula does.
#include "common.h"
#include "swiglu_math.h"
#include "vec.h"

namespace nmb {
namespace {

struct SwigluArgs {
  int64_t g_ld, u_ld, d_ld, dg_ld, du_ld, o_ld;
  int64_t rows, cols, vec_cols, total;
};

// Launch shape (both kernels): wavefront w takes kVec x 64 consecutive 16-byte
// vectors of the flattened [rows, cols / V] index space (one coalesced
// 1 KB access per k, split only where a row ends), every load issued before
// any is used; the row of a vector index comes from a multiply-high division.
// Indices past the end re-read the last vector and are not stored.
constexpr int kVec = 2;

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename T>
__device__ __forceinline__ void unpack(const uint4& raw, float (&out)[VecTraits<T>::N]) {
  T e[VecTraits<T>::N];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < VecTraits<T>::N; ++i) out[i] = to_f32(e[i]);
}

// row and vector column of vector slot k of this lane (clamped to the last
// vector); fd divides by the vectors per row
__device__ __forceinline__ void locate(const SwigluArgs& a, const FastDiv& fd, int k, bool& ok,
                                       int64_t& row, int64_t& vcol) {
  const uint32_t w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t i = (w * kVec + k) * 64 + (threadIdx.x & 63);
  ok = i < static_cast<uint32_t>(a.total);
  const uint32_t ic = ok ? i : static_cast<uint32_t>(a.total) - 1;
  const uint32_t r = fast_div(ic, fd);
  row = r;
  vcol = ic - r * fd.d;
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         T* __restrict__ o, SwigluArgs a,
                                                         FastDiv fd) {
  constexpr int V = VecTraits<T>::N;
  bool ok[kVec];
  int64_t row[kVec], c[kVec];
  uint4 graw[kVec], uraw[kVec];
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    locate(a, fd, k, ok[k], row[k], c[k]);
    c[k] *= V;
    graw[k] = ld16(g + row[k] * a.g_ld + c[k]);
    uraw[k] = ld16(u + row[k] * a.u_ld + c[k]);
  }
  // every vector computed before any store: a wait after a store would cover
  // every outstanding load (loads and stores share one counter)
  float ov[kVec][V];
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    float gv[V], uv[V];
    unpack<T>(graw[k], gv);
    unpack<T>(uraw[k], uv);
#pragma unroll
    for (int e = 0; e < V; ++e) ov[k][e] = swiglu_t<T>(gv[e], uv[e]);
  }
#pragma unroll
  for (int k = 0; k < kVec; ++k)
    if (ok[k]) store_vec<T>(o + row[k] * a.o_ld + c[k], ov[k]);
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         const T* __restrict__ dout,
                                                         T* __restrict__ dg, T* __restrict__ du,
                                                         T* __restrict__ o, SwigluArgs a,
                                                         FastDiv fd) {
  constexpr int V = VecTraits<T>::N;
  bool ok[kVec];
  int64_t row[kVec], c[kVec];
  uint4 graw[kVec], uraw[kVec], draw[kVec];
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    locate(a, fd, k, ok[k], row[k], c[k]);
    c[k] *= V;
    graw[k] = ld16(g + row[k] * a.g_ld + c[k]);
    uraw[k] = ld16(u + row[k] * a.u_ld + c[k]);
    draw[k] = ld16(dout + row[k] * a.d_ld + c[k]);
  }
  // every vector computed before any store (see the forward)
  float dgv[kVec][V], duv[kVec][V], ov[kVec][V];
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    float gv[V], uv[V], dv[V];
    unpack<T>(graw[k], gv);
    unpack<T>(uraw[k], uv);
    unpack<T>(draw[k], dv);
#pragma unroll
    for (int e = 0; e < V; ++e) swiglu_bwd_elem<T>(gv[e], uv[e], dv[e], dgv[k][e], duv[k][e], ov[k][e]);
  }
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    if (!ok[k]) continue;
    store_vec<T>(dg + row[k] * a.dg_ld + c[k], dgv[k]);
    store_vec<T>(du + row[k] * a.du_ld + c[k], duv[k]);
    if (o != nullptr) store_vec<T>(o + row[k] * a.o_ld + c[k], ov[k]);
  }
}

// one wavefront per kVec x 64 vectors, four per workgroup
unsigned swiglu_blocks(const SwigluArgs& a) {
  return static_cast<unsigned>((a.total + 256 * kVec - 1) / (256 * kVec));
}

template <typename T>
int launch_fwd(const void* g, int64_t g_ld, const void* u, int64_t u_ld, void* o, int64_t o_ld,
               int64_t rows, int64_t cols, hipStream_t stream) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE(g && u && o, "swiglu_fwd: null tensor");
  NMB_REQUIRE(rows >= 0 && cols > 0 && g_ld >= cols && u_ld >= cols && o_ld >= cols,
              "swiglu_fwd: invalid shape or leading dimension");
  NMB_REQUIRE_SUPPORTED(cols % V == 0 && g_ld % V == 0 && u_ld % V == 0 && o_ld % V == 0,
                        "swiglu_fwd: columns and leading dimensions must be multiples of %d", V);
  NMB_REQUIRE(aligned16(g) && aligned16(u) && aligned16(o),
              "swiglu_fwd: tensors must be 16-byte aligned");
  SwigluArgs a{};
  a.g_ld = g_ld;
  a.u_ld = u_ld;
  a.o_ld = o_ld;
  a.rows = rows;
  a.cols = cols;
  a.vec_cols = cols / V;
  a.total = rows * a.vec_cols;
  if (a.total == 0) return NMB_OK;
  NMB_REQUIRE_SUPPORTED(a.total < (int64_t{1} << 31) - 256 * kVec,
                        "swiglu_fwd: more than 2^31 vectors of %d elements", V);
  hipLaunchKernelGGL((swiglu_fwd_kernel<T>), dim3(swiglu_blocks(a)), dim3(256), 0,
                     stream, static_cast<const T*>(g), static_cast<const T*>(u),
                     static_cast<T*>(o), a, make_fastdiv(static_cast<uint32_t>(a.vec_cols)));
  NMB_CHECK_LAUNCH("swiglu_fwd");
  return NMB_OK;
}

template <typename T>
int launch_bwd(const void* g, int64_t g_ld, const void* u, int64_t u_ld, const void* d,
               int64_t d_ld, void* dg, int64_t dg_ld, void* du, int64_t du_ld, void* o,
               int64_t o_ld, int64_t rows, int64_t cols, hipStream_t stream) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE(g && u && d && dg && du, "swiglu_bwd: null tensor");
  NMB_REQUIRE(rows >= 0 && cols > 0 && g_ld >= cols && u_ld >= cols && d_ld >= cols &&
                  dg_ld >= cols && du_ld >= cols && (o == nullptr || o_ld >= cols),
              "swiglu_bwd: invalid shape or leading dimension");
  NMB_REQUIRE_SUPPORTED(cols % V == 0 && g_ld % V == 0 && u_ld % V == 0 && d_ld % V == 0 &&
                            dg_ld % V == 0 && du_ld % V == 0 && (o == nullptr || o_ld % V == 0),
                        "swiglu_bwd: columns and leading dimensions must be multiples of %d", V);
  NMB_REQUIRE(aligned16(g) && aligned16(u) && aligned16(d) && aligned16(dg) && aligned16(du) &&
                  (o == nullptr || aligned16(o)),
              "swiglu_bwd: tensors must be 16-byte aligned");
  SwigluArgs a{};
  a.g_ld = g_ld;
  a.u_ld = u_ld;
  a.d_ld = d_ld;
  a.dg_ld = dg_ld;
  a.du_ld = du_ld;
  a.o_ld = o_ld;
  a.rows = rows;
  a.cols = cols;
  a.vec_cols = cols / V;
  a.total = rows * a.vec_cols;
  if (a.total == 0) return NMB_OK;
  NMB_REQUIRE_SUPPORTED(a.total < (int64_t{1} << 31) - 256 * kVec,
                        "swiglu_bwd: more than 2^31 vectors of %d elements", V);
  hipLaunchKernelGGL((swiglu_bwd_kernel<T>), dim3(swiglu_blocks(a)), dim3(256), 0,
                     stream, static_cast<const T*>(g), static_cast<const T*>(u),
                     static_cast<const T*>(d), static_cast<T*>(dg), static_cast<T*>(du),
                     static_cast<T*>(o), a, make_fastdiv(static_cast<uint32_t>(a.vec_cols)));
  NMB_CHECK_LAUNCH("swiglu_bwd");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_swiglu_fwd(const void* gate, int64_t gate_ld, const void* up, int64_t up_ld,
                              void* out, int64_t out_ld, int64_t rows, int64_t cols, int dtype,
                              hipStream_t stream) {
  if (dtype == NMB_BF16)
    return nmb::launch_fwd<nmb::bf16>(gate, gate_ld, up, up_ld, out, out_ld, rows, cols, stream);
  if (dtype == NMB_F32)
    return nmb::launch_fwd<float>(gate, gate_ld, up, up_ld, out, out_ld, rows, cols, stream);
  NMB_REQUIRE_SUPPORTED(false, "swiglu_fwd: unsupported dtype code %d", dtype);
}

extern "C" int nmb_swiglu_bwd(const void* gate, int64_t gate_ld, const void* up, int64_t up_ld,
                              const void* dout, int64_t dout_ld, void* dgate, int64_t dgate_ld,
                              void* dup, int64_t dup_ld, void* out, int64_t out_ld, int64_t rows,
                              int64_t cols, int dtype, hipStream_t stream) {
  if (dtype == NMB_BF16)
    return nmb::launch_bwd<nmb::bf16>(gate, gate_ld, up, up_ld, dout, dout_ld, dgate, dgate_ld,
                                      dup, dup_ld, out, out_ld, rows, cols, stream);
  if (dtype == NMB_F32)
    return nmb::launch_bwd<float>(gate, gate_ld, up, up_ld, dout, dout_ld, dgate, dgate_ld, dup,
                                  dup_ld, out, out_ld, rows, cols, stream);
  NMB_REQUIRE_SUPPORTED(false, "swiglu_bwd: unsupported dtype code %d", dtype);
}
