// SwiGLU forward and fused recompute-backward for gfx950.
//
// Follows GPTMLP.forward's `F.silu(gate) * up` (reference models/gpt/mlp.py:77)
// with the reference's rounding points: s = cast(silu(gate)) computed in fp32,
// out = cast(s * up).  The backward is the autograd of that expression:
//   d_up = cast(d_out * s);  ds = cast(d_out * up);
//   d_gate = cast(ds * sigmoid(g) * (1 + g * (1 - sigmoid(g))))
// and it re-emits `out` for the down-projection weight gradient, so the
// forward never has to keep it.  Pure HBM streaming with 16-byte accesses.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

__device__ __forceinline__ float sigmoid_f(float g) { return __fdiv_rn(1.0f, 1.0f + expf(-g)); }

struct SwigluArgs {
  int64_t g_ld, u_ld, d_ld, dg_ld, du_ld, o_ld;
  int64_t rows, cols, vec_cols, total;
};

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         T* __restrict__ o, SwigluArgs a) {
  constexpr int V = VecTraits<T>::N;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / a.vec_cols;
    const int64_t c = (i - r * a.vec_cols) * V;
    float gv[V], uv[V], ov[V];
    load_vec<T>(g + r * a.g_ld + c, gv);
    load_vec<T>(u + r * a.u_ld + c, uv);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float s = round_as<T>(__fdiv_rn(gv[k], 1.0f + expf(-gv[k])));
      ov[k] = mul_rn(s, uv[k]);
    }
    store_vec<T>(o + r * a.o_ld + c, ov);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         const T* __restrict__ dout,
                                                         T* __restrict__ dg, T* __restrict__ du,
                                                         T* __restrict__ o, SwigluArgs a) {
  constexpr int V = VecTraits<T>::N;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / a.vec_cols;
    const int64_t c = (i - r * a.vec_cols) * V;
    float gv[V], uv[V], dv[V], dgv[V], duv[V], ov[V];
    load_vec<T>(g + r * a.g_ld + c, gv);
    load_vec<T>(u + r * a.u_ld + c, uv);
    load_vec<T>(dout + r * a.d_ld + c, dv);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float sig = sigmoid_f(gv[k]);
      const float s = round_as<T>(__fdiv_rn(gv[k], 1.0f + expf(-gv[k])));
      ov[k] = mul_rn(s, uv[k]);
      duv[k] = mul_rn(dv[k], s);
      const float ds = round_as<T>(mul_rn(dv[k], uv[k]));
      dgv[k] = ds * sig * (1.0f + gv[k] * (1.0f - sig));
    }
    store_vec<T>(dg + r * a.dg_ld + c, dgv);
    store_vec<T>(du + r * a.du_ld + c, duv);
    if (o != nullptr) store_vec<T>(o + r * a.o_ld + c, ov);
  }
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
  int64_t blocks = (a.total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL((swiglu_fwd_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, static_cast<const T*>(g), static_cast<const T*>(u),
                     static_cast<T*>(o), a);
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
  int64_t blocks = (a.total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL((swiglu_bwd_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, static_cast<const T*>(g), static_cast<const T*>(u),
                     static_cast<const T*>(d), static_cast<T*>(dg), static_cast<T*>(du),
                     static_cast<T*>(o), a);
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
