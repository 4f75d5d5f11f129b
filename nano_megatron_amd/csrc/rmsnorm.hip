// RMSNorm forward/backward for gfx950.
//
// Follows RMSNorm.forward (reference nn/norms.py:38-41):
//   var = mean(fp32(x)^2); n = fp32(x) * rsqrt(var + eps); y = cast(n) * cast(w)
// and the gradient of that expression:
//   g = dy * w;  dx = rstd * (g - n * mean(g * n));  dw = sum_rows(dy * cast(n)).
//
// Layout: one 64-lane wavefront owns one row; each lane holds ITERS 16-byte
// vectors of the row in registers, so x is read from HBM exactly once.  The
// row statistic is a wavefront butterfly reduction.  dw is reduced
// deterministically: per-workgroup partial sums (fixed row order) into an fp32
// workspace, then a column-sum kernel with a fixed order.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

constexpr int kWaves = 4;
constexpr int kBwdBlocks = 256;

// Loads are issued unconditionally: a lane whose 16-byte vector lies past the
// row's end reads column 0 instead and drops the value at unpack time.  (A
// load under a lane condition is followed by a wait for its data where the
// branches join, which serialises a wave's loads.)
__device__ __forceinline__ int clamp_col(int it, int lane, int vec, int cols) {
  const int c = (it * 64 + lane) * vec;
  return c < cols ? c : 0;
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename T>
__device__ __forceinline__ void unpack_masked(const uint4& raw, bool keep, float (&out)[VecTraits<T>::N]) {
  T e[VecTraits<T>::N];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < VecTraits<T>::N; ++i) out[i] = keep ? to_f32(e[i]) : 0.f;
}

// 16 bytes of T from V floats (bf16: pairs through one two-wide conversion,
// v_cvt_pk_bf16_f32, straight into the register that is stored)
template <typename T>
__device__ __forceinline__ uint4 pack16(const float (&v)[VecTraits<T>::N]) {
  uint4 r;
  if constexpr (sizeof(T) == 2) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const b2 p = __builtin_convertvector(f2{v[2 * j], v[2 * j + 1]}, b2);
      __builtin_memcpy(&w[j], &p, 4);
    }
    r = uint4{w[0], w[1], w[2], w[3]};
  } else {
    __builtin_memcpy(&r, v, 16);
  }
  return r;
}

template <typename T>
__device__ __forceinline__ float inv_rms(float sum_sq, int cols, float eps) {
  const float var = __fdiv_rn(sum_sq, static_cast<float>(cols));
  // rsqrt as torch evaluates it on the CPU: a correctly rounded square root,
  // then a correctly rounded division (sqrtf is the correctly rounded one;
  // this HIP header maps __fsqrt_rn to the approximate hardware square root)
  return __fdiv_rn(1.0f, sqrtf(add_rn(var, eps)));
}

// FULL: the row is exactly ITERS vectors per lane (no column masks)
template <typename T, int ITERS, bool FULL>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ y,
                                                          float* __restrict__ rstd, int64_t rows,
                                                          int cols, float eps) {
  constexpr int V = VecTraits<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const T* xr = x + row * cols;
  // every load (x and w) is issued before any value is used
  uint4 xraw[ITERS], wraw[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int c = FULL ? (it * 64 + lane) * V : clamp_col(it, lane, V, cols);
    xraw[it] = ld16(xr + c);
    wraw[it] = ld16(w + c);
  }
  float v[ITERS][V];
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    unpack_masked<T>(xraw[it], FULL || (it * 64 + lane) * V < cols, v[it]);
#pragma unroll
    for (int i = 0; i < V; ++i) ss += v[it][i] * v[it][i];
  }
  ss = wave_sum(ss);
  const float r = inv_rms<T>(ss, cols, eps);
  // the weights are needed here (an empty asm use), so their loads stay with
  // those of x instead of being sunk into the conditional stores below
#pragma unroll
  for (int it = 0; it < ITERS; ++it) asm volatile("" ::"v"(wraw[it].x), "v"(wraw[it].y), "v"(wraw[it].z), "v"(wraw[it].w));
  T* yr = y + row * cols;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    // computed by every lane (only the store is conditional), so no load is
    // moved into the conditional block
    const int c = (it * 64 + lane) * V;
    float wv[V], o[V];
    unpack_masked<T>(wraw[it], true, wv);
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = mul_rn(round_as<T>(mul_rn(v[it][i], r)), wv[i]);
    if (FULL || c < cols) store_vec<T>(yr + c, o);
  }
  if (rstd != nullptr && lane == 0) rstd[row] = r;
}

// Backward: 8 wavefronts per workgroup; the workgroup walks its rows in groups
// of 8 x rows_per_wave, wave w taking rows w, w + 8, w + 16, ... of a group.
// A wave issues the loads of all its rows of a group (x, dy and the residual
// gradient, 8 rows' worth of 16-byte vectors per lane) before it computes any,
// so one memory latency covers several rows and a CU keeps ~200 KB of reads in
// flight.
constexpr int kBwdWaves = 8;
constexpr int rows_per_wave(int iters) { return iters <= 2 ? 4 : 1; }

// One row: dx = rstd * (g - n * mean(g * n)) (+ the residual gradient), with
// g = round(dy * w) and n = x * rstd; acc += round(dy * round(n)) (the weight
// gradient's per-row term, rounded as the reference's product tensor is).
// dx of the row goes to out (packed), not to memory: the caller stores a
// wave's rows after computing all of them.  FULL: whole tiles (the row is
// exactly ITERS vectors per lane and every block row exists), so nothing is
// masked and no branch splits the stores.
template <typename T, int ITERS, bool RES, bool FULL>
__device__ __forceinline__ void bwd_row(const uint4 (&xr)[ITERS], const uint4 (&dr)[ITERS],
                                        const uint4 (&rr)[ITERS],
                                        const float (&wv)[ITERS][VecTraits<T>::N],
                                        float (&acc)[ITERS][VecTraits<T>::N], uint4 (&out)[ITERS],
                                        int lane, int cols, float eps) {
  constexpr int V = VecTraits<T>::N;
  float xv[ITERS][V], dv[ITERS][V];
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const bool in_row = FULL || (it * 64 + lane) * V < cols;
    unpack_masked<T>(xr[it], in_row, xv[it]);
    unpack_masked<T>(dr[it], in_row, dv[it]);
#pragma unroll
    for (int i = 0; i < V; ++i) ss += xv[it][i] * xv[it][i];
  }
  ss = wave_sum(ss);
  const float r = inv_rms<T>(ss, cols, eps);
  float dot = 0.f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float n = mul_rn(xv[it][i], r);
      const float g = round_as<T>(mul_rn(dv[it][i], wv[it][i]));
      dot = add_rn(dot, mul_rn(g, n));
      acc[it][i] += round_as<T>(mul_rn(dv[it][i], round_as<T>(n)));
      xv[it][i] = n;
      dv[it][i] = g;
    }
  }
  dot = wave_sum(dot);
  const float mean_dot = __fdiv_rn(dot, static_cast<float>(cols));
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    float o[V];
    // each product and difference rounded on its own (no contraction), as
    // the reference's separate tensor operations round them
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = mul_rn(r, sub_rn(dv[it][i], mul_rn(xv[it][i], mean_dot)));
    if constexpr (RES) {
      float rv[V];
      unpack_masked<T>(rr[it], true, rv);
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] += rv[i];
    }
    out[it] = pack16<T>(o);
  }
}

template <typename T, int ITERS>
__device__ __forceinline__ void load_row(const T* __restrict__ p, float (&v)[ITERS][VecTraits<T>::N],
                                         int lane, int cols) {
  constexpr int V = VecTraits<T>::N;
  uint4 raw[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) raw[it] = ld16(p + clamp_col(it, lane, V, cols));
#pragma unroll
  for (int it = 0; it < ITERS; ++it) unpack_masked<T>(raw[it], (it * 64 + lane) * V < cols, v[it]);
}

template <typename T, int ITERS, bool RES, bool FULL>
__global__ __launch_bounds__(512) void rmsnorm_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ dy,
    const T* __restrict__ dres, T* __restrict__ dx, float* __restrict__ partial, int64_t rows,
    int cols, float eps, int64_t rows_per_block) {
  constexpr int V = VecTraits<T>::N;
  extern __shared__ float s_dw[];  // [4][cols]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float wv[ITERS][V];
  float acc[ITERS][V];
  load_row<T, ITERS>(w, wv, lane, cols);
#pragma unroll
  for (int it = 0; it < ITERS; ++it)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[it][i] = 0.f;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  constexpr int kRowsPerWave = rows_per_wave(ITERS);
  for (int64_t base = r0; base < r1; base += kBwdWaves * kRowsPerWave) {
    uint4 xr[kRowsPerWave][ITERS], dr[kRowsPerWave][ITERS], rr[kRowsPerWave][ITERS];
#pragma unroll
    for (int k = 0; k < kRowsPerWave; ++k) {
      const int64_t row = base + wave + kBwdWaves * k;
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        // rows past the block's end read row r0 (never used)
        const int64_t o = (FULL || row < r1 ? row : r0) * cols + (FULL ? (it * 64 + lane) * V : clamp_col(it, lane, V, cols));
        xr[k][it] = ld16(x + o);
        dr[k][it] = ld16(dy + o);
        rr[k][it] = RES ? ld16(dres + o) : uint4{0, 0, 0, 0};
      }
    }
    // rows are computed as their loads land (loads complete in order); the
    // stores wait until every row of the group is done, because a wait after
    // a store covers every outstanding load (loads and stores share one
    // counter and complete out of order)
    uint4 dxo[kRowsPerWave][ITERS];
#pragma unroll
    for (int k = 0; k < kRowsPerWave; ++k) {
      const int64_t row = base + wave + kBwdWaves * k;
      if (FULL || row < r1)  // wave-uniform
        bwd_row<T, ITERS, RES, FULL>(xr[k], dr[k], rr[k], wv, acc, dxo[k], lane, cols, eps);
    }
#pragma unroll
    for (int k = 0; k < kRowsPerWave; ++k) {
      const int64_t row = base + wave + kBwdWaves * k;
      if (FULL || row < r1) {  // wave-uniform
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
          const int c = (it * 64 + lane) * V;
          if (FULL || c < cols) *reinterpret_cast<uint4*>(dx + row * cols + c) = dxo[k][it];
        }
      }
    }
  }
  // fold the 8 wave partials in two rounds through 4 LDS rows (<= 64 KiB)
  const int slot = wave & 3;
  if (wave >= 4) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = (it * 64 + lane) * V;
      if (c < cols) {
#pragma unroll
        for (int i = 0; i < V; ++i) s_dw[slot * cols + c + i] = acc[it][i];
      }
    }
  }
  __syncthreads();
  if (wave < 4) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = (it * 64 + lane) * V;
      if (c < cols) {
#pragma unroll
        for (int i = 0; i < V; ++i) s_dw[slot * cols + c + i] += acc[it][i];
      }
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < cols; c += 512) {
    const float t = (s_dw[c] + s_dw[cols + c]) + (s_dw[2 * cols + c] + s_dw[3 * cols + c]);
    partial[static_cast<int64_t>(blockIdx.x) * cols + c] = t;
  }
}

// dw[c] = sum_b partial[b][c] in a fixed order.  Block: 16 row groups x 16
// columns (64-byte segments); each thread issues its (at most 16) loads
// back to back, then the row groups are combined in LDS.
template <typename T>
__global__ __launch_bounds__(256) void column_sum_kernel(const float* __restrict__ partial,
                                                         int nblocks, int cols,
                                                         T* __restrict__ out) {
  __shared__ float s[16][17];
  const int cl = threadIdx.x & 15;
  const int rg = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + cl;
  float acc = 0.f;
  if (c < cols) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int b = rg + 16 * j;
      v[j] = b < nblocks ? partial[static_cast<int64_t>(b) * cols + c] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc += v[j];
  }
  s[rg][cl] = acc;
  __syncthreads();
  if (rg == 0 && c < cols) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += s[k][cl];
    out[c] = from_f32<T>(t);
  }
}

int iters_for(int cols, int vec) { return (cols + 64 * vec - 1) / (64 * vec); }

void bwd_grid(int64_t rows, int* nblocks, int64_t* rows_per_block) {
  int64_t nb = (rows + kBwdWaves - 1) / kBwdWaves;
  if (nb > kBwdBlocks) nb = kBwdBlocks;
  if (nb < 1) nb = 1;
  int64_t rpb = (rows + nb - 1) / nb;
  rpb = (rpb + kBwdWaves - 1) / kBwdWaves * kBwdWaves;
  nb = (rows + rpb - 1) / rpb;
  if (nb < 1) nb = 1;
  *nblocks = static_cast<int>(nb);
  *rows_per_block = rpb;
}

template <typename T>
int check_common(const void* x, const void* w, int64_t rows, int64_t cols) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE(x != nullptr && w != nullptr, "rmsnorm: null tensor pointer");
  NMB_REQUIRE(rows >= 0 && cols > 0, "rmsnorm: invalid shape rows=%lld cols=%lld",
              (long long)rows, (long long)cols);
  NMB_REQUIRE_SUPPORTED(cols % V == 0, "rmsnorm: hidden size %lld must be a multiple of %d",
                        (long long)cols, V);
  NMB_REQUIRE_SUPPORTED(iters_for(static_cast<int>(cols), V) <= 8,
                        "rmsnorm: hidden size %lld exceeds the supported maximum %d",
                        (long long)cols, 8 * 64 * V);
  return NMB_OK;
}

template <typename T>
int fwd_impl(const void* x, const void* w, void* y, float* rstd, int64_t rows, int64_t cols,
             float eps, hipStream_t stream) {
  int st = check_common<T>(x, w, rows, cols);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(y != nullptr, "rmsnorm_fwd: null output");
  NMB_REQUIRE(aligned16(x) && aligned16(w) && aligned16(y),
              "rmsnorm_fwd: tensors must be 16-byte aligned");
  if (rows == 0) return NMB_OK;
  const dim3 grid(static_cast<unsigned>((rows + kWaves - 1) / kWaves));
  const int c = static_cast<int>(cols);
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* yp = static_cast<T*>(y);
  switch (iters_for(c, VecTraits<T>::N)) {
#define NMB_CASE(I)                                                                               \
  case I:                                                                                         \
    if (c == I * 64 * VecTraits<T>::N)                                                            \
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, I, true>), grid, dim3(256), 0, stream, xp, wp, yp, \
                         rstd, rows, c, eps);                                                     \
    else                                                                                          \
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, I, false>), grid, dim3(256), 0, stream, xp, wp,    \
                         yp, rstd, rows, c, eps);                                                 \
    break;
    NMB_CASE(1) NMB_CASE(2) NMB_CASE(3) NMB_CASE(4) NMB_CASE(5) NMB_CASE(6) NMB_CASE(7)
    NMB_CASE(8)
#undef NMB_CASE
  }
  NMB_CHECK_LAUNCH("rmsnorm_fwd");
  return NMB_OK;
}

template <typename T>
int bwd_rows_impl(const void* x, const void* w, const void* dy, const void* dres, void* dx, void* ws,
                  size_t ws_bytes, int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  int st = check_common<T>(x, w, rows, cols);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(dy != nullptr && dx != nullptr, "rmsnorm_bwd: null tensor");
  NMB_REQUIRE(aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx) &&
                  (dres == nullptr || aligned16(dres)),
              "rmsnorm_bwd: tensors must be 16-byte aligned");
  int nblocks;
  int64_t rpb;
  bwd_grid(rows, &nblocks, &rpb);
  const size_t need = static_cast<size_t>(nblocks) * static_cast<size_t>(cols) * sizeof(float);
  NMB_REQUIRE(nblocks <= 256, "rmsnorm_bwd: internal grid exceeds the column-sum capacity");
  NMB_REQUIRE(ws != nullptr && ws_bytes >= need,
              "rmsnorm_bwd: workspace of %zu bytes is smaller than the %zu required", ws_bytes,
              need);
  const int c = static_cast<int>(cols);
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  const T* dyp = static_cast<const T*>(dy);
  const T* drp = static_cast<const T*>(dres);
  T* dxp = static_cast<T*>(dx);
  float* part = static_cast<float*>(ws);
  const size_t lds = static_cast<size_t>(4) * cols * sizeof(float);
  switch (iters_for(c, VecTraits<T>::N)) {
#define NMB_LAUNCH(I, RES, FULL)                                                                     \
  hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, I, RES, FULL>), dim3(nblocks), dim3(512), lds, stream, xp, \
                     wp, dyp, drp, dxp, part, rows, c, eps, rpb)
#define NMB_CASE(I)                                                                              \
  case I:                                                                                        \
    if (c == I * 64 * VecTraits<T>::N && rows == nblocks * rpb &&                              \
        rpb % (kBwdWaves * rows_per_wave(I)) == 0) {                                             \
      if (drp != nullptr) NMB_LAUNCH(I, true, true); else NMB_LAUNCH(I, false, true);            \
    } else {                                                                                     \
      if (drp != nullptr) NMB_LAUNCH(I, true, false); else NMB_LAUNCH(I, false, false);          \
    }                                                                                            \
    break;
    NMB_CASE(1) NMB_CASE(2) NMB_CASE(3) NMB_CASE(4) NMB_CASE(5) NMB_CASE(6) NMB_CASE(7)
    NMB_CASE(8)
#undef NMB_CASE
#undef NMB_LAUNCH
  }
  NMB_CHECK_LAUNCH("rmsnorm_bwd");
  return NMB_OK;
}

template <typename T>
int bwd_dw_impl(const void* ws, size_t ws_bytes, int64_t rows, int64_t cols, void* dw, hipStream_t stream) {
  NMB_REQUIRE(dw != nullptr && rows >= 0 && cols > 0, "rmsnorm_bwd_dw: bad arguments");
  int nblocks;
  int64_t rpb;
  bwd_grid(rows, &nblocks, &rpb);
  const size_t need = static_cast<size_t>(nblocks) * static_cast<size_t>(cols) * sizeof(float);
  NMB_REQUIRE(ws != nullptr && ws_bytes >= need,
              "rmsnorm_bwd_dw: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  const int c = static_cast<int>(cols);
  hipLaunchKernelGGL((column_sum_kernel<T>), dim3((c + 15) / 16), dim3(256), 0, stream,
                     static_cast<const float*>(ws), nblocks, c, static_cast<T*>(dw));
  NMB_CHECK_LAUNCH("rmsnorm_bwd(dw)");
  return NMB_OK;
}

template <typename T>
int bwd_impl(const void* x, const void* w, const void* dy, const void* dres, void* dx, void* dw,
             void* ws, size_t ws_bytes, int64_t rows, int64_t cols, float eps,
             hipStream_t stream) {
  NMB_REQUIRE(dw != nullptr, "rmsnorm_bwd: null tensor");
  const int st = bwd_rows_impl<T>(x, w, dy, dres, dx, ws, ws_bytes, rows, cols, eps, stream);
  if (st != NMB_OK) return st;
  return bwd_dw_impl<T>(ws, ws_bytes, rows, cols, dw, stream);
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                               int64_t cols, float eps, int dtype, hipStream_t stream) {
  NMB_REQUIRE(eps > 0.f, "rmsnorm_fwd: eps must be positive, got %g", (double)eps);
  if (dtype == NMB_BF16) return nmb::fwd_impl<nmb::bf16>(x, w, y, rstd, rows, cols, eps, stream);
  if (dtype == NMB_F32) return nmb::fwd_impl<float>(x, w, y, rstd, rows, cols, eps, stream);
  NMB_REQUIRE_SUPPORTED(false, "rmsnorm_fwd: unsupported dtype code %d", dtype);
}

extern "C" int nmb_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, size_t* bytes) {
  NMB_REQUIRE(bytes != nullptr && rows >= 0 && cols > 0, "rmsnorm_bwd_workspace_bytes: bad args");
  int nb;
  int64_t rpb;
  nmb::bwd_grid(rows, &nb, &rpb);
  *bytes = static_cast<size_t>(nb) * static_cast<size_t>(cols) * sizeof(float);
  return NMB_OK;
}

extern "C" int nmb_rmsnorm_bwd(const void* x, const void* w, const void* dy,
                               const void* residual_grad, void* dx, void* dw, void* workspace,
                               size_t workspace_bytes, int64_t rows, int64_t cols, float eps,
                               int dtype, hipStream_t stream) {
  NMB_REQUIRE(eps > 0.f, "rmsnorm_bwd: eps must be positive, got %g", (double)eps);
  if (dtype == NMB_BF16)
    return nmb::bwd_impl<nmb::bf16>(x, w, dy, residual_grad, dx, dw, workspace, workspace_bytes,
                                    rows, cols, eps, stream);
  if (dtype == NMB_F32)
    return nmb::bwd_impl<float>(x, w, dy, residual_grad, dx, dw, workspace, workspace_bytes,
                                rows, cols, eps, stream);
  NMB_REQUIRE_SUPPORTED(false, "rmsnorm_bwd: unsupported dtype code %d", dtype);
}

extern "C" int nmb_rmsnorm_bwd_rows(const void* x, const void* w, const void* dy,
                                    const void* residual_grad, void* dx, void* workspace,
                                    size_t workspace_bytes, int64_t rows, int64_t cols, float eps,
                                    int dtype, hipStream_t stream) {
  NMB_REQUIRE(eps > 0.f, "rmsnorm_bwd: eps must be positive, got %g", (double)eps);
  if (dtype == NMB_BF16)
    return nmb::bwd_rows_impl<nmb::bf16>(x, w, dy, residual_grad, dx, workspace, workspace_bytes, rows,
                                         cols, eps, stream);
  if (dtype == NMB_F32)
    return nmb::bwd_rows_impl<float>(x, w, dy, residual_grad, dx, workspace, workspace_bytes, rows, cols,
                                     eps, stream);
  NMB_REQUIRE_SUPPORTED(false, "rmsnorm_bwd: unsupported dtype code %d", dtype);
}

extern "C" int nmb_rmsnorm_bwd_dw(const void* workspace, size_t workspace_bytes, int64_t rows,
                                  int64_t cols, void* dw, int dtype, hipStream_t stream) {
  if (dtype == NMB_BF16) return nmb::bwd_dw_impl<nmb::bf16>(workspace, workspace_bytes, rows, cols, dw, stream);
  if (dtype == NMB_F32) return nmb::bwd_dw_impl<float>(workspace, workspace_bytes, rows, cols, dw, stream);
  NMB_REQUIRE_SUPPORTED(false, "rmsnorm_bwd_dw: unsupported dtype code %d", dtype);
}
