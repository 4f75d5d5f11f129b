// fp32 GEMM on the fp32 MFMA (v_mfma_f32_16x16x4_f32) for gfx950.
//
// The dense projections of the fp32 parity configuration (reference
// nn.Linear / F.linear at nn/kernels/torch_backend.py:19-20 and
// tensor_parallel/layers.py:214, and their autograd products, in fp32):
//   D[M, N] = alpha * op(A)[M, K] * op(B)[K, N] + beta * C[M, N]   (row-major)
// with the operand layouts of nmb_gemm_bf16 (A [M, K] or [K, M]; B [N, K] or
// [K, N]).  Every product is an exact fp32 product accumulated in fp32 by the
// matrix core, so results agree with an fp32 reference GEMM to the rounding of
// the summation order.
//
// Workgroup tile 64 x 64, four wavefronts of 32 x 32 (2 x 2 MFMA tiles of
// 16 x 16), K tiles of 16 staged in LDS as [k][m] and [k][n] (one row per k,
// padded by 4 floats so the 16 lanes of a fragment read hit distinct banks).
// Operand tiles are read element-wise with bounds checks (any shape, any
// leading dimension, no alignment requirement); the configuration is a
// parity path, not a throughput one.
#include "common.h"

namespace nmb {
namespace {

constexpr int kTile = 64;
constexpr int kKT = 16;
constexpr int kPad = kTile + 4;

struct GemmF32Args {
  const float* a;
  const float* b;
  const float* c;
  float* d;
  int64_t lda, ldb, ldc, ldd;
  int M, N, K;
  float alpha, beta;
};

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A_KC: A stored [M, K] (K contiguous), else [K, M].  B_KC: B stored [N, K],
// else [K, N].
template <bool A_KC, bool B_KC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32Args g) {
  __shared__ float sA[kKT][kPad];
  __shared__ float sB[kKT][kPad];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, q = lane >> 4;
  const int m0 = static_cast<int>(blockIdx.y) * kTile;
  const int n0 = static_cast<int>(blockIdx.x) * kTile;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < g.K; k0 += kKT) {
    // 64 x 16 elements per operand tile, four per thread; the index order
    // follows the contiguous dimension so neighbouring lanes read neighbours
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + 256 * e;
      int r, k;
      if (A_KC) { r = idx / kKT; k = idx % kKT; } else { k = idx / kTile; r = idx % kTile; }
      const int m = m0 + r, kk = k0 + k;
      float v = 0.f;
      if (m < g.M && kk < g.K) v = A_KC ? g.a[static_cast<int64_t>(m) * g.lda + kk] : g.a[static_cast<int64_t>(kk) * g.lda + m];
      sA[k][r] = v;
      if (B_KC) { r = idx / kKT; k = idx % kKT; } else { k = idx / kTile; r = idx % kTile; }
      const int n = n0 + r, kb = k0 + k;
      float w = 0.f;
      if (n < g.N && kb < g.K) w = B_KC ? g.b[static_cast<int64_t>(n) * g.ldb + kb] : g.b[static_cast<int64_t>(kb) * g.ldb + n];
      sB[k][r] = w;
    }
    __syncthreads();
    // MFMA 16x16x4: lane (l16, q) supplies A[row l16][k q] and B[k q][col l16]
#pragma unroll
    for (int kk = 0; kk < kKT; kk += 4) {
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = sA[kk + q][wm + 16 * i + l16];
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = sB[kk + q][wn + 16 * j + l16];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_f32(fa[i], fb[j], acc[i][j]);
    }
    __syncthreads();
  }

  // acc[i][j][e] = D[m0 + wm + 16 i + 4 q + e][n0 + wn + 16 j + l16]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 16 * j + l16;
      if (n >= g.N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm + 16 * i + 4 * q + e;
        if (m >= g.M) continue;
        float v = g.alpha * acc[i][j][e];
        if (g.beta != 0.f) v += g.beta * g.c[static_cast<int64_t>(m) * g.ldc + n];
        g.d[static_cast<int64_t>(m) * g.ldd + n] = v;
      }
    }
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_gemm_f32(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k, float alpha,
                            const float* a, int64_t lda, const float* b, int64_t ldb, float beta,
                            const float* c, int64_t ldc, float* d, int64_t ldd, hipStream_t stream) {
  NMB_REQUIRE(a_layout == 0 || a_layout == 1, "gemm_f32: a_layout must be 0 ([M,K]) or 1 ([K,M])");
  NMB_REQUIRE(b_layout == 0 || b_layout == 1, "gemm_f32: b_layout must be 0 ([N,K]) or 1 ([K,N])");
  NMB_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
              "gemm_f32: invalid shape %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  NMB_REQUIRE(d != nullptr && (k == 0 || (a != nullptr && b != nullptr)), "gemm_f32: null operand");
  NMB_REQUIRE(beta == 0.f || c != nullptr, "gemm_f32: beta != 0 needs C");
  const bool a_kc = a_layout == 0, b_kc = b_layout == 0;
  NMB_REQUIRE(lda >= (a_kc ? k : m) && ldb >= (b_kc ? k : n) && ldd >= n && (beta == 0.f || ldc >= n),
              "gemm_f32: leading dimension too small");
  if (m == 0 || n == 0) return NMB_OK;
  const int64_t gy = (m + nmb::kTile - 1) / nmb::kTile, gx = (n + nmb::kTile - 1) / nmb::kTile;
  NMB_REQUIRE(gy <= 65535 && gx < (int64_t{1} << 31), "gemm_f32: problem too large for one launch");
  nmb::GemmF32Args g{a, b, c, d, lda, ldb, ldc, ldd, static_cast<int>(m), static_cast<int>(n),
                     static_cast<int>(k), alpha, beta};
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (a_kc && b_kc) hipLaunchKernelGGL((nmb::gemm_f32_kernel<true, true>), grid, dim3(256), 0, stream, g);
  else if (a_kc) hipLaunchKernelGGL((nmb::gemm_f32_kernel<true, false>), grid, dim3(256), 0, stream, g);
  else if (b_kc) hipLaunchKernelGGL((nmb::gemm_f32_kernel<false, true>), grid, dim3(256), 0, stream, g);
  else hipLaunchKernelGGL((nmb::gemm_f32_kernel<false, false>), grid, dim3(256), 0, stream, g);
  NMB_CHECK_LAUNCH("gemm_f32");
  return NMB_OK;
}
