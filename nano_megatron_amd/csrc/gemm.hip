// bf16 GEMM with fp32 accumulation for gfx950 (v_mfma_f32_16x16x32_bf16).
//
// The dense projections of the block (reference nn.Linear / F.linear at
// nn/kernels/torch_backend.py:19-20 and tensor_parallel/layers.py:214, and
// their autograd products):
//   D[M, N] = alpha * op(A)[M, K] * op(B)[K, N] + beta * C[M, N]   (row-major)
// with A stored K-contiguous ([M, K]) or M-contiguous ([K, M]) and B stored
// K-contiguous ([N, K], a weight used as W^T) or N-contiguous ([K, N]).
//
// Workgroup tile BM x BN x 64 with 4 wavefronts in a 2 x 2 arrangement; each
// wavefront owns a (BM/2) x (BN/2) block of 16 x 16 MFMA tiles whose fp32
// accumulators live in AGPRs.  Both operands are staged in LDS K-contiguous
// ([row][k], 8 elements of padding) so every MFMA fragment is one 16-byte LDS
// read; an M/N-contiguous operand is transposed on the way in (pairs of k rows
// written as 32-bit words).  LDS is double-buffered and the next K tile's
// global reads are issued before the current tile's MFMAs, one barrier per K
// tile.  Each MFMA computes a D^T tile (B fragment as the A operand), so a
// lane ends up with four consecutive columns of one output row and stores
// them as one 8-byte write.  Blocks are mapped so that consecutive tiles along
// N -- which share the A row block -- run on the same XCD.
#include "common.h"

namespace nmb {
namespace {

constexpr int BK = 64;
constexpr int LDS_K = BK + 8;  // row stride (elements) of both LDS tiles

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = static_cast<bf16>(0.f);
  return z;
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// A thread's share of one R-row x 64-k operand tile (R = BM or BN) in flight
// between global memory and LDS.
//  KC (k contiguous): item = (row, 16-byte k chunk), 8 consecutive k of a row.
//  RC (row contiguous): item = (k pair, 16-byte row chunk): rows 8c..8c+7 at
//     k and k+1, written to LDS as 32-bit (k, k+1) words.
template <int R, bool KC>
struct OperandTile {
  static constexpr int kItems = KC ? R * (BK / 8) : (BK / 2) * (R / 8);
  static constexpr int kPer = kItems / 256;
  static_assert(kItems % 256 == 0, "tile must split evenly over 256 threads");
  bf16x8 a[kPer], b[kPer];

  // src points at element (row 0, k 0) of this tile; ld is the row stride of
  // the stored matrix (elements); rows/ks give the valid extent.
  __device__ __forceinline__ void load(const bf16* __restrict__ src, int64_t ld, int rows, int ks) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i;
      if (KC) {
        const int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        a[i] = (r < rows && kc < ks) ? ld8(src + static_cast<int64_t>(r) * ld + kc) : zero8();
      } else {
        const int rc = (c % (R / 8)) * 8, kp = (c / (R / 8)) * 2;
        // stored [k][row]: row chunk rc..rc+7 of k rows kp and kp+1
        a[i] = (kp < ks && rc < rows) ? ld8(src + static_cast<int64_t>(kp) * ld + rc) : zero8();
        b[i] = (kp + 1 < ks && rc < rows) ? ld8(src + static_cast<int64_t>(kp + 1) * ld + rc) : zero8();
      }
    }
  }

  __device__ __forceinline__ void store(bf16* __restrict__ dst) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i;
      if (KC) {
        const int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        *reinterpret_cast<bf16x8*>(dst + r * LDS_K + kc) = a[i];
      } else {
        const int rc = (c % (R / 8)) * 8, kp = (c / (R / 8)) * 2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          bf16 pr[2] = {a[i][e], b[i][e]};
          uint32_t w;
          __builtin_memcpy(&w, pr, 4);
          *reinterpret_cast<uint32_t*>(dst + (rc + e) * LDS_K + kp) = w;
        }
      }
    }
  }
};

struct GemmArgs {
  const bf16* a;
  const bf16* b;
  const bf16* c;
  bf16* d;
  int64_t lda, ldb, ldc, ldd;
  int M, N, K;
  float alpha, beta;
  int tiles_n, items, per_xcd;
};

template <int BM, int BN, bool A_KC, bool B_KC>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;    // 16x16 MFMA tiles per wave
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];
  // LDS: [A buffer 0][A buffer 1][B buffer 0][B buffer 1]
  auto sA = [&](int buf) { return smem + buf * (BM * LDS_K); };
  auto sB = [&](int buf) { return smem + 2 * BM * LDS_K + buf * (BN * LDS_K); };

  const int L = static_cast<int>(blockIdx.x);
  const int w = (L % 8) * g.per_xcd + L / 8;
  if (w >= g.items) return;
  const int m0 = (w / g.tiles_n) * BM;
  const int n0 = (w % g.tiles_n) * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, q4 = lane >> 4;
  const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;

  // operand tile origins: A row block m0, B row (= output column) block n0
  const bf16* a_base = A_KC ? g.a + static_cast<int64_t>(m0) * g.lda : g.a + m0;
  const bf16* b_base = B_KC ? g.b + static_cast<int64_t>(n0) * g.ldb : g.b + n0;
  const int rows_a = min(BM, g.M - m0), rows_b = min(BN, g.N - n0);
  auto a_tile = [&](int k0) {
    return A_KC ? a_base + k0 : a_base + static_cast<int64_t>(k0) * g.lda;
  };
  auto b_tile = [&](int k0) {
    return B_KC ? b_base + k0 : b_base + static_cast<int64_t>(k0) * g.ldb;
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  OperandTile<BM, A_KC> ta;
  OperandTile<BN, B_KC> tb;
  const int nk = (g.K + BK - 1) / BK;
  ta.load(a_tile(0), g.lda, rows_a, min(BK, g.K));
  tb.load(b_tile(0), g.ldb, rows_b, min(BK, g.K));
  ta.store(sA(0));
  tb.store(sB(0));
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      const int k1 = (kt + 1) * BK;
      ta.load(a_tile(k1), g.lda, rows_a, min(BK, g.K - k1));
      tb.load(b_tile(k1), g.ldb, rows_b, min(BK, g.K - k1));
    }
    const bf16* pa = sA(cur) + (wm + l16) * LDS_K + q4 * 8;
    const bf16* pb = sB(cur) + (wn + l16) * LDS_K + q4 * 8;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = ld8(pa + i * 16 * LDS_K + kk);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = ld8(pb + j * 16 * LDS_K + kk);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(fb[j], fa[i], acc[i][j]);
    }
    if (kt + 1 < nk) {
      ta.store(sA(cur ^ 1));
      tb.store(sB(cur ^ 1));
    }
    __syncthreads();
  }

  // acc[i][j][e] = D[m0 + wm + 16 i + l16][n0 + wn + 16 j + 4 q4 + e]
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm + 16 * i + l16;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn + 16 * j + 4 * q4;
      if (n >= g.N) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = g.alpha * acc[i][j][e];
      if (g.beta != 0.f) {
        const bf16* cp = g.c + static_cast<int64_t>(m) * g.ldc + n;
        if (n + 4 <= g.N) {
          const bf16x4 cv = *reinterpret_cast<const bf16x4*>(cp);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += g.beta * static_cast<float>(cv[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < g.N) v[e] += g.beta * static_cast<float>(cp[e]);
        }
      }
      bf16* dp = g.d + static_cast<int64_t>(m) * g.ldd + n;
      if (n + 4 <= g.N) {
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = static_cast<bf16>(v[e]);
        *reinterpret_cast<bf16x4*>(dp) = ov;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < g.N) dp[e] = static_cast<bf16>(v[e]);
      }
    }
  }
}

template <int BM, int BN, bool A_KC, bool B_KC>
int launch(GemmArgs g, hipStream_t stream) {
  const int tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  const int64_t items = static_cast<int64_t>(tiles_m) * g.tiles_n;
  NMB_REQUIRE(items < (int64_t{1} << 30), "gemm: too many tiles");
  g.items = static_cast<int>(items);
  g.per_xcd = static_cast<int>((items + 7) / 8);
  const size_t lds = static_cast<size_t>(2 * (BM + BN) * LDS_K) * sizeof(bf16);
  static bool configured = false;  // raise the dynamic-LDS limit once per instantiation
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, A_KC, B_KC>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) {
      set_error("gemm: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
      return NMB_EHIP;
    }
    configured = true;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, A_KC, B_KC>), dim3(static_cast<unsigned>(g.per_xcd * 8)),
                     dim3(256), lds, stream, g);
  NMB_CHECK_LAUNCH("gemm");
  return NMB_OK;
}

template <int BM, int BN>
int dispatch_layout(bool a_kc, bool b_kc, const GemmArgs& g, hipStream_t s) {
  if (a_kc && b_kc) return launch<BM, BN, true, true>(g, s);
  if (a_kc && !b_kc) return launch<BM, BN, true, false>(g, s);
  if (!a_kc && b_kc) return launch<BM, BN, false, true>(g, s);
  return launch<BM, BN, false, false>(g, s);
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_gemm_bf16(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k,
                             float alpha, const void* a, int64_t lda, const void* b, int64_t ldb,
                             float beta, const void* c, int64_t ldc, void* d, int64_t ldd,
                             hipStream_t stream) {
  NMB_REQUIRE(a != nullptr && b != nullptr && d != nullptr, "gemm: null operand");
  NMB_REQUIRE(a_layout == 0 || a_layout == 1, "gemm: a_layout must be 0 ([M,K]) or 1 ([K,M])");
  NMB_REQUIRE(b_layout == 0 || b_layout == 1, "gemm: b_layout must be 0 ([N,K]) or 1 ([K,N])");
  NMB_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
              "gemm: invalid shape %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  NMB_REQUIRE(beta == 0.f || c != nullptr, "gemm: beta != 0 needs C");
  const bool a_kc = a_layout == 0, b_kc = b_layout == 0;
  // 16-byte operand reads: the contiguous dimension and the leading dimensions
  // must be multiples of 8 elements, pointers 16-byte aligned
  NMB_REQUIRE_SUPPORTED((a_kc ? k : m) % 8 == 0 && (b_kc ? k : n) % 8 == 0 && lda % 8 == 0 &&
                            ldb % 8 == 0,
                        "gemm: contiguous extents and leading dimensions must be multiples of 8");
  NMB_REQUIRE(nmb::aligned16(a) && nmb::aligned16(b), "gemm: A and B must be 16-byte aligned");
  NMB_REQUIRE(lda >= (a_kc ? k : m) && ldb >= (b_kc ? k : n) && ldd >= n && (beta == 0.f || ldc >= n),
              "gemm: leading dimension too small");
  NMB_REQUIRE(ldd % 4 == 0 && (beta == 0.f || ldc % 4 == 0) &&
                  (reinterpret_cast<uintptr_t>(d) & 7) == 0 &&
                  (beta == 0.f || (reinterpret_cast<uintptr_t>(c) & 7) == 0),
              "gemm: C/D rows must be 8-byte aligned");
  if (m == 0 || n == 0) return NMB_OK;
  nmb::GemmArgs g{};
  g.a = static_cast<const nmb::bf16*>(a);
  g.b = static_cast<const nmb::bf16*>(b);
  g.c = static_cast<const nmb::bf16*>(c);
  g.d = static_cast<nmb::bf16*>(d);
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.ldd = ldd;
  g.M = static_cast<int>(m);
  g.N = static_cast<int>(n);
  g.K = static_cast<int>(k);
  g.alpha = alpha;
  g.beta = beta;
  return nmb::dispatch_layout<256, 256>(a_kc, b_kc, g, stream);
}
