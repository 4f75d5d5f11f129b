// bf16 GEMM with fp32 accumulation for gfx950 (v_mfma_f32_16x16x32_bf16).
//
// The dense projections of the block (reference nn.Linear / F.linear at
// nn/kernels/torch_backend.py:19-20 and tensor_parallel/layers.py:214, and
// their autograd products):
//   D[M, N] = alpha * op(A)[M, K] * op(B)[K, N] + beta * C[M, N]   (row-major)
// with A stored K-contiguous ([M, K]) or M-contiguous ([K, M]) and B stored
// K-contiguous ([N, K], a weight used as W^T) or N-contiguous ([K, N]).
//
// Configurations (a plan per shape picks one): 256 x 256 or 256 x 128 output
// tiles of 8 wavefronts, one workgroup per CU, 64-deep K tiles; 128 x 128 or
// 128 x 256 tiles of 4 wavefronts, two workgroups per CU, 32-deep K tiles.
// Every one runs two wavefronts per SIMD: one wavefront per SIMD leaves the
// MFMA unit idle through every LDS and barrier wait, and with the compiler's
// accumulator allocation issues MFMAs at ~60% of the peak rate.
//
// Operands go from HBM straight into LDS (buffer_load ... lds, 16 bytes per
// lane, no VGPR round trip), each in the layout it has in memory:
//  * K-contiguous tile [rows][BKT k]: 2 BKT-byte rows, the 16-byte k chunk c
//    of row r stored in slot c ^ kc_swizzle(r).  An MFMA fragment (16 rows x
//    8 k per lane group) is one ds_read_b128 per lane.
//  * M/N-contiguous tile [BKT k][R]: 2R-byte k rows, the 32-byte chunk pair p
//    of k row k stored at pair slot p ^ rc_swizzle(k).  A fragment is two
//    ds_read_b64_tr_b16 per lane: in each group of 16 lanes, lane i receives
//    element i & 3 of the 8 bytes addressed by lane 4j + i/4 (j = 0..3), so
//    lanes pointing at [k + i/4][n0 + 4 (i & 3)] deliver column n0 + i,
//    k .. k + 3 -- the K-contiguous fragment without a transposing store.
// Row, column and k tails: the loads of invalid chunks get an offset past the
// buffer's num_records, which the hardware returns as zeros.
//
// LDS holds S = 2-4 K-tile stages (as many as fit the workgroup's share);
// after the barrier that publishes tile kt, the loads of tile kt + S - 1 go
// into the stage everyone has finished reading (one barrier per K tile).
// Each MFMA computes a D^T tile (B fragment as the A operand), so a lane ends
// up with four consecutive columns of one output row; the epilogues stage the
// tile through LDS and store whole rows.  Blocks are mapped so that the tiles
// an XCD (with its own L2) runs together form a 4 x 8 block of tiles.
//
// Split K (small M x N, long K -- the weight gradients): split s of a tile
// covers K range [s * kps, (s + 1) * kps) and writes fp32 partials to the
// caller's workspace; a second kernel sums the splits in a fixed order
// (deterministic) and applies alpha, beta and the bf16 rounding (or writes
// fp32, for nmb_gemm_bf16_f32out).
#include <algorithm>

#include "common.h"
#include "lds_dma.h"
#include "swiglu_math.h"

namespace nmb {
namespace {

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// 16-byte chunk slots of the K-contiguous tile.  64-deep K tiles (128-byte
// rows, 8 chunks): row r keeps chunk c in slot c ^ (r & 7).  32-deep K tiles
// (64-byte rows, 4 chunks): slot c ^ ((r >> 1) & 3).  With these a fragment
// read (16 rows x 16 bytes in each group of 16 lanes) has no LDS bank
// conflicts on gfx950 (SQ_LDS_BANK_CONFLICT reads zero; c ^ (r & 3), no
// swizzle, and ((r >> 1) & 3) ^ ((r >> 3) & 1) give two-way conflicts).
template <int BKT>
__device__ __forceinline__ int kc_swizzle(int r) {
  return BKT == 64 ? (r & 7) : ((r >> 1) & 3);
}
// 32-byte pair slots of the M/N-contiguous tile: k row k keeps pair p in slot
// p ^ rc_swizzle(k), so that the 8 k rows of a half-wave transposed read
// (k .. k + 3 and k + 8 .. k + 11) land on distinct banks.
__device__ __forceinline__ int rc_swizzle(int k) { return (k & 3) | ((k >> 1) & 4); }

// One wave's share of the loads of an R-row operand tile per BKT-deep K tile:
// R * BKT / 512 load instructions of 1 KB (64 lanes x 16 B), spread over NW
// waves.
template <int R, bool KC, int BKT, int NW>
struct Loader {
  static constexpr int kPer = R * BKT / (512 * NW);
  static constexpr int kCpr = BKT / 8;   // K-contiguous: 16-byte chunks per row
  static constexpr int kRpi = 64 / kCpr; // K-contiguous: rows per instruction
  static constexpr int kChunks = R / 8;  // M/N-contiguous: 16-byte chunks per k row
  static_assert(kPer >= 1 && R * BKT % (512 * NW) == 0, "tile must split evenly over the waves");
  static_assert(KC || R == 128 || R == 256, "M/N-contiguous tiles have 128 or 256 columns");
  i32x4 rsrc;
  uint32_t off[kPer];  // byte offset at k0 = 0, kOOB for an invalid row / column
  int kin[kPer];       // k index (within the K tile) where this lane's chunk starts
  uint32_t kstride;    // bytes per unit of k

  // base: element (row0, k 0) of the tile (K-contiguous) or (k 0, col0)
  // (M/N-contiguous); valid: rows (K-contiguous) or columns of the tile inside
  // the matrix; bytes: extent of the matrix from base.
  __device__ void init(const bf16* base, int64_t ld, int valid, uint32_t bytes, int wave, int lane) {
    rsrc = make_rsrc(base, bytes);
    kstride = KC ? 2u : static_cast<uint32_t>(2 * ld);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = wave * kPer + j;
      if (KC) {
        // instruction i fills rows kRpi i ..; lane p: row kRpi i + p / kCpr, slot p % kCpr
        const int r = kRpi * i + lane / kCpr;
        const int c = (lane % kCpr) ^ kc_swizzle<BKT>(r);
        kin[j] = 8 * c;
        off[j] = r < valid ? static_cast<uint32_t>((r * ld + 8 * c) * 2) : kOOB;
      } else {
        const int q = 64 * i + lane;
        const int kr = q / kChunks, s = q % kChunks;
        const int c = s ^ (2 * rc_swizzle(kr));  // pair swizzle keeps the chunk's low bit
        kin[j] = kr;
        off[j] = 8 * c < valid ? static_cast<uint32_t>((kr * ld + 8 * c) * 2) : kOOB;
      }
    }
  }

  // SwiGLU tiles (K-contiguous [2F, K] weights, gate rows then up rows): tile
  // row r reads gate (r & 32 clear) or up row j0 + 32 (r / 64) + r % 32, so a
  // wave's 64 columns hold 32 gate columns and the matching 32 up columns.
  __device__ void init_pairs(const bf16* base, int64_t ld, int f, int j0, uint32_t bytes, int wave,
                             int lane) {
    static_assert(KC, "paired rows need K-contiguous weights");
    rsrc = make_rsrc(base, bytes);
    kstride = 2u;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = wave * kPer + j;
      const int r = kRpi * i + lane / kCpr;
      const int c = (lane % kCpr) ^ kc_swizzle<BKT>(r);
      const int col = j0 + 32 * (r >> 6) + (r & 31);
      const int64_t row = col + ((r >> 5) & 1) * static_cast<int64_t>(f);
      kin[j] = 8 * c;
      off[j] = col < f ? static_cast<uint32_t>((row * ld + 8 * c) * 2) : kOOB;
    }
  }

  // loads K tile [k0, k0 + BKT) (zeros at and past k_end) into the LDS tile
  __device__ __forceinline__ void issue(const bf16* tile, int k0, int k_end, int wave) const {
    const uint32_t koff = static_cast<uint32_t>(k0) * kstride;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const bool ok = off[j] != kOOB && k0 + kin[j] < k_end;
      load_lds16(rsrc, tile + 512 * (wave * kPer + j), ok ? off[j] + koff : kOOB);
    }
  }
  // The same with scalar arithmetic only for a whole K tile: m0 is the LDS
  // byte address of this wave's first 1 KB of the tile (uniform) and the K
  // advance rides in the instruction's scalar offset; a partial last K tile
  // zeroes its chunks past k_end per lane.
  __device__ __forceinline__ void issue_s(uint32_t m0, int k0, int k_end) const {
    const uint32_t koff = static_cast<uint32_t>(k0) * kstride;
    if (k0 + BKT <= k_end) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) load_lds16s(rsrc, m0 + 1024u * j, off[j], koff);
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const bool ok = off[j] != kOOB && k0 + kin[j] < k_end;
        load_lds16s(rsrc, m0 + 1024u * j, ok ? off[j] : kOOB, koff);
      }
    }
  }
};

// Per-lane LDS offsets (elements) of the MFMA fragments of T 16-row groups of
// an R-row operand tile, starting at tile row row0: fragment t of k32 step kk
// gives lane l op[row0 + 16 t + l % 16][kk + 8 (l / 16) .. + 7].
template <int R, bool KC, int T, int BKT>
struct Frags {
  // K-contiguous: one offset (the swizzle depends on l % 16 only; the group
  // offset 16 t BKT is an immediate, and for kk = 32 the chunk (4 + g) ^ x is
  // (g ^ x) ^ 4).  M/N-contiguous: the two transposed reads of each fragment
  // (the swizzle does not depend on k bit 5).
  int off[KC ? 1 : 2 * T];

  __device__ void init(int row0, int lane) {
    const int l16 = lane & 15, g = lane >> 4;
    if (KC) {
      off[0] = (row0 + l16) * BKT + 8 * (g ^ kc_swizzle<BKT>(l16));
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // lane p of group g: k row 8 g + 4 h + p / 4, columns 16 pair + 4 (p & 3) .. + 3
          const int k = 8 * g + 4 * h + (l16 >> 2);
          const int pair = (row0 >> 4) + t;
          off[2 * t + h] = k * R + 16 * (pair ^ rc_swizzle(k)) + 4 * (l16 & 3);
        }
    }
  }

  __device__ __forceinline__ bf16x8 get(const bf16* tile, int t, int kk) const {
    if (KC) return ld8(tile + t * 16 * BKT + (kk ? (off[0] ^ 32) : off[0]));
    return ld_tr(tile + off[2 * t] + kk * R, tile + off[2 * t + 1] + kk * R);
  }
};

struct GemmArgs {
  const bf16* a;
  const bf16* b;
  const bf16* c;
  bf16* d;
  float* partial;  // split K: [splits][M][N] fp32
  int64_t lda, ldb, ldc, ldd;
  int M, N, K;
  float alpha, beta;
  int tiles_n, tiles, splits, kps, items, per_xcd;
  // RoPE epilogue (head dim RD > 0): the first rope_cols output columns are
  // heads of RD rotated by the position of their row
  const float* rope_cos;  // fp32 [n_pos, RD/2]
  const float* rope_sin;
  const int32_t* rope_pos;  // [batch, pos_bstride] or null: rope_offset + row % rope_seq
  int64_t rope_pos_bstride;
  int rope_offset, rope_seq, rope_n_pos, rope_cols;
  // SwiGLU epilogue: the [M, 2F] gate/up product (nullable; d nullable too)
  bf16* gu;
  int64_t ldgu;
  // SwiGLU-backward epilogue: the forward's [M, 2F] gate/up product (read)
  // and its gradient (written); D receives the re-emitted activation
  const bf16* swb_gu;
  int64_t swb_ldgu;
  bf16* swb_dgu;
  int64_t swb_lddgu;
  // fp32 output (nullable): D32 = alpha A B + beta D32, written in place of D
  // (C and D unused); unsplit plans store it from the tile, split ones from
  // the reduction
  float* d32;
  int64_t ldd32;
};

// Columns of D covered by one TBN-wide tile: TBN, or TBN / 2 with the SwiGLU
// epilogue (each output column takes a gate and an up column of the product).
template <int TBN, bool SWI>
constexpr int out_cols() { return SWI ? TBN / 2 : TBN; }

// LDS stages of a configuration (K tiles in flight + 1) within the
// workgroup's share of 160 KB.
template <int TBM, int TBN, int NW, int BKT>
struct Stages {
  static constexpr int kStageBytes = (TBM + TBN) * BKT * 2;
  static constexpr int kBudget = NW == 4 ? 80 * 1024 : 160 * 1024;
  static constexpr int S = kBudget / kStageBytes >= 4 ? 4 : kBudget / kStageBytes;
  static_assert(S >= 2, "two LDS stages at least");
};

// Byte offsets of K-tile stage st of the A and B operand tiles from sA and
// sB: consecutive stages.
template <int TBM, int TBN, int BKT>
struct LinearStages {
  __device__ static uint32_t a(int st) { return static_cast<uint32_t>(st) * (TBM * BKT * 2u); }
  __device__ static uint32_t b(int st) { return static_cast<uint32_t>(st) * (TBN * BKT * 2u); }
};

// Called at the start of every K tile, after the barrier (no-op).
struct NoHook {
  __device__ void operator()(int, int) const {}
};

__device__ __forceinline__ const bf16* at_byte(const void* base, uint32_t off) {
  return reinterpret_cast<const bf16*>(reinterpret_cast<const char*>(base) + off);
}

// The K loop of one tile: acc[i][j] += the wave's 16 x 16 MFMA tiles of
// op(A) op(B) over [k_begin, k_end), the operands streamed through the S LDS
// stages (at sA + Map::a(stage), sB + Map::b(stage)) by the loaders (the
// wave tile at rows wm, columns wn).  The first `pre` K tiles may have been
// issued by the caller already (into their stages, by the same loaders, with
// nothing issued after them); hook(kt, nk) runs at the start of each K tile,
// after the barrier.  Returns with every load of the loop complete; the other
// waves may still read the last stage.
template <int TBM, int TBN, int NW, int BKT, bool A_KC, bool B_KC, int TM, int TN,
          class Map = LinearStages<TBM, TBN, BKT>, class Hook = NoHook>
__device__ __forceinline__ void k_loop(const Loader<TBM, A_KC, BKT, NW>& la,
                                       const Loader<TBN, B_KC, BKT, NW>& lb, bf16 (*sA)[TBM * BKT],
                                       bf16 (*sB)[TBN * BKT], f32x4 (&acc)[TM][TN], int wm, int wn,
                                       int k_begin, int k_end, int wave, int lane, int pre = 0,
                                       const Hook& hook = Hook{}) {
  constexpr int KSTEPS = BKT / 32;
  constexpr int S = Stages<TBM, TBN, NW, BKT>::S;
  Frags<TBM, A_KC, TM, BKT> fra;
  Frags<TBN, B_KC, TN, BKT> frb;
  fra.init(wm, lane);
  frb.init(wn, lane);

  // S - 1 K tiles in flight.  Each K tile kt: wait until this wave's loads of
  // tile kt have landed (those of later tiles may stay in flight), barrier
  // (everyone's have; everyone is done with the stage read last iteration),
  // all fragment reads, the loads of tile kt + S - 1 into that freed stage,
  // then the MFMAs.
  constexpr int kLoads = Loader<TBM, A_KC, BKT, NW>::kPer + Loader<TBN, B_KC, BKT, NW>::kPer;
  const int nk = (k_end - k_begin + BKT - 1) / BKT;
  // scalar load issue (fewer VALU instructions in the loop): 1-4% faster on
  // the 256 x 128 and 128-row tiles, 2-4% slower on 256 x 256 (measured)
  constexpr bool kScalarIssue = !(TBM == 256 && TBN == 256);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t a_lds = lds_offset(&sA[0][0]) + 1024u * wave_u * Loader<TBM, A_KC, BKT, NW>::kPer;
  const uint32_t b_lds = lds_offset(&sB[0][0]) + 1024u * wave_u * Loader<TBN, B_KC, BKT, NW>::kPer;
  auto issue = [&](int kt) {
    const int st = kt % S;
    if constexpr (kScalarIssue) {
      la.issue_s(a_lds + Map::a(st), k_begin + kt * BKT, k_end);
      lb.issue_s(b_lds + Map::b(st), k_begin + kt * BKT, k_end);
    } else {
      la.issue(at_byte(&sA[0][0], Map::a(st)), k_begin + kt * BKT, k_end, wave);
      lb.issue(at_byte(&sB[0][0], Map::b(st)), k_begin + kt * BKT, k_end, wave);
    }
  };
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p >= pre && p < nk) issue(p);
  for (int kt = 0; kt < nk; ++kt) {
    // tiles issued after tile kt: min(nk - 1, kt + S - 2) - kt
    const int after = min(nk - 1, kt + S - 2) - kt;
    if (after >= 2) wait_vmcnt<2 * kLoads>();
    else if (after == 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
    lds_barrier();
    hook(kt, nk);
    const int st = kt % S;
    const bf16* ta = at_byte(&sA[0][0], Map::a(st));
    const bf16* tb = at_byte(&sB[0][0], Map::b(st));
    bf16x8 fa[KSTEPS][TM], fb[KSTEPS][TN];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[ks][j] = frb.get(tb, j, 32 * ks);
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[ks][i] = fra.get(ta, i, 32 * ks);
    }
    if constexpr (KSTEPS == 2) {
      // The wave issues in order and a full LDS queue stalls it, MFMAs
      // included: let the step-0 MFMAs start after the step-0 reads and put one
      // step-1 read between every two of them (scheduling hints only).
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(fb[0][j], fa[0][i], acc[i][j]);
      constexpr int R = TM + TN;
      __builtin_amdgcn_sched_group_barrier(0x100, R, 0);  // step-0 LDS reads
#pragma unroll
      for (int r = 0; r < R; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one step-1 LDS read
      }
      if constexpr (TM * TN > 2 * R) __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - 2 * R, 0);
      if (kt + S - 1 < nk) issue(kt + S - 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(fb[1][j], fa[1][i], acc[i][j]);
    } else {
      if (kt + S - 1 < nk) issue(kt + S - 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(fb[0][j], fa[0][i], acc[i][j]);
    }
  }

}

// One workgroup's work: item L of the launch (XCD-ordered as below), on the
// operand stages sA and sB in LDS.
//
// TBM x TBN output tile, NW wavefronts (4: 2 x 2, two workgroups per CU;
// 8: 2 x 4 or 4 x 2, one workgroup per CU), BKT-deep K tiles.  RD > 0: RoPE
// epilogue on heads of RD.  SWI: B is [2F, K] (gate rows, then up rows), N = F,
// and D = swiglu(gate product, up product).
template <int TBM, int TBN, int NW, int BKT, bool A_KC, bool B_KC, int RD, bool SWI, bool SWB>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int L,
                                          bf16 (*sA)[TBM * BKT],
                                          bf16 (*sB)[TBN * BKT]) {
  constexpr int WAVES_N = NW == 4 ? 2 : (TBN == 256 ? 4 : 2);
  constexpr int WAVES_M = NW / WAVES_N;
  constexpr int WM = TBM / WAVES_M, WN = TBN / WAVES_N;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;              // 16 x 16 MFMA tiles per wave
  constexpr int S = Stages<TBM, TBN, NW, BKT>::S;

  const int w = (L % 8) * g.per_xcd + L / 8;
  if (w >= g.items) return;
  const int split = w / g.tiles;
  const int t = w % g.tiles;
  // grouped order: 4 tile rows at a time, walking the rows fastest, so the
  // 32 workgroups an XCD runs together cover 4 rows x 8 columns of tiles and
  // share their operand blocks in its L2
  constexpr int GM = 4;
  const int tiles_m = g.tiles / g.tiles_n;
  const int grp = t / (GM * g.tiles_n);
  const int gsize = min(tiles_m - grp * GM, GM);
  const int r = t - grp * GM * g.tiles_n;
  const int m0 = (grp * GM + r % gsize) * TBM;
  const int n0 = (r / gsize) * out_cols<TBN, SWI>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave / WAVES_N) * WM, wn = (wave % WAVES_N) * WN;
  const int k_begin = split * g.kps;
  const int k_end = min(g.K, k_begin + g.kps);

  Loader<TBM, A_KC, BKT, NW> la;
  Loader<TBN, B_KC, BKT, NW> lb;
  {
    // tile origins and the extents (bytes) of the matrices from there
    const bf16* a0 = A_KC ? g.a + static_cast<int64_t>(m0) * g.lda : g.a + m0;
    const bf16* b0 = B_KC ? g.b + static_cast<int64_t>(n0) * g.ldb : g.b + n0;
    const int va = min(TBM, g.M - m0), vb = min(TBN, g.N - n0);
    const int64_t ea = A_KC ? (static_cast<int64_t>(va - 1) * g.lda + g.K) * 2
                            : (static_cast<int64_t>(g.K - 1) * g.lda + (g.M - m0)) * 2;
    const int64_t eb = B_KC ? (static_cast<int64_t>(vb - 1) * g.ldb + g.K) * 2
                            : (static_cast<int64_t>(g.K - 1) * g.ldb + (g.N - n0)) * 2;
    la.init(a0, g.lda, va, static_cast<uint32_t>(ea), wave, lane);
    if constexpr (SWI) {
      const int64_t e2 = (static_cast<int64_t>(2 * g.N - 1) * g.ldb + g.K) * 2;
      lb.init_pairs(g.b, g.ldb, g.N, n0, static_cast<uint32_t>(e2), wave, lane);
    } else {
      lb.init(b0, g.ldb, vb, static_cast<uint32_t>(eb), wave, lane);
    }
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  k_loop<TBM, TBN, NW, BKT, A_KC, B_KC, TM, TN>(la, lb, sA, sB, acc, wm, wn, k_begin, k_end, wave, lane);

  // acc[i][j][e] = D[m0 + wm + 16 i + l16][n0 + wn + 16 j + 4 q4 + e]
  const int l16 = lane & 15, q4 = lane >> 4;
  // fp32 rows of the tile through LDS in passes of PR tile rows (as many as
  // the operand stages hold); the row's 16-byte slot s sits at s ^ (r & 15),
  // so a fragment's 16 rows hit distinct banks.  stage_f32(p0) writes this
  // wave's rows [p0, p0 + PR) of acc (alpha and beta are applied as the rows
  // are stored).
  constexpr int ROW_BYTES = TBN * 4;
  constexpr int RA = (S * TBM * BKT * 2) / ROW_BYTES;  // rows in sA, the rest in sB
  constexpr int CAP = RA + (S * TBN * BKT * 2) / ROW_BYTES;
  constexpr int PR = CAP >= TBM ? TBM : (CAP >= 128 ? 128 : (CAP >= 64 ? 64 : 32));
  static_assert(PR <= CAP && PR % 16 == 0 && TBM % PR == 0, "fp32 rows per pass");
  auto slot_at = [&](int lr, int slot) -> float* {
    float* rp = lr < RA ? reinterpret_cast<float*>(&sA[0][0]) + lr * TBN
                        : reinterpret_cast<float*>(&sB[0][0]) + (lr - RA) * TBN;
    return rp + 4 * (slot ^ (lr & 15));
  };
  auto stage_f32 = [&](int p0) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int lr = wm + 16 * i + l16 - p0;
      if (lr < 0 || lr >= PR) continue;  // uniform over the 16 rows of a fragment
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *reinterpret_cast<f32x4*>(slot_at(lr, (wn + 16 * j + 4 * q4) >> 2)) = acc[i][j];
    }
  };
  if (g.splits > 1 || g.d32 != nullptr) {
    // fp32 partials, each row stored by whole 16-byte slots; or, unsplit with
    // an fp32 output, D32 = alpha acc + beta D32 (as the reduction forms it)
    const bool direct = g.splits == 1;
    float* part = direct ? g.d32 : g.partial + static_cast<int64_t>(split) * g.M * g.N;
    const int64_t ldp = direct ? g.ldd32 : g.N;
    constexpr int LPR = TBN / 4, RPI = 64 / LPR, ROWS_PER_WAVE = PR / NW;
    static_assert(ROWS_PER_WAVE % RPI == 0, "whole store instructions per wave");
    const int sl = lane % LPR;
#pragma unroll
    for (int p0 = 0; p0 < TBM; p0 += PR) {
      __syncthreads();  // the operand stages (first pass) or the last pass's rows are free
      stage_f32(p0);
      __syncthreads();
#pragma unroll
      for (int it = 0; it < ROWS_PER_WAVE / RPI; ++it) {
        const int lr = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
        f32x4 v = *reinterpret_cast<const f32x4*>(slot_at(lr, sl));
        const int m = m0 + p0 + lr, n = n0 + 4 * sl;
        if (m < g.M && n < g.N) {
          f32x4* dst = reinterpret_cast<f32x4*>(part + static_cast<int64_t>(m) * ldp + n);
          if (direct) {
            const f32x4 old = g.beta != 0.f ? *dst : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = g.alpha * v[e];
              if (g.beta != 0.f) v[e] += g.beta * old[e];
            }
          }
          *dst = v;
        }
      }
    }
    return;
  }
  if constexpr (SWI) {
    // acc[i][j] (j & 2 clear) holds gate columns, acc[i][j + 2] the matching up
    // columns: output column n0 + 32 ((wn + 16 j) / 64) + 16 (j & 1) + 4 q4 + e.
    // The swiglu kernel's roundings: gate and up to bf16, then the activation;
    // the rounded gate and up go to gu when it is given.
    static_assert(WN % 64 == 0 && RD == 0, "a wave's columns pair whole 32-column groups");
    // the product only (the recompute): no activation math in this epilogue,
    // whose time adds to the kernel's (every workgroup reaches it together)
    const bool act = g.d != nullptr;
    if constexpr (TBN == 256 && NW == 8) {
      // The product only: through LDS, as the plain epilogue below, the
      // [gate | up] tile (256 x 256: the tile's 128 gate columns, then its 128
      // up columns) stored as whole rows (3.9% faster at 8192 x 5472 x 1024;
      // with the activation, whose 128-column tile gains less than the extra
      // pass costs, the stores stay direct).
      if (!act) {
        constexpr int H = TBN / 2;
        constexpr int RPA = (S * TBM * BKT) / TBN;
        auto at = [&](int r, int c) -> bf16* {
          bf16* rp = r < RPA ? &sA[0][0] + r * TBN : &sB[0][0] + (r - RPA) * TBN;
          return rp + 8 * ((c >> 3) ^ (r & 15)) + (c & 4);
        };
        __syncthreads();  // every wave is done with the operand stages
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            if (j & 2) continue;
            const int r = wm + 16 * i + l16;
            const int oc = 32 * ((wn + 16 * j) >> 6) + 16 * (j & 1) + 4 * q4;
            bf16x4 gv, uv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              gv[e] = static_cast<bf16>(acc[i][j][e]);
              uv[e] = static_cast<bf16>(acc[i][j + 2][e]);
            }
            *reinterpret_cast<bf16x4*>(at(r, oc)) = gv;
            *reinterpret_cast<bf16x4*>(at(r, H + oc)) = uv;
          }
        }
        __syncthreads();
        constexpr int LPR = TBN / 8, RPI = 64 / LPR;  // 32 lanes per row: 16 gate, 16 up
        constexpr int ROWS_PER_WAVE = TBM / NW;
        const int sl = lane % LPR;
        const int half = sl / (LPR / 2), col = 8 * (sl % (LPR / 2));
#pragma unroll
        for (int it = 0; it < ROWS_PER_WAVE / RPI; ++it) {
          const int r = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
          const bf16x8 v = *reinterpret_cast<const bf16x8*>(at(r, 8 * sl));
          const int m = m0 + r, n = n0 + col;
          if (m < g.M && n < g.N && g.gu != nullptr)
            *reinterpret_cast<bf16x8*>(g.gu + static_cast<int64_t>(m) * g.ldgu + half * g.N + n) = v;
        }
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm + 16 * i + l16;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (j & 2) continue;
        const int n = n0 + 32 * ((wn + 16 * j) >> 6) + 16 * (j & 1) + 4 * q4;
        if (n >= g.N) continue;
        bf16x4 gv, uv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gv[e] = static_cast<bf16>(acc[i][j][e]);
          uv[e] = static_cast<bf16>(acc[i][j + 2][e]);
        }
        if (g.gu != nullptr) {
          bf16* row = g.gu + static_cast<int64_t>(m) * g.ldgu;
          *reinterpret_cast<bf16x4*>(row + n) = gv;
          *reinterpret_cast<bf16x4*>(row + g.N + n) = uv;
        }
        if (act) {
          bf16x4 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ov[e] = static_cast<bf16>(swiglu_t<bf16>(static_cast<float>(gv[e]), static_cast<float>(uv[e])));
          *reinterpret_cast<bf16x4*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = ov;
        }
      }
    }
    return;
  }
  if constexpr (RD == 0) {
    // with a residual add (beta != 0): the fp32 products go through LDS, and
    // each lane then reads 8 columns of C, adds and stores them as 16 bytes
    // (D = bf16(alpha * acc + beta * C), one rounding)
    if (g.beta != 0.f) {
      constexpr int LPR = TBN / 8, RPI = 64 / LPR, ROWS_PER_WAVE = PR / NW;
      constexpr int IT = ROWS_PER_WAVE / RPI;
      static_assert(ROWS_PER_WAVE % RPI == 0, "whole store instructions per wave");
      const int sl = lane % LPR;
      if constexpr (PR == TBM) {
        // One pass (the whole tile): every C row of the wave is loaded while
        // the products are staged and every row computed before the first
        // store (loads and stores share one counter and complete out of
        // order, so a wait after a store would also wait for it).  Lanes past
        // the matrix load element (m0, n0), which exists, and store nothing.
        bf16x8 cv[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int lr = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
          const int m = m0 + lr, n = n0 + 8 * sl;
          const bool ok = m < g.M && n < g.N;
          cv[it] = *reinterpret_cast<const bf16x8*>(g.c + static_cast<int64_t>(ok ? m : m0) * g.ldc +
                                                    (ok ? n : n0));
        }
        __syncthreads();  // every wave is done with the operand stages
        stage_f32(0);
        __syncthreads();
        bf16x8 ov[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int lr = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
          const f32x4 lo = *reinterpret_cast<const f32x4*>(slot_at(lr, 2 * sl));
          const f32x4 hi = *reinterpret_cast<const f32x4*>(slot_at(lr, 2 * sl + 1));
          float v[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = g.alpha * lo[e];
            v[4 + e] = g.alpha * hi[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) ov[it][e] = static_cast<bf16>(v[e] + g.beta * static_cast<float>(cv[it][e]));
        }
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int lr = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
          const int m = m0 + lr, n = n0 + 8 * sl;
          if (m < g.M && n < g.N) *reinterpret_cast<bf16x8*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = ov[it];
        }
        return;
      }
      // several passes (the later passes' accumulators are still held: no
      // registers for a pass of C rows)
#pragma unroll
      for (int p0 = 0; p0 < TBM; p0 += PR) {
        __syncthreads();  // the operand stages (first pass) or the last pass's rows are free
        stage_f32(p0);
        __syncthreads();
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int lr = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
          const int m = m0 + p0 + lr, n = n0 + 8 * sl;
          if (m >= g.M || n >= g.N) continue;
          const f32x4 lo = *reinterpret_cast<const f32x4*>(slot_at(lr, 2 * sl));
          const f32x4 hi = *reinterpret_cast<const f32x4*>(slot_at(lr, 2 * sl + 1));
          const bf16x8 cv = *reinterpret_cast<const bf16x8*>(g.c + static_cast<int64_t>(m) * g.ldc + n);
          float v[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = g.alpha * lo[e];
            v[4 + e] = g.alpha * hi[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += g.beta * static_cast<float>(cv[e]);
          bf16x8 ov;
#pragma unroll
          for (int e = 0; e < 8; ++e) ov[e] = static_cast<bf16>(v[e]);
          *reinterpret_cast<bf16x8*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = ov;
        }
      }
      return;
    }
  }
  // The bf16 result tile goes to global memory through LDS: each lane first
  // writes its 4-column pieces into a row-major copy of the tile in the
  // operand stages (16-byte slots of row r at slot ^ (r & 15), so the 16 rows
  // of a fragment hit distinct banks), then every lane stores 16 contiguous
  // bytes and a wave whole tile rows.  Stored straight from the fragments, an
  // instruction writes 32 bytes in each of 16 rows; through LDS the step's
  // products with no residual add run up to 4.5% faster (bit-identical).
  constexpr int RPA = (S * TBM * BKT) / TBN;  // tile rows that fit in sA, the rest in sB
  static_assert(RPA + S * BKT >= TBM, "the bf16 tile fits in the operand stages");
  static_assert(TBN % 128 == 0, "16-byte slots of a tile row, swizzled by 4 row bits");
  auto tile_at = [&](int r, int c) -> bf16* {  // tile element (r, c), c a multiple of 4
    bf16* rp = r < RPA ? &sA[0][0] + r * TBN : &sB[0][0] + (r - RPA) * TBN;
    return rp + 8 * ((c >> 3) ^ (r & 15)) + (c & 4);
  };
  __syncthreads();  // every wave is done with the operand stages
  if constexpr (RD > 0) {
    static_assert(WN % RD == 0, "a wave's columns cover whole heads");
    // RoPE as the rotary kernel does it (reference nn/rotary.py:36-38, 65-70):
    // q rounded to bf16, cos/sin rounded to bf16, a rounding after each
    // product and after the sum.  Column pairs (d, d + RD/2) of a head are
    // tiles j and j + RD/32 of the same lane.
    constexpr int HALF = RD / 2;
    constexpr int JP = HALF / 16;  // first-half column tiles of a head
    // The cos/sin values of row tile i + 1 are loaded before row tile i is
    // rotated, so the table loads of consecutive row tiles overlap instead of
    // each row tile waiting for its own.  A lane reads 4 consecutive values
    // per first-half column tile (16-byte loads; the host checks the tables'
    // alignment); rows past the matrix read a valid row and are not stored.
    f32x4 tc[2][JP], ts[2][JP];
    bool tbad[2];
    auto load_tab = [&](int i, int b) {
      const int m = min(m0 + wm + 16 * i + l16, g.M - 1);
      const int sq = m % g.rope_seq;
      int pos = g.rope_pos != nullptr
                    ? g.rope_pos[static_cast<int64_t>(m / g.rope_seq) * g.rope_pos_bstride + sq]
                    : g.rope_offset + sq;
      // an out-of-table position is a caller error: read a valid row and poison the result
      tbad[b] = pos < 0 || pos >= g.rope_n_pos;
      if (tbad[b]) pos = 0;
      const float* crow = g.rope_cos + static_cast<int64_t>(pos) * HALF + 4 * q4;
      const float* srow = g.rope_sin + static_cast<int64_t>(pos) * HALF + 4 * q4;
#pragma unroll
      for (int h = 0; h < JP; ++h) {
        tc[b][h] = *reinterpret_cast<const f32x4*>(crow + 16 * h);
        ts[b][h] = *reinterpret_cast<const f32x4*>(srow + 16 * h);
      }
    };
    load_tab(0, 0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int b = i & 1;
      if (i + 1 < TM) load_tab(i + 1, b ^ 1);
      const int r = wm + 16 * i + l16;
      const int m = m0 + r;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int c = wn + 16 * j + 4 * q4;
        if (n0 + c >= g.N) continue;
        if ((16 * j) % RD >= HALF) {
          if (n0 + wn + 16 * j < g.rope_cols) continue;  // written with its first-half partner
        } else if (n0 + wn + 16 * j < g.rope_cols) {
          const int h = ((16 * j) % RD) / 16;
          bf16x4 o1, o2;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x1 = round_as<bf16>(acc[i][j][e]);
            const float x2 = round_as<bf16>(acc[i][(j + JP) % TN][e]);
            const float cs = round_as<bf16>(tc[b][h][e]);
            const float sn = round_as<bf16>(ts[b][h][e]);
            float r1 = round_as<bf16>(add_rn(round_as<bf16>(mul_rn(x1, cs)), round_as<bf16>(mul_rn(-x2, sn))));
            float r2 = round_as<bf16>(add_rn(round_as<bf16>(mul_rn(x2, cs)), round_as<bf16>(mul_rn(x1, sn))));
            if (tbad[b]) r1 = r2 = __builtin_nanf("");
            o1[e] = static_cast<bf16>(r1);
            o2[e] = static_cast<bf16>(r2);
          }
          *reinterpret_cast<bf16x4*>(tile_at(r, c)) = o1;
          *reinterpret_cast<bf16x4*>(tile_at(r, c + HALF)) = o2;
          continue;
        }
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = static_cast<bf16>(acc[i][j][e]);
        *reinterpret_cast<bf16x4*>(tile_at(r, c)) = ov;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm + 16 * i + l16;
      const int m = m0 + r;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int c = wn + 16 * j + 4 * q4;
        const int n = n0 + c;
        if (n >= g.N) continue;
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = static_cast<bf16>(g.alpha * acc[i][j][e]);
        *reinterpret_cast<bf16x4*>(tile_at(r, c)) = ov;
      }
    }
  }
  __syncthreads();
  // tile rows -> global: TBN / 8 lanes per row, 64 / (TBN / 8) rows per instruction
  constexpr int LPR = TBN / 8;
  constexpr int RPI = 64 / LPR;
  constexpr int ROWS_PER_WAVE = TBM / NW;
  static_assert(ROWS_PER_WAVE % RPI == 0, "whole store instructions per wave");
  const int sl = lane % LPR;
  if constexpr (SWB) {
    // The SwiGLU backward on the tile (ds = bf16(acc), as the product would be
    // stored): 8 columns of a row per lane, g and u read from the gate/up
    // product (every load issued before any store: a wait after a store
    // covers every outstanding load), dg and du written to its gradient and
    // silu(g) u to D when it is given; bit-identical to the product followed
    // by the SwiGLU backward kernel (same element function).
    static_assert(RD == 0 && !SWI, "one epilogue at a time");
    constexpr int IT = ROWS_PER_WAVE / RPI;
    constexpr int CH = IT > 8 ? 8 : IT;  // rows in flight per lane (registers)
    static_assert(IT % CH == 0, "whole chunks");
#pragma unroll
    for (int c0 = 0; c0 < IT; c0 += CH) {
      uint4 graw[CH], uraw[CH];
#pragma unroll
      for (int ci = 0; ci < CH; ++ci) {
        const int it = c0 + ci;
        const int r = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
        const int m = m0 + r, n = n0 + 8 * sl;
        // out-of-range lanes read row m0, column 0 (in range; never used)
        const bool ok = m < g.M && n < g.N;
        const bf16* row = g.swb_gu + static_cast<int64_t>(ok ? m : m0) * g.swb_ldgu + (ok ? n : 0);
        graw[ci] = *reinterpret_cast<const uint4*>(row);
        uraw[ci] = *reinterpret_cast<const uint4*>(row + g.N);
      }
#pragma unroll
      for (int ci = 0; ci < CH; ++ci) {
        const int it = c0 + ci;
        const int r = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
        const int m = m0 + r, n = n0 + 8 * sl;
        const bf16x8 dsv = *reinterpret_cast<const bf16x8*>(tile_at(r, 8 * sl));
        bf16x8 gv, uv, dgo, duo, oo;
        __builtin_memcpy(&gv, &graw[ci], 16);
        __builtin_memcpy(&uv, &uraw[ci], 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float dgf, duf, of;
          swiglu_bwd_elem<bf16>(static_cast<float>(gv[e]), static_cast<float>(uv[e]), static_cast<float>(dsv[e]),
                                dgf, duf, of);
          dgo[e] = static_cast<bf16>(dgf);
          duo[e] = static_cast<bf16>(duf);
          oo[e] = static_cast<bf16>(of);
        }
        if (m < g.M && n < g.N) {
          bf16* drow = g.swb_dgu + static_cast<int64_t>(m) * g.swb_lddgu;
          *reinterpret_cast<bf16x8*>(drow + n) = dgo;
          *reinterpret_cast<bf16x8*>(drow + g.N + n) = duo;
          if (g.d != nullptr) *reinterpret_cast<bf16x8*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = oo;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int it = 0; it < ROWS_PER_WAVE / RPI; ++it) {
    const int r = wave * ROWS_PER_WAVE + it * RPI + lane / LPR;
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(tile_at(r, 8 * sl));
    const int m = m0 + r, n = n0 + 8 * sl;
    if (m < g.M && n < g.N) *reinterpret_cast<bf16x8*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = v;
  }
}

template <int TBM, int TBN, int NW, int BKT, bool A_KC, bool B_KC, int RD, bool SWI = false,
          bool SWB = false>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) void gemm_kernel(GemmArgs g) {
  constexpr int S = Stages<TBM, TBN, NW, BKT>::S;
  __shared__ __attribute__((aligned(1024))) bf16 sA[S][TBM * BKT];
  __shared__ __attribute__((aligned(1024))) bf16 sB[S][TBN * BKT];
  gemm_tile<TBM, TBN, NW, BKT, A_KC, B_KC, RD, SWI, SWB>(g, static_cast<int>(blockIdx.x), sA, sB);
}

// Two products in one launch of 8-wavefront workgroups: the first g1.per_xcd
// * 8 workgroups run configuration 1's tiles of g1, the rest configuration
// 2's of g2 (the Q/K/V projection: the q/k columns with RoPE in 256 x 256
// tiles, the v columns in 256 x 128; the v tiles start on CUs as the longer
// ones finish, with no launch boundary between them).  The stages of either
// configuration share one LDS array.
template <int TBM1, int TBN1, int BKT1, int RD1, int TBM2, int TBN2, int BKT2, bool B_KC>
__global__ __launch_bounds__(512, 1) void gemm_pair_kernel(GemmArgs g1, GemmArgs g2) {
  constexpr int S1 = Stages<TBM1, TBN1, 8, BKT1>::S, S2 = Stages<TBM2, TBN2, 8, BKT2>::S;
  constexpr int A1 = S1 * TBM1 * BKT1, B1 = S1 * TBN1 * BKT1;
  constexpr int A2 = S2 * TBM2 * BKT2, B2 = S2 * TBN2 * BKT2;
  constexpr int kElems = A1 + B1 > A2 + B2 ? A1 + B1 : A2 + B2;
  __shared__ __attribute__((aligned(1024))) bf16 smem[kElems];
  static_assert(A1 % 512 == 0 && A2 % 512 == 0, "B stages stay 1 KB aligned");
  const int L = static_cast<int>(blockIdx.x);
  const int n1 = g1.per_xcd * 8;
  if (L < n1) {
    gemm_tile<TBM1, TBN1, 8, BKT1, true, B_KC, RD1, false, false>(
        g1, L, reinterpret_cast<bf16(*)[TBM1 * BKT1]>(smem), reinterpret_cast<bf16(*)[TBN1 * BKT1]>(smem + A1));
  } else {
    gemm_tile<TBM2, TBN2, 8, BKT2, true, B_KC, 0, false, false>(
        g2, L - n1, reinterpret_cast<bf16(*)[TBM2 * BKT2]>(smem), reinterpret_cast<bf16(*)[TBN2 * BKT2]>(smem + A2));
  }
}

// The MLP backward's two products for one 256-row x 128-column tile of F,
// with the SwiGLU backward as the epilogue and nothing in between in memory:
//   phase 1: [g|u] = A1 [Wg; Wu]^T (g1: A1 = n2 [M, K1], B = the paired
//            [2F, K1] gate/up weight, as nmb_gemm_bf16_swiglu reads it),
//   phase 2: ds = A2 Wd (g2: A2 = dY [M, K2], B = Wd [F, K2] or [K2, F]),
//   epilogue: dg, du = swiglu_bwd(g, u, ds) into dgu [M, 2F] and
//            silu(g) u into act [M, F] (the activation the Wd gradient reads).
// Both phases use the same wave tiling (4 x 2 waves, 64 rows x 64 F columns
// each), so the lane holding g, u of an element (phase 1's 16 x 16 tiles j
// and j + 2 of a gate / up column pair) holds its ds too (phase 2's tile
// (j & 1) + 2 (j >> 2)).  g, u and ds are rounded to bf16 as the separate
// products store them and every K sum runs in the order of the other
// kernels, so the outputs equal nmb_gemm_bf16_swiglu (product only) followed
// by nmb_gemm_bf16_swiglu_bwd bit for bit, without [g|u] ever being written.
// Phase 2's three stages in the 160 KB of LDS, placed so that its first two
// (A 32 KB + B 16 KB each) fall where phase 1's last K tile does not read
// (phase 1 reads stage 1 in its last tile when its tile count is even: A at
// [32, 64) KB and B at [96, 128) KB): A at 0, 64, 32 KB, B at 128, 144, 96 KB.
struct GuSwbPhase2Stages {
  __device__ static uint32_t a(int st) { return st == 0 ? 0u : (st == 1 ? 65536u : 32768u); }
  __device__ static uint32_t b(int st) { return st == 0 ? 131072u : (st == 1 ? 147456u : 98304u); }
};

template <bool B2_KC>
__global__ __launch_bounds__(512, 1) void gemm_gu_swb_kernel(GemmArgs g1, GemmArgs g2) {
  constexpr int TBM = 256, TB1 = 256, TB2 = 128, NW = 8, BKT = 64, WAVES_N = 2;
  constexpr int WM = TBM / (NW / WAVES_N), WN1 = TB1 / WAVES_N, WN2 = TB2 / WAVES_N;
  constexpr int TM = WM / 16, TN1 = WN1 / 16, TN2 = WN2 / 16;
  constexpr int S1 = Stages<TBM, TB1, NW, BKT>::S, S2 = Stages<TBM, TB2, NW, BKT>::S;
  constexpr int A1 = S1 * TBM * BKT, B1 = S1 * TB1 * BKT;
  constexpr int kElems = 160 * 1024 / 2;
  static_assert(S1 == 2 && S2 == 3 && A1 + B1 <= kElems, "the stage placement assumes 2 + 3 stages");
  static_assert(A1 % 512 == 0, "B stages stay 1 KB aligned");
  static_assert(TN1 == 2 * TN2, "a wave's gate/up columns pair with its ds columns");
  __shared__ __attribute__((aligned(1024))) bf16 smem[kElems];

  const int L = static_cast<int>(blockIdx.x);
  const int w = (L % 8) * g2.per_xcd + L / 8;
  if (w >= g2.items) return;
  // grouped order as in gemm_tile: 4 tile rows at a time
  constexpr int GM = 4;
  const int tiles_m = g2.tiles / g2.tiles_n;
  const int grp = w / (GM * g2.tiles_n);
  const int gsize = min(tiles_m - grp * GM, GM);
  const int r = w - grp * GM * g2.tiles_n;
  const int m0 = (grp * GM + r % gsize) * TBM;
  const int f0 = (r / gsize) * TB2;
  const int M = g2.M, F = g2.N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave / WAVES_N) * WM, wc = wave % WAVES_N;
  const int va = min(TBM, M - m0);

  // phase 2's loaders (ds = dY Wd for the same tile)
  auto init2 = [&](Loader<TBM, true, BKT, NW>& la, Loader<TB2, B2_KC, BKT, NW>& lb, int lane) {
    la.init(g2.a + static_cast<int64_t>(m0) * g2.lda, g2.lda, va,
            static_cast<uint32_t>((static_cast<int64_t>(va - 1) * g2.lda + g2.K) * 2), wave, lane);
    const int vb = min(TB2, F - f0);
    const bf16* b0 = B2_KC ? g2.b + static_cast<int64_t>(f0) * g2.ldb : g2.b + f0;
    const int64_t eb = B2_KC ? (static_cast<int64_t>(vb - 1) * g2.ldb + g2.K) * 2
                             : (static_cast<int64_t>(g2.K - 1) * g2.ldb + (F - f0)) * 2;
    lb.init(b0, g2.ldb, vb, static_cast<uint32_t>(eb), wave, lane);
  };
  // Phase 2's first two K tiles are loaded during phase 1's last K tile (into
  // stages that tile does not read), so that phase 2 starts on landed data
  // instead of waiting a full load latency.  Phase 1 ends in its stage 1 when
  // it has an even number of K tiles; otherwise phase 2 loads them itself.
  const int nk1 = (g1.K + BKT - 1) / BKT, nk2 = (g2.K + BKT - 1) / BKT;
  const int pre2 = (nk1 >= 2 && nk1 % 2 == 0) ? min(S2 - 1, nk2) : 0;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto prefetch2 = [&](int kt, int nk) {
    if (pre2 == 0 || kt != nk - 1) return;
    Loader<TBM, true, BKT, NW> la;
    Loader<TB2, B2_KC, BKT, NW> lb;
    // the lane index made opaque, so that the offsets are formed here and not
    // hoisted out of phase 1's loop into registers held (or spilled) across it
    int ln = lane;
    asm volatile("" : "+v"(ln));
    init2(la, lb, ln);
    // as k_loop issues them (scalar issue for 256 x 128 tiles)
    const uint32_t a_lds = lds_offset(smem) + 1024u * wave_u * Loader<TBM, true, BKT, NW>::kPer;
    const uint32_t b_lds = lds_offset(smem) + 1024u * wave_u * Loader<TB2, B2_KC, BKT, NW>::kPer;
    for (int p = 0; p < pre2; ++p) {
      la.issue_s(a_lds + GuSwbPhase2Stages::a(p), p * BKT, g2.K);
      lb.issue_s(b_lds + GuSwbPhase2Stages::b(p), p * BKT, g2.K);
    }
  };

  // phase 1: the gate/up product of the tile's F columns (128 gate, 128 up)
  f32x4 acc1[TM][TN1];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN1; ++j) acc1[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    Loader<TBM, true, BKT, NW> la;
    Loader<TB1, true, BKT, NW> lb;
    la.init(g1.a + static_cast<int64_t>(m0) * g1.lda, g1.lda, va,
            static_cast<uint32_t>((static_cast<int64_t>(va - 1) * g1.lda + g1.K) * 2), wave, lane);
    lb.init_pairs(g1.b, g1.ldb, F, f0,
                  static_cast<uint32_t>((static_cast<int64_t>(2 * F - 1) * g1.ldb + g1.K) * 2), wave, lane);
    k_loop<TBM, TB1, NW, BKT, true, true, TM, TN1, LinearStages<TBM, TB1, BKT>, decltype(prefetch2)>(
        la, lb, reinterpret_cast<bf16(*)[TBM * BKT]>(smem), reinterpret_cast<bf16(*)[TB1 * BKT]>(smem + A1),
        acc1, wm, wc * WN1, 0, g1.K, wave, lane, 0, prefetch2);
  }
  // g and u as the product stores them (bf16); column tile jj of phase 2 is
  // gate tile (jj & 1) + 4 (jj >> 1) of phase 1, its up partner 2 tiles on
  bf16x4 gv[TM][TN2], uv[TM][TN2];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jj = 0; jj < TN2; ++jj) {
      const int j = (jj & 1) + 4 * (jj >> 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gv[i][jj][e] = static_cast<bf16>(acc1[i][j][e]);
        uv[i][jj][e] = static_cast<bf16>(acc1[i][j + 2][e]);
      }
    }
  __syncthreads();  // every wave is done with phase 1's stages

  // phase 2: ds = dY Wd for the same tile
  f32x4 acc2[TM][TN2];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN2; ++j) acc2[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    Loader<TBM, true, BKT, NW> la;
    Loader<TB2, B2_KC, BKT, NW> lb;
    init2(la, lb, lane);
    k_loop<TBM, TB2, NW, BKT, true, B2_KC, TM, TN2, GuSwbPhase2Stages>(
        la, lb, reinterpret_cast<bf16(*)[TBM * BKT]>(smem), reinterpret_cast<bf16(*)[TB2 * BKT]>(smem),
        acc2, wm, wc * WN2, 0, g2.K, wave, lane, pre2);
  }

  // the SwiGLU backward on the tile: lane (l16, q4) holds row wm + 16 i + l16,
  // F columns wc 64 + 16 jj + 4 q4 .. + 3 of every (i, jj)
  const int l16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm + 16 * i + l16;
    if (m >= M) continue;
    bf16* drow = g2.swb_dgu + static_cast<int64_t>(m) * g2.swb_lddgu;
#pragma unroll
    for (int jj = 0; jj < TN2; ++jj) {
      const int n = f0 + wc * WN2 + 16 * jj + 4 * q4;
      if (n >= F) continue;
      bf16x4 dgo, duo, oo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float dgf, duf, of;
        swiglu_bwd_elem<bf16>(static_cast<float>(gv[i][jj][e]), static_cast<float>(uv[i][jj][e]),
                              round_as<bf16>(acc2[i][jj][e]), dgf, duf, of);
        dgo[e] = static_cast<bf16>(dgf);
        duo[e] = static_cast<bf16>(duf);
        oo[e] = static_cast<bf16>(of);
      }
      *reinterpret_cast<bf16x4*>(drow + n) = dgo;
      *reinterpret_cast<bf16x4*>(drow + F + n) = duo;
      if (g2.d != nullptr) *reinterpret_cast<bf16x4*>(g2.d + static_cast<int64_t>(m) * g2.ldd + n) = oo;
    }
  }
}

// D = alpha * sum_s partial[s] + beta * C, splits summed in order; 8 columns
// per thread (N % 8 == 0).
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs g) {
  const int64_t groups = static_cast<int64_t>(g.M) * (g.N / 8);
  const int64_t mn = static_cast<int64_t>(g.M) * g.N;
  for (int64_t x = blockIdx.x * 256ll + threadIdx.x; x < groups; x += gridDim.x * 256ll) {
    const int m = static_cast<int>(x / (g.N / 8));
    const int n = static_cast<int>(x % (g.N / 8)) * 8;
    const float* p = g.partial + static_cast<int64_t>(m) * g.N + n;
    f32x4 s0 = *reinterpret_cast<const f32x4*>(p);
    f32x4 s1 = *reinterpret_cast<const f32x4*>(p + 4);
    for (int s = 1; s < g.splits; ++s) {
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(p + s * mn);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(p + s * mn + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s0[e] += a0[e];
        s1[e] += a1[e];
      }
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = g.alpha * s0[e];
      v[4 + e] = g.alpha * s1[e];
    }
    if (g.d32 != nullptr) {
      // fp32 output: D32 = alpha sum + beta D32
      f32x4* dst = reinterpret_cast<f32x4*>(g.d32 + static_cast<int64_t>(m) * g.ldd32 + n);
      if (g.beta != 0.f) {
        const f32x4 o0 = dst[0], o1 = dst[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] += g.beta * o0[e];
          v[4 + e] += g.beta * o1[e];
        }
      }
      dst[0] = f32x4{v[0], v[1], v[2], v[3]};
      dst[1] = f32x4{v[4], v[5], v[6], v[7]};
      continue;
    }
    if (g.beta != 0.f) {
      const bf16x8 cv = ld8(g.c + static_cast<int64_t>(m) * g.ldc + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += g.beta * static_cast<float>(cv[e]);
    }
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = static_cast<bf16>(v[e]);
    *reinterpret_cast<bf16x8*>(g.d + static_cast<int64_t>(m) * g.ldd + n) = ov;
  }
}

// Kernel configurations: tile, wavefronts per workgroup, K-tile depth, and the
// measured throughput of one workgroup on these shapes (FLOP/s), used to rank
// the configurations of a product.
struct Config {
  int tbm, tbn, nw, bkt;
  double rate;
};
constexpr Config kConfigs[] = {
    {256, 256, 8, 64, 3.9e12},  // one workgroup per CU
    {256, 128, 8, 64, 3.0e12},
    {128, 128, 4, 32, 1.6e12},  // two workgroups per CU
    {128, 256, 4, 32, 1.7e12},
};

struct Plan {
  int config;     // index into kConfigs
  int splits;     // 1: no split K
  int kps;        // K per split (multiple of the config's K tile)
  double time;    // the estimate the plan was chosen by (seconds)
};

// Configuration and K split for an M x N x K product on 256 CUs.  Products
// with both operands M/N-contiguous (the weight gradients) or too few output
// tiles for the CUs use the two-workgroups-per-CU configurations with a K
// split; the others the one-workgroup configurations.  Among those, the
// least estimated time = rounds of workgroups over the CUs x tile time + the
// fp32 partials written and read back (~5 TB/s).
// Columns of one wavefront's share of a configuration's tile.
constexpr int wave_cols(const Config& c) { return c.nw == 4 ? c.tbn / 2 : (c.tbn == 256 ? c.tbn / 4 : c.tbn / 2); }

Plan plan_for(int64_t m, int64_t n, int64_t k, bool a_kc, bool b_kc, int rope_head_dim = 0,
              bool whole_k = false) {
  constexpr int64_t kCUs = 256;
  constexpr double kBytesPerS = 5e12;
  const int64_t big_tiles = ((m + 255) / 256) * ((n + 127) / 128);
  const bool small = (!a_kc && !b_kc) || big_tiles < kCUs;
  Plan best{small ? 2 : 1, 1, 0, 0.0};
  double best_t = -1.0;
  // pass 0: the configurations of the problem's size class; pass 1 (RoPE only,
  // when none of those fits the head): any configuration that fits
  for (int pass = 0; pass < 2 && best_t < 0; ++pass) {
    for (int c = 0; c < static_cast<int>(sizeof(kConfigs) / sizeof(kConfigs[0])); ++c) {
      const Config& cf = kConfigs[c];
      // the RoPE epilogue needs whole heads per wavefront and no K split
      if (pass == 0 && (cf.nw == 4) != small) continue;
      if (rope_head_dim > 0 && wave_cols(cf) % rope_head_dim != 0) continue;
      if (pass == 1 && rope_head_dim == 0) continue;
      const int64_t slots = cf.nw == 4 ? 2 * kCUs : kCUs;
      const int64_t tiles = ((m + cf.tbm - 1) / cf.tbm) * ((n + cf.tbn - 1) / cf.tbn);
      const int64_t kt = std::max<int64_t>((k + cf.bkt - 1) / cf.bkt, 1);  // K tiles
      for (int64_t s = 1; s <= (small && rope_head_dim == 0 && !whole_k ? 16 : 1); ++s) {
        const int64_t tps = (kt + s - 1) / s;  // K tiles per split
        const int64_t splits = (kt + tps - 1) / tps;
        if (splits != s || (s > 1 && tps * cf.bkt < 512)) continue;
        const int64_t rounds = (tiles * splits + slots - 1) / slots;
        double t = static_cast<double>(rounds) * 2.0 * cf.tbm * cf.tbn * (tps * cf.bkt) / cf.rate;
        if (splits > 1) t += static_cast<double>(splits) * m * n * 8 / kBytesPerS;
        if (best_t < 0 || t < best_t * 0.999) {
          best_t = t;
          best = Plan{c, static_cast<int>(splits), static_cast<int>(tps * cf.bkt), t};
        }
      }
    }
  }
  // Weight gradients (both operands M/N-contiguous, long K): also the 256 x 256
  // configuration in a single round of workgroups, each split at least 1024
  // deep; its per-workgroup rate on this layout was measured at ~5.8e12 FLOP/s
  // (the 16-tile-row 32-deep tiles of the other family read twice the LDS
  // bytes per MFMA through the transposing reads).
  if (!a_kc && !b_kc && rope_head_dim == 0 && !whole_k) {
    constexpr double kRateMN = 5.8e12;
    const Config& cf = kConfigs[0];
    const int64_t tiles = ((m + cf.tbm - 1) / cf.tbm) * ((n + cf.tbn - 1) / cf.tbn);
    const int64_t kt = std::max<int64_t>((k + cf.bkt - 1) / cf.bkt, 1);
    for (int64_t s = 1; s <= 16; ++s) {
      const int64_t tps = (kt + s - 1) / s;
      const int64_t splits = (kt + tps - 1) / tps;
      if (splits != s || tiles * splits > kCUs || (s > 1 && tps * cf.bkt < 1024)) continue;
      double t = 2.0 * cf.tbm * cf.tbn * (tps * cf.bkt) / kRateMN;
      if (splits > 1) t += static_cast<double>(splits) * m * n * 8 / kBytesPerS;
      if (t < best_t * 0.999) {
        best_t = t;
        best = Plan{0, static_cast<int>(splits), static_cast<int>(tps * cf.bkt), t};
      }
    }
  }
  return best;
}

// Tile count and the XCD-ordered work split of a launch of TBM x TBN tiles.
template <int TBM, int TBN, bool SWI = false>
int prepare(GemmArgs& g) {
  const int tiles_m = (g.M + TBM - 1) / TBM;
  g.tiles_n = (g.N + out_cols<TBN, SWI>() - 1) / out_cols<TBN, SWI>();
  const int64_t tiles = static_cast<int64_t>(tiles_m) * g.tiles_n;
  const int64_t items = tiles * g.splits;
  NMB_REQUIRE(items < (int64_t{1} << 30), "gemm: too many tiles");
  g.tiles = static_cast<int>(tiles);
  g.items = static_cast<int>(items);
  g.per_xcd = static_cast<int>((items + 7) / 8);
  return NMB_OK;
}

template <int TBM, int TBN, int NW, int BKT, bool A_KC, bool B_KC, int RD = 0, bool SWI = false,
          bool SWB = false>
int launch(GemmArgs g, hipStream_t stream) {
  const int st = prepare<TBM, TBN, SWI>(g);
  if (st != NMB_OK) return st;
  hipLaunchKernelGGL((gemm_kernel<TBM, TBN, NW, BKT, A_KC, B_KC, RD, SWI, SWB>),
                     dim3(static_cast<unsigned>(g.per_xcd * 8)), dim3(NW * 64), 0, stream, g);
  NMB_CHECK_LAUNCH("gemm");
  if (g.splits > 1) {
    const int64_t groups = static_cast<int64_t>(g.M) * (g.N / 8);
    const int64_t blocks = std::min<int64_t>((groups + 255) / 256, 4096);
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, g);
    NMB_CHECK_LAUNCH("gemm split reduce");
  }
  return NMB_OK;
}

template <int TBM, int TBN, int NW, int BKT>
int dispatch_layout(bool a_kc, bool b_kc, const GemmArgs& g, hipStream_t s) {
  if (a_kc && b_kc) return launch<TBM, TBN, NW, BKT, true, true>(g, s);
  if (a_kc && !b_kc) return launch<TBM, TBN, NW, BKT, true, false>(g, s);
  if (!a_kc && b_kc) return launch<TBM, TBN, NW, BKT, false, true>(g, s);
  return launch<TBM, TBN, NW, BKT, false, false>(g, s);
}

template <int RD>
int dispatch_rope(int config, bool b_kc, const GemmArgs& g, hipStream_t s) {
  if constexpr (RD == 64) {
    switch (config) {
      case 0: return b_kc ? launch<256, 256, 8, 64, true, true, RD>(g, s) : launch<256, 256, 8, 64, true, false, RD>(g, s);
      case 1: return b_kc ? launch<256, 128, 8, 64, true, true, RD>(g, s) : launch<256, 128, 8, 64, true, false, RD>(g, s);
      case 2: return b_kc ? launch<128, 128, 4, 32, true, true, RD>(g, s) : launch<128, 128, 4, 32, true, false, RD>(g, s);
      default: break;
    }
  }
  return b_kc ? launch<128, 256, 4, 32, true, true, RD>(g, s) : launch<128, 256, 4, 32, true, false, RD>(g, s);
}

// The RoPE columns in 256 x 256 tiles (g1) and the rest in 256 x 128 (g2),
// unsplit, in one launch.
template <int RD>
int launch_rope_pair(bool b_kc, GemmArgs g1, GemmArgs g2, hipStream_t s) {
  int st = prepare<256, 256>(g1);
  if (st != NMB_OK) return st;
  st = prepare<256, 128>(g2);
  if (st != NMB_OK) return st;
  const unsigned blocks = static_cast<unsigned>(g1.per_xcd + g2.per_xcd) * 8u;
  if (b_kc)
    hipLaunchKernelGGL((gemm_pair_kernel<256, 256, 64, RD, 256, 128, 64, true>), dim3(blocks), dim3(512), 0, s, g1, g2);
  else
    hipLaunchKernelGGL((gemm_pair_kernel<256, 256, 64, RD, 256, 128, 64, false>), dim3(blocks), dim3(512), 0, s, g1, g2);
  NMB_CHECK_LAUNCH("gemm pair");
  return NMB_OK;
}

int dispatch_swiglu_bwd(int config, bool b_kc, const GemmArgs& g, hipStream_t s) {
  switch (config) {
    case 0: return b_kc ? launch<256, 256, 8, 64, true, true, 0, false, true>(g, s)
                        : launch<256, 256, 8, 64, true, false, 0, false, true>(g, s);
    case 1: return b_kc ? launch<256, 128, 8, 64, true, true, 0, false, true>(g, s)
                        : launch<256, 128, 8, 64, true, false, 0, false, true>(g, s);
    case 2: return b_kc ? launch<128, 128, 4, 32, true, true, 0, false, true>(g, s)
                        : launch<128, 128, 4, 32, true, false, 0, false, true>(g, s);
    default: return b_kc ? launch<128, 256, 4, 32, true, true, 0, false, true>(g, s)
                         : launch<128, 256, 4, 32, true, false, 0, false, true>(g, s);
  }
}

int dispatch_swiglu(int config, const GemmArgs& g, hipStream_t s) {
  switch (config) {
    case 0: return launch<256, 256, 8, 64, true, true, 0, true>(g, s);
    case 1: return launch<256, 128, 8, 64, true, true, 0, true>(g, s);
    case 2: return launch<128, 128, 4, 32, true, true, 0, true>(g, s);
    default: return launch<128, 256, 4, 32, true, true, 0, true>(g, s);
  }
}

int64_t workspace_for(const Plan& p, int64_t m, int64_t n) {
  return p.splits > 1 ? static_cast<int64_t>(p.splits) * m * n * 4 : 0;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_gemm_bf16_workspace_bytes(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k,
                                             int64_t* bytes) {
  NMB_REQUIRE(bytes != nullptr, "gemm: null bytes");
  NMB_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
              "gemm: invalid shape");
  *bytes = nmb::workspace_for(nmb::plan_for(m, n, k, a_layout == 0, b_layout == 0), m, n);
  return NMB_OK;
}

namespace nmb {
namespace {

// Argument checks shared by the GEMM entry points.
int check_gemm(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k, const void* a, int64_t lda,
               const void* b, int64_t ldb, bool use_c, const void* c, int64_t ldc, const void* d,
               int64_t ldd) {
  NMB_REQUIRE(a != nullptr && b != nullptr && d != nullptr, "gemm: null operand");
  NMB_REQUIRE(a_layout == 0 || a_layout == 1, "gemm: a_layout must be 0 ([M,K]) or 1 ([K,M])");
  NMB_REQUIRE(b_layout == 0 || b_layout == 1, "gemm: b_layout must be 0 ([N,K]) or 1 ([K,N])");
  NMB_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
              "gemm: invalid shape %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  NMB_REQUIRE(!use_c || c != nullptr, "gemm: beta != 0 needs C");
  const bool a_kc = a_layout == 0, b_kc = b_layout == 0;
  // 16-byte operand chunks: the contiguous dimensions and the leading
  // dimensions are multiples of 8 elements and the pointers 16-byte aligned
  NMB_REQUIRE_SUPPORTED((a_kc ? k : m) % 8 == 0 && (b_kc ? k : n) % 8 == 0 && n % 8 == 0 &&
                            lda % 8 == 0 && ldb % 8 == 0 && ldd % 8 == 0 && (!use_c || ldc % 8 == 0),
                        "gemm: N, the contiguous extents and leading dimensions must be multiples of 8");
  NMB_REQUIRE(aligned16(a) && aligned16(b) && aligned16(d) && (!use_c || aligned16(c)),
              "gemm: operands must be 16-byte aligned");
  NMB_REQUIRE(lda >= (a_kc ? k : m) && ldb >= (b_kc ? k : n) && ldd >= n && (!use_c || ldc >= n),
              "gemm: leading dimension too small");
  // the loads address a tile's operand with 32-bit byte offsets
  const int64_t span_a = a_kc ? int64_t{256} * lda : k * lda;
  const int64_t span_b = b_kc ? int64_t{256} * ldb : k * ldb;
  NMB_REQUIRE_SUPPORTED(2 * span_a < (int64_t{1} << 31) && 2 * span_b < (int64_t{1} << 31),
                        "gemm: an operand tile spans more than 2 GiB");
  return NMB_OK;
}

GemmArgs make_args(int64_t m, int64_t n, int64_t k, float alpha, const void* a, int64_t lda,
                   const void* b, int64_t ldb, float beta, const void* c, int64_t ldc, void* d,
                   int64_t ldd, void* workspace, const Plan& p) {
  GemmArgs g{};
  g.a = static_cast<const bf16*>(a);
  g.b = static_cast<const bf16*>(b);
  g.c = static_cast<const bf16*>(c);
  g.d = static_cast<bf16*>(d);
  g.partial = static_cast<float*>(workspace);
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.ldd = ldd;
  g.M = static_cast<int>(m);
  g.N = static_cast<int>(n);
  g.K = static_cast<int>(k);
  g.alpha = alpha;
  g.beta = beta;
  g.splits = p.splits;
  g.kps = p.kps;
  return g;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_gemm_bf16(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k,
                             float alpha, const void* a, int64_t lda, const void* b, int64_t ldb,
                             float beta, const void* c, int64_t ldc, void* d, int64_t ldd,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const int st = nmb::check_gemm(a_layout, b_layout, m, n, k, a, lda, b, ldb, beta != 0.f, c, ldc, d, ldd);
  if (st != NMB_OK) return st;
  if (m == 0 || n == 0) return NMB_OK;
  const bool a_kc = a_layout == 0, b_kc = b_layout == 0;
  const nmb::Plan p = nmb::plan_for(m, n, k, a_kc, b_kc);
  const int64_t need = nmb::workspace_for(p, m, n);
  NMB_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
              "gemm: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)workspace_bytes);
  NMB_REQUIRE(need == 0 || nmb::aligned16(workspace), "gemm: workspace must be 16-byte aligned");
  const nmb::GemmArgs g = nmb::make_args(m, n, k, alpha, a, lda, b, ldb, beta, c, ldc, d, ldd, workspace, p);
  switch (p.config) {
    case 0: return nmb::dispatch_layout<256, 256, 8, 64>(a_kc, b_kc, g, stream);
    case 1: return nmb::dispatch_layout<256, 128, 8, 64>(a_kc, b_kc, g, stream);
    case 2: return nmb::dispatch_layout<128, 128, 4, 32>(a_kc, b_kc, g, stream);
    default: return nmb::dispatch_layout<128, 256, 4, 32>(a_kc, b_kc, g, stream);
  }
}

extern "C" int nmb_gemm_bf16_f32out(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k,
                                    float alpha, const void* a, int64_t lda, const void* b,
                                    int64_t ldb, float beta, float* d32, int64_t ldd32,
                                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  // the bf16 checks (D32 stands in for D: non-null, 16-byte aligned), then D32's leading dimension
  const int st = nmb::check_gemm(a_layout, b_layout, m, n, k, a, lda, b, ldb, false, nullptr, 0, d32, n);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(ldd32 >= n && ldd32 % 4 == 0,
              "gemm_f32out: D32 leading dimension must be >= N and a multiple of 4");
  if (m == 0 || n == 0) return NMB_OK;
  const bool a_kc = a_layout == 0, b_kc = b_layout == 0;
  const nmb::Plan p = nmb::plan_for(m, n, k, a_kc, b_kc);
  const int64_t need = nmb::workspace_for(p, m, n);
  NMB_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
              "gemm_f32out: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)workspace_bytes);
  NMB_REQUIRE(need == 0 || nmb::aligned16(workspace), "gemm_f32out: workspace must be 16-byte aligned");
  nmb::GemmArgs g = nmb::make_args(m, n, k, alpha, a, lda, b, ldb, beta, nullptr, 0, nullptr, 0, workspace, p);
  g.d32 = d32;
  g.ldd32 = ldd32;
  switch (p.config) {
    case 0: return nmb::dispatch_layout<256, 256, 8, 64>(a_kc, b_kc, g, stream);
    case 1: return nmb::dispatch_layout<256, 128, 8, 64>(a_kc, b_kc, g, stream);
    case 2: return nmb::dispatch_layout<128, 128, 4, 32>(a_kc, b_kc, g, stream);
    default: return nmb::dispatch_layout<128, 256, 4, 32>(a_kc, b_kc, g, stream);
  }
}

extern "C" int nmb_gemm_bf16_rope(int b_layout, int64_t m, int64_t n, int64_t k, const void* a,
                                  int64_t lda, const void* b, int64_t ldb, void* d, int64_t ldd,
                                  const float* cos_table, const float* sin_table, int64_t n_pos,
                                  const int32_t* positions, int64_t pos_batch_stride,
                                  int64_t pos_offset, int64_t seq, int64_t head_dim,
                                  int64_t rope_cols, hipStream_t stream) {
  const int st = nmb::check_gemm(0, b_layout, m, n, k, a, lda, b, ldb, false, nullptr, 0, d, ldd);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(cos_table != nullptr && sin_table != nullptr && n_pos > 0 && n_pos < (1 << 30),
              "gemm_rope: cos/sin tables of n_pos rows needed");
  // the epilogue reads 4 table values per 16-byte load
  NMB_REQUIRE(nmb::aligned16(cos_table) && nmb::aligned16(sin_table),
              "gemm_rope: cos/sin tables must be 16-byte aligned");
  NMB_REQUIRE_SUPPORTED(head_dim == 64 || head_dim == 128, "gemm_rope: head_dim %lld (64 or 128 supported)",
                        (long long)head_dim);
  NMB_REQUIRE(rope_cols >= 0 && rope_cols <= n && rope_cols % head_dim == 0,
              "gemm_rope: rope_cols %lld must be a multiple of head_dim within N", (long long)rope_cols);
  NMB_REQUIRE(seq > 0 && seq < (1 << 30) && m % seq == 0, "gemm_rope: M (%lld) must be batch x seq (%lld)",
              (long long)m, (long long)seq);
  if (positions == nullptr) {
    NMB_REQUIRE(pos_offset >= 0 && pos_offset + seq <= n_pos,
                "gemm_rope: positions [%lld, %lld) exceed the cos/sin table of %lld rows",
                (long long)pos_offset, (long long)(pos_offset + seq), (long long)n_pos);
  } else {
    NMB_REQUIRE(pos_batch_stride >= 0, "gemm_rope: negative position batch stride");
  }
  if (m == 0 || n == 0) return NMB_OK;
  const bool b_kc = b_layout == 0;
  // the product's first n_cols columns (q and k heads up to rope_cols) with the RoPE epilogue
  auto rope_args = [&](const nmb::Plan& pl, int64_t n_cols) {
    nmb::GemmArgs g = nmb::make_args(m, n_cols, k, 1.f, a, lda, b, ldb, 0.f, nullptr, 0, d, ldd, nullptr, pl);
    g.rope_cos = cos_table;
    g.rope_sin = sin_table;
    g.rope_pos = positions;
    g.rope_pos_bstride = pos_batch_stride;
    g.rope_offset = static_cast<int>(positions == nullptr ? pos_offset : 0);
    g.rope_seq = static_cast<int>(seq);
    g.rope_n_pos = static_cast<int>(n_pos);
    g.rope_cols = static_cast<int>(rope_cols);
    return g;
  };
  nmb::Plan p = nmb::plan_for(m, n, k, true, b_kc, static_cast<int>(head_dim));
  int64_t n_rope = n;
  if (rope_cols > 0 && rope_cols < n) {
    // The columns past rope_cols (v) need no rotation: as a plain product of
    // their own they can take a tile shape that fills the CUs in whole rounds
    // where the full width cannot (8192 x 3072: 1.5 rounds of 256 x 256 tiles
    // or three short ones of 256 x 128; split: one round of each).  Every tile
    // shape accumulates K in the same order, so the bits do not change.
    const nmb::Plan pr = nmb::plan_for(m, rope_cols, k, true, b_kc, static_cast<int>(head_dim));
    const nmb::Plan pv = nmb::plan_for(m, n - rope_cols, k, true, b_kc, 0, true);
    if (pr.time + pv.time < p.time) {
      const nmb::bf16* bv = static_cast<const nmb::bf16*>(b) + (b_kc ? rope_cols * ldb : rope_cols);
      nmb::bf16* dv = static_cast<nmb::bf16*>(d) + rope_cols;
      const nmb::GemmArgs gv = nmb::make_args(m, n - rope_cols, k, 1.f, a, lda, bv, ldb, 0.f, nullptr, 0,
                                              dv, ldd, nullptr, pv);
      if (head_dim == 64 && pr.config == 0 && pv.config == 1 && pr.splits == 1 && pv.splits == 1) {
        // both parts in one launch (5% faster at 8192 x 3072 x 1024 than two, same bits)
        return nmb::launch_rope_pair<64>(b_kc, rope_args(pr, rope_cols), gv, stream);
      }
      int st2 = NMB_OK;
      switch (pv.config) {
        case 0: st2 = nmb::dispatch_layout<256, 256, 8, 64>(true, b_kc, gv, stream); break;
        case 1: st2 = nmb::dispatch_layout<256, 128, 8, 64>(true, b_kc, gv, stream); break;
        case 2: st2 = nmb::dispatch_layout<128, 128, 4, 32>(true, b_kc, gv, stream); break;
        default: st2 = nmb::dispatch_layout<128, 256, 4, 32>(true, b_kc, gv, stream); break;
      }
      if (st2 != NMB_OK) return st2;
      p = pr;
      n_rope = rope_cols;
    }
  }
  const nmb::GemmArgs g = rope_args(p, n_rope);
  return head_dim == 64 ? nmb::dispatch_rope<64>(p.config, b_layout == 0, g, stream)
                        : nmb::dispatch_rope<128>(p.config, b_layout == 0, g, stream);
}

extern "C" int nmb_gemm_bf16_swiglu(int64_t m, int64_t f, int64_t k, const void* a, int64_t lda,
                                    const void* b, int64_t ldb, void* d, int64_t ldd, void* gu,
                                    int64_t ldgu, hipStream_t stream) {
  NMB_REQUIRE(d != nullptr || gu != nullptr, "gemm_swiglu: neither d nor gu given");
  // B is [2F, K]; D is [M, F]; gu is [M, 2F]
  const int st = nmb::check_gemm(0, 0, m, f, k, a, lda, b, ldb, false, nullptr, 0,
                                 d != nullptr ? d : gu, d != nullptr ? ldd : ldgu);
  if (st != NMB_OK) return st;
  NMB_REQUIRE_SUPPORTED(f % 8 == 0, "gemm_swiglu: F (%lld) must be a multiple of 8", (long long)f);
  NMB_REQUIRE(gu == nullptr || (ldgu >= 2 * f && ldgu % 8 == 0 && nmb::aligned16(gu)),
              "gemm_swiglu: gu must be 16-byte aligned with a leading dimension >= 2F, a multiple of 8");
  // the paired loads address the whole [2F, K] weight with 32-bit byte offsets
  NMB_REQUIRE_SUPPORTED(2 * (2 * f * ldb) < (int64_t{1} << 31),
                        "gemm_swiglu: the gate/up weight spans more than 2 GiB");
  if (m == 0 || f == 0) return NMB_OK;
  const nmb::Plan p = nmb::plan_for(m, 2 * f, k, true, true, 0, true);
  nmb::GemmArgs g = nmb::make_args(m, f, k, 1.f, a, lda, b, ldb, 0.f, nullptr, 0, d, ldd, nullptr, p);
  g.gu = static_cast<nmb::bf16*>(gu);
  g.ldgu = ldgu;
  return nmb::dispatch_swiglu(p.config, g, stream);
}

extern "C" int nmb_gemm_bf16_swiglu_bwd(int b_layout, int64_t m, int64_t f, int64_t k, const void* a,
                                        int64_t lda, const void* b, int64_t ldb, const void* gu, int64_t ldgu,
                                        void* dgu, int64_t lddgu, void* act, int64_t ldact,
                                        hipStream_t stream) {
  // ds = A B is [M, F]; gu and dgu are [M, 2F]; act (nullable) is [M, F]
  NMB_REQUIRE(dgu != nullptr && gu != nullptr, "gemm_swiglu_bwd: null gu or dgu");
  const int st = nmb::check_gemm(0, b_layout, m, f, k, a, lda, b, ldb, false, nullptr, 0, dgu, lddgu);
  if (st != NMB_OK) return st;
  NMB_REQUIRE_SUPPORTED(f % 8 == 0, "gemm_swiglu_bwd: F (%lld) must be a multiple of 8", (long long)f);
  NMB_REQUIRE(ldgu >= 2 * f && ldgu % 8 == 0 && nmb::aligned16(gu) && lddgu >= 2 * f && lddgu % 8 == 0,
              "gemm_swiglu_bwd: gu and dgu must be 16-byte aligned [M, 2F] with leading dimensions multiples of 8");
  NMB_REQUIRE(act == nullptr || (ldact >= f && ldact % 8 == 0 && nmb::aligned16(act)),
              "gemm_swiglu_bwd: act must be 16-byte aligned [M, F] with a leading dimension multiple of 8");
  if (m == 0 || f == 0) return NMB_OK;
  const bool b_kc = b_layout == 0;
  const nmb::Plan p = nmb::plan_for(m, f, k, true, b_kc, 0, true);
  nmb::GemmArgs g = nmb::make_args(m, f, k, 1.f, a, lda, b, ldb, 0.f, nullptr, 0, act, ldact, nullptr, p);
  g.swb_gu = static_cast<const nmb::bf16*>(gu);
  g.swb_ldgu = ldgu;
  g.swb_dgu = static_cast<nmb::bf16*>(dgu);
  g.swb_lddgu = lddgu;
  return nmb::dispatch_swiglu_bwd(p.config, b_kc, g, stream);
}

extern "C" int nmb_gemm_bf16_gate_up_swiglu_bwd(int64_t m, int64_t f, int64_t k1, const void* a1, int64_t lda1,
                                                const void* wgu, int64_t ldwgu, int64_t k2, const void* a2,
                                                int64_t lda2, int b_layout, const void* wd, int64_t ldwd,
                                                void* dgu, int64_t lddgu, void* act, int64_t ldact,
                                                hipStream_t stream) {
  // [g|u] = a1 wgu^T ([M, K1] x [2F, K1]), ds = a2 wd ([M, K2] x op(wd) [K2, F]); dgu [M, 2F], act [M, F]
  NMB_REQUIRE(dgu != nullptr, "gemm_gate_up_swiglu_bwd: null dgu");
  int st = nmb::check_gemm(0, 0, m, f, k1, a1, lda1, wgu, ldwgu, false, nullptr, 0, dgu, lddgu);
  if (st != NMB_OK) return st;
  st = nmb::check_gemm(0, b_layout, m, f, k2, a2, lda2, wd, ldwd, false, nullptr, 0, dgu, lddgu);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(lddgu >= 2 * f, "gemm_gate_up_swiglu_bwd: dgu needs a leading dimension >= 2F");
  NMB_REQUIRE(act == nullptr || (ldact >= f && ldact % 8 == 0 && nmb::aligned16(act)),
              "gemm_gate_up_swiglu_bwd: act must be 16-byte aligned [M, F] with a leading dimension multiple of 8");
  NMB_REQUIRE_SUPPORTED(2 * (2 * f * ldwgu) < (int64_t{1} << 31),
                        "gemm_gate_up_swiglu_bwd: the gate/up weight spans more than 2 GiB");
  if (m == 0 || f == 0) return NMB_OK;
  const nmb::Plan none{0, 1, 0, 0.0};
  nmb::GemmArgs g1 = nmb::make_args(m, f, k1, 1.f, a1, lda1, wgu, ldwgu, 0.f, nullptr, 0, nullptr, 0, nullptr, none);
  nmb::GemmArgs g2 = nmb::make_args(m, f, k2, 1.f, a2, lda2, wd, ldwd, 0.f, nullptr, 0, act, ldact, nullptr, none);
  g2.swb_dgu = static_cast<nmb::bf16*>(dgu);
  g2.swb_lddgu = lddgu;
  st = nmb::prepare<256, 128>(g2);
  if (st != NMB_OK) return st;
  if (b_layout == 0)
    hipLaunchKernelGGL((nmb::gemm_gu_swb_kernel<true>), dim3(static_cast<unsigned>(g2.per_xcd * 8)), dim3(512),
                       0, stream, g1, g2);
  else
    hipLaunchKernelGGL((nmb::gemm_gu_swb_kernel<false>), dim3(static_cast<unsigned>(g2.per_xcd * 8)), dim3(512),
                       0, stream, g1, g2);
  NMB_CHECK_LAUNCH("gemm gate_up swiglu_bwd");
  return NMB_OK;
}
