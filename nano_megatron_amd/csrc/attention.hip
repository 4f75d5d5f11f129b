// Causal / non-causal MHA-GQA attention forward and backward for gfx950.
//
// Follows TorchKernelBackend.local_attention (reference
// nn/kernels/torch_backend.py:25-76: softmax(Q K^T * scale + mask) V with the
// mask key_pos <= sequence_offset + query_pos) and the ring maths of
// context_parallel/ring.py:104-250 (online max/sum merge over K/V blocks with
// absolute-position causal masks, lse = m + log l; backward
// delta = rowsum(dO * O), P = exp(S - lse), dS = P (dP - delta)).
//
// bf16 path (head_dim 64 or 128): v_mfma_f32_16x16x32_bf16, fp32 accumulate.
//   Forward and dQ kernels compute S^T = K Q^T so that every lane holds the
//   scores of ONE query (lane % 16) for 16 keys: the softmax statistics are
//   per-lane scalars, the O^T / dQ^T accumulators are rescaled per lane, and the
//   probabilities feed the next MFMA as its B operand straight from registers
//   (the 32-deep K index of that MFMA is a fixed permutation of keys that the
//   A operand, read from LDS with transposing reads, follows as well).
//   The dK/dV kernel uses S = Q K^T the same way with the roles of queries and
//   keys exchanged.  K/V (or Q/dO) tiles stream from HBM into LDS by direct
//   loads, once per workgroup, in their row-major layout.
//   GQA reads KV head h / (Hq / Hkv) directly; the dK/dV workgroup of a KV
//   head loops over its query heads, so no repeat is materialised and no
//   atomics are used (deterministic).
// fp32 path: one wavefront per query (or key) row, fp32 FMA, for the fp32
//   parity configuration.
#include <math.h>

#include <atomic>
#include <mutex>

#include "common.h"
#include "dropout_math.h"
#include "lds_dma.h"

namespace nmb {
namespace {

constexpr int kMaxBlocks = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct KVBlocks {
  const void* k[kMaxBlocks];
  const void* v[kMaxBlocks];
  void* dk[kMaxBlocks];
  void* dv[kMaxBlocks];
  int64_t koff[kMaxBlocks];
};

struct AttnShape {
  int B, Hq, Hkv, Sq, Sk, nblk, causal;
  int64_t q_sb, q_ss, q_sh;
  int64_t kv_sb, kv_ss, kv_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t q_offset;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
};

// The RoPE backward fused into the dQ / dK stores: the gradient of the
// rotated q (k) is rotated by -theta (reference nn/rotary.py:27-38; the
// transpose of rotate_half is -rotate_half), with the rotary kernel's
// roundings, the position of local token index i being pos[b * pos_bstride + i]
// or pos_offset + i.
struct RopeGrad {
  const float* cos;  // fp32 [n_pos, D/2]
  const float* sin;
  const int32_t* pos;
  int64_t pos_bstride, pos_offset;
  int n_pos;
};

// Rotation by -theta of the pair (x1, x2) = (g[d], g[d + D/2]) at table entry
// (crow, srow)[d]; bad poisons (out-of-table position).
__device__ __forceinline__ void rope_back(float x1, float x2, float cf, float sf, bool bad, bf16& o1, bf16& o2) {
  const float c = round_as<bf16>(cf);
  const float sn = -round_as<bf16>(sf);
  float r1 = round_as<bf16>(add_rn(round_as<bf16>(mul_rn(x1, c)), round_as<bf16>(mul_rn(-x2, sn))));
  float r2 = round_as<bf16>(add_rn(round_as<bf16>(mul_rn(x2, c)), round_as<bf16>(mul_rn(x1, sn))));
  if (bad) r1 = r2 = __builtin_nanf("");
  o1 = static_cast<bf16>(r1);
  o2 = static_cast<bf16>(r2);
}

__device__ __forceinline__ int64_t rope_pos(const RopeGrad& rg, int b, int i, bool* bad) {
  int64_t pos = rg.pos != nullptr ? static_cast<int64_t>(rg.pos[b * rg.pos_bstride + i]) : rg.pos_offset + i;
  *bad = pos < 0 || pos >= rg.n_pos;
  return *bad ? 0 : pos;
}

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

// exp2 as the raw v_exp_f32: results below 2^-126 flush to 0, which is
// immaterial for softmax weights (the library exp2 adds a 5-instruction
// denormal range fix-up around every exponential).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Number of 64-key tiles of a block that any query up to absolute position
// q_last can see.
__device__ __forceinline__ int visible_key_tiles(const AttnShape& p, int64_t koff, int64_t q_last) {
  int n = (p.Sk + 63) >> 6;
  if (p.causal) {
    const int64_t lim = q_last - koff;
    if (lim < 0) return 0;
    const int64_t t = (lim >> 6) + 1;
    if (t < n) n = static_cast<int>(t);
  }
  return n;
}

// Blocks are dispatched round-robin over the 8 XCDs (block L runs on XCD L % 8,
// each XCD with its own L2).  Work item w = (L % 8) * per_xcd + L / 8 puts
// consecutive items -- the q-tiles of one head, which read the same K/V -- on
// the same XCD.  Returns -1 for the padding blocks of the last round.
__device__ __forceinline__ int xcd_item(int items, int per_xcd) {
  const int L = static_cast<int>(blockIdx.x);
  const int w = (L % 8) * per_xcd + L / 8;
  return w < items ? w : -1;
}

// Advance (blk, kt) to the next visible K/V tile of the concatenated blocks;
// nt holds the visible tile count of block blk (recomputed only when the
// block changes).
__device__ __forceinline__ void next_tile(const AttnShape& p, const KVBlocks& kv, int64_t q_last,
                                          int& blk, int& kt, int& nt) {
  if (++kt < nt) return;
  kt = 0;
  for (++blk; blk < p.nblk; ++blk) {
    nt = visible_key_tiles(p, kv.koff[blk], q_last);
    if (nt > 0) return;
  }
}

__device__ __forceinline__ int first_block(const AttnShape& p, const KVBlocks& kv, int64_t q_last,
                                           int& nt) {
  int blk = 0;
  nt = 0;
  for (; blk < p.nblk; ++blk) {
    nt = visible_key_tiles(p, kv.koff[blk], q_last);
    if (nt > 0) break;
  }
  return blk;
}

// Largest tile-relative key index (key = k0 + index) visible to a query at
// absolute position qa: keys beyond Sk are never visible, and with causal
// masking key position koff + k0 + index must not exceed qa.
__device__ __forceinline__ int mask_limit(const AttnShape& p, int64_t koff, int k0, int64_t qa) {
  int64_t lim = static_cast<int64_t>(p.Sk) - 1 - k0;
  if (p.causal) {
    const int64_t c = qa - koff - k0;
    if (c < lim) lim = c;
  }
  if (lim < -1) lim = -1;
  if (lim > 1 << 20) lim = 1 << 20;
  return static_cast<int>(lim);
}

// ---------------------------------------------------------------- forward
// Workgroup = NWV wavefronts x TQ column tiles of 16 queries of one (batch,
// head): column tile t of wave w holds queries 16 NWV t + 16 w .. +15 of the
// workgroup's 16 NWV TQ queries, so under causal masking every wave sees about
// the same keys (balanced), and a tile whose first key lies beyond all queries
// of a column tile is skipped for that column tile (wave-uniform).  K/V stream
// through LDS in 64-key tiles, three tiles ahead of the one computed.  Scores
// stay raw; exp2(s * c - m * c) folds the softmax scale into one FMA per score.
// log2-domain lse for P = exp2(S * scale_log2 - lse2); a query with no visible
// key (lse = -inf) maps to +inf so that every P of its row is 0.
__device__ __forceinline__ float lse_to_log2(float v) {
  return v == -__builtin_inff() ? __builtin_inff() : v * kLog2e;
}

// 64-row x D bf16 tiles (K, V, Q, dO) stream from HBM straight into LDS
// (buffer_load ... lds: no register round trip), kStages deep, so kStages - 1
// tiles are in flight while one is computed.  A tile keeps the row-major
// layout with its 16-byte chunks swizzled: chunk c of row r in slot
// c ^ swz(r).  The swizzle serves both fragment kinds without bank conflicts
// (SQ_LDS_BANK_CONFLICT reads zero for each kind alone on gfx950):
//  * row fragments (an MFMA operand holding 8 consecutive columns of a row per
//    lane; 16 rows per lane group): one ds_read_b128;
//  * column fragments (8 rows of one column per lane: rows r0 + 4g .. +3 and
//    r0 + 16 + 4g .. +3 of a 32-row chunk, the key/query order in which the
//    score accumulators hold P and dS): two ds_read_b64_tr_b16.
// (2 ((r >> 1) & 3) + ((r >> 3) & 1) at D 64 and 2 (r & 7) + ((r >> 3) & 1) at
// D 128 keep the column reads conflict-free but give every row read a two-way
// conflict; r & 15 at D 128 the reverse.)
template <int D>
struct Tile64 {
  static constexpr int kElems = 64 * D;
  __device__ static int swz(int r) { return D == 64 ? (r & 7) : 2 * (r & 7); }
  __device__ static int at(int r, int col) { return r * D + 8 * ((col >> 3) ^ swz(r)) + (col & 7); }
  // row r, columns col .. col + 7 (col a multiple of 8)
  __device__ static bf16x8 row8(const bf16* t, int r, int col) { return ld8(t + at(r, col)); }
  // lane (l16, g): column c0 + l16, rows r0 + 4g .. +3 then r0 + 16 + 4g .. +3
  __device__ static bf16x8 col8(const bf16* t, int r0, int c0, int l16, int g) {
    const int r = r0 + 4 * g + (l16 >> 2), cc = c0 + 4 * (l16 & 3);
    return ld_tr(t + at(r, cc), t + at(r + 16, cc));
  }
};

// One wave's share (of NW waves) of the direct loads of a 64-row tile: load j
// fills LDS bytes [1024 (wave P + j), + 1024) of the tile; lane l's 16 bytes
// are chunk slot s of row r there, read from global chunk s ^ swz(r).
template <int D, int NW = 4>
struct TileStream {
  using Tile = Tile64<D>;
  static constexpr int P = Tile::kElems * 2 / 1024 / NW;  // 1 KB loads per wave per tile
  static_assert(P >= 1 && Tile::kElems * 2 % (1024 * NW) == 0, "a tile splits evenly over the waves");
  uint32_t off[P];  // byte offset from row 0 of the tile
  int row[P];

  __device__ void init(int64_t row_stride, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int e = (1024 * (wave * P + j) + 16 * lane) / 2;  // element offset within the tile
      const int r = e / D, sl = (e % D) / 8;
      row[j] = r;
      off[j] = static_cast<uint32_t>(r * row_stride * 2) + 16u * static_cast<uint32_t>(sl ^ Tile::swz(r));
    }
  }

  // rows r0 .. r0 + 63 (r0 * row bytes = r0_bytes) of a matrix of nrows rows;
  // rows at and past nrows read as zeros
  __device__ __forceinline__ void issue(const i32x4& rs, bf16* dst, int r0, int nrows, uint32_t r0_bytes,
                                        int wave) const {
#pragma unroll
    for (int j = 0; j < P; ++j)
      load_lds16(rs, dst + 512 * (wave * P + j), r0 + row[j] < nrows ? r0_bytes + off[j] : kOOB);
  }
};

// FL (from LSE): the softmax statistics are given (lse read, not written), so
// P = exp2(S * scale_log2 - lse2) directly: no running maximum, rescale or
// row sum, and O = P V needs no final division.
//
// NWV wavefronts per workgroup (4 or 8).  With 8 at head dim 64 a workgroup
// holds 512 queries, all of one (batch, head) at sequence length 512, so a CU
// runs one head's whole causal triangle with every wave busy to the end,
// instead of a light and a heavy query tile whose light half leaves one wave
// per SIMD for the second half.  For longer sequences (many query tiles per
// head) two column tiles per wave and three 4-wave workgroups per CU (three
// waves per SIMD, three LDS stages) hide more latency.
template <int D, int TQ, int NWV, bool FL>
__global__ __launch_bounds__(64 * NWV, (D == 64 && NWV == 4) ? (TQ <= 2 ? 3 : 2) : 1) void attn_fwd_kernel(
    const bf16* __restrict__ q, KVBlocks kv, bf16* __restrict__ o, float* __restrict__ lse,
    AttnShape p, int n_qt, int items, int per_xcd) {
  constexpr int CT = 16 * NWV;  // query stride between a wave's column tiles
  constexpr int BQ = CT * TQ, BK = 64, KS = D / 32, DT = D / 16;
  constexpr int kStages = (D == 64 && NWV == 4 && TQ <= 2) ? 3 : 4;  // 48 or 64 KB of LDS at D 64
  // two column tiles: fragments read per MFMA step (fewer registers); four:
  // fragments held across the column tiles (the scores of four would not fit)
  constexpr bool kPhased = TQ <= 2;
  using Tile = Tile64<D>;
  constexpr int kLoads = 2 * TileStream<D, NWV>::P;  // this wave's loads per K/V tile pair
  __shared__ __attribute__((aligned(1024))) bf16 sK[kStages][Tile::kElems];
  __shared__ __attribute__((aligned(1024))) bf16 sV[kStages][Tile::kElems];

  const int w = xcd_item(items, per_xcd);
  if (w < 0) return;
  const int bh = w / n_qt;
  const int qt = n_qt - 1 - (w % n_qt);  // heavy causal tiles first within a head
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int l16 = lane & 15, g = lane >> 4;
  const int hk = h / (p.Hq / p.Hkv);
  const int qbase = qt * BQ + 16 * wave;  // column tile t: qbase + CT t + l16
  const float c = p.scale_log2;

  const bf16* qb = q + b * p.q_sb + h * p.q_sh;
  bf16x8 qf[TQ][KS];
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const int qi = qbase + CT * t + l16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[t][ks] = qi < p.Sq ? ld8(qb + static_cast<int64_t>(qi) * p.q_ss + ks * 32 + g * 8) : zero8();
  }
  // acc[t][DT] (without FL) accumulates the row sum of P: its A operand is a
  // ones row (lane group 0, l16 == 0), so the P V MFMAs sum P and the sum is
  // rescaled together with O
  constexpr int NA = FL ? DT : DT + 1;
  float m[TQ];
  f32x4 acc[TQ][NA];
  bf16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = static_cast<bf16>(l16 == 0 ? 1.f : 0.f);
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    m[t] = -__builtin_inff();
    if constexpr (FL) {
      // m holds lse2 of this lane's query (+inf for a query past the end)
      const int qi = qbase + CT * t + l16;
      m[t] = qi < p.Sq ? lse_to_log2(lse[(static_cast<int64_t>(b) * p.Hq + h) * p.Sq + qi])
                       : __builtin_inff();
    }
#pragma unroll
    for (int dt = 0; dt < NA; ++dt) acc[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Q (and the given LSE) land before the first K/V tile load is issued.  The
  // compiler counts only its own loads: one still pending where the loop
  // starts makes it wait for every outstanding load, the K/V tiles in flight
  // included, before the first MFMA of every iteration.
  wait_vmcnt<0>();
  const int64_t qa_wg_last = p.q_offset + min(qt * BQ + BQ - 1, p.Sq - 1);
  const int64_t kv_off = b * p.kv_sb + hk * p.kv_sh;
  // bytes from (b, key 0, hk) to the end of the last key row of a block (< 2^31, checked by the host)
  const uint32_t kv_bytes = static_cast<uint32_t>(((p.Sk - 1) * p.kv_ss + D) * 2);
  const uint32_t row_bytes = static_cast<uint32_t>(p.kv_ss * 2);
  TileStream<D, NWV> ld;
  ld.init(p.kv_ss, wave, lane);

  bf16* ob = o + b * p.o_sb + h * p.o_sh;
  float* lb = lse + (static_cast<int64_t>(b) * p.Hq + h) * p.Sq;
  // O (and the LSE) of column tile t, normalised by its row sum
  auto store_tile = [&](int t) {
    int qi = qbase + CT * t + l16;
    // opaque to the optimiser: the store addresses are formed here, not
    // hoisted out of the key-tile loop into registers held across it
    asm volatile("" : "+v"(qi));
    // the row sum sits in element 0 of the sum tile in lane group 0; every
    // lane group of the query needs it
    float l = 0.f;
    if constexpr (!FL) l = xor32_sum(xor16_sum(g == 0 ? acc[t][NA - 1][0] : 0.f));
    if (qi >= p.Sq) return;
    const float inv = FL ? 1.f : (l > 0.f ? 1.f / l : 0.f);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      bf16x4 wv;
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[e] = static_cast<bf16>(acc[t][dt][e] * inv);
      *reinterpret_cast<bf16x4*>(ob + static_cast<int64_t>(qi) * p.o_ss + dt * 16 + g * 4) = wv;
    }
    if (!FL && g == 0) lb[qi] = l > 0.f ? (m[t] * c + log2f(l)) * kLn2 : -__builtin_inff();
  };
  // With one K/V block the key tiles come in ascending order, and under
  // causal masking a column tile is finished at the last tile it sees: its
  // output is stored then, so that the stores overlap the remaining tiles'
  // work instead of all following the loop (for the four-column-tile waves of
  // short sequences, where that burst is a large part of the kernel).  (The stores count in vmcnt
  // beside the tile loads; as loads complete in order, the wait at the top
  // of the loop still implies that the oldest tile has landed.)
  bool stored[TQ];
  int fin[TQ];  // first key (tile-relative to the block) of column tile t's last tile, or -1
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    stored[t] = false;
    fin[t] = -1;
    if (p.nblk == 1) {
      int64_t last_key = p.Sk - 1;
      if (p.causal) last_key = min(last_key, p.q_offset + min(qbase + CT * t + 15, p.Sq - 1) - kv.koff[0]);
      if (last_key >= 0) fin[t] = static_cast<int>(last_key / BK) * BK;
    }
  }

  // compute cursor (blk, kt) and load cursor (pblk, pkt) over the visible tiles
  int nt = 0;
  int blk = first_block(p, kv, qa_wg_last, nt), kt = 0;
  int pnt = nt, pblk = blk, pkt = 0;
  // loads of the load cursor's tile into a stage; past the last tile, loads of
  // zeros (every iteration issues and waits for the same number of loads)
  auto issue = [&](int stage) {
    if (pblk < p.nblk) {
      const uint32_t r0b = static_cast<uint32_t>(pkt * BK) * row_bytes;
      ld.issue(make_rsrc(static_cast<const bf16*>(kv.k[pblk]) + kv_off, kv_bytes), sK[stage], pkt * BK, p.Sk, r0b, wave);
      ld.issue(make_rsrc(static_cast<const bf16*>(kv.v[pblk]) + kv_off, kv_bytes), sV[stage], pkt * BK, p.Sk, r0b, wave);
      next_tile(p, kv, qa_wg_last, pblk, pkt, pnt);
    } else {
      const i32x4 rz = make_rsrc(kv.k[0], 0);
      ld.issue(rz, sK[stage], 0, 0, 0u, wave);
      ld.issue(rz, sV[stage], 0, 0, 0u, wave);
    }
  };
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) issue(st);

  for (int it = 0; blk < p.nblk; ++it) {
    // this wave's loads of tile it have landed (those of the next kStages - 2
    // may still fly); after the barrier, everyone's have, and nobody reads the
    // stage of tile it - 1 any more: refill it with tile it + kStages - 1
    wait_vmcnt<(kStages - 2) * kLoads>();
    lds_barrier();
    issue((it + kStages - 1) % kStages);
    const bf16* tk = sK[it % kStages];
    const bf16* tv = sV[it % kStages];
    const int64_t koff = kv.koff[blk];
    const int k0 = kt * BK;
    next_tile(p, kv, qa_wg_last, blk, kt, nt);
    // per column tile: is any key of this tile visible, is masking needed?
    bool live[TQ], need_mask[TQ];
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      const int64_t qfirst = p.q_offset + qbase + CT * t;
      const int64_t qlast = p.q_offset + min(qbase + CT * t + 15, p.Sq - 1);
      live[t] = !(p.causal && koff + k0 > qlast) && (qbase + CT * t < p.Sq);
      need_mask[t] = (k0 + BK > p.Sk) || (p.causal && koff + k0 + BK - 1 > qfirst);
    }

    // softmax of one column tile's scores (in place, then packed into P, the
    // B operand of the P V MFMAs); rescales that tile's O and row sum
    auto softmax = [&](int t, f32x4 (&sc)[4], bf16x8 (&pt)[2]) {
      float tmax = -__builtin_inff();
      if (need_mask[t]) {
        // last visible tile-relative key index of this lane's query
        const int lim = mask_limit(p, koff, k0, p.q_offset + qbase + CT * t + l16);
#pragma unroll
        for (int mk = 0; mk < 4; ++mk)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // branch-free select: a conditional store into the vector element
            // under short-circuit control flow is not reliably kept
            const float sv = sc[mk][e];
            sc[mk][e] = (mk * 16 + g * 4 + e > lim) ? -__builtin_inff() : sv;
          }
      }
      if constexpr (FL) {
#pragma unroll
        for (int mk = 0; mk < 4; ++mk)
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[mk][e] = fast_exp2(fmaf(sc[mk][e], c, -m[t]));
      } else {
#pragma unroll
        for (int mk = 0; mk < 4; ++mk)
#pragma unroll
          for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, sc[mk][e]);
        tmax = xor32_max(xor16_max(tmax));
        // Lazy rescaling: the running maximum m moves only when the tile's
        // maximum exceeds it by more than 8 in the exp2 domain; otherwise P
        // stays below 2^8 and the fp32 accumulators absorb it.  O and the row
        // sum are rescaled together, so O / sum and m + log(sum) are unchanged.
        const bool grow = tmax > m[t] && (m[t] == -__builtin_inff() || (tmax - m[t]) * c > 8.f);
        if (__any(grow)) {  // wave-uniform
          const float alpha = grow ? fast_exp2((m[t] - tmax) * c) : 1.f;  // m = -inf: alpha = 0
          m[t] = grow ? tmax : m[t];
#pragma unroll
          for (int dt = 0; dt < NA; ++dt) acc[t][dt] *= alpha;
        }
        // no visible key yet: m = -inf, every score -inf, P = 0
        const float mc = m[t] == -__builtin_inff() ? 0.f : m[t] * c;
#pragma unroll
        for (int mk = 0; mk < 4; ++mk)
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[mk][e] = fast_exp2(fmaf(sc[mk][e], c, -mc));
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pt[s2][e] = static_cast<bf16>(sc[2 * s2][e]);
          pt[s2][4 + e] = static_cast<bf16>(sc[2 * s2 + 1][e]);
        }
    };
    if constexpr (kPhased) {
      // Three phases over the wave's column tiles: scores of every live
      // column tile (K fragments read per k step), softmax, then P V (V^T
      // fragments read per d tile).  Each fragment is still read from LDS once
      // per tile, but none is held across the phases.
      f32x4 s[TQ][4];
      bf16x8 pf[TQ][2];
#pragma unroll
      for (int t = 0; t < TQ; ++t)
#pragma unroll
        for (int mk = 0; mk < 4; ++mk) s[t][mk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 kk[4];
#pragma unroll
        for (int mk = 0; mk < 4; ++mk) kk[mk] = Tile::row8(tk, mk * 16 + l16, ks * 32 + g * 8);
#pragma unroll
        for (int t = 0; t < TQ; ++t)
          if (live[t]) {
#pragma unroll
            for (int mk = 0; mk < 4; ++mk) s[t][mk] = mfma16(kk[mk], qf[t][ks], s[t][mk]);
          }
      }
#pragma unroll
      for (int t = 0; t < TQ; ++t)
        if (live[t]) softmax(t, s[t], pf[t]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        bf16x8 vv[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) vv[s2] = Tile::col8(tv, 32 * s2, dt * 16, l16, g);
#pragma unroll
        for (int t = 0; t < TQ; ++t)
          if (live[t]) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) acc[t][dt] = mfma16(vv[s2], pf[t][s2], acc[t][dt]);
          }
      }
      if constexpr (!FL) {
#pragma unroll
        for (int t = 0; t < TQ; ++t)
          if (live[t]) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) acc[t][NA - 1] = mfma16(ones, pf[t][s2], acc[t][NA - 1]);
          }
      }
    } else {
      // K and V^T fragments of this tile, read from LDS once and held while
      // each column tile of the wave runs scores, softmax and P V in turn
      bf16x8 kfr[KS][4], vfr[DT][2];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int mk = 0; mk < 4; ++mk) kfr[ks][mk] = Tile::row8(tk, mk * 16 + l16, ks * 32 + g * 8);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) vfr[dt][s2] = Tile::col8(tv, 32 * s2, dt * 16, l16, g);
#pragma unroll
      for (int t = 0; t < TQ; ++t) {
        if (!live[t]) continue;
        f32x4 s[4];
#pragma unroll
        for (int mk = 0; mk < 4; ++mk) s[mk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int mk = 0; mk < 4; ++mk) s[mk] = mfma16(kfr[ks][mk], qf[t][ks], s[mk]);
        bf16x8 pf[2];
        softmax(t, s, pf);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) acc[t][dt] = mfma16(vfr[dt][s2], pf[s2], acc[t][dt]);
        if constexpr (!FL) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) acc[t][NA - 1] = mfma16(ones, pf[s2], acc[t][NA - 1]);
        }
      }
    }
    if constexpr (!kPhased) {
#pragma unroll
      for (int t = 0; t < TQ; ++t)
        if (live[t] && k0 == fin[t]) {
          store_tile(t);
          stored[t] = true;
        }
    }
  }
  // no load may still write this workgroup's LDS when it ends
  wait_vmcnt<0>();
#pragma unroll
  for (int t = 0; t < TQ; ++t)
    if (!stored[t]) store_tile(t);
}

// ---------------------------------------------------------------- delta (fp32 path)
// delta[b, h, i] = sum_d dO[b, i, h, d] * O[b, i, h, d] (fp32).
template <typename T>
__global__ __launch_bounds__(256) void attn_delta_kernel(const T* __restrict__ o,
                                                         const T* __restrict__ dout,
                                                         float* __restrict__ delta, AttnShape p,
                                                         int D) {
  const int64_t rows = static_cast<int64_t>(p.B) * p.Sq * p.Hq;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; r < rows;
       r += static_cast<int64_t>(gridDim.x) * 256) {
    const int h = static_cast<int>(r % p.Hq);
    const int64_t bi = r / p.Hq;
    const int i = static_cast<int>(bi % p.Sq);
    const int b = static_cast<int>(bi / p.Sq);
    const int64_t off = b * p.o_sb + static_cast<int64_t>(i) * p.o_ss + h * p.o_sh;
    float s = 0.f;
    for (int d = 0; d < D; ++d) s += to_f32(o[off + d]) * to_f32(dout[off + d]);
    delta[(static_cast<int64_t>(b) * p.Hq + h) * p.Sq + i] = s;
  }
}

// ---------------------------------------------------------------- dQ
// Same tiling as the forward (S^T = K Q^T per wave), NW waves of 32 queries.
// The prologue computes delta = rowsum(dO * O) for the workgroup's queries
// from the registers that hold dO and writes it for the dK/dV kernel, which
// runs next on the stream.  At head dim 128, 8 waves (two per SIMD).
template <int D, bool ROPE, int NW>
__global__ __launch_bounds__(64 * NW, D == 64 ? 2 : 1) void attn_bwd_dq_kernel(
    const bf16* __restrict__ q, KVBlocks kv, const bf16* __restrict__ o,
    const bf16* __restrict__ dout, const float* __restrict__ lse, float* __restrict__ delta,
    float* __restrict__ lse2_out, bf16* __restrict__ dq, AttnShape p, int n_qt, int items, int per_xcd,
    RopeGrad rg) {
  constexpr int BQ = 32 * NW, BK = 64, KS = D / 32, DT = D / 16;
  constexpr int kStages = 4;
  using Tile = Tile64<D>;
  constexpr int kLoads = 2 * TileStream<D, NW>::P;  // this wave's loads per K/V tile pair
  __shared__ __attribute__((aligned(1024))) bf16 sK[kStages][Tile::kElems];
  __shared__ __attribute__((aligned(1024))) bf16 sV[kStages][Tile::kElems];

  const int w = xcd_item(items, per_xcd);
  if (w < 0) return;
  // item = (b * Hq + h) * n_pairs + pair.  At head dim 64 pair j covers query
  // tiles n_qt - 1 - j and j one after the other (equal causal work per
  // workgroup; the middle tile of an odd n_qt is alone); at 128 a workgroup
  // takes one query tile (heavy ones first).
  constexpr bool kPair = D == 64;
  const int n_pairs = kPair ? (n_qt + 1) / 2 : n_qt;
  const int bh = w / n_pairs;
  const int pj = w % n_pairs;
  const int n_sub = kPair && n_qt - 1 - pj != pj ? 2 : 1;
  auto qtile = [&](int sub) { return sub == 0 ? n_qt - 1 - pj : pj; };
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int l16 = lane & 15, g = lane >> 4;
  const int hk = h / (p.Hq / p.Hkv);
  const float c = p.scale_log2;

  const bf16* qb = q + b * p.q_sb + h * p.q_sh;
  const bf16* ob = o + b * p.o_sb + h * p.o_sh;
  const bf16* db = dout + b * p.o_sb + h * p.o_sh;
  const float* lb = lse + (static_cast<int64_t>(b) * p.Hq + h) * p.Sq;
  float* deb = delta + (static_cast<int64_t>(b) * p.Hq + h) * p.Sq;
  float* l2b = lse2_out + (static_cast<int64_t>(b) * p.Hq + h) * p.Sq;
  bf16* dqb = dq + b * p.q_sb + h * p.q_sh;
  bf16x8 qf[2][KS], df[2][KS];
  float lse2[2], dl[2];
  f32x4 acc[2][DT];
  int q0 = 0;  // this wave's first query of the current sub-item
  // a sub-item's Q and dO fragments, delta = rowsum(dO * O) and the base-2
  // LSE (both also written for the dK/dV kernel, which runs next); dQ to zero
  auto start = [&](int sub) {
    q0 = qtile(sub) * BQ + wave * 32;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int qi = q0 + 16 * t + l16;
      const bool ok = qi < p.Sq;
      float part = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[t][ks] = ok ? ld8(qb + static_cast<int64_t>(qi) * p.q_ss + ks * 32 + g * 8) : zero8();
        df[t][ks] = ok ? ld8(db + static_cast<int64_t>(qi) * p.o_ss + ks * 32 + g * 8) : zero8();
        const bf16x8 of = ok ? ld8(ob + static_cast<int64_t>(qi) * p.o_ss + ks * 32 + g * 8) : zero8();
#pragma unroll
        for (int e = 0; e < 8; ++e) part += static_cast<float>(df[t][ks][e]) * static_cast<float>(of[e]);
      }
      part = xor32_sum(xor16_sum(part));
      dl[t] = part;
      lse2[t] = ok ? lse_to_log2(lb[qi]) : __builtin_inff();
      if (ok && g == 0) {
        deb[qi] = part;
        l2b[qi] = lse2[t];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // lane holds dQ[q0 + 16 t + l16][d = 16 dt + 4 g + e]; d and d + D/2 are dt and dt + DT/2
  auto finish = [&]() {
    if constexpr (ROPE) {
      // every cos/sin value (4 consecutive d per 16-byte load) is loaded and
      // every output computed before the first store: loads and stores share
      // one counter, so a wait after a store would also wait for it.  A query
      // past the sequence reads a valid row and stores nothing.
      f32x4 cw[2][DT / 2], sw[2][DT / 2];
      bool bad[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int64_t pos = rope_pos(rg, b, min(q0 + 16 * t + l16, p.Sq - 1), &bad[t]);
#pragma unroll
        for (int dt = 0; dt < DT / 2; ++dt) {
          cw[t][dt] = *reinterpret_cast<const f32x4*>(rg.cos + pos * (D / 2) + dt * 16 + g * 4);
          sw[t][dt] = *reinterpret_cast<const f32x4*>(rg.sin + pos * (D / 2) + dt * 16 + g * 4);
        }
      }
      bf16x4 w1[2][DT / 2], w2[2][DT / 2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            bf16 r1, r2;
            rope_back(round_as<bf16>(acc[t][dt][e] * p.scale), round_as<bf16>(acc[t][dt + DT / 2][e] * p.scale),
                      cw[t][dt][e], sw[t][dt][e], bad[t], r1, r2);
            w1[t][dt][e] = r1;
            w2[t][dt][e] = r2;
          }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int qi = q0 + 16 * t + l16;
        if (qi >= p.Sq) continue;
#pragma unroll
        for (int dt = 0; dt < DT / 2; ++dt) {
          *reinterpret_cast<bf16x4*>(dqb + static_cast<int64_t>(qi) * p.q_ss + dt * 16 + g * 4) = w1[t][dt];
          *reinterpret_cast<bf16x4*>(dqb + static_cast<int64_t>(qi) * p.q_ss + D / 2 + dt * 16 + g * 4) = w2[t][dt];
        }
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int qi = q0 + 16 * t + l16;
      if (qi >= p.Sq) continue;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        bf16x4 wv;
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[e] = static_cast<bf16>(acc[t][dt][e] * p.scale);
        *reinterpret_cast<bf16x4*>(dqb + static_cast<int64_t>(qi) * p.q_ss + dt * 16 + g * 4) = wv;
      }
    }
  };
  // last absolute query position of a sub-item's workgroup tile
  auto wg_last = [&](int sub) { return p.q_offset + min(qtile(sub) * BQ + BQ - 1, p.Sq - 1); };

  const int64_t kv_off = b * p.kv_sb + hk * p.kv_sh;
  const uint32_t kv_bytes = static_cast<uint32_t>(((p.Sk - 1) * p.kv_ss + D) * 2);
  const uint32_t row_bytes = static_cast<uint32_t>(p.kv_ss * 2);
  TileStream<D, NW> ld;
  ld.init(p.kv_ss, wave, lane);

  // K/V tiles stream through LDS as in the forward: the visible tiles of the
  // first sub-item, then those of the second (load cursor psub/pblk/pkt,
  // compute cursor csub/blk/kt)
  int pnt = 0, psub = 0;
  int pblk = first_block(p, kv, wg_last(0), pnt), pkt = 0;
  auto advance_load = [&]() {
    next_tile(p, kv, wg_last(psub), pblk, pkt, pnt);
    while (pblk >= p.nblk && psub + 1 < n_sub) {
      ++psub;
      pblk = first_block(p, kv, wg_last(psub), pnt);
      pkt = 0;
    }
  };
  if (pblk >= p.nblk && n_sub == 2) {  // the first sub-item sees no key
    psub = 1;
    pblk = first_block(p, kv, wg_last(1), pnt);
  }
  auto issue = [&](int stage) {
    if (pblk < p.nblk) {
      const uint32_t r0b = static_cast<uint32_t>(pkt * BK) * row_bytes;
      ld.issue(make_rsrc(static_cast<const bf16*>(kv.k[pblk]) + kv_off, kv_bytes), sK[stage], pkt * BK, p.Sk, r0b, wave);
      ld.issue(make_rsrc(static_cast<const bf16*>(kv.v[pblk]) + kv_off, kv_bytes), sV[stage], pkt * BK, p.Sk, r0b, wave);
      advance_load();
    } else {
      const i32x4 rz = make_rsrc(kv.k[0], 0);
      ld.issue(rz, sK[stage], 0, 0, 0u, wave);
      ld.issue(rz, sV[stage], 0, 0, 0u, wave);
    }
  };
  start(0);
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) issue(st);

  int nt = 0, csub = 0;
  int blk = first_block(p, kv, wg_last(0), nt), kt = 0;
  for (int it = 0;; ++it) {
    bool switched = false;
    while (blk >= p.nblk && csub + 1 < n_sub) {
      // the next sub-item: store this one's dQ, load the next one's Q/dO; the
      // stores share vmcnt with the tile loads and need not retire in order,
      // so this iteration waits for everything
      finish();
      ++csub;
      start(csub);
      blk = first_block(p, kv, wg_last(csub), nt);
      kt = 0;
      switched = true;
    }
    if (blk >= p.nblk) break;
    if (switched) wait_vmcnt<0>();
    else wait_vmcnt<(kStages - 2) * kLoads>();
    lds_barrier();
    issue((it + kStages - 1) % kStages);
    const bf16* tk = sK[it % kStages];
    const bf16* tv = sV[it % kStages];
    const int64_t koff = kv.koff[blk];
    const int k0 = kt * BK;
    next_tile(p, kv, wg_last(csub), blk, kt, nt);
    const int64_t qa_wave_first = p.q_offset + q0;
    const int64_t qa_wave_last = p.q_offset + min(q0 + 31, p.Sq - 1);
    if (p.causal && koff + k0 > qa_wave_last) continue;
    const bool need_mask = (k0 + BK > p.Sk) || (p.causal && koff + k0 + BK - 1 > qa_wave_first);

    bf16x8 dsf[2][2];
    int lim[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
      lim[t] = need_mask ? mask_limit(p, koff, k0, p.q_offset + q0 + 16 * t + l16) : BK;
    // per 16-key slice mk: S^T and dP^T (K and V row fragments), then
    // dS = P (dP - delta) packed into the B operand of the dQ MFMAs; only one
    // slice's scores are live at a time.  A tile that every query of the wave
    // sees in full takes the element loop without the mask selects: at D 64
    // a second copy of the whole slice loop, at D 128 (where that copy would
    // spill) a branch per slice around the element loop.
    auto slices = [&](auto masked) {
#pragma unroll
    for (int mk = 0; mk < 4; ++mk) {
      f32x4 s[2], dp[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 ak = Tile::row8(tk, mk * 16 + l16, ks * 32 + g * 8);
        const bf16x8 av = Tile::row8(tv, mk * 16 + l16, ks * 32 + g * 8);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          s[t] = mfma16(ak, qf[t][ks], s[t]);
          dp[t] = mfma16(av, df[t][ks], dp[t]);
        }
      }
      auto elems = [&](auto sel) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float pv = fast_exp2(fmaf(s[t][e], c, -lse2[t]));
            if constexpr (decltype(sel)::value) pv = (mk * 16 + g * 4 + e > lim[t]) ? 0.f : pv;
            dsf[mk >> 1][t][4 * (mk & 1) + e] = static_cast<bf16>(pv * (dp[t][e] - dl[t]));
          }
      };
      if constexpr (decltype(masked)::value && D == 128) {
        if (need_mask) elems(std::true_type{});
        else elems(std::false_type{});
      } else {
        elems(masked);
      }
    }
    };
    if constexpr (D == 64) {
      if (need_mask) slices(std::true_type{});
      else slices(std::false_type{});
    } else {
      slices(std::true_type{});
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const bf16x8 a = Tile::col8(tk, 32 * s2, dt * 16, l16, g);
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t][dt] = mfma16(a, dsf[s2][t], acc[t][dt]);
      }
    }
  }
  // no load may still write this workgroup's LDS when it ends
  wait_vmcnt<0>();
  finish();
}

// ---------------------------------------------------------------- dK, dV
// Workgroup = 128 keys of one (batch, KV head, block).  Head dim 64: 4 waves,
// key tile j (16 keys) of wave w holds keys 64 j + 16 w .. +15 of the
// workgroup's range (interleaved, so causal work is balanced across waves),
// so each Q/dO fragment read from LDS feeds two MFMA tiles.  Head dim 128:
// 8 waves of one 16-key tile each (two waves per SIMD; the dK/dV accumulators
// of a second tile would not fit beside them).  Loops over the query heads of the GQA group and
// over the 64-query tiles that can see these keys, with the next Q/dO tile's
// global reads in flight during the current tile's MFMA work.
template <int D, bool ROPE, int NW>
__global__ __launch_bounds__(64 * NW, D == 64 ? 2 : 1) void attn_bwd_dkdv_kernel(
    const bf16* __restrict__ q, KVBlocks kv, const bf16* __restrict__ dout,
    const float* __restrict__ lse2, const float* __restrict__ delta, AttnShape p, int n_kt,
    int items, int per_xcd, RopeGrad rg) {
  // KT key tiles of 16 per wave, KSTR keys apart
  constexpr int BQ = 64, KT = 128 / (16 * NW), KSTR = 16 * NW, BKW = KSTR * KT, KS = D / 32, DT = D / 16;
  static_assert(BKW == 128, "128 keys per workgroup");
  constexpr int kStages = 4;
  // P and dS per 32-query half (fewer registers: two waves per SIMD at D 128)
  // or for all 64 queries at once (more independent MFMAs: faster at D 64)
  constexpr bool kSliced = D == 128;
  using Tile = Tile64<D>;
  // this wave's loads per query tile: Q, dO, and one 256-byte row statistic
  // (even waves fetch lse2, odd waves delta)
  constexpr int kLoads = 2 * TileStream<D, NW>::P + 1;
  __shared__ __attribute__((aligned(1024))) bf16 sQ[kStages][Tile::kElems];
  __shared__ __attribute__((aligned(1024))) bf16 sD[kStages][Tile::kElems];
  __shared__ __attribute__((aligned(256))) float sStat[kStages][NW][BQ];

  const int w = xcd_item(items, per_xcd);
  if (w < 0) return;
  // item = ((b * nblk + blk) * Hkv + hk) * n_pairs + pair.  At head dim 64
  // pair j covers key tiles j and n_kt - 1 - j one after the other, so under
  // causal masking every workgroup sees about the same number of query tiles
  // (the middle tile of an odd n_kt is alone); at 128 the registers of a
  // second tile's state do not fit, and a workgroup takes one key tile.
  constexpr bool kPair = D == 64;
  const int n_pairs = kPair ? (n_kt + 1) / 2 : n_kt;
  const int pj = w % n_pairs;
  const int rest = w / n_pairs;
  const int hk = rest % p.Hkv;
  const int bb = rest / p.Hkv;
  const int blk = bb % p.nblk;
  const int b = bb / p.nblk;
  const int n_sub = kPair && n_kt - 1 - pj != pj ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t koff = kv.koff[blk];
  const int group = p.Hq / p.Hkv;
  const float c = p.scale_log2;
  const int n_qt = (p.Sq + BQ - 1) / BQ;

  // per sub-item (key tile): first visible query tile and the iteration count
  auto sub_tile = [&](int sub) { return sub == 0 ? pj : n_kt - 1 - pj; };
  auto qt_begin_of = [&](int sub) {
    int first_q = 0;
    if (p.causal) {
      const int64_t fq = koff + sub_tile(sub) * BKW - p.q_offset;
      first_q = fq <= 0 ? 0 : (fq >= p.Sq ? p.Sq : static_cast<int>(fq));
    }
    return first_q / BQ;
  };
  const int qtb0 = qt_begin_of(0), qtb1 = n_sub == 2 ? qt_begin_of(1) : 0;
  const int n_iter0 = group * (n_qt - qtb0);
  const int n_iter1 = n_sub == 2 ? group * (n_qt - qtb1) : 0;
  const int total = n_iter0 + n_iter1;

  const int64_t kv_off = b * p.kv_sb + hk * p.kv_sh;
  const bf16* kb = static_cast<const bf16*>(kv.k[blk]) + kv_off;
  const bf16* vb = static_cast<const bf16*>(kv.v[blk]) + kv_off;
  bf16* dkb = static_cast<bf16*>(kv.dk[blk]) + kv_off;
  bf16* dvb = static_cast<bf16*>(kv.dv[blk]) + kv_off;
  bf16x8 kf[KT][KS], vf[KT][KS];
  f32x4 dka[KT][DT], dva[KT][DT];
  int kbase = 0;  // key tile j of this wave: kbase + KSTR j + l16
  // a sub-item's K/V fragments into registers and its accumulators to zero
  auto start = [&](int sub) {
    kbase = sub_tile(sub) * BKW + 16 * wave;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const int key = kbase + KSTR * j + l16;
      const bool ok = key < p.Sk;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[j][ks] = ok ? ld8(kb + static_cast<int64_t>(key) * p.kv_ss + ks * 32 + g * 8) : zero8();
        vf[j][ks] = ok ? ld8(vb + static_cast<int64_t>(key) * p.kv_ss + ks * 32 + g * 8) : zero8();
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dka[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        dva[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  // lane holds dK[key = kbase + KSTR j + 4 g + e][d = 16 dt + l16]
  auto finish = [&]() {
    if constexpr (ROPE) {
      // d = 16 dt + l16 and d + D/2 are dt and dt + DT/2 (one K/V block: key =
      // token index).  Every cos/sin value is loaded and every output computed
      // before the first store (a wait after a store would also wait for it);
      // a key past the sequence reads a valid row and stores nothing.
      float cw[KT][4][DT / 2], sw[KT][4][DT / 2];
      bool bad[KT][4];
#pragma unroll
      for (int j = 0; j < KT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t pos = rope_pos(rg, b, min(kbase + KSTR * j + g * 4 + e, p.Sk - 1), &bad[j][e]);
#pragma unroll
          for (int dt = 0; dt < DT / 2; ++dt) {
            cw[j][e][dt] = rg.cos[pos * (D / 2) + dt * 16 + l16];
            sw[j][e][dt] = rg.sin[pos * (D / 2) + dt * 16 + l16];
          }
        }
      bf16 ko[KT][4][DT], vo[KT][4][DT];
#pragma unroll
      for (int j = 0; j < KT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
          for (int dt = 0; dt < DT / 2; ++dt)
            rope_back(round_as<bf16>(dka[j][dt][e] * p.scale), round_as<bf16>(dka[j][dt + DT / 2][e] * p.scale),
                      cw[j][e][dt], sw[j][e][dt], bad[j][e], ko[j][e][dt], ko[j][e][dt + DT / 2]);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) vo[j][e][dt] = static_cast<bf16>(dva[j][dt][e]);
        }
#pragma unroll
      for (int j = 0; j < KT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = kbase + KSTR * j + g * 4 + e;
          if (key >= p.Sk) continue;
          bf16* dkr = dkb + static_cast<int64_t>(key) * p.kv_ss;
          bf16* dvr = dvb + static_cast<int64_t>(key) * p.kv_ss;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            dkr[dt * 16 + l16] = ko[j][e][dt];
            dvr[dt * 16 + l16] = vo[j][e][dt];
          }
        }
      return;
    }
#pragma unroll
    for (int j = 0; j < KT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kbase + KSTR * j + g * 4 + e;
        if (key >= p.Sk) continue;
        bf16* dkr = dkb + static_cast<int64_t>(key) * p.kv_ss;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) dkr[dt * 16 + l16] = static_cast<bf16>(dka[j][dt][e] * p.scale);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          dvb[static_cast<int64_t>(key) * p.kv_ss + dt * 16 + l16] = static_cast<bf16>(dva[j][dt][e]);
      }
  };
  // Stream tile i is query tile qt of query head hk * group + ih: the first
  // sub-item's tiles qtb0 .. n_qt - 1 of each head of the group in turn, then
  // from stream tile n_iter0 on the second's from qtb1.  The loads and the
  // compute each walk it one tile per step (no division per iteration).
  const int qt_first = n_iter0 > 0 ? qtb0 : qtb1;
  auto step_qt = [&](int next, int& qt) {  // qt of stream tile next, from that of next - 1
    const bool wrap = next == n_iter0 || qt + 1 == n_qt;
    qt = wrap ? (next < n_iter0 ? qtb0 : qtb1) : qt + 1;
    return wrap;
  };
  // Q / dO tiles and their row statistics stream through LDS (kStages deep),
  // across the two sub-items.  Past the last iteration the loads read zeros.
  TileStream<D, NW> lq, ldo;
  lq.init(p.q_ss, wave, lane);
  ldo.init(p.o_ss, wave, lane);
  const uint32_t q_bytes = static_cast<uint32_t>(((p.Sq - 1) * p.q_ss + D) * 2);
  const uint32_t o_bytes = static_cast<uint32_t>(((p.Sq - 1) * p.o_ss + D) * 2);
  int l_ih = 0, l_qt = qt_first;  // the next tile to load
  auto issue = [&](int it, int stage) {
    if (it < total) {
      const int h = hk * group + l_ih, q0 = l_qt * BQ;
      if (step_qt(it + 1, l_qt)) l_ih = it + 1 == n_iter0 ? 0 : l_ih + 1;
      lq.issue(make_rsrc(q + b * p.q_sb + h * p.q_sh, q_bytes), sQ[stage], q0, p.Sq,
               static_cast<uint32_t>(q0) * static_cast<uint32_t>(p.q_ss * 2), wave);
      ldo.issue(make_rsrc(dout + b * p.o_sb + h * p.o_sh, o_bytes), sD[stage], q0, p.Sq,
                static_cast<uint32_t>(q0) * static_cast<uint32_t>(p.o_ss * 2), wave);
      const float* stat = ((wave & 1) ? delta : lse2) + (static_cast<int64_t>(b) * p.Hq + h) * p.Sq;
      load_lds4(make_rsrc(stat, static_cast<uint32_t>(p.Sq * 4)), &sStat[stage][wave][0],
                q0 + lane < p.Sq ? static_cast<uint32_t>(4 * (q0 + lane)) : kOOB);
    } else {
      const i32x4 rz = make_rsrc(q, 0);
      lq.issue(rz, sQ[stage], 0, 0, 0u, wave);
      ldo.issue(rz, sD[stage], 0, 0, 0u, wave);
      load_lds4(rz, &sStat[stage][wave][0], kOOB);
    }
  };
  start(0);
  // K/V in registers before the first Q/dO tile load is issued (as in the
  // forward: a pending compiler-visible load at the loop would make every
  // iteration wait for the tiles in flight)
  wait_vmcnt<0>();
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) issue(st, st);
  bool switched = false;
  int c_qt = qt_first;  // the tile computed
  for (int it = 0; it < total; ++it) {
    if (it == n_iter0 && n_sub == 2) {
      // first iteration of the second key tile: store the first one's dK/dV
      // and load the second's K/V; the stores share vmcnt with the tile
      // loads and need not retire in order, so wait for everything
      finish();
      start(1);
      switched = true;
      wait_vmcnt<0>();
    } else {
      wait_vmcnt<(kStages - 2) * kLoads>();
    }
    lds_barrier();
    issue(it + kStages - 1, (it + kStages - 1) % kStages);
    const bf16* tq = sQ[it % kStages];
    const bf16* td = sD[it % kStages];
    const float* sL = sStat[it % kStages][0];
    const float* sDl = sStat[it % kStages][1];
    const int q0 = c_qt * BQ;
    step_qt(it + 1, c_qt);
    const int64_t qa_last = p.q_offset + min(q0 + BQ - 1, p.Sq - 1);
    bool live[KT], need_mask[KT];
    bool any = false;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const int kt0 = kbase + KSTR * j;
      live[j] = kt0 < p.Sk && !(p.causal && koff + kt0 > qa_last);
      need_mask[j] = (kt0 + 16 > p.Sk) || (p.causal && koff + kt0 + 15 > p.q_offset + q0);
      any = any || live[j];
    }
    if (!any) continue;
    // The MFMAs below run for every key tile of the wave, live or not, with no
    // branch between them, so that LDS reads and MFMAs are scheduled together;
    // a tile that is not live gets zero P and dS (its keys are all masked) and
    // adds nothing to dK and dV.

    if constexpr (kSliced) {
      // tile-relative queries [qmin, qend) see key tile j's key of this lane
      // (qend: the queries past Sq, whose zero-filled rows must not count)
      int qmin[KT];
      const int qend = min(BQ, p.Sq - q0);
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        qmin[j] = 0;
        if (need_mask[j]) {
          const int key = kbase + KSTR * j + l16;
          int64_t f = p.causal ? koff + key - p.q_offset - q0 : 0;
          if (key >= p.Sk) f = BQ;
          qmin[j] = f < 0 ? 0 : (f > BQ ? BQ : static_cast<int>(f));
        }
      }
      // per 32-query half s2: S = Q K^T and dP = dO V^T for its two 16-query
      // slices (lane holds S[q = 16 mq + 4 g + e][key = kbase + KSTR j + l16]),
      // P and dS = P (dP - delta) packed into the A operands, then the dV += P^T dO
      // and dK += dS^T Q MFMAs over the half's dO^T / Q^T column fragments
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        f32x4 s[2][KT], dp[2][KT];
#pragma unroll
        for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
          for (int j = 0; j < KT; ++j) {
            s[m2][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            dp[m2][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
        for (int m2 = 0; m2 < 2; ++m2) {
          const int mq = 2 * s2 + m2;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 aq = Tile::row8(tq, mq * 16 + l16, ks * 32 + g * 8);
            const bf16x8 ad = Tile::row8(td, mq * 16 + l16, ks * 32 + g * 8);
#pragma unroll
            for (int j = 0; j < KT; ++j) {
              s[m2][j] = mfma16(aq, kf[j][ks], s[m2][j]);
              dp[m2][j] = mfma16(ad, vf[j][ks], dp[m2][j]);
            }
          }
        }
        bf16x8 pa[KT], da[KT];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          if (!live[j]) {  // formed, not visible: adds nothing
            pa[j] = da[j] = zero8();
            continue;
          }
          if (!need_mask[j] && qend == BQ) {
            // every query of the tile sees every key of the tile: no selects
#pragma unroll
            for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int ql = (2 * s2 + m2) * 16 + g * 4 + e;
                const float pv = fast_exp2(fmaf(s[m2][j][e], c, -sL[ql]));
                pa[j][4 * m2 + e] = static_cast<bf16>(pv);
                da[j][4 * m2 + e] = static_cast<bf16>(pv * (dp[m2][j][e] - sDl[ql]));
              }
          } else {
#pragma unroll
            for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int ql = (2 * s2 + m2) * 16 + g * 4 + e;
                float pv = fast_exp2(fmaf(s[m2][j][e], c, -sL[ql]));
                pv = (ql < qmin[j] || ql >= qend) ? 0.f : pv;
                pa[j][4 * m2 + e] = static_cast<bf16>(pv);
                da[j][4 * m2 + e] = static_cast<bf16>(pv * (dp[m2][j][e] - sDl[ql]));
              }
          }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 bd = Tile::col8(td, 32 * s2, dt * 16, l16, g);
          const bf16x8 bq = Tile::col8(tq, 32 * s2, dt * 16, l16, g);
#pragma unroll
          for (int j = 0; j < KT; ++j) {
            dva[j][dt] = mfma16(pa[j], bd, dva[j][dt]);
            dka[j][dt] = mfma16(da[j], bq, dka[j][dt]);
          }
        }
      }
    } else {
      // S = Q K^T and dP = dO V^T: lane holds S[q = 16 mq + 4 g + e][key = kbase + KSTR j + l16]
      f32x4 s[4][KT], dp[4][KT];
#pragma unroll
      for (int mq = 0; mq < 4; ++mq)
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          s[mq][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[mq][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int mq = 0; mq < 4; ++mq) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 aq = Tile::row8(tq, mq * 16 + l16, ks * 32 + g * 8);
          const bf16x8 ad = Tile::row8(td, mq * 16 + l16, ks * 32 + g * 8);
#pragma unroll
          for (int j = 0; j < KT; ++j) {
            s[mq][j] = mfma16(aq, kf[j][ks], s[mq][j]);
            dp[mq][j] = mfma16(ad, vf[j][ks], dp[mq][j]);
          }
        }
      }
      bf16x8 pa[2][KT], da[2][KT];
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        if (!live[j]) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) pa[s2][j] = da[s2][j] = zero8();
          continue;
        }
        // tile-relative queries [qmin, qend) see this lane's key (qend: the
        // queries past Sq, whose zero-filled rows must not count)
        int qmin = 0;
        const int qend = min(BQ, p.Sq - q0);
        if (need_mask[j]) {
          const int key = kbase + KSTR * j + l16;
          int64_t f = p.causal ? koff + key - p.q_offset - q0 : 0;
          if (key >= p.Sk) f = BQ;
          qmin = f < 0 ? 0 : (f > BQ ? BQ : static_cast<int>(f));
        }
        if (!need_mask[j] && qend == BQ) {
          // every query of the tile sees every key of the tile: no selects
#pragma unroll
          for (int mq = 0; mq < 4; ++mq)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int ql = mq * 16 + g * 4 + e;
              const float pv = fast_exp2(fmaf(s[mq][j][e], c, -sL[ql]));
              s[mq][j][e] = pv;
              dp[mq][j][e] = pv * (dp[mq][j][e] - sDl[ql]);
            }
        } else {
#pragma unroll
          for (int mq = 0; mq < 4; ++mq)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int ql = mq * 16 + g * 4 + e;
              float pv = fast_exp2(fmaf(s[mq][j][e], c, -sL[ql]));
              pv = (ql < qmin || ql >= qend) ? 0.f : pv;
              s[mq][j][e] = pv;
              dp[mq][j][e] = pv * (dp[mq][j][e] - sDl[ql]);
            }
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pa[s2][j][e] = static_cast<bf16>(s[2 * s2][j][e]);
            pa[s2][j][4 + e] = static_cast<bf16>(s[2 * s2 + 1][j][e]);
            da[s2][j][e] = static_cast<bf16>(dp[2 * s2][j][e]);
            da[s2][j][4 + e] = static_cast<bf16>(dp[2 * s2 + 1][j][e]);
          }
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8 bd = Tile::col8(td, 32 * s2, dt * 16, l16, g);
          const bf16x8 bq = Tile::col8(tq, 32 * s2, dt * 16, l16, g);
#pragma unroll
          for (int j = 0; j < KT; ++j) {
            dva[j][dt] = mfma16(pa[s2][j], bd, dva[j][dt]);
            dka[j][dt] = mfma16(da[s2][j], bq, dka[j][dt]);
          }
        }
      }
    }
  }
  // no load may still write this workgroup's LDS when it ends
  wait_vmcnt<0>();
  if (n_sub == 2 && !switched) {  // the second key tile saw no query tile
    finish();
    start(1);
  }
  finish();
}

// ---------------------------------------------------------------- generic path
// One wavefront per query row; lane owns head_dim elements lane and lane + 64
// (head_dim <= 128).  The fp32 configuration's attention, and attention with
// an explicit mask in any supported dtype (the reference passes attention_mask
// to SDPA, nn/kernels/torch_backend.py:60-76): MK 0 no mask, 1 a boolean mask
// (one byte per entry, nonzero = attend), 2 an additive mask in the attention
// dtype (added to the scaled scores; -inf drops the key).  A query row with no
// visible key gives zeros and lse = -inf, as the safe softmax of the
// reference's SDPA does.  Attention dropout (SDPA's dropout_p, applied to the
// normalised probabilities): probability (b, h, i, j) is multiplied by the
// dropout_math.h factor of index ((b * Hq + h) * Sq + i) * Sk + j; l and the
// lse stay those of the undropped softmax.
struct MaskRef {
  const void* p;
  int64_t sb, sh, sq, sk;  // element strides of [batch, q_heads, seq_q, seq_k] (0: broadcast)
};

template <typename T, int MK>
__device__ __forceinline__ bool visible(const MaskRef& mr, int b, int h, int64_t i, int64_t j, float& add) {
  if constexpr (MK == 0) {
    return true;
  } else {
    const int64_t off = b * mr.sb + h * mr.sh + i * mr.sq + j * mr.sk;
    if constexpr (MK == 1) {
      return static_cast<const uint8_t*>(mr.p)[off] != 0;
    } else {
      add = to_f32(static_cast<const T*>(mr.p)[off]);
      return add != -__builtin_inff();
    }
  }
}

template <typename T>
__device__ __forceinline__ float dot_row(const T* a, const T* b, int D, int lane) {
  float s = 0.f;
  for (int d = lane; d < D; d += 64) s += to_f32(a[d]) * to_f32(b[d]);
  return wave_sum(s);
}

template <typename T, int MK>
__global__ __launch_bounds__(64) void attn_fwd_generic_kernel(const T* __restrict__ q, KVBlocks kv,
                                                              T* __restrict__ o, float* __restrict__ lse,
                                                              AttnShape p, int D, MaskRef mr,
                                                              DropoutParams dp) {
  const int lane = threadIdx.x;
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.Hq / p.Hkv);
  const T* qr = q + b * p.q_sb + static_cast<int64_t>(i) * p.q_ss + h * p.q_sh;
  const int64_t qa = p.q_offset + i;
  const uint64_t prow = ((static_cast<uint64_t>(b) * p.Hq + h) * p.Sq + i) * p.Sk;  // dropout index base
  float m = -__builtin_inff(), l = 0.f;
  float acc[2] = {0.f, 0.f};
  for (int blk = 0; blk < p.nblk; ++blk) {
    const T* kb = static_cast<const T*>(kv.k[blk]) + b * p.kv_sb + hk * p.kv_sh;
    const T* vb = static_cast<const T*>(kv.v[blk]) + b * p.kv_sb + hk * p.kv_sh;
    const int64_t koff = kv.koff[blk];
    for (int j = 0; j < p.Sk; ++j) {
      if (p.causal && koff + j > qa) break;
      float add = 0.f;
      if (!visible<T, MK>(mr, b, h, i, j, add)) continue;
      const T* kr = kb + static_cast<int64_t>(j) * p.kv_ss;
      const T* vr = vb + static_cast<int64_t>(j) * p.kv_ss;
      const float sc = dot_row(qr, kr, D, lane) * p.scale + add;
      const float mnew = fmaxf(m, sc);
      const float alpha = expf(m - mnew);
      const float pv = expf(sc - mnew);
      l = l * alpha + pv;
      const float pz = pv * drop_factor(dp, prow + j);  // dropout acts after the normalisation
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int d = lane + 64 * c;
        if (d < D) acc[c] = acc[c] * alpha + pz * to_f32(vr[d]);
      }
      m = mnew;
    }
  }
  T* orow = o + b * p.o_sb + static_cast<int64_t>(i) * p.o_ss + h * p.o_sh;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int d = lane + 64 * c;
    if (d < D) orow[d] = from_f32<T>(acc[c] * inv);
  }
  if (lane == 0)
    lse[(static_cast<int64_t>(b) * p.Hq + h) * p.Sq + i] = l > 0.f ? m + logf(l) : -__builtin_inff();
}

template <typename T, int MK>
__global__ __launch_bounds__(64) void attn_bwd_dq_generic_kernel(
    const T* __restrict__ q, KVBlocks kv, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, T* __restrict__ dq,
    AttnShape p, int D, MaskRef mr, DropoutParams dp) {
  const int lane = threadIdx.x;
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.Hq / p.Hkv);
  const T* qr = q + b * p.q_sb + static_cast<int64_t>(i) * p.q_ss + h * p.q_sh;
  const T* dr = dout + b * p.o_sb + static_cast<int64_t>(i) * p.o_ss + h * p.o_sh;
  const int64_t row = (static_cast<int64_t>(b) * p.Hq + h) * p.Sq + i;
  const uint64_t prow = static_cast<uint64_t>(row) * p.Sk;
  const float ls = lse[row], dl = delta[row];
  const int64_t qa = p.q_offset + i;
  float acc[2] = {0.f, 0.f};
  if (ls != -__builtin_inff()) {
    for (int blk = 0; blk < p.nblk; ++blk) {
      const T* kb = static_cast<const T*>(kv.k[blk]) + b * p.kv_sb + hk * p.kv_sh;
      const T* vb = static_cast<const T*>(kv.v[blk]) + b * p.kv_sb + hk * p.kv_sh;
      const int64_t koff = kv.koff[blk];
      for (int j = 0; j < p.Sk; ++j) {
        if (p.causal && koff + j > qa) break;
        float add = 0.f;
        if (!visible<T, MK>(mr, b, h, i, j, add)) continue;
        const T* kr = kb + static_cast<int64_t>(j) * p.kv_ss;
        const T* vr = vb + static_cast<int64_t>(j) * p.kv_ss;
        const float pv = expf(dot_row(qr, kr, D, lane) * p.scale + add - ls);
        // dropout: dP = Z (dO . V) with Z = keep / (1 - p); delta = rowsum(dO o O) still
        // equals sum_j P Z (dO . V), so dS = P (dP - delta)
        const float ds = pv * (drop_factor(dp, prow + j) * dot_row(dr, vr, D, lane) - dl);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int d = lane + 64 * c;
          if (d < D) acc[c] += ds * to_f32(kr[d]);
        }
      }
    }
  }
  T* out = dq + b * p.q_sb + static_cast<int64_t>(i) * p.q_ss + h * p.q_sh;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int d = lane + 64 * c;
    if (d < D) out[d] = from_f32<T>(acc[c] * p.scale);
  }
}

template <typename T, int MK>
__global__ __launch_bounds__(64) void attn_bwd_dkdv_generic_kernel(
    const T* __restrict__ q, KVBlocks kv, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, AttnShape p, int D, MaskRef mr,
    DropoutParams dp) {
  const int lane = threadIdx.x;
  const int j = blockIdx.x, hk = blockIdx.y;
  const int blk = static_cast<int>(blockIdx.z) % p.nblk;
  const int b = static_cast<int>(blockIdx.z) / p.nblk;
  const int group = p.Hq / p.Hkv;
  const int64_t koff = kv.koff[blk];
  const int64_t kvo = b * p.kv_sb + static_cast<int64_t>(j) * p.kv_ss + hk * p.kv_sh;
  const T* kr = static_cast<const T*>(kv.k[blk]) + kvo;
  const T* vr = static_cast<const T*>(kv.v[blk]) + kvo;
  float dk[2] = {0.f, 0.f}, dv[2] = {0.f, 0.f};
  int i0 = 0;
  if (p.causal) {
    const int64_t fq = koff + j - p.q_offset;
    i0 = fq <= 0 ? 0 : (fq >= p.Sq ? p.Sq : static_cast<int>(fq));
  }
  for (int hi = 0; hi < group; ++hi) {
    const int h = hk * group + hi;
    for (int i = i0; i < p.Sq; ++i) {
      const int64_t row = (static_cast<int64_t>(b) * p.Hq + h) * p.Sq + i;
      const float ls = lse[row];
      if (ls == -__builtin_inff()) continue;
      float add = 0.f;
      if (!visible<T, MK>(mr, b, h, i, j, add)) continue;
      const T* qr = q + b * p.q_sb + static_cast<int64_t>(i) * p.q_ss + h * p.q_sh;
      const T* dr = dout + b * p.o_sb + static_cast<int64_t>(i) * p.o_ss + h * p.o_sh;
      const float pv = expf(dot_row(qr, kr, D, lane) * p.scale + add - ls);
      const float z = drop_factor(dp, static_cast<uint64_t>(row) * p.Sk + j);
      const float ds = pv * (z * dot_row(dr, vr, D, lane) - delta[row]);
      const float pz = pv * z;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int d = lane + 64 * c;
        if (d < D) {
          dv[c] += pz * to_f32(dr[d]);
          dk[c] += ds * to_f32(qr[d]);
        }
      }
    }
  }
  T* dkr = static_cast<T*>(kv.dk[blk]) + kvo;
  T* dvr = static_cast<T*>(kv.dv[blk]) + kvo;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int d = lane + 64 * c;
    if (d < D) {
      dkr[d] = from_f32<T>(dk[c] * p.scale);
      dvr[d] = from_f32<T>(dv[c]);
    }
  }
}

// ---------------------------------------------------------------- host side
int fill_shape(AttnShape* p, KVBlocks* kv, const void* q, const void* const* kb,
               const void* const* vb, const int64_t* koff, int nblk, int64_t B, int64_t Hq,
               int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, const int64_t* qs,
               const int64_t* kvs, const int64_t* os, int causal, int64_t q_offset, float scale,
               int dtype) {
  NMB_REQUIRE(q != nullptr && kb != nullptr && vb != nullptr && koff != nullptr && qs != nullptr &&
                  kvs != nullptr && os != nullptr,
              "attention: null argument");
  NMB_REQUIRE(nblk >= 1 && nblk <= kMaxBlocks, "attention: n_blocks must be in [1, %d], got %d",
              kMaxBlocks, nblk);
  NMB_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0 && D > 0,
              "attention: invalid shape");
  NMB_REQUIRE(Hq % Hkv == 0, "query heads (%lld) must be divisible by KV heads (%lld)",
              (long long)Hq, (long long)Hkv);
  NMB_REQUIRE(B <= 65535 && Hq <= 65535 && Sq <= 0x3fffffff && Sk <= 0x3fffffff,
              "attention: shape exceeds the launch grid");
  if (dtype == NMB_BF16) {
    NMB_REQUIRE_SUPPORTED(D == 64 || D == 128, "attention (bf16): head_dim must be 64 or 128, got %lld",
                          (long long)D);
    for (int i = 0; i < 3; ++i)
      NMB_REQUIRE_SUPPORTED(qs[i] % 8 == 0 && kvs[i] % 8 == 0 && os[i] % 8 == 0,
                            "attention (bf16): strides must be multiples of 8 elements");
    NMB_REQUIRE(aligned16(q), "attention: q must be 16-byte aligned");
  } else if (dtype == NMB_F32) {
    NMB_REQUIRE_SUPPORTED(D <= 128, "attention (fp32): head_dim must be <= 128, got %lld",
                          (long long)D);
  } else {
    NMB_REQUIRE_SUPPORTED(false, "attention: unsupported dtype code %d", dtype);
  }
  for (int i = 0; i < nblk; ++i) {
    NMB_REQUIRE(kb[i] != nullptr && vb[i] != nullptr, "attention: null K/V block %d", i);
    NMB_REQUIRE(dtype != NMB_BF16 || (aligned16(kb[i]) && aligned16(vb[i])),
                "attention: K/V blocks must be 16-byte aligned");
    kv->k[i] = kb[i];
    kv->v[i] = vb[i];
    kv->koff[i] = koff[i];
    kv->dk[i] = nullptr;
    kv->dv[i] = nullptr;
  }
  p->B = static_cast<int>(B);
  p->Hq = static_cast<int>(Hq);
  p->Hkv = static_cast<int>(Hkv);
  p->Sq = static_cast<int>(Sq);
  p->Sk = static_cast<int>(Sk);
  p->nblk = nblk;
  p->causal = causal ? 1 : 0;
  p->q_sb = qs[0];
  p->q_ss = qs[1];
  p->q_sh = qs[2];
  p->kv_sb = kvs[0];
  p->kv_ss = kvs[1];
  p->kv_sh = kvs[2];
  p->o_sb = os[0];
  p->o_ss = os[1];
  p->o_sh = os[2];
  p->q_offset = q_offset;
  p->scale = scale > 0.f ? scale : static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
  p->scale_log2 = p->scale * kLog2e;
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

using nmb::AttnShape;
using nmb::KVBlocks;

namespace {
// Launch geometry of the XCD-mapped kernels: a 1-D grid of 8 * per_xcd blocks.
void xcd_grid(int64_t items, int* per_xcd, unsigned* blocks) {
  const int64_t per = (items + 7) / 8;
  *per_xcd = static_cast<int>(per);
  *blocks = static_cast<unsigned>(per * 8);
}
}  // namespace

namespace nmb {
namespace {

int attn_fwd_impl(bool from_lse, const void* q, const void* const* k_blocks,
                            const void* const* v_blocks, const int64_t* k_offsets, int n_blocks,
                            void* o, float* lse, int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t seq_q, int64_t seq_k, int64_t head_dim,
                            const int64_t* q_strides, const int64_t* kv_strides,
                            const int64_t* o_strides, int causal, int64_t q_offset, float scale,
                            int dtype, hipStream_t stream) {
  AttnShape p;
  KVBlocks kv;
  int st = nmb::fill_shape(&p, &kv, q, k_blocks, v_blocks, k_offsets, n_blocks, batch, q_heads,
                           kv_heads, seq_q, seq_k, head_dim, q_strides, kv_strides, o_strides,
                           causal, q_offset, scale, dtype);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(o != nullptr && lse != nullptr, "attn_fwd: null output");
  if (batch == 0 || seq_q == 0) return NMB_OK;
  if (dtype == NMB_BF16) {
    NMB_REQUIRE(nmb::aligned16(o), "attn_fwd: o must be 16-byte aligned");
    // the forward addresses a K/V block through a 32-bit buffer offset
    NMB_REQUIRE_SUPPORTED(seq_k == 0 || ((seq_k - 1) * kv_strides[1] + head_dim) * 2 < (int64_t{1} << 31),
                          "attn_fwd: a K/V block spans more than 2 GiB");
    // queries per workgroup: NWV waves x TQ column tiles of 16.  D 64: 8 waves x 4
    // for 512 .. 1023 queries, 4 x 2 (three workgroups per CU) from 1024, else
    // 4 x 4; D 128: 8 x 2 (two waves per SIMD)
    const bool long_seq = head_dim == 64 && seq_q >= 1024;
    const int nwv = (head_dim == 64 && seq_q >= 512 && !long_seq) || head_dim == 128 ? 8 : 4;
    const int bq = 16 * nwv * (head_dim == 64 && !long_seq ? 4 : 2);
    const int n_qt = static_cast<int>((seq_q + bq - 1) / bq);
    const int64_t items = static_cast<int64_t>(n_qt) * q_heads * batch;
    NMB_REQUIRE(items < (int64_t{1} << 30), "attn_fwd: problem too large for one launch");
    int per_xcd;
    unsigned blocks;
    xcd_grid(items, &per_xcd, &blocks);
    const nmb::bf16* qp = static_cast<const nmb::bf16*>(q);
    nmb::bf16* op = static_cast<nmb::bf16*>(o);
#define NMB_FWD(DD, TT, NW, FF)                                                                        \
  hipLaunchKernelGGL((nmb::attn_fwd_kernel<DD, TT, NW, FF>), dim3(blocks), dim3(64 * NW), 0, stream, qp, kv, \
                     op, lse, p, n_qt, static_cast<int>(items), per_xcd)
    if (head_dim == 64 && nwv == 8) {
      if (from_lse) NMB_FWD(64, 4, 8, true); else NMB_FWD(64, 4, 8, false);
    } else if (long_seq) {
      if (from_lse) NMB_FWD(64, 2, 4, true); else NMB_FWD(64, 2, 4, false);
    } else if (head_dim == 64) {
      if (from_lse) NMB_FWD(64, 4, 4, true); else NMB_FWD(64, 4, 4, false);
    } else {
      if (from_lse) NMB_FWD(128, 2, 8, true); else NMB_FWD(128, 2, 8, false);
    }
#undef NMB_FWD
  } else {
    NMB_REQUIRE_SUPPORTED(!from_lse, "attn_fwd_from_lse: bf16 only");
    const dim3 grid(static_cast<unsigned>(seq_q), static_cast<unsigned>(q_heads),
                    static_cast<unsigned>(batch));
    hipLaunchKernelGGL((nmb::attn_fwd_generic_kernel<float, 0>), grid, dim3(64), 0, stream,
                       static_cast<const float*>(q), kv, static_cast<float*>(o), lse, p,
                       static_cast<int>(head_dim), nmb::MaskRef{}, nmb::DropoutParams{0, 0, 1.f});
  }
  NMB_CHECK_LAUNCH("attn_fwd");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_attn_fwd(const void* q, const void* const* k_blocks,
                            const void* const* v_blocks, const int64_t* k_offsets, int n_blocks,
                            void* o, float* lse, int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t seq_q, int64_t seq_k, int64_t head_dim,
                            const int64_t* q_strides, const int64_t* kv_strides,
                            const int64_t* o_strides, int causal, int64_t q_offset, float scale,
                            int dtype, hipStream_t stream) {
  return nmb::attn_fwd_impl(false, q, k_blocks, v_blocks, k_offsets, n_blocks, o, lse, batch, q_heads,
                            kv_heads, seq_q, seq_k, head_dim, q_strides, kv_strides, o_strides, causal,
                            q_offset, scale, dtype, stream);
}

extern "C" int nmb_attn_fwd_from_lse(const void* q, const void* const* k_blocks,
                                     const void* const* v_blocks, const int64_t* k_offsets,
                                     int n_blocks, const float* lse, void* o, int64_t batch,
                                     int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                                     int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                     const int64_t* kv_strides, const int64_t* o_strides,
                                     int causal, int64_t q_offset, float scale, int dtype,
                                     hipStream_t stream) {
  // the kernel only reads lse in this mode
  return nmb::attn_fwd_impl(true, q, k_blocks, v_blocks, k_offsets, n_blocks, o,
                            const_cast<float*>(lse), batch, q_heads, kv_heads, seq_q, seq_k,
                            head_dim, q_strides, kv_strides, o_strides, causal, q_offset, scale,
                            dtype, stream);
}

extern "C" int nmb_attn_bwd_workspace_bytes(int64_t batch, int64_t q_heads, int64_t seq_q,
                                            size_t* bytes) {
  NMB_REQUIRE(bytes != nullptr && batch >= 0 && q_heads >= 0 && seq_q >= 0,
              "attn_bwd_workspace_bytes: bad args");
  *bytes = 2 * static_cast<size_t>(batch * q_heads * seq_q) * sizeof(float);
  return NMB_OK;
}

namespace nmb {
namespace {

int attn_bwd_impl(const void* q, const void* const* k_blocks,
                            const void* const* v_blocks, const int64_t* k_offsets, int n_blocks,
                            const void* o, const void* dout, const float* lse, void* dq,
                            void* const* dk_blocks, void* const* dv_blocks, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t q_heads,
                            int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                            const int64_t* q_strides, const int64_t* kv_strides,
                            const int64_t* o_strides, int causal, int64_t q_offset, float scale,
                            int dtype, hipStream_t stream, const RopeGrad* rope) {
  AttnShape p;
  KVBlocks kv;
  int st = nmb::fill_shape(&p, &kv, q, k_blocks, v_blocks, k_offsets, n_blocks, batch, q_heads,
                           kv_heads, seq_q, seq_k, head_dim, q_strides, kv_strides, o_strides,
                           causal, q_offset, scale, dtype);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(o != nullptr && dout != nullptr && lse != nullptr && dq != nullptr &&
                  dk_blocks != nullptr && dv_blocks != nullptr,
              "attn_bwd: null argument");
  for (int i = 0; i < n_blocks; ++i) {
    NMB_REQUIRE(dk_blocks[i] != nullptr && dv_blocks[i] != nullptr, "attn_bwd: null dK/dV block");
    kv.dk[i] = dk_blocks[i];
    kv.dv[i] = dv_blocks[i];
  }
  const size_t need = 2 * static_cast<size_t>(batch * q_heads * seq_q) * sizeof(float);
  NMB_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "attn_bwd: workspace of %zu bytes is smaller than the %zu required",
              workspace_bytes, need);
  if (batch == 0) return NMB_OK;
  // workspace: delta [B, Hq, Sq], then the log2-domain lse [B, Hq, Sq]
  float* delta = static_cast<float*>(workspace);
  float* lse2 = delta + batch * q_heads * seq_q;
  const int D = static_cast<int>(head_dim);
  if (dtype == NMB_BF16) {
    NMB_REQUIRE(nmb::aligned16(dq) && nmb::aligned16(dout) && nmb::aligned16(o),
                "attn_bwd: dq/dout/o must be 16-byte aligned");
    // the kernels address K/V, Q and dO through 32-bit buffer offsets
    NMB_REQUIRE_SUPPORTED(
        (seq_k == 0 || ((seq_k - 1) * kv_strides[1] + head_dim) * 2 < (int64_t{1} << 31)) &&
            (seq_q == 0 || (((seq_q - 1) * q_strides[1] + head_dim) * 2 < (int64_t{1} << 31) &&
                            ((seq_q - 1) * o_strides[1] + head_dim) * 2 < (int64_t{1} << 31))),
        "attn_bwd: a Q, dO or K/V block spans more than 2 GiB");
    const nmb::bf16* qp = static_cast<const nmb::bf16*>(q);
    const nmb::bf16* opp = static_cast<const nmb::bf16*>(o);
    const nmb::bf16* dp = static_cast<const nmb::bf16*>(dout);
    nmb::bf16* dqp = static_cast<nmb::bf16*>(dq);
    // the dQ kernel also writes delta, which the dK/dV kernel reads: keep this order
    if (seq_q > 0) {
      // query tiles of 128 (D 64, two per workgroup) or 256 (D 128, 8 waves)
      const int bq = D == 64 ? 128 : 256;
      const int n_qt = static_cast<int>((seq_q + bq - 1) / bq);
      const int64_t items = static_cast<int64_t>(D == 64 ? (n_qt + 1) / 2 : n_qt) * q_heads * batch;
      NMB_REQUIRE(items < (int64_t{1} << 30), "attn_bwd: problem too large for one launch");
      int per_xcd;
      unsigned blocks;
      xcd_grid(items, &per_xcd, &blocks);
      const RopeGrad rg = rope != nullptr ? *rope : RopeGrad{};
#define NMB_DQ(DD, RR, NW)                                                                            \
  hipLaunchKernelGGL((nmb::attn_bwd_dq_kernel<DD, RR, NW>), dim3(blocks), dim3(64 * NW), 0, stream, qp, \
                     kv, opp, dp, lse, delta, lse2, dqp, p, n_qt, static_cast<int>(items), per_xcd, rg)
      if (D == 64) {
        if (rope) NMB_DQ(64, true, 4); else NMB_DQ(64, false, 4);
      } else {
        if (rope) NMB_DQ(128, true, 8); else NMB_DQ(128, false, 8);
      }
#undef NMB_DQ
      NMB_CHECK_LAUNCH("attn_bwd(dq)");
    }
    if (seq_k > 0) {
      const int n_kt = static_cast<int>((seq_k + 127) / 128);  // 128-key tiles, two per workgroup at D 64
      const int64_t items = static_cast<int64_t>(D == 64 ? (n_kt + 1) / 2 : n_kt) * kv_heads * batch * n_blocks;
      NMB_REQUIRE(items < (int64_t{1} << 30), "attn_bwd: problem too large for one launch");
      int per_xcd;
      unsigned blocks;
      xcd_grid(items, &per_xcd, &blocks);
      const RopeGrad rg = rope != nullptr ? *rope : RopeGrad{};
#define NMB_DKDV(DD, RR, NW)                                                                            \
  hipLaunchKernelGGL((nmb::attn_bwd_dkdv_kernel<DD, RR, NW>), dim3(blocks), dim3(64 * NW), 0, stream, qp, \
                     kv, dp, lse2, delta, p, n_kt, static_cast<int>(items), per_xcd, rg)
      if (D == 64) {
        if (rope) NMB_DKDV(64, true, 4); else NMB_DKDV(64, false, 4);
      } else {
        if (rope) NMB_DKDV(128, true, 8); else NMB_DKDV(128, false, 8);
      }
#undef NMB_DKDV
      NMB_CHECK_LAUNCH("attn_bwd(dkdv)");
    }
  } else {
    if (seq_q > 0) {
      int64_t rows = batch * q_heads * seq_q;
      int64_t blocks = (rows + 255) / 256;
      if (blocks > 8192) blocks = 8192;
      hipLaunchKernelGGL(nmb::attn_delta_kernel<float>, dim3(static_cast<unsigned>(blocks)),
                         dim3(256), 0, stream, static_cast<const float*>(o),
                         static_cast<const float*>(dout), delta, p, D);
      NMB_CHECK_LAUNCH("attn_bwd(delta)");
    }
    const float* qp = static_cast<const float*>(q);
    const float* dp = static_cast<const float*>(dout);
    if (seq_q > 0) {
      const dim3 grid(static_cast<unsigned>(seq_q), static_cast<unsigned>(q_heads),
                      static_cast<unsigned>(batch));
      hipLaunchKernelGGL((nmb::attn_bwd_dq_generic_kernel<float, 0>), grid, dim3(64), 0, stream, qp, kv,
                         dp, lse, delta, static_cast<float*>(dq), p, D, nmb::MaskRef{},
                         nmb::DropoutParams{0, 0, 1.f});
      NMB_CHECK_LAUNCH("attn_bwd(dq,f32)");
    }
    if (seq_k > 0) {
      const dim3 grid(static_cast<unsigned>(seq_k), static_cast<unsigned>(kv_heads),
                      static_cast<unsigned>(batch * n_blocks));
      hipLaunchKernelGGL((nmb::attn_bwd_dkdv_generic_kernel<float, 0>), grid, dim3(64), 0, stream, qp,
                         kv, dp, lse, delta, p, D, nmb::MaskRef{}, nmb::DropoutParams{0, 0, 1.f});
      NMB_CHECK_LAUNCH("attn_bwd(dkdv,f32)");
    }
  }
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_attn_bwd(const void* q, const void* const* k_blocks,
                            const void* const* v_blocks, const int64_t* k_offsets, int n_blocks,
                            const void* o, const void* dout, const float* lse, void* dq,
                            void* const* dk_blocks, void* const* dv_blocks, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t q_heads,
                            int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                            const int64_t* q_strides, const int64_t* kv_strides,
                            const int64_t* o_strides, int causal, int64_t q_offset, float scale,
                            int dtype, hipStream_t stream) {
  return nmb::attn_bwd_impl(q, k_blocks, v_blocks, k_offsets, n_blocks, o, dout, lse, dq, dk_blocks,
                            dv_blocks, workspace, workspace_bytes, batch, q_heads, kv_heads, seq_q,
                            seq_k, head_dim, q_strides, kv_strides, o_strides, causal, q_offset,
                            scale, dtype, stream, nullptr);
}

namespace nmb {
namespace {

// Shape, mask and dropout of the masked entry points: one K/V block at key
// offset 0; the generic kernels load elements one at a time, so any head_dim
// <= 128 and any strides (of bf16 or fp32 data) are accepted.  mask_kind 0
// (no mask) serves attention with dropout alone.
int masked_setup(AttnShape* p, KVBlocks* kv, MaskRef* mr, DropoutParams* dp, const void* q, const void* k,
                 const void* v, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                 int64_t seq_k, int64_t head_dim, const int64_t* qs, const int64_t* kvs, const int64_t* os,
                 const void* mask, int mask_kind, const int64_t* ms, int causal, int64_t q_offset,
                 float scale, float dropout_p, uint64_t seed, int dtype) {
  NMB_REQUIRE_SUPPORTED(dtype == NMB_BF16 || dtype == NMB_F32, "attention (masked): unsupported dtype code %d",
                        dtype);
  NMB_REQUIRE(mask_kind == 0 || mask_kind == 1 || mask_kind == 2,
              "attention (masked): mask_kind must be 0 (none), 1 (boolean) or 2 (additive), got %d",
              mask_kind);
  NMB_REQUIRE(dropout_p >= 0.f && dropout_p < 1.f, "attention (masked): dropout_p must be in [0, 1), got %g",
              static_cast<double>(dropout_p));
  if (mask_kind != 0) {
    NMB_REQUIRE(mask != nullptr && ms != nullptr, "attention (masked): null mask");
    NMB_REQUIRE(ms[0] >= 0 && ms[1] >= 0 && ms[2] >= 0 && ms[3] >= 0,
                "attention (masked): mask strides must be non-negative");
  }
  const void* kb[1] = {k};
  const void* vb[1] = {v};
  const int64_t koff[1] = {0};
  const int st = fill_shape(p, kv, q, kb, vb, koff, 1, batch, q_heads, kv_heads, seq_q, seq_k, head_dim,
                            qs, kvs, os, causal, q_offset, scale, NMB_F32);
  if (st != NMB_OK) return st;
  *mr = mask_kind != 0 ? MaskRef{mask, ms[0], ms[1], ms[2], ms[3]} : MaskRef{};
  *dp = make_dropout(static_cast<double>(dropout_p), seed);
  return NMB_OK;
}

template <typename T>
void masked_fwd_launch(const AttnShape& p, const KVBlocks& kv, const MaskRef& mr, const DropoutParams& dp,
                       int kind, const void* q, void* o, float* lse, int D, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.Sq), static_cast<unsigned>(p.Hq), static_cast<unsigned>(p.B));
  const T* qp = static_cast<const T*>(q);
  T* op = static_cast<T*>(o);
  if (kind == 0)
    hipLaunchKernelGGL((attn_fwd_generic_kernel<T, 0>), grid, dim3(64), 0, stream, qp, kv, op, lse, p, D, mr, dp);
  else if (kind == 1)
    hipLaunchKernelGGL((attn_fwd_generic_kernel<T, 1>), grid, dim3(64), 0, stream, qp, kv, op, lse, p, D, mr, dp);
  else
    hipLaunchKernelGGL((attn_fwd_generic_kernel<T, 2>), grid, dim3(64), 0, stream, qp, kv, op, lse, p, D, mr, dp);
}

template <typename T>
void masked_bwd_launch(const AttnShape& p, const KVBlocks& kv, const MaskRef& mr, const DropoutParams& drop,
                       int kind, const void* q, const void* o, const void* dout, const float* lse, float* delta,
                       void* dq, int D, hipStream_t stream) {
  const T* qp = static_cast<const T*>(q);
  const T* dp = static_cast<const T*>(dout);
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  if (rows > 0) {
    int64_t blocks = (rows + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(attn_delta_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const T*>(o), dp, delta, p, D);
    const dim3 grid(static_cast<unsigned>(p.Sq), static_cast<unsigned>(p.Hq), static_cast<unsigned>(p.B));
    T* dqp = static_cast<T*>(dq);
    if (kind == 0)
      hipLaunchKernelGGL((attn_bwd_dq_generic_kernel<T, 0>), grid, dim3(64), 0, stream, qp, kv, dp, lse, delta,
                         dqp, p, D, mr, drop);
    else if (kind == 1)
      hipLaunchKernelGGL((attn_bwd_dq_generic_kernel<T, 1>), grid, dim3(64), 0, stream, qp, kv, dp, lse, delta,
                         dqp, p, D, mr, drop);
    else
      hipLaunchKernelGGL((attn_bwd_dq_generic_kernel<T, 2>), grid, dim3(64), 0, stream, qp, kv, dp, lse, delta,
                         dqp, p, D, mr, drop);
  }
  if (p.Sk > 0 && p.B > 0) {
    const dim3 grid(static_cast<unsigned>(p.Sk), static_cast<unsigned>(p.Hkv), static_cast<unsigned>(p.B));
    if (kind == 0)
      hipLaunchKernelGGL((attn_bwd_dkdv_generic_kernel<T, 0>), grid, dim3(64), 0, stream, qp, kv, dp, lse,
                         delta, p, D, mr, drop);
    else if (kind == 1)
      hipLaunchKernelGGL((attn_bwd_dkdv_generic_kernel<T, 1>), grid, dim3(64), 0, stream, qp, kv, dp, lse,
                         delta, p, D, mr, drop);
    else
      hipLaunchKernelGGL((attn_bwd_dkdv_generic_kernel<T, 2>), grid, dim3(64), 0, stream, qp, kv, dp, lse,
                         delta, p, D, mr, drop);
  }
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_attn_masked_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                                   int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                                   int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                   const int64_t* kv_strides, const int64_t* o_strides, const void* mask,
                                   int mask_kind, const int64_t* mask_strides, int causal,
                                   int64_t q_offset, float scale, float dropout_p, uint64_t seed, int dtype,
                                   hipStream_t stream) {
  AttnShape p;
  KVBlocks kv;
  nmb::MaskRef mr;
  nmb::DropoutParams dp;
  const int st = nmb::masked_setup(&p, &kv, &mr, &dp, q, k, v, batch, q_heads, kv_heads, seq_q, seq_k,
                                   head_dim, q_strides, kv_strides, o_strides, mask, mask_kind, mask_strides,
                                   causal, q_offset, scale, dropout_p, seed, dtype);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(o != nullptr && lse != nullptr, "attn_masked_fwd: null output");
  if (batch == 0 || seq_q == 0) return NMB_OK;
  if (dtype == NMB_BF16)
    nmb::masked_fwd_launch<nmb::bf16>(p, kv, mr, dp, mask_kind, q, o, lse, static_cast<int>(head_dim), stream);
  else
    nmb::masked_fwd_launch<float>(p, kv, mr, dp, mask_kind, q, o, lse, static_cast<int>(head_dim), stream);
  NMB_CHECK_LAUNCH("attn_masked_fwd");
  return NMB_OK;
}

extern "C" int nmb_attn_masked_bwd(const void* q, const void* k, const void* v, const void* o,
                                   const void* dout, const float* lse, void* dq, void* dk, void* dv,
                                   void* workspace, size_t workspace_bytes, int64_t batch,
                                   int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                   int64_t head_dim, const int64_t* q_strides, const int64_t* kv_strides,
                                   const int64_t* o_strides, const void* mask, int mask_kind,
                                   const int64_t* mask_strides, int causal, int64_t q_offset, float scale,
                                   float dropout_p, uint64_t seed, int dtype, hipStream_t stream) {
  AttnShape p;
  KVBlocks kv;
  nmb::MaskRef mr;
  nmb::DropoutParams dp;
  const int st = nmb::masked_setup(&p, &kv, &mr, &dp, q, k, v, batch, q_heads, kv_heads, seq_q, seq_k,
                                   head_dim, q_strides, kv_strides, o_strides, mask, mask_kind, mask_strides,
                                   causal, q_offset, scale, dropout_p, seed, dtype);
  if (st != NMB_OK) return st;
  NMB_REQUIRE(o != nullptr && dout != nullptr && lse != nullptr && dq != nullptr && dk != nullptr &&
                  dv != nullptr,
              "attn_masked_bwd: null argument");
  const size_t need = static_cast<size_t>(batch * q_heads * seq_q) * sizeof(float);
  NMB_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "attn_masked_bwd: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
              need);
  kv.dk[0] = dk;
  kv.dv[0] = dv;
  if (batch == 0) return NMB_OK;
  float* delta = static_cast<float*>(workspace);
  if (dtype == NMB_BF16)
    nmb::masked_bwd_launch<nmb::bf16>(p, kv, mr, dp, mask_kind, q, o, dout, lse, delta, dq,
                                      static_cast<int>(head_dim), stream);
  else
    nmb::masked_bwd_launch<float>(p, kv, mr, dp, mask_kind, q, o, dout, lse, delta, dq,
                                  static_cast<int>(head_dim), stream);
  NMB_CHECK_LAUNCH("attn_masked_bwd");
  return NMB_OK;
}

extern "C" int nmb_attn_bwd_rope(const void* q, const void* k, const void* v, const void* o,
                                 const void* dout, const float* lse, void* dq, void* dk, void* dv,
                                 void* workspace, size_t workspace_bytes, int64_t batch,
                                 int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
                                 const int64_t* q_strides, const int64_t* kv_strides,
                                 const int64_t* o_strides, int causal, int64_t q_offset,
                                 float scale, const float* cos_table, const float* sin_table,
                                 int64_t n_pos,
                                 const int32_t* positions, int64_t pos_batch_stride,
                                 int64_t pos_offset, hipStream_t stream) {
  NMB_REQUIRE(cos_table != nullptr && sin_table != nullptr && n_pos > 0 && n_pos < (1 << 30),
              "attn_bwd_rope: cos/sin tables of n_pos rows needed");
  // the dQ stores read 4 table values per 16-byte load
  NMB_REQUIRE(nmb::aligned16(cos_table) && nmb::aligned16(sin_table),
              "attn_bwd_rope: cos/sin tables must be 16-byte aligned");
  NMB_REQUIRE_SUPPORTED(head_dim == 64 || head_dim == 128, "attn_bwd_rope: head_dim %lld (64 or 128 supported)",
                        (long long)head_dim);
  if (positions == nullptr) {
    NMB_REQUIRE(pos_offset >= 0 && pos_offset + seq <= n_pos,
                "attn_bwd_rope: positions [%lld, %lld) exceed the cos/sin table of %lld rows",
                (long long)pos_offset, (long long)(pos_offset + seq), (long long)n_pos);
  } else {
    NMB_REQUIRE(pos_batch_stride >= 0, "attn_bwd_rope: negative position batch stride");
  }
  const nmb::RopeGrad rg{cos_table, sin_table, positions, pos_batch_stride,
                         positions == nullptr ? pos_offset : 0, static_cast<int>(n_pos)};
  const void* kb[1] = {k};
  const void* vb[1] = {v};
  void* dkb[1] = {dk};
  void* dvb[1] = {dv};
  const int64_t koff[1] = {0};
  // one K/V block whose keys are the queries' tokens (self-attention of the local sequence)
  return nmb::attn_bwd_impl(q, kb, vb, koff, 1, o, dout, lse, dq, dkb, dvb, workspace,
                            workspace_bytes, batch, q_heads, kv_heads, seq, seq, head_dim, q_strides,
                            kv_strides, o_strides, causal, q_offset, scale, NMB_BF16, stream, &rg);
}

// ---------------------------------------------------------------- backward without allocation
// nmb_attn_bwd_noalloc: nmb_attn_bwd with its workspace (delta and the base-2
// lse, fp32 [B, Hq, Sq] each) in a fixed device array instead of a caller
// buffer, for callers that cannot allocate.  Each device holds its own copy of
// the array until the process ends; every call on a device uses that copy, so
// calls that overlap on one device (two streams, two threads) race.  Nothing
// in it needs clearing: the dQ kernel writes every delta and lse entry of the
// call before the dK/dV kernel reads them (same stream).
namespace {

constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;  // B x Hq x Sq <= 1M query rows
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

// device address of `scratch` per device, looked up once with that device current
std::atomic<void*> g_scratch_address[kMaxDevices];
std::mutex g_scratch_mutex;

int scratch_for_stream(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) {
    nmb::set_error("attn_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return NMB_EHIP;
  }
  if (stream != nullptr) {
    int dev = -1;
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) {
      nmb::set_error("attn_bwd_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
      return NMB_EHIP;
    }
    NMB_REQUIRE(dev == current,
                "attn_bwd_noalloc: the stream belongs to device %d but device %d is current", dev,
                current);
  }
  NMB_REQUIRE(current >= 0 && current < kMaxDevices, "attn_bwd_noalloc: device %d out of range",
              current);
  void* p = g_scratch_address[current].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_address[current].load(std::memory_order_relaxed);
    if (p == nullptr) {
      // the array's name is a host-side stand-in: kernels get this address
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        nmb::set_error("attn_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       current, hipGetErrorString(e));
        return NMB_EHIP;
      }
      g_scratch_address[current].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NMB_OK;
}

}  // namespace

extern "C" int nmb_attn_bwd_noalloc(const void* q, const void* const* k_blocks,
                                    const void* const* v_blocks, const int64_t* k_offsets,
                                    int n_blocks, const void* o, const void* dout, const float* lse,
                                    void* dq, void* const* dk_blocks, void* const* dv_blocks,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t seq_q, int64_t seq_k, int64_t head_dim,
                                    const int64_t* q_strides, const int64_t* kv_strides,
                                    const int64_t* o_strides, int causal, int64_t q_offset,
                                    float scale, int dtype, hipStream_t stream) {
  NMB_REQUIRE(batch >= 0 && q_heads >= 0 && seq_q >= 0 && batch <= 65535 && q_heads <= 65535 &&
                  seq_q <= 0x3fffffff,
              "attn_bwd_noalloc: invalid shape");
  const size_t need = 2 * static_cast<size_t>(batch * q_heads * seq_q) * sizeof(float);
  NMB_REQUIRE(need <= kNoAllocScratchBytes,
              "attn_bwd_noalloc: %zu bytes of scratch needed, at most %zu available "
              "(batch x q_heads x seq_q <= %zu)",
              need, kNoAllocScratchBytes, kNoAllocScratchBytes / (2 * sizeof(float)));
  void* ws = nullptr;
  const int st = scratch_for_stream(stream, &ws);
  if (st != NMB_OK) return st;
  return nmb::attn_bwd_impl(q, k_blocks, v_blocks, k_offsets, n_blocks, o, dout, lse, dq, dk_blocks,
                            dv_blocks, ws, kNoAllocScratchBytes, batch, q_heads, kv_heads, seq_q,
                            seq_k, head_dim, q_strides, kv_strides, o_strides, causal, q_offset,
                            scale, dtype, stream, nullptr);
}
