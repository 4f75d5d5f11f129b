// Token embedding forward and backward for gfx950.
//
// Follows VocabParallelEmbedding.forward at TP=1 (reference
// tensor_parallel/embedding.py:60-74: F.embedding, a row gather of the [V, H]
// table) and its backward, the scatter-add of the output gradient rows into
// the table gradient.  An id outside [0, V) yields a zero row and adds nothing
// to the table gradient (embedding.py:63-68 masks ids outside the partition).  The table is tied to the LM head (models/gpt/model.py:
// 125-142), so the backward can take the LM head's table gradient and return
// the sum, in the order autograd accumulates them: bf16(lm + bf16(rows)).
//
// Backward without atomics (deterministic): workgroup (row block, column
// chunk) owns RV table rows x CH columns.  It takes the token ids in rounds of
// 2048 (8 consecutive ids per thread, loaded together), lists the tokens whose
// id falls in its rows in token order (a workgroup prefix sum of each
// thread's hits), and once the ids are done (or the list is full) adds their
// gradient chunks, sixteen rows' loads in flight at a time, to fp32
// accumulators in LDS in list order, then writes its rows once.  Every output-gradient element is read by one workgroup; the ids
// (8 bytes per token) are read by all of them from L2.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

constexpr int RV = 16;        // table rows per workgroup
constexpr int CH = 1024;      // columns per workgroup (4 per thread)
constexpr int kPer = 8;       // token ids per thread per round
constexpr int kRound = 256 * kPer;  // tokens per round
constexpr int kList = 3072;    // listed tokens held before their rows are added (12 KB of LDS)
constexpr int kBatch = 16;     // gradient rows loaded together

template <typename T>
__global__ __launch_bounds__(256) void embedding_fwd_kernel(const T* __restrict__ table,
                                                            const int64_t* __restrict__ ids,
                                                            T* __restrict__ out, int64_t n_tokens,
                                                            int64_t vocab, int64_t hidden) {
  constexpr int V = VecTraits<T>::N;
  const int64_t vecs = hidden / V;
  const int64_t total = n_tokens * vecs;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t t = i / vecs;
    const int64_t c = (i - t * vecs) * V;
    const int64_t id = ids[t];
    float v[V];
    if (id >= 0 && id < vocab) {
      load_vec<T>(table + id * hidden + c, v);
    } else {
      // an id outside the table's [0, vocab) gives a zero row and reads
      // nothing, as the reference masks ids outside its partition
      // (tensor_parallel/embedding.py:63-68; at TP=1 the partition is the table)
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = 0.f;
    }
    store_vec<T>(out + t * hidden + c, v);
  }
}

// 4 consecutive elements of T (8 bytes of bf16, 16 of fp32) as floats
template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&v)[4]) {
  if constexpr (sizeof(T) == 2) {
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    T e[4];
    __builtin_memcpy(e, &raw, 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = to_f32(e[i]);
  } else {
    const float4 raw = *reinterpret_cast<const float4*>(p);
    v[0] = raw.x;
    v[1] = raw.y;
    v[2] = raw.z;
    v[3] = raw.w;
  }
}

template <typename T>
__global__ __launch_bounds__(256, 2) void embedding_bwd_kernel(const T* __restrict__ dout,
                                                               const int64_t* __restrict__ ids,
                                                               const T* __restrict__ grad_in,
                                                               T* __restrict__ grad_out,
                                                               int64_t n_tokens, int64_t vocab,
                                                               int64_t hidden) {
  __shared__ float4 acc[RV * CH / 4];  // 64 KB: row r, this thread's 4 columns at [r * CH / 4 + thread]
  __shared__ int list[kList];          // matching tokens in token order: token * RV + row
  __shared__ int wave_total[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row_blocks = (vocab + RV - 1) / RV;
  const int64_t v0 = (blockIdx.x % row_blocks) * RV;
  const int64_t c0 = (blockIdx.x / row_blocks) * CH;
  const int cols = static_cast<int>(min<int64_t>(CH, hidden - c0));
  const int c = threadIdx.x * 4;  // this thread's 4 columns
  const int cc = c < cols ? c : 0;  // (a thread past the chunk's columns loads column 0, unused)
#pragma unroll
  for (int r = 0; r < RV; ++r) acc[r * (CH / 4) + threadIdx.x] = make_float4(0.f, 0.f, 0.f, 0.f);

  // the tied LM head's rows of this block, loaded first: nothing depends on
  // them until the end (rows past the table read its last row, not stored)
  float prior[RV][4];
#pragma unroll
  for (int r = 0; r < RV; ++r) {
    if (grad_in != nullptr) {
      load4<T>(grad_in + min(v0 + r, vocab - 1) * hidden + c0 + cc, prior[r]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) prior[r][e] = 0.f;
    }
  }

  // the listed gradient rows, in token order, into the accumulators: all of
  // a batch's loads in flight together
  int listed = 0;  // workgroup-uniform
  auto add_listed = [&]() {
    if (c < cols) {
      for (int k0 = 0; k0 < listed; k0 += kBatch) {
        float v[kBatch][4];
        int row[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int e = list[min(k0 + u, listed - 1)];
          row[u] = e % RV;
          load4<T>(dout + static_cast<int64_t>(e / RV) * hidden + c0 + c, v[u]);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (k0 + u < listed) {  // (no break: the loaded rows stay in registers)
            float4& a = acc[row[u] * (CH / 4) + threadIdx.x];
            float4 t = a;
            t.x += v[u][0];
            t.y += v[u][1];
            t.z += v[u][2];
            t.w += v[u][3];
            a = t;
          }
        }
      }
    }
    listed = 0;
  };

  // the ids in rounds of kPer consecutive tokens per thread, the next round's
  // in flight while this round's are listed; the rows are added once the
  // list is full or the ids are done, so that their loads are not spread
  // over the rounds one latency each
  int64_t id[kPer], next[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) next[j] = -1;
  auto load_ids = [&](int64_t base, int64_t (&dst)[kPer]) {
    const int64_t t0 = base + threadIdx.x * kPer;
#pragma unroll
    for (int j = 0; j < kPer; ++j) dst[j] = t0 + j < n_tokens ? ids[t0 + j] : -1;
  };
  load_ids(0, id);
  for (int64_t base = 0; base < n_tokens; base += kRound) {
    if (listed > kList - kRound) {
      // a full round may not fit: add what is listed first (every thread is
      // past the previous round's list writes: second barrier below)
      add_listed();
      __syncthreads();  // every thread is done reading the list
    }
    const int t_off = static_cast<int>(base) + threadIdx.x * kPer;
    int hits = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) hits += id[j] >= v0 && id[j] < v0 + RV;
    // exclusive prefix of the hits over the workgroup (thread order = token order)
    int incl = hits;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wave_total[wave] = incl;
    __syncthreads();  // wave totals ready
    int pos = listed + incl - hits;
    for (int w = 0; w < wave; ++w) pos += wave_total[w];
    const int total = wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (id[j] >= v0 && id[j] < v0 + RV) list[pos++] = (t_off + j) * RV + static_cast<int>(id[j] - v0);
    listed += total;
    __syncthreads();  // the round's list entries are visible; wave totals read
    if (base + kRound < n_tokens) load_ids(base + kRound, next);
#pragma unroll
    for (int j = 0; j < kPer; ++j) id[j] = next[j];
  }
  add_listed();
  __syncthreads();
  if (c >= cols) return;
#pragma unroll
  for (int r = 0; r < RV; ++r) {
    if (v0 + r >= vocab) break;
    const int64_t o = (v0 + r) * hidden + c0 + c;
    const float4 a4 = acc[r * (CH / 4) + threadIdx.x];
    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the embedding's own gradient is rounded to the table dtype before the
      // tied LM-head gradient is added (autograd adds two gradient tensors)
      const float mine = round_as<T>(av[e]);
      out[e] = grad_in != nullptr ? add_rn(prior[r][e], mine) : mine;
    }
    if constexpr (sizeof(T) == 2) {
      T ov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = from_f32<T>(out[e]);
      uint2 raw;
      __builtin_memcpy(&raw, ov, 8);
      *reinterpret_cast<uint2*>(grad_out + o) = raw;
    } else {
      *reinterpret_cast<float4*>(grad_out + o) = make_float4(out[0], out[1], out[2], out[3]);
    }
  }
}

template <typename T>
int fwd_impl(const void* table, const int64_t* ids, void* out, int64_t n_tokens, int64_t vocab,
             int64_t hidden, hipStream_t stream) {
  constexpr int V = VecTraits<T>::N;
  NMB_REQUIRE_SUPPORTED(hidden % V == 0, "embedding: hidden (%lld) must be a multiple of %d",
                        (long long)hidden, V);
  NMB_REQUIRE(aligned16(table) && aligned16(out), "embedding: tensors must be 16-byte aligned");
  const int64_t total = n_tokens * (hidden / V);
  if (total == 0) return NMB_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((embedding_fwd_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, static_cast<const T*>(table), ids, static_cast<T*>(out), n_tokens,
                     vocab, hidden);
  NMB_CHECK_LAUNCH("embedding_fwd");
  return NMB_OK;
}

template <typename T>
int bwd_impl(const void* dout, const int64_t* ids, const void* grad_in, void* grad_out,
             int64_t n_tokens, int64_t vocab, int64_t hidden, hipStream_t stream) {
  NMB_REQUIRE_SUPPORTED(hidden % 4 == 0, "embedding_bwd: hidden (%lld) must be a multiple of 4",
                        (long long)hidden);
  const int64_t blocks = ((vocab + RV - 1) / RV) * ((hidden + CH - 1) / CH);
  NMB_REQUIRE(blocks < (int64_t{1} << 31), "embedding_bwd: table too large");
  // the token list holds token * RV + row in 32 bits
  NMB_REQUIRE_SUPPORTED(n_tokens < (int64_t{1} << 27), "embedding_bwd: %lld tokens exceed the supported 2^27",
                        (long long)n_tokens);
  // rows of 4 elements are read as one 8-byte (bf16) or 16-byte (fp32) access
  const uintptr_t align = 4 * sizeof(T) - 1;
  NMB_REQUIRE((reinterpret_cast<uintptr_t>(dout) & align) == 0 &&
                  (reinterpret_cast<uintptr_t>(grad_out) & align) == 0 &&
                  (grad_in == nullptr || (reinterpret_cast<uintptr_t>(grad_in) & align) == 0),
              "embedding_bwd: dout, grad_in and grad_out must be aligned to %d bytes",
              static_cast<int>(align + 1));
  if (blocks == 0) return NMB_OK;
  hipLaunchKernelGGL((embedding_bwd_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, static_cast<const T*>(dout), ids, static_cast<const T*>(grad_in),
                     static_cast<T*>(grad_out), n_tokens, vocab, hidden);
  NMB_CHECK_LAUNCH("embedding_bwd");
  return NMB_OK;
}

}  // namespace
}  // namespace nmb

extern "C" int nmb_embedding_fwd(const void* table, const int64_t* ids, void* out, int64_t n_tokens,
                                 int64_t vocab, int64_t hidden, int dtype, hipStream_t stream) {
  NMB_REQUIRE(table != nullptr && ids != nullptr && out != nullptr, "embedding_fwd: null argument");
  NMB_REQUIRE(n_tokens >= 0 && vocab > 0 && hidden > 0, "embedding_fwd: invalid shape");
  if (dtype == NMB_BF16) return nmb::fwd_impl<nmb::bf16>(table, ids, out, n_tokens, vocab, hidden, stream);
  if (dtype == NMB_F32) return nmb::fwd_impl<float>(table, ids, out, n_tokens, vocab, hidden, stream);
  NMB_REQUIRE_SUPPORTED(false, "embedding_fwd: unsupported dtype %d", dtype);
  return NMB_EUNSUPPORTED;
}

extern "C" int nmb_embedding_bwd(const void* dout, const int64_t* ids, const void* grad_in,
                                 void* grad_out, int64_t n_tokens, int64_t vocab, int64_t hidden,
                                 int dtype, hipStream_t stream) {
  NMB_REQUIRE(dout != nullptr && ids != nullptr && grad_out != nullptr, "embedding_bwd: null argument");
  NMB_REQUIRE(n_tokens >= 0 && vocab > 0 && hidden > 0, "embedding_bwd: invalid shape");
  if (dtype == NMB_BF16)
    return nmb::bwd_impl<nmb::bf16>(dout, ids, grad_in, grad_out, n_tokens, vocab, hidden, stream);
  if (dtype == NMB_F32)
    return nmb::bwd_impl<float>(dout, ids, grad_in, grad_out, n_tokens, vocab, hidden, stream);
  NMB_REQUIRE_SUPPORTED(false, "embedding_bwd: unsupported dtype %d", dtype);
  return NMB_EUNSUPPORTED;
}
