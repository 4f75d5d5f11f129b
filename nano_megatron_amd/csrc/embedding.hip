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
// chunk) owns RV table rows x CH columns.  It walks the token ids in order,
// 256 at a time, compacts the tokens whose id falls in its rows into an LDS
// list (wavefront ballots + a block prefix, so the list keeps token order),
// and adds their gradient chunks to fp32 accumulators in LDS, then writes the
// rows once.  Every output-gradient element is read by one workgroup; the ids
// (8 bytes per token) are read by all of them from L2.
#include "common.h"
#include "vec.h"

namespace nmb {
namespace {

constexpr int RV = 16;     // table rows per workgroup
constexpr int CH = 1024;   // columns per workgroup (4 per thread)

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

template <typename T>
__global__ __launch_bounds__(256) void embedding_bwd_kernel(const T* __restrict__ dout,
                                                            const int64_t* __restrict__ ids,
                                                            const T* __restrict__ grad_in,
                                                            T* __restrict__ grad_out,
                                                            int64_t n_tokens, int64_t vocab,
                                                            int64_t hidden) {
  __shared__ float acc[RV * CH];     // 64 KB
  __shared__ int list_t[256];        // matching tokens of the current pass, in order
  __shared__ int list_r[256];
  __shared__ int wave_count[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row_blocks = (vocab + RV - 1) / RV;
  const int64_t v0 = (blockIdx.x % row_blocks) * RV;
  const int64_t c0 = (blockIdx.x / row_blocks) * CH;
  const int cols = static_cast<int>(min<int64_t>(CH, hidden - c0));
  const int c = threadIdx.x * 4;  // this thread's 4 columns
  for (int i = threadIdx.x; i < RV * CH; i += 256) acc[i] = 0.f;

  for (int64_t base = 0; base < n_tokens; base += 256) {
    const int64_t t = base + threadIdx.x;
    const int64_t id = t < n_tokens ? ids[t] : -1;
    const bool hit = id >= v0 && id < v0 + RV;
    const uint64_t mask = __ballot(hit);
    const int before = __builtin_popcountll(mask & ((uint64_t{1} << lane) - 1));
    if (lane == 0) wave_count[wave] = __builtin_popcountll(mask);
    __syncthreads();  // wave counts ready; the previous pass's list is consumed
    int off = 0;
    for (int w = 0; w < wave; ++w) off += wave_count[w];
    const int total = wave_count[0] + wave_count[1] + wave_count[2] + wave_count[3];
    if (hit) {
      list_t[off + before] = static_cast<int>(threadIdx.x);
      list_r[off + before] = static_cast<int>(id - v0);
    }
    __syncthreads();
    if (c < cols) {
      for (int k = 0; k < total; ++k) {
        const T* src = dout + (base + list_t[k]) * hidden + c0 + c;
        float* a = acc + list_r[k] * CH + c;
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] += to_f32(src[e]);
      }
    }
  }
  __syncthreads();
  if (c >= cols) return;
  for (int r = 0; r < RV && v0 + r < vocab; ++r) {
    const int64_t o = (v0 + r) * hidden + c0 + c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the embedding's own gradient is rounded to the table dtype before the
      // tied LM-head gradient is added (autograd adds two gradient tensors)
      const float mine = round_as<T>(acc[r * CH + c + e]);
      const float prior = grad_in != nullptr ? to_f32(grad_in[o + e]) : 0.f;
      grad_out[o + e] = from_f32<T>(grad_in != nullptr ? add_rn(prior, mine) : mine);
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
