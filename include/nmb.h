/*
 * nmb.h -- C ABI of libnmb.so, the MI355X (gfx950) kernels behind the
 * activation-checkpointed GPT block of pyy233/Nano-Megatron.
 *
 * Every entry point:
 *   - takes raw device pointers owned by the caller, plain sizes and strides
 *     (in elements), a dtype code and the caller's hipStream_t;
 *   - enqueues work on that stream and returns without synchronising;
 *   - returns NMB_OK or an error status, never throws, and records a message
 *     readable with nmb_last_error() on the same thread;
 *   - allocates no device memory: scratch comes in as a caller workspace.
 * All functions are reentrant; the PyTorch autograd device thread calls the
 * backward entry points while the main thread may call forward ones.
 *
 * The "replaces" notes cite the reference interface, as file:line under
 * pyy233/Nano-Megatron src/nano_megatron/.
 */
#ifndef NMB_H
#define NMB_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes; the Python host maps EINVAL/EUNSUPPORTED to ValueError and
 * EHIP to RuntimeError, as the reference raises ValueError on contract
 * violations (nn/kernels/torch_backend.py:45-55, nn/norms.py:34-37). */
#define NMB_OK 0
#define NMB_EINVAL 1
#define NMB_EUNSUPPORTED 2
#define NMB_EHIP 3

/* dtype codes: the path computes in fp32 (config 1) or bf16 storage with fp32
 * arithmetic (configs 2-5). */
#define NMB_F32 0
#define NMB_BF16 1

/* Message of the last failed call on this thread ("" if none). */
const char* nmb_last_error(void);

/* ABI version; bumped on any signature change. */
int nmb_abi_version(void);

/* ------------------------------------------------------------ RMSNorm
 * replaces RMSNorm.forward (nn/norms.py:33-41) and its autograd backward;
 * seam: KernelBackend.rms_norm (nn/kernels/interface.py:20-21,
 * nn/kernels/torch_backend.py:22-23).
 * x, y: [rows, cols] contiguous; w: [cols]; rstd (nullable): [rows] fp32.
 * y = cast(x * rsqrt(mean(x^2) + eps)) * w with fp32 statistics. */
int nmb_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                    int64_t cols, float eps, int dtype, hipStream_t stream);

/* Bytes of workspace nmb_rmsnorm_bwd needs for this shape. */
int nmb_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, size_t* bytes);

/* dx = rstd * (g - n * mean(g * n)) with g = dy * w, n = x * rstd (rstd
 * recomputed from x), plus residual_grad if non-null; dw = sum_rows(dy * n)
 * reduced deterministically through the workspace. */
int nmb_rmsnorm_bwd(const void* x, const void* w, const void* dy, const void* residual_grad,
                    void* dx, void* dw, void* workspace, size_t workspace_bytes, int64_t rows,
                    int64_t cols, float eps, int dtype, hipStream_t stream);

/* nmb_rmsnorm_bwd in its two launches, for a caller that runs the weight
 * gradient's column sum on another stream (ordered after the first by the
 * caller): nmb_rmsnorm_bwd_rows writes dx and the per-workgroup dw partials
 * into the workspace; nmb_rmsnorm_bwd_dw sums them into dw in a fixed order
 * (the same bits as nmb_rmsnorm_bwd).  Same reference function. */
int nmb_rmsnorm_bwd_rows(const void* x, const void* w, const void* dy, const void* residual_grad,
                         void* dx, void* workspace, size_t workspace_bytes, int64_t rows,
                         int64_t cols, float eps, int dtype, hipStream_t stream);
int nmb_rmsnorm_bwd_dw(const void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                       void* dw, int dtype, hipStream_t stream);

/* ------------------------------------------------------------ RoPE
 * replaces RotaryEmbedding.forward + apply_rotary_pos_emb
 * (nn/rotary.py:27-38, 55-70) as called at models/gpt/attention.py:180-181.
 * nmb_rope_table fills cos/sin [n_pos, half] fp32 with cos(p * inv_freq[i]).
 * nmb_rope_apply rotates x [batch, seq, heads, 2*half] (strides in elements
 * for b, s, h; the last dim contiguous) into out (same strides; may alias x):
 *   out = x * cos + rotate_half(x) * sin        (inverse = 0)
 *   out = x * cos - rotate_half(x) * sin        (inverse = 1, the backward)
 * position of (b, s) = positions[b * pos_batch_stride + s] if positions is
 * non-null, else pos_offset + s. */
int nmb_rope_table(float* cos_table, float* sin_table, const float* inv_freq, int64_t n_pos,
                   int64_t half, hipStream_t stream);

int nmb_rope_apply(const void* x, void* out, const float* cos_table, const float* sin_table,
                   int64_t n_pos, const int32_t* positions, int64_t pos_batch_stride,
                   int64_t pos_offset, int64_t batch, int64_t seq, int64_t heads,
                   int64_t head_dim, const int64_t* x_strides, const int64_t* out_strides,
                   int inverse, int dtype, hipStream_t stream);

/* ------------------------------------------------------------ SwiGLU
 * replaces F.silu(gate) * up (models/gpt/mlp.py:77).
 * All operands are [rows, cols] with a row stride (elements). */
int nmb_swiglu_fwd(const void* gate, int64_t gate_ld, const void* up, int64_t up_ld, void* out,
                   int64_t out_ld, int64_t rows, int64_t cols, int dtype, hipStream_t stream);

/* Fused recompute-backward: from gate, up and d_out produce d_gate, d_up and
 * (if out is non-null) the recomputed out = silu(gate) * up that the
 * down-projection weight gradient needs. */
int nmb_swiglu_bwd(const void* gate, int64_t gate_ld, const void* up, int64_t up_ld,
                   const void* dout, int64_t dout_ld, void* dgate, int64_t dgate_ld, void* dup,
                   int64_t dup_ld, void* out, int64_t out_ld, int64_t rows, int64_t cols,
                   int dtype, hipStream_t stream);

/* ------------------------------------------------------------ attention
 * replaces TorchKernelBackend.local_attention (nn/kernels/torch_backend.py:
 * 25-76; seam nn/kernels/interface.py:22-25) and the ring maths of
 * _ring_forward/_ring_backward (context_parallel/ring.py:104-250).
 *
 * q: [batch, seq_q, q_heads, head_dim]; each of the n_blocks K/V blocks:
 * [batch, seq_k, kv_heads, head_dim]; o like q.  Strides are arrays of 3
 * int64 (batch, seq, head) in elements; head_dim is contiguous.  K and V (and
 * dK, dV) share kv_strides; dq shares q_strides; dO shares o_strides.
 * Query i has absolute position q_offset + i; key j of block b has position
 * k_offsets[b] + j.  With causal != 0 a key is visible iff its position is
 * <= the query's.  Query head h reads KV head h / (q_heads / kv_heads) (GQA
 * without materialised repeats).  The blocks are one concatenated key
 * sequence for the online softmax.  lse: [batch, q_heads, seq_q] fp32,
 * natural log; a query with no visible key gets o = 0 and lse = -inf.
 * scale <= 0 selects 1/sqrt(head_dim). */
int nmb_attn_fwd(const void* q, const void* const* k_blocks, const void* const* v_blocks,
                 const int64_t* k_offsets, int n_blocks, void* o, float* lse, int64_t batch,
                 int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                 int64_t head_dim, const int64_t* q_strides, const int64_t* kv_strides,
                 const int64_t* o_strides, int causal, int64_t q_offset, float scale, int dtype,
                 hipStream_t stream);

/* The forward's output recomputed from its saved LSE (the reference
 * recomputes attention in the checkpointed backward, nn/activation_checkpoint.py:
 * 73-100 / context_parallel/ring.py:169-250 recompute P from the LSE): with the
 * softmax statistics known, P = exp(S - lse) directly, no running maximum or
 * rescale; o = P V.  Same arguments as nmb_attn_fwd, lse read.  Equal to the
 * forward's o within bf16 rounding (not bit for bit: the forward normalises
 * at the end).  bf16 only. */
int nmb_attn_fwd_from_lse(const void* q, const void* const* k_blocks, const void* const* v_blocks,
                          const int64_t* k_offsets, int n_blocks, const float* lse, void* o,
                          int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                          int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                          const int64_t* kv_strides, const int64_t* o_strides, int causal,
                          int64_t q_offset, float scale, int dtype, hipStream_t stream);

/* Bytes of workspace nmb_attn_bwd needs: the fp32 delta = rowsum(dO * O) and,
 * for bf16, the softmax LSE in base 2 (both [batch, q_heads, seq_q]). */
int nmb_attn_bwd_workspace_bytes(int64_t batch, int64_t q_heads, int64_t seq_q, size_t* bytes);

/* Backward from the saved lse: dq (overwritten), and per block dk, dv
 * (overwritten).  Deterministic: no atomics. */
int nmb_attn_bwd(const void* q, const void* const* k_blocks, const void* const* v_blocks,
                 const int64_t* k_offsets, int n_blocks, const void* o, const void* dout,
                 const float* lse, void* dq, void* const* dk_blocks, void* const* dv_blocks,
                 void* workspace, size_t workspace_bytes, int64_t batch, int64_t q_heads,
                 int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                 const int64_t* q_strides, const int64_t* kv_strides, const int64_t* o_strides,
                 int causal, int64_t q_offset, float scale, int dtype, hipStream_t stream);

/* nmb_attn_bwd without a workspace argument and without any allocation: no
 * counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch (delta and the base-2 LSE, fp32
 * [batch, q_heads, seq_q] each) lives in a fixed 8 MiB device array, one per
 * device, held until the process ends: batch x q_heads x seq_q must be at
 * most 1,048,576 (EINVAL beyond).  Every call on a device uses that device's
 * array, so calls that overlap on one device (two streams or threads) race;
 * the stream must belong to the current device.  Same results as
 * nmb_attn_bwd, bit for bit. */
int nmb_attn_bwd_noalloc(const void* q, const void* const* k_blocks, const void* const* v_blocks,
                         const int64_t* k_offsets, int n_blocks, const void* o, const void* dout,
                         const float* lse, void* dq, void* const* dk_blocks, void* const* dv_blocks,
                         int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                         int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                         const int64_t* kv_strides, const int64_t* o_strides, int causal,
                         int64_t q_offset, float scale, int dtype, hipStream_t stream);

/* nmb_attn_bwd for one K/V block that holds the queries' own tokens (the
 * block's self-attention; reference models/gpt/attention.py:180-206) with the
 * RoPE backward of q and k fused into the dQ / dK stores (replaces
 * nmb_attn_bwd + two nmb_rope_apply(inverse = 1); nn/rotary.py:27-38): dq and
 * dk come out rotated by -theta with the rotary kernel's roundings, bit for
 * bit.  Token i's position is positions[b * pos_batch_stride + i] (int32,
 * nullable) or pos_offset + i.  bf16 only; head_dim 64 or 128. */
int nmb_attn_bwd_rope(const void* q, const void* k, const void* v, const void* o, const void* dout,
                      const float* lse, void* dq, void* dk, void* dv, void* workspace,
                      size_t workspace_bytes, int64_t batch, int64_t q_heads, int64_t kv_heads,
                      int64_t seq, int64_t head_dim, const int64_t* q_strides,
                      const int64_t* kv_strides, const int64_t* o_strides, int causal,
                      int64_t q_offset, float scale, const float* cos_table, const float* sin_table,
                      int64_t n_pos, const int32_t* positions, int64_t pos_batch_stride,
                      int64_t pos_offset, hipStream_t stream);

/* Attention with an explicit mask and/or dropout: local_attention called
 * with attention_mask or dropout_p > 0 (reference nn/kernels/torch_backend.py:
 * 60-76: the mask goes to SDPA, ANDed with the causal mask when causal, and
 * SDPA applies dropout_p to the normalised probabilities).  One K/V block at
 * key offset 0; layouts and strides as nmb_attn_fwd / nmb_attn_bwd.
 * mask_kind 0: no mask (mask and mask_strides ignored); 1: a boolean mask,
 * one byte per entry, nonzero = attend; 2: an additive mask of the attention
 * dtype, added to the scaled scores (-inf drops the key).  mask_strides: the
 * mask's element strides over [batch, q_heads, seq_q, seq_k], 0 for a
 * broadcast dimension.  A query row with no visible key gives a zero output
 * row, lse = -inf and zero gradients (SDPA's safe softmax).  dropout_p in
 * [0, 1): probability (b, h, i, j) is kept iff bits >= floor(p * 2^32) and then
 * scaled by 1 / (1 - p), with bits the 32-bit half (idx & 1) of SplitMix64's
 * output for counter idx >> 1 under `seed` (SplitMix64: Steele, Lea and Flood,
 * OOPSLA 2014) at idx = ((b * q_heads + h) * seq_q + i) * seq_k + j; lse is
 * that of the undropped softmax, and the backward, given the same seed,
 * regenerates the mask.  The mask cannot equal torch's Philox stream, so
 * dropout matches the reference in distribution, not bit for bit.  bf16 or
 * fp32, head_dim <= 128, any strides; computed in fp32 one query row per
 * wavefront (a parity path: no configuration of the reference uses a mask
 * or attention dropout).  Backward workspace: nmb_attn_bwd_workspace_bytes
 * (only its first half, the delta rows, is used). */
int nmb_attn_masked_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                        int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                        const int64_t* kv_strides, const int64_t* o_strides, const void* mask,
                        int mask_kind, const int64_t* mask_strides, int causal, int64_t q_offset,
                        float scale, float dropout_p, uint64_t seed, int dtype, hipStream_t stream);
int nmb_attn_masked_bwd(const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse, void* dq, void* dk, void* dv,
                        void* workspace, size_t workspace_bytes, int64_t batch, int64_t q_heads,
                        int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                        const int64_t* q_strides, const int64_t* kv_strides,
                        const int64_t* o_strides, const void* mask, int mask_kind,
                        const int64_t* mask_strides, int causal, int64_t q_offset, float scale,
                        float dropout_p, uint64_t seed, int dtype, hipStream_t stream);

/* ------------------------------------------------------------ dropout
 * replaces parallel_dropout (nn/dropout.py:47-70, F.dropout) and the residual
 * add around it in GPTLayer.forward (models/gpt/layer.py:114-137) and after
 * the embedding (models/gpt/model.py:203-212).
 * out[i] = cast(residual[i] + cast(keep(i) ? x[i] / (1 - p) : 0)) over n
 * contiguous elements of dtype, residual nullable (then 0); keep(i) is the
 * SplitMix64 mask of nmb_attn_masked_fwd at idx = i.  Without a residual the
 * call is also the dropout's backward (dx = dropout(dout), same seed).  out
 * may alias x or residual.  p in [0, 1); p = 0 is the identity. */
int nmb_dropout_add(const void* x, const void* residual, void* out, int64_t n, float p, uint64_t seed,
                    int dtype, hipStream_t stream);

/* ------------------------------------------------------------ embedding
 * replaces VocabParallelEmbedding.forward at TP=1 (tensor_parallel/
 * embedding.py:60-74, F.embedding) and its backward.
 * table / out / dout / grads: row-major [vocab, hidden] and [n_tokens, hidden]
 * of dtype; ids: int64 [n_tokens].  An id outside [0, vocab) gives a zero row
 * and contributes nothing to the table gradient (the reference masks ids
 * outside its partition to zero rows, tensor_parallel/embedding.py:63-68).
 * Backward: grad_out = grad_in + sum over tokens of dout rows (fp32 sums in
 * token order, rounded to dtype, then added to grad_in, as autograd adds the
 * tied LM head's gradient: models/gpt/model.py:125-142); grad_in may be null
 * (then 0) and may alias grad_out.  Deterministic (no atomics). */
int nmb_embedding_fwd(const void* table, const int64_t* ids, void* out, int64_t n_tokens,
                      int64_t vocab, int64_t hidden, int dtype, hipStream_t stream);
int nmb_embedding_bwd(const void* dout, const int64_t* ids, const void* grad_in, void* grad_out,
                      int64_t n_tokens, int64_t vocab, int64_t hidden, int dtype,
                      hipStream_t stream);

/* ------------------------------------------------------------ cross entropy
 * replaces _VocabParallelCrossEntropy.forward/backward at TP=1
 * (tensor_parallel/cross_entropy.py:30-86) applied to one chunk of tied
 * LM-head logits (tensor_parallel/layers.py:207-214).
 * logits: [rows, vocab] with row stride ld; targets: int64 [rows].
 * Forward: loss[r] = lse[r] - z[r, t_r] (0 if t_r == ignore_index), lse in
 * fp32 over fp32-converted logits. */
int nmb_ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t rows,
               int64_t vocab, int64_t ignore_index, float* loss, float* lse, int dtype,
               hipStream_t stream);

/* Backward in place: logits[r, j] <- (exp(z - lse[r]) - [j == t_r]) * grad[r],
 * rows with an ignored target become 0. grad: fp32 [rows]. */
int nmb_ce_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t rows, int64_t vocab,
               int64_t ignore_index, const float* lse, const float* grad, int dtype,
               hipStream_t stream);

/* ------------------------------------------------------------ GEMM
 * replaces the dense projections nn.Linear / F.linear (nn/kernels/
 * torch_backend.py:19-20, tensor_parallel/layers.py:214) and their autograd
 * products, bf16 in / bf16 out with fp32 accumulation:
 *   D[M, N] = alpha * op(A)[M, K] * op(B)[K, N] + beta * C[M, N]   (row-major)
 * a_layout 0: A stored [M, K] (row stride lda); 1: A stored [K, M].
 * b_layout 0: B stored [N, K] (a weight used as W^T); 1: B stored [K, N].
 * C may alias D.  N, the contiguous extents and lda/ldb/ldc/ldd must be
 * multiples of 8; all pointers 16-byte aligned.  Small M x N with long K is
 * split along K: fp32 partials go to the caller's workspace (size from
 * nmb_gemm_bf16_workspace_bytes, 0 when unsplit) and are summed in a fixed
 * order (deterministic). */
int nmb_gemm_bf16_workspace_bytes(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k,
                                  int64_t* bytes);
int nmb_gemm_bf16(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k, float alpha,
                  const void* a, int64_t lda, const void* b, int64_t ldb, float beta,
                  const void* c, int64_t ldc, void* d, int64_t ldd, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream);

/* bf16 GEMM with an fp32 output, for sums of products rounded to bf16 once
 * (the tied LM-head gradient dE = sum over token chunks of G_c^T x_c, which
 * the reference forms as one product G^T X with one rounding:
 * tensor_parallel/layers.py:207-214 under autograd):
 *   D32[M, N] = alpha * op(A) * op(B) + beta * D32   (fp32, row-major)
 * Operands, layouts, checks and workspace as nmb_gemm_bf16 (same plan, so
 * nmb_gemm_bf16_workspace_bytes gives the size); ldd32 >= N, a multiple of 4,
 * D32 16-byte aligned. */
int nmb_gemm_bf16_f32out(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k, float alpha,
                         const void* a, int64_t lda, const void* b, int64_t ldb, float beta,
                         float* d32, int64_t ldd32, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream);

/* fp32 GEMM on the fp32 matrix cores, for the fp32 parity configuration
 * (replaces the same nn.Linear / F.linear products in fp32):
 *   D[M, N] = alpha * op(A) * op(B) + beta * C, layouts as nmb_gemm_bf16
 * (a_layout 0: A [M, K], 1: [K, M]; b_layout 0: B [N, K], 1: [K, N]); any
 * shape, leading dimension and alignment; C may alias D; exact fp32 products
 * accumulated in fp32. */
int nmb_gemm_f32(int a_layout, int b_layout, int64_t m, int64_t n, int64_t k, float alpha,
                 const float* a, int64_t lda, const float* b, int64_t ldb, float beta,
                 const float* c, int64_t ldc, float* d, int64_t ldd, hipStream_t stream);

/* GEMM with the rotary embedding as its epilogue: the Q/K/V projection and
 * RoPE of q and k in one pass (reference models/gpt/attention.py:172-181 with
 * nn/rotary.py:27-38, 55-70; replaces nmb_gemm_bf16 + two nmb_rope_apply).
 *   D = A B (A row-major [M, K]; b_layout as in nmb_gemm_bf16), then each of
 *   the first rope_cols columns of D, read as heads of head_dim (64 or 128),
 *   is rotated with the reference's roundings: q = bf16(D), cos/sin = bf16 of
 *   the fp32 tables [n_pos, head_dim/2], bf16 after each product and the sum.
 * Row m is token (m / seq, m % seq); its position is positions[(m / seq) *
 * pos_batch_stride + m % seq] (int32, nullable) or pos_offset + m % seq.
 * The result equals nmb_gemm_bf16 followed by nmb_rope_apply on the q and k
 * columns bit for bit.  No workspace (never split along K). */
int nmb_gemm_bf16_rope(int b_layout, int64_t m, int64_t n, int64_t k, const void* a, int64_t lda,
                       const void* b, int64_t ldb, void* d, int64_t ldd, const float* cos_table,
                       const float* sin_table, int64_t n_pos, const int32_t* positions,
                       int64_t pos_batch_stride, int64_t pos_offset, int64_t seq, int64_t head_dim,
                       int64_t rope_cols, hipStream_t stream);

/* The gate/up projection GEMM with the SwiGLU activation as its epilogue
 * (reference models/gpt/mlp.py:44-70, 77: gate_proj, up_proj, F.silu(gate) *
 * up; replaces nmb_gemm_bf16 of [Wg; Wu] + nmb_swiglu_fwd).
 *   P = A [Wg; Wu]^T, A row-major [M, K], b = [2F, K] K-contiguous (rows 0..F-1
 *   the gate weight, F..2F-1 the up weight, row stride ldb);
 *   gu (nullable) [M, 2F] receives bf16(P);
 *   d (nullable) [M, F] receives bf16(silu(bf16(P_gate)) * bf16(P_up)) with
 *   the roundings of nmb_swiglu_fwd.
 * One plan per shape, never split along K: gu is the same bits whether or not
 * d is written, and d equals nmb_swiglu_fwd of that gu bit for bit.  F, K,
 * lda, ldb, ldd, ldgu multiples of 8; no workspace. */
int nmb_gemm_bf16_swiglu(int64_t m, int64_t f, int64_t k, const void* a, int64_t lda, const void* b,
                         int64_t ldb, void* d, int64_t ldd, void* gu, int64_t ldgu,
                         hipStream_t stream);

/* The down projection's input gradient with the SwiGLU backward as its
 * epilogue (autograd of models/gpt/mlp.py:77-78: ds = dY Wd, then the
 * backward of silu(gate) * up; replaces nmb_gemm_bf16 + nmb_swiglu_bwd):
 *   ds = bf16(A B), A row-major [M, K] (dY), b_layout as nmb_gemm_bf16
 *   (Wd used as [K, F]: b_layout 1 for the row-major [K, F] weight);
 *   gu [M, 2F] holds the gate/up product (gate columns 0..F-1, up F..2F-1);
 *   dgu [M, 2F] receives (d gate | d up); act (nullable) [M, F] receives
 *   silu(gate) * up for the down projection's weight gradient.
 * Bit-identical to nmb_gemm_bf16 followed by nmb_swiglu_bwd (same element
 * function, ds rounded to bf16 first); never split along K; F, K and the
 * leading dimensions multiples of 8; no workspace; no intermediate ds in
 * memory. */
int nmb_gemm_bf16_swiglu_bwd(int b_layout, int64_t m, int64_t f, int64_t k, const void* a,
                             int64_t lda, const void* b, int64_t ldb, const void* gu, int64_t ldgu,
                             void* dgu, int64_t lddgu, void* act, int64_t ldact, hipStream_t stream);

/* The MLP backward of a recomputed block in one kernel (autograd of
 * models/gpt/mlp.py:72-78 with the gate/up product recomputed, as a
 * checkpointed layer's backward re-runs it): per 256 x 128 tile of F,
 *   [g|u] = bf16(A1 Wgu^T)   A1 [M, K1] row-major (n2), Wgu [2F, K1] row-major
 *                            ([Wg; Wu], paired as nmb_gemm_bf16_swiglu reads it),
 *   ds = bf16(A2 op(Wd))     A2 [M, K2] row-major (dY), b_layout as above,
 * then the SwiGLU backward: dgu [M, 2F] = (d gate | d up), act (nullable)
 * [M, F] = silu(g) u.  Bit-identical to nmb_gemm_bf16_swiglu (product only)
 * followed by nmb_gemm_bf16_swiglu_bwd, without the [M, 2F] product in
 * memory; never split along K; F, K1, K2 and the leading dimensions
 * multiples of 8; no workspace. */
int nmb_gemm_bf16_gate_up_swiglu_bwd(int64_t m, int64_t f, int64_t k1, const void* a1, int64_t lda1,
                                     const void* wgu, int64_t ldwgu, int64_t k2, const void* a2,
                                     int64_t lda2, int b_layout, const void* wd, int64_t ldwd, void* dgu,
                                     int64_t lddgu, void* act, int64_t ldact, hipStream_t stream);

/* ------------------------------------------------------------ optimizer
 * replaces FlatShardZeROStrategy.clip_grad_norm + optimizer_step at DP=1
 * (data_parallel/_zero.py:130-199; defaults config/schema.py:439-445):
 * global grad-norm clip (max_norm <= 0: no clip) and fp32-master AdamW with
 * decoupled weight decay, writing the master, both moments and the
 * parameter (cast to param_dtype) in one pass.
 * params / grads: DEVICE arrays of n_tensors device pointers; offsets: DEVICE
 * array of n_tensors + 1 element prefix sums (offsets[n] = total_elements);
 * master / exp_avg / exp_avg_sq: flat fp32 [total_elements] in that order.
 * norm_out (nullable, device, 2 floats): receives the pre-clip norm and the
 * clip coefficient.  Deterministic (fixed-order reductions).  The
 * hyper-parameters are doubles, as the reference's Python floats are: the
 * derived scalars (1 - beta, 1 - lr wd, sqrt(bias correction 2), lr / bias
 * correction 1) are formed in double and rounded to fp32 once, as torch rounds
 * a Python scalar meeting an fp32 tensor; the update then runs the
 * reference's tensor operations in their order, each rounded once.  Valid
 * hyper-parameters: lr >= 0 (a schedule may end at 0), eps > 0, betas in
 * [0, 1), step >= 1. */
int nmb_adamw_workspace_bytes(int64_t total_elements, size_t* bytes);

int nmb_adamw_step(const uint64_t* params, const uint64_t* grads, const int64_t* offsets,
                   int n_tensors, int64_t total_elements, float* master, float* exp_avg,
                   float* exp_avg_sq, int param_dtype, int grad_dtype, double lr, double beta1,
                   double beta2, double eps, double weight_decay, int64_t step, float max_norm,
                   float* norm_out, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* nmb_adamw_step with the update's scalars read from device memory, so that a
 * captured HIP graph of the training step (one capture of the trainer's step,
 * training/trainer.py:424-474, replayed every step) picks up each step's bias
 * corrections and learning rate: the launch arguments of a graph are fixed
 * when it is captured.  The record (nmb_adamw_hyper_bytes bytes, 4-byte
 * aligned, in device memory) is what nmb_adamw_hyper writes into host memory
 * for (lr, beta1, beta2, eps, weight_decay, step): the same fp32 scalars
 * nmb_adamw_step forms, so both entry points update bit-identically.  The
 * caller copies the record to the device before each replay. */
int nmb_adamw_hyper_bytes(size_t* bytes);
int nmb_adamw_hyper(double lr, double beta1, double beta2, double eps, double weight_decay,
                    int64_t step, void* record);
int nmb_adamw_step_hyper(const uint64_t* params, const uint64_t* grads, const int64_t* offsets,
                         int n_tensors, int64_t total_elements, float* master, float* exp_avg,
                         float* exp_avg_sq, int param_dtype, int grad_dtype, const void* hyper,
                         float max_norm, float* norm_out, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NMB_H */
