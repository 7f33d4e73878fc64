/*
 * eth_amd.h -- C-ABI of the MI355X (gfx950) implementation of one ETH
 * pipeline stage's training step.
 *
 * Plain pointers, sizes and a hipStream_t (passed as void*); no framework
 * types.  Every function returns ETH_OK (0) or an error code and, on error,
 * leaves a message in eth_last_error() (thread-local).  All device pointers
 * must point to memory of the current HIP device; all work is enqueued on
 * `stream` and nothing here synchronizes the host or allocates device memory.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the YuMJie/ETH tree).
 */
#ifndef ETH_AMD_H
#define ETH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ETH_OK = 0, ETH_ERR_INVALID = 1, ETH_ERR_HIP = 2 };
enum { ETH_F32 = 0, ETH_F16 = 1, ETH_BF16 = 2 };

/* Library identity and error reporting. */
int eth_abi_version(void);
const char* eth_last_error(void);

/* Fill n floats with `value` (graph-safe replacement for hipMemsetAsync). */
int eth_fill_f32(float* dst, int64_t n, float value, void* stream);

/* ------------------------------------------------------------------------
 * Block-wise gradient synchronization, local half.
 *
 * A bucket payload is described by a device table of chunks.  Each chunk is a
 * 2-D strided block of one main_grad tensor (rows x row_len elements, rows
 * `src_stride` elements apart) that occupies payload[dst, dst+rows*row_len).
 * The host splits every TensorSegmentSpec of a LocalFragmentBindingSpec into
 * chunks of at most ETH_CHUNK_ELEMS elements, once, when the plan is bound.
 * ---------------------------------------------------------------------- */
#define ETH_CHUNK_ELEMS 16384

typedef struct eth_chunk {
  uint64_t src;        /* device address of the chunk's first source element */
  int64_t dst;         /* element offset of the chunk inside the payload */
  int64_t src_stride;  /* elements between successive rows of the source */
  int32_t rows;        /* rows in the chunk (1 for a contiguous run) */
  int32_t row_len;     /* contiguous elements per row */
  float scale;         /* LocalFragmentBindingSpec.contribution_scale */
  int32_t flags;       /* ETH_CHUNK_NORM | ETH_CHUNK_SHADOWED */
} eth_chunk_t;

#define ETH_CHUNK_NORM 1     /* counts toward the optimizer L2 norm */
#define ETH_CHUNK_SHADOWED 2 /* a later bucket of the same pass packs over this
                              * chunk's payload range: its unpack skips the
                              * ETH_UNPACK_WRITEBACK store, which nothing could
                              * read before it is overwritten */

/* Pack: payload[dst + i] = src[i] * scale (the multiply is skipped when
 * scale == 1, so the copy is bit-exact).
 * Replaces GradientBucketExecutor._pack / _segment_view
 * (eth/runtime/megatron/grad_sync/executor.py:173-226). */
int eth_bucket_pack(const eth_chunk_t* chunks, int64_t n_chunks, void* payload,
                    int dtype, void* stream);

/* Unpack after the bucket's all-reduce:
 *   v = payload[i] * normalization_scale       (skipped when == 1)
 *   if (flags & ETH_UNPACK_WRITEBACK) payload[i] = v  (not in ETH_CHUNK_SHADOWED
 *                                                      chunks)
 *   g = v * inv_loss_scale                      (only with ETH_UNPACK_UNSCALE)
 *   src[i] = g;  found_inf |= !isfinite(v);  partials[chunk] = sum g^2 over
 *   ETH_CHUNK_NORM chunks (only with ETH_UNPACK_STATS).
 * `partials` (one double per chunk, indexed from partial_base) and
 * `found_inf` (one float, set to 1.0 on a non-finite value, never cleared
 * here) are only touched with ETH_UNPACK_STATS.
 * Replaces payload.mul_ + GradientBucketExecutor._unpack
 * (executor.py:228-261) fused with
 * torch._amp_foreach_non_finite_check_and_unscale_
 * (optimizer/optimizer.py:436-461) and the per-tensor pow(2).sum() of
 * CanonicalOptimizerSemantics.clip_grad_norm
 * (grad_sync/optimizer_semantics.py:563-595). */
#define ETH_UNPACK_WRITEBACK 1
#define ETH_UNPACK_UNSCALE 2
#define ETH_UNPACK_STATS 4
int eth_bucket_unpack(const eth_chunk_t* chunks, int64_t n_chunks, void* payload,
                      int dtype, float normalization_scale, float inv_loss_scale,
                      int flags, float* found_inf, double* partials,
                      int64_t partial_base, void* stream);

/* One bucket of a sync pass: its chunk table, payload and first partial slot. */
typedef struct eth_bucket {
  const eth_chunk_t* chunks; /* device chunk table */
  int64_t n_chunks;
  void* payload;             /* device payload (the rank's scratch buffer) */
  int64_t partial_base;      /* first slot of the bucket's L2 partials */
  int32_t dtype;             /* ETH_F32 / ETH_F16 / ETH_BF16 */
  int32_t reserved;          /* 0 */
} eth_bucket_t;

/* A whole sync pass over `n_buckets` buckets (host array, in order) whose
 * all-reduce is the identity -- every process group of the pass holds this
 * rank alone -- with the pass's scale, flags and statistics buffers
 * (ETH_UNPACK_UNSCALE applies to fp32 payloads only).  Every entry is
 * checked before the first launch.  One host call instead of two per
 * bucket, so the host stays ahead of the GPU through the pass.
 * Without `staging` (NULL): for each bucket, eth_bucket_pack then
 * eth_bucket_unpack, the launches of the per-bucket calls in their order.
 * With `staging` (16-byte aligned, two halves of `staging_half_bytes`, each
 * at least the largest payload of the pass): bucket i is packed into half
 * (i & 1) and unpacked from it, and one launch unpacks bucket i-1 while it
 * packs bucket i (n_buckets + 1 launches instead of 2 * n_buckets).  The
 * gradients, statistics and the payload buffers' final contents are
 * bit-identical to the per-bucket calls: a chunk that no later bucket packs
 * over (not ETH_CHUNK_SHADOWED) stores its payload values -- normalized,
 * when normalization_scale != 1 -- into the bucket's payload buffer, which
 * is what the per-bucket sequence leaves there.
 * Replaces the bucket loop of GradientBucketExecutor.execute
 * (eth/runtime/megatron/grad_sync/executor.py:248-260) for a single-rank
 * data-parallel group. */
int eth_bucket_sync_local(const eth_bucket_t* buckets, int64_t n_buckets,
                          float normalization_scale, float inv_loss_scale, int flags,
                          float* found_inf, double* partials, void* staging,
                          int64_t staging_half_bytes, void* stream);

/* Standalone unscale + inf/nan check + sum of squares over chunk-described
 * fp32 gradients, in place (g *= inv_scale when ETH_UNPACK_UNSCALE).  Used
 * when gradients did not pass through eth_bucket_unpack this step.
 * Replaces torch._amp_foreach_non_finite_check_and_unscale_
 * (optimizer/optimizer.py:452-453) + the canonical L2 statistic
 * (grad_sync/optimizer_semantics.py:584-587).
 * With ETH_STATS_SCALED_OVERFLOW (and without ETH_UNPACK_UNSCALE) the
 * gradients are left as they are and `inv_loss_scale` carries the loss
 * scale instead: found_inf is also set where g * scale is not finite, i.e.
 * where the loss-scaled value of an already unscaled gradient (a tied
 * embedding sum formed after the unpack) would have overflowed. */
#define ETH_STATS_SCALED_OVERFLOW 8
int eth_grad_stats(const eth_chunk_t* chunks, int64_t n_chunks, float inv_loss_scale,
                   int flags, float* found_inf, double* partials, int64_t partial_base,
                   void* stream);

/* The tied word-embedding sum fused with those post-sync statistics: for
 * every element of the chunks (the root's fp32 main grad), s = root + copy
 * (the copy's element at the same offset from `copy` as the root's from
 * `root`) is stored into both, and the chunk's statistics are taken of s as
 * eth_grad_stats(..., inv_loss_scale = loss_scale,
 * flags = ETH_STATS_SCALED_OVERFLOW) takes them: found_inf where
 * s * loss_scale is not finite, partials[partial_base + chunk] = sum of s^2
 * for ETH_CHUNK_NORM chunks.  The bits equal eth_tied_grad_sum followed by
 * that eth_grad_stats call, in one pass instead of two.  Replaces the
 * same-rank branch of synchronize_shared_weights_grads
 * (eth/runtime/megatron/training.py:489-531) together with the root's share
 * of the unscale check and L2 statistic (optimizer/optimizer.py:452-453,
 * grad_sync/optimizer_semantics.py:584-587). */
int eth_tied_grad_sum_stats(const eth_chunk_t* chunks, int64_t n_chunks, float* root,
                            float* copy, float loss_scale, float* found_inf,
                            double* partials, int64_t partial_base, void* stream);

/* The fp16-contract widening copy fused with the statistics: 16-bit main
 * grads (`dtype` bf16 / fp16; chunk.src, strided rows as in a bucket table)
 * into contiguous fp32 gradients out[chunk.dst ...], g = float(x) (exact),
 * then, as eth_grad_stats does on g: g *= inv_loss_scale with
 * ETH_UNPACK_UNSCALE; found_inf and partials[partial_base + chunk] with
 * ETH_UNPACK_STATS.  One pass instead of a copy and an in-place unscale.
 * Replaces main_param.grad = main_grad.float() of
 * Float16OptimizerWithFloat16Params._copy_model_grads_to_main_grads
 * (optimizer/optimizer.py:388-404) fused with
 * torch._amp_foreach_non_finite_check_and_unscale_ (:452-453) and the
 * canonical L2 statistic (grad_sync/optimizer_semantics.py:584-587). */
int eth_widen_grad_stats(const eth_chunk_t* chunks, int64_t n_chunks, float* out, int dtype,
                         float inv_loss_scale, int flags, float* found_inf, double* partials,
                         int64_t partial_base, void* stream);

/* Reduce `n` per-chunk partials into stats[0] = sum of squares (double) and
 * stats[1] = L2 norm; stats[2] = clip coefficient max_norm/(norm+1e-6)
 * (1.0 when max_norm <= 0).  Deterministic order.
 * Replaces the all_reduce + sqrt + coefficient of
 * grad_sync/optimizer_semantics.py:584-592. */
int eth_grad_norm_finalize(const double* partials, int64_t n, double max_norm,
                           double* stats, void* stream);

/* ------------------------------------------------------------------------
 * Fused AdamW with fp32 master weights (decoupled weight decay), one launch
 * over a tensor table.  Per element, in fp32, following torch.optim.AdamW
 * (the reference's fallback for apex FusedAdam,
 * eth/runtime/megatron/optimizer/__init__.py:28-34,66-72):
 *   g  = grad * clip          (clip = stats[2] when stats != NULL and < 1)
 *   p  = p * (1 - lr*wd)
 *   m  = lerp(m, g, 1-beta1)
 *   v  = v*beta2 + (1-beta2)*g*g
 *   p += -(lr/bc1) * m / (sqrt(v)/sqrt(bc2) + eps)
 *   model = cast(p)           (bf16/fp16 model copy when `model` != 0;
 *                              Float16Optimizer._copy_main_params_to_model_params,
 *                              optimizer/optimizer.py:475-479)
 * The whole launch is a no-op when found_inf != NULL and *found_inf != 0
 * (the skipped step of optimizer/optimizer.py:501-512).
 * ---------------------------------------------------------------------- */
typedef struct eth_adam_tensor {
  uint64_t param;       /* fp32 master weights */
  uint64_t grad;        /* fp32 gradient */
  uint64_t exp_avg;     /* fp32 */
  uint64_t exp_avg_sq;  /* fp32 */
  uint64_t model;       /* bf16/fp16 model copy, or 0 */
  int64_t numel;
  double lr;
  double weight_decay;
} eth_adam_tensor_t;

typedef struct eth_adam_chunk {
  int32_t tensor;  /* index into the tensor table */
  int32_t n;       /* elements in this chunk (<= ETH_CHUNK_ELEMS) */
  int64_t start;   /* first element of the chunk inside the tensor */
} eth_adam_chunk_t;

int eth_adam_step(const eth_adam_tensor_t* tensors, const eth_adam_chunk_t* chunks,
                  int64_t n_chunks, double beta1, double beta2, double eps,
                  int64_t step, int model_dtype, const double* stats,
                  const float* found_inf, void* stream);

/* ------------------------------------------------------------------------
 * Dense GEMM on the matrix cores (bf16/fp16 in, fp32 accumulate):
 *   C[m*ldc + n] (+)= alpha * sum_k A(m,k) * B(k,n)  (+ bias[n])
 * A(m,k) = a_kcontig ? A[m*lda + k] : A[k*lda + m]
 * B(k,n) = b_kcontig ? B[n*ldb + k] : B[k*ldb + n]
 * c_dtype: ETH_BF16 / ETH_F16 (rounded store) or ETH_F32 (store, or add into
 * C with ETH_GEMM_ACCUMULATE).  bias (in_dtype, length N) with ETH_GEMM_BIAS.
 * Requires K % 8 == 0, lda/ldb % 8 == 0, 16-byte aligned A/B, and M % 8 == 0
 * (N % 8 == 0) when A (B) is not K-contiguous.
 * Replaces F.linear in ColumnParallelLinear/RowParallelLinear forward
 * (eth/runtime/megatron/mpu/layers.py:357-370,452-470), their autograd
 * backward products, and the main_grad.add_(grad) hook of
 * model/distributed.py:116-123 (wgrad with ETH_GEMM_ACCUMULATE).
 * ---------------------------------------------------------------------- */
#define ETH_GEMM_ACCUMULATE 1
#define ETH_GEMM_BIAS 2
int eth_gemm(const void* A, int64_t lda, int a_kcontig, const void* B, int64_t ldb,
             int b_kcontig, void* C, int64_t ldc, int c_dtype, const void* bias,
             int64_t M, int64_t N, int64_t K, int in_dtype, int flags, float alpha,
             void* stream);

/* Split-K form of the fp32 product (C += A B with accumulate != 0, else
 * C = A B; alpha 1, no bias) for grids too small to fill the chip, such as
 * the [h, h] weight gradient of the attention projection: `splits` k-ranges
 * (K % (128 * splits) == 0) write fp32 partial products into the caller's
 * workspace of eth_gemm_splitk_workspace(M, N, splits) bytes, which a second
 * kernel sums in split order (deterministic) and adds into or stores to C.
 * N % 4 == 0, 16-byte aligned C rows.
 * Same reference seam as eth_gemm's ETH_GEMM_ACCUMULATE form
 * (model/distributed.py:116-123 over mpu/layers.py:452-470). */
int64_t eth_gemm_splitk_workspace(int64_t M, int64_t N, int splits);
int eth_gemm_splitk(const void* A, int64_t lda, int a_kcontig, const void* B, int64_t ldb, int b_kcontig,
                    float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int in_dtype, int splits,
                    int accumulate, float* workspace, void* stream);

/* ------------------------------------------------------------------------
 * LayerNorm (bf16/fp16 rows of `cols` elements, cols % 8 == 0, <= 8192).
 * Forward writes y and fp32 mean / rstd per row; backward writes dx and
 * stores (accumulate == 0) or adds (accumulate != 0) fp32 dgamma / dbeta,
 * using `workspace` of eth_ln_bwd_workspace(rows, cols) floats.
 * Replaces fused_mix_prec_layer_norm_cuda.forward_affine / backward_affine
 * (eth/runtime/megatron/fused_kernels/layer_norm_cuda.cpp:121-201) as used
 * by MixedFusedLayerNorm (model/fused_layer_norm.py:30-89).
 * ---------------------------------------------------------------------- */
int eth_ln_fwd(const void* x, const void* gamma, const void* beta, void* y, float* mean,
               float* rstd, int64_t rows, int64_t cols, float eps, int dtype, void* stream);
int64_t eth_ln_bwd_workspace(int64_t rows, int64_t cols);
int eth_ln_bwd(const void* dy, const void* x, const float* mean, const float* rstd,
               const void* gamma, void* dx, float* dgamma, float* dbeta, float* workspace,
               int64_t rows, int64_t cols, int accumulate, int dtype, void* stream);

/* The final LayerNorm of a GPT stage with its transpose folded in: x is a
 * [seq, batch, cols] tensor, y is written [batch, seq, cols], mean / rstd in
 * y's row order (eth_ln_fwd_sb); the backward takes dy [batch, seq, cols]
 * and writes dx [seq, batch, cols] (eth_ln_bwd_sb, workspace as for
 * eth_ln_bwd with rows = seq * batch).  The kernels of eth_ln_fwd /
 * eth_ln_bwd read and write x through the row permutation, so the results
 * equal a transposed copy followed by those calls bit for bit.
 * Replaces hidden_states.transpose(0, 1).contiguous() + FusedLayerNorm of
 * the final-layernorm op (eth/runtime/megatron/model/flex_ops.py:552-553)
 * and the copy its backward makes. */
int eth_ln_fwd_sb(const void* x, const void* gamma, const void* beta, void* y, float* mean,
                  float* rstd, int64_t seq, int64_t batch, int64_t cols, float eps, int dtype,
                  void* stream);
int eth_ln_bwd_sb(const void* dy, const void* x, const float* mean, const float* rstd,
                  const void* gamma, void* dx, float* dgamma, float* dbeta, float* workspace,
                  int64_t seq, int64_t batch, int64_t cols, int accumulate, int dtype, void* stream);
/* LayerNorm backward fused with the residual branch that read the same
 * input: dx = bf16(bf16(dx_ln) + dresid), the sum autograd forms when a
 * tensor feeds both the LayerNorm and the later residual add
 * (ParallelLayerNormOp publishing hidden_states_1/2, flex_ops.py:488-664,
 * consumed by bias_dropout_add, flex_ops.py:104-134).  With colsum_part
 * non-NULL it also stores per-row-group column sums of the stored dx,
 * colsum_part[eth_ln_bwd_groups(rows, cols)][cols] (fp32): folded by
 * eth_reduce_partials they are the bias gradient of the bias-dropout-add at
 * p == 0 that produced this LayerNorm's input (the sum over the broadcast
 * dimensions that autograd of `x + bias` forms there).  dresid == NULL is
 * eth_ln_bwd. */
int64_t eth_ln_bwd_groups(int64_t rows, int64_t cols);
int eth_ln_bwd_residual(const void* dy, const void* x, const float* mean, const float* rstd,
                        const void* gamma, const void* dresid, void* dx, float* dgamma,
                        float* dbeta, float* colsum_part, float* workspace, int64_t rows,
                        int64_t cols, int accumulate, int dtype, void* stream);
/* The bias-dropout-add that ends a sub-block and the LayerNorm that starts
 * the next, in one pass over the rows: h = residual + dropout(x + b, p,
 * seed) is stored exactly as eth_bias_dropout_add_fwd stores it (same mask),
 * and y, mean, rstd are eth_ln_fwd of the stored h, bit for bit; h is not
 * read back from HBM.  Replaces the op pair enc-post-attention-dropout ->
 * enc-2nd-layernorm (and enc-post-MLP-dropout -> the next layer's
 * enc-1st-layernorm): bias_dropout_add (flex_ops.py:104-134) followed by
 * MixedFusedLayerNorm's forward_affine (model/fused_layer_norm.py:62-89). */
int eth_bda_ln_fwd(const void* x, const void* bias, const void* residual, void* h,
                   const void* gamma, const void* beta, void* y, float* mean, float* rstd,
                   int64_t rows, int64_t cols, float p, uint64_t seed, float eps, int dtype,
                   void* stream);

/* ------------------------------------------------------------------------
 * Elementwise ops of the GPT block ([rows, cols] row-major, cols % 8 == 0).
 * eth_bias_gelu_fwd/bwd: y = gelu_tanh(x + b), dx = dy * gelu_tanh'(x + b)
 *   (ParallelMlpGeLUOp, eth/runtime/megatron/model/flex_ops.py:1882-1906,60-63).
 * eth_bias_dropout_add_fwd: out = residual + dropout(x + b, p, seed); p == 0
 *   is the identity (bias_dropout_add_fused_train, flex_ops.py:104-134).
 * eth_dropout_bwd: dx = dy * keep / (1 - p) with the same (seed, index) mask.
 * eth_col_sum: out[c] (+)= sum_r x[r*ld + c] in fp32 -- the bias gradients
 *   of the linear / bias-dropout-add / bias-GELU ops; `workspace` holds
 *   eth_col_sum_workspace(rows, cols) floats.
 * ---------------------------------------------------------------------- */
int eth_bias_gelu_fwd(const void* x, const void* bias, void* y, int64_t rows, int64_t cols,
                      int dtype, void* stream);
int eth_bias_gelu_bwd(const void* dy, const void* x, const void* bias, void* dx, int64_t rows,
                      int64_t cols, int dtype, void* stream);
int eth_bias_dropout_add_fwd(const void* x, const void* bias, const void* residual, void* out,
                             int64_t rows, int64_t cols, float p, uint64_t seed, int dtype,
                             void* stream);
int eth_dropout_bwd(const void* dy, void* dx, int64_t rows, int64_t cols, float p,
                    uint64_t seed, int dtype, void* stream);
int64_t eth_col_sum_workspace(int64_t rows, int64_t cols);
int eth_col_sum(const void* x, int64_t ld, int64_t rows, int64_t cols, float* out,
                float* workspace, int accumulate, int dtype, void* stream);
/* Bias-GELU backward with its bias gradient in the same pass: dx as
 * eth_bias_gelu_bwd, and dbias (+)= column sums of the stored dx (fp32) --
 * what ParallelMlpGeLUOp's backward (flex_ops.py:1882-1906 with
 * model/fused_bias_gelu.py:39-45, bias grad = the same tensor as the input
 * grad, summed by the caller) followed by eth_col_sum computes, without
 * reading dx back.  `workspace` holds eth_bias_gelu_bwd_workspace(rows,
 * cols) floats. */
int64_t eth_bias_gelu_bwd_workspace(int64_t rows, int64_t cols);
int eth_bias_gelu_bwd_dbias(const void* dy, const void* x, const void* bias, void* dx,
                            float* dbias, float* workspace, int64_t rows, int64_t cols,
                            int accumulate, int dtype, void* stream);
/* out[c] (+)= sum_g part[g * ld + c] (fp32, cols % 4 == 0, ld % 4 == 0, part
 * 16-byte aligned), summed in a fixed order: folds the column-sum partials
 * of eth_ln_bwd_residual into a bias gradient. */
int eth_reduce_partials(const float* part, int64_t groups, int64_t cols, int64_t ld, float* out,
                        int accumulate, void* stream);

/* ------------------------------------------------------------------------
 * Causal attention (softmax(Q K^T / sqrt(hn) + causal -inf) V per batch and
 * head), flash-style, head_dim 64 or 128, seq % 128 == 0.  Every tensor is
 * addressed as base + s*stride[0] + b*stride[1] + h*stride[2] + d with d
 * contiguous and rows 16-byte aligned, so q/k/v may be views into the
 * [s, b, np, 3*hn] QKV output and dq/dk/dv into its gradient.
 * lse ([batch*heads, seq] fp32) is written by the forward and read by the
 * backward; delta ([batch*heads, seq] fp32) is backward scratch.
 * Replaces ParallelFlashAtten / F.scaled_dot_product_attention(is_causal=True)
 * (eth/runtime/megatron/model/flex_ops.py:66-96,1401-1426) and its autograd
 * backward.
 * ---------------------------------------------------------------------- */
typedef struct eth_attn_desc {
  int32_t batch, heads, seq, head_dim, dtype;
  int64_t q_strides[3], k_strides[3], v_strides[3], o_strides[3];
  int64_t do_strides[3], dq_strides[3], dk_strides[3], dv_strides[3];
} eth_attn_desc_t;

int eth_attn_fwd(const eth_attn_desc_t* desc, const void* q, const void* k, const void* v,
                 void* out, float* lse, void* stream);
int eth_attn_bwd(const eth_attn_desc_t* desc, const void* q, const void* k, const void* v,
                 const void* out, const void* dout, const float* lse, float* delta, void* dq,
                 void* dk, void* dv, void* stream);

/* ------------------------------------------------------------------------
 * Vocabulary side of the first / last stage.
 * eth_embedding_fwd: out[s, b, :] = word[tokens[b, s]] + pos[positions[b, s]]
 *   (tokens/positions int64 [batch, seq]; out [seq, batch, hidden]); replaces
 *   Embedding_v1.forward (eth/runtime/megatron/model/flex_ops.py:450-485,
 *   VocabParallelEmbedding mpu/layers.py:136-205 at TP = 1).
 * eth_embedding_bwd: fp32 dword[tok] += dout, dpos[pos] += dout, bitwise
 *   deterministic: the ids are sorted with their dout rows (in `workspace`
 *   of eth_embedding_bwd_workspace(batch, seq) bytes) and each table row is
 *   summed by one workgroup in dout-row order.  Inputs of more than 32768
 *   tokens run as consecutive chunks of whole sequence positions (at most
 *   32768 dout rows each, in sequence order), each adding its own ordered
 *   sums; batch <= 32768, and bits(vocab - 1) + bits(rows per chunk - 1)
 *   <= 32.  Either table may be NULL.
 *   Replaces the embedding's autograd backward (embedding_dense_backward, a
 *   sort + segmented reduction) and the main_grad.add_ hook of
 *   model/distributed.py:116-123.
 * eth_xent_fwd / eth_xent_bwd: per-row loss = logsumexp(z) - z[label] from
 *   16-bit logits [rows, ld], saving lse; dz = (softmax - onehot) * dloss
 *   (any row count: eth_xent_bwd launches 65535 rows at a time).
 *   Replace vocab_parallel_cross_entropy(logits.float(), labels)
 *   (mpu/cross_entropy.py:36-115; flex_ops.py:1976-1981).
 * Out-of-range ids are clamped and flagged in *bad_index (set to 1).
 * ---------------------------------------------------------------------- */
int eth_embedding_fwd(const int64_t* tokens, const int64_t* positions, const void* word,
                      const void* pos, void* out, int64_t batch, int64_t seq, int64_t hidden,
                      int64_t vocab, int64_t max_pos, int* bad_index, int dtype, void* stream);
int64_t eth_embedding_bwd_workspace(int64_t batch, int64_t seq);
int eth_embedding_bwd(const int64_t* tokens, const int64_t* positions, const void* dout,
                      float* dword, float* dpos, void* workspace, int64_t batch, int64_t seq,
                      int64_t hidden, int64_t vocab, int64_t max_pos, int dtype, void* stream);
/* Allocation-free form of eth_embedding_bwd, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  The sort keys live in a static device array of 2 * 32768 keys
 * (256 KiB per GPU, held until the process ends) instead of a caller
 * workspace; batch * seq beyond 32768 is rejected.  Every call on one GPU
 * uses that GPU's array, so calls that overlap on one GPU race.  Same
 * arguments and results as eth_embedding_bwd otherwise; calls no
 * allocating routine. */
int eth_embedding_bwd_noalloc(const int64_t* tokens, const int64_t* positions, const void* dout,
                              float* dword, float* dpos, int64_t batch, int64_t seq, int64_t hidden,
                              int64_t vocab, int64_t max_pos, int dtype, void* stream);
int eth_xent_fwd(const void* logits, int64_t ld, const int64_t* labels, float* loss, float* lse,
                 int64_t rows, int64_t vocab, int* bad_index, int dtype, void* stream);
int eth_xent_bwd(const void* logits, int64_t ld, const int64_t* labels, const float* lse,
                 const float* dloss, void* dlogits, int64_t ldd, int64_t rows, int64_t vocab,
                 int dtype, void* stream);

/* Tied word-embedding gradients on one rank: root = copy = root + copy (fp32,
 * 16-byte aligned).  Replaces the same-rank branch of
 * synchronize_shared_weights_grads (eth/runtime/megatron/training.py:489-531). */
int eth_tied_grad_sum(float* root, float* copy, int64_t n, void* stream);
/* The same for 16-bit (bf16 / fp16, `dtype`) main grads, as fp16 training
 * without fp32 gradient accumulation keeps them (the reference's default,
 * eth/runtime/megatron/model/distributed.py:69-103): each sum is formed in
 * fp32 and rounded once, as an all-reduce sum in that dtype rounds it. */
int eth_tied_grad_sum_half(void* root, void* copy, int64_t n, int dtype, void* stream);

/* The deterministic synthetic batch of `n_samples` samples (`sample_ids`: a
 * HOST array) of `seq` positions, row-major [n_samples, seq] on the device:
 * tokens = (id * 1103515245 + p * 12345) mod vocab (int64, wrapping products,
 * non-negative residues), loss_mask = ((id + p) mod 4 != 0) as fp32 1 / 0,
 * position_ids = p.  One launch per 64 samples, the ids passed by value.
 * Replaces the token / loss-mask / position-id tensors of
 * synthetic_gpt_batch (eth/runtime/megatron/grad_sync/loss.py:100-119); the
 * boolean attention mask it also returns is not built here (the causal
 * attention kernels imply it). */
int eth_synthetic_batch(const int64_t* sample_ids, int64_t n_samples, int64_t seq, int64_t vocab,
                        int64_t* tokens, float* loss_mask, int64_t* position_ids, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ETH_AMD_H */
