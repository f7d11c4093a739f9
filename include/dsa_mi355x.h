/*
 * dsa_mi355x.h - C ABI of the MI355X (gfx950) DeepSeek sparse-attention (DSA) kernels.
 *
 * Every entry point takes raw device pointers, int64 sizes, scalar parameters and a
 * hipStream_t passed as void*.  It enqueues work asynchronously on that stream and
 * returns DSA_OK (0) or a non-zero dsa_status; it never throws.  On error the message
 * is available from dsa_last_error() (thread-local).  The caller owns every buffer.
 * Tensors are dense row-major ("BSND" in the reference's terms) unless a leading
 * dimension argument says otherwise.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * torchtitan-npu reference repository):
 *   dsa_lightning_indexer        torch_npu.npu_lightning_indexer (scores + top-k in one call;
 *   (= dsa_indexer_fwd +          the two halves are also exported on their own)
 *      dsa_topk)                 (converters/kernels/dsa.py:217-226;
 *                                 ops/aclnn/lightning_indexer/binding.cpp:12-36)
 *   dsa_sparse_mla_fwd           torch_npu.npu_sparse_flash_attention, attention_mode=2
 *                                (converters/kernels/dsa.py:238-253;
 *                                 ops/aclnn/sparse_attn_sharedkv/binding.cpp:30-60)
 *   dsa_sparse_mla_bwd           its autograd backward / npu_sparse_attn_sharedkv_grad
 *                                (ops/aclnn/sparse_attn_sharedkv/binding.cpp:62-88)
 *   dsa_attn_mass +
 *   dsa_indexer_kl_grad          torch_npu.npu_sparse_lightning_indexer_grad_kl_loss
 *                                (converters/kernels/dsa.py:159-177;
 *                                 ops/aclnn/sparse_lightning_indexer_grad_kl_loss/binding.cpp:12-36)
 *   dsa_quantize_fp8_rows        the fp8-e4m3 per-row quantisation this build adds in front of
 *                                npu_lightning_indexer (the reference indexes in bf16 and marks fp8
 *                                as a QAT step: models/deepseek_v4/model.py:646, :822)
 *   dsa_sparse_mla_{fwd,bwd}_sink
 *   (and dsa_attn_sink_fold +
 *   dsa_attn_sink_grad)          the per-head sink of SparseAttention.forward (models/deepseek_v4/
 *                                model.py:573-623) inside npu_sparse_attn_shared_kv{,_grad}
 *                                (converters/kernels/npu_smla.py:351-400;
 *                                 ops/aclnn/sparse_attn_sharedkv/binding.cpp:30-88)
 *   dsa_compressor_fwd           Compressor._forward_bsnd pooling + RMSNorm
 *                                (models/deepseek_v4/model.py:183-221; torch-only in the reference)
 *   dsa_compressor_fwd_tnd       Compressor._forward_tnd (models/deepseek_v4/model.py:223-274)
 *   dsa_mla_absorb               the MLA absorb einsums (models/deepseek_v32/model.py:520-535, :574-575)
 *   dsa_tnd_metadata             build_smla_attention_masks (models/deepseek_v4/tnd.py:97-164) on the device
 *   dsa_indexer_prep             the indexer's RoPE + rotate_activation (+ this build's fp8 quantisation)
 *                                (models/deepseek_v32/model.py:196-221, :264-282;
 *                                 models/deepseek_v4/model.py:343-357; torch-only in the reference)
 *   dsa_*_varlen                 the A5 packed-varlen ("TND") ops taking cu_seqlens_q / cu_seqlens_k:
 *                                lightning_indexer (converters/kernels/npu_smla.py:754-768),
 *                                sparse_flash_mla{,_grad} (:457-479, :540-568),
 *                                sparse_lightning_indexer_kl_loss_grad (:584-598)
 *   dsa_lightning_indexer_tnd,   the same packed batches with cu_seqlens on the device (no host read):
 *   dsa_tnd_global_indices       npu_lightning_indexer with actual_seq_lengths tensors
 *                                (ops/aclnn/lightning_indexer/binding.cpp:14), and sequence-local
 *                                slots as global key rows for the fixed-length attention / KL calls
 */
#ifndef DSA_MI355X_H
#define DSA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dsa_dtype { DSA_F32 = 0, DSA_BF16 = 1, DSA_FP8_E4M3 = 2 };

enum dsa_status {
  DSA_OK = 0,
  DSA_ERR_INVALID_ARG = 1,   /* null pointer, bad size, unsupported combination */
  DSA_ERR_LAUNCH = 2,        /* the HIP runtime reported an error */
  DSA_ERR_UNSUPPORTED = 3    /* valid request this build does not implement */
};

/* Thread-local text of the last error (empty string if none). */
const char* dsa_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int dsa_abi_version(void);

/*
 * Per-kernel timing (no counterpart in the reference; for benchmarks and profiling).
 * dsa_kernel_timing(1) drops earlier records and makes every later kernel launch of this
 * library record a HIP event before and after itself on its stream; dsa_kernel_timing(0)
 * stops recording.  dsa_kernel_timing_count() waits for the recorded events, sums the
 * elapsed times per kernel name and returns the number of distinct kernels (or < 0 with
 * dsa_last_error); dsa_kernel_timing_get(i, ...) returns entry i: its name (truncated to
 * name_cap - 1 bytes), the summed milliseconds and the number of launches.  While
 * enabled, each launch creates two events and takes a lock; leave it off in production.
 */
int dsa_kernel_timing(int enable);
int dsa_kernel_timing_count(void);
int dsa_kernel_timing_get(int i, char* name, int64_t name_cap, double* total_ms, int64_t* launches);

/*
 * Lightning-indexer scores (reference: bf16_index, models/deepseek_v32/model.py:224-236;
 * LiCompute, models/deepseek_v4/model.py:647-652).
 *   scores[b, s, t] = k_scale[b,t] * sum_h w[b,s,h] * q_scale[b,s,h] * relu(q[b,s,h,:] . k[b,t,:])
 * for t < (s + q_offset + 1) / cmp_ratio, and -inf for every other t < s_k.
 *   q        [B, S, H_I, D_I]   bf16 or fp8-e4m3 (q_dtype)
 *   q_scale  [B, S, H_I] fp32 or NULL (== 1)
 *   k        [B, S_k, D_I]      same dtype as q
 *   k_scale  [B, S_k] fp32 or NULL (== 1)
 *   w        [B, S, H_I] fp32
 *   scores   [B, S, ld_scores] fp32, ld_scores >= S_k
 * D_I must be 128 (MFMA path) ; H_I a multiple of 16 and <= 128.
 */
int dsa_indexer_fwd(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                    float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                    int64_t head_dim, int64_t ld_scores, int64_t q_offset, int64_t cmp_ratio, void* stream);

/*
 * dsa_indexer_fwd with a caller workspace (same reference interface: npu_lightning_indexer,
 * converters/kernels/dsa.py:217-226).  For fp8-e4m3 operands with H_I = 64 and D_I = 128 the
 * workspace holds, per query row, four fp8 pieces of u = sum_h (w q_scale / 2)[h] q[h, :] and
 * their power-of-two scales, written by a pre-pass; the score kernel then takes
 *   sum_h c_h relu(x_h) = sum_h (c_h / 2) |x_h| + u . k
 * with u . k on the MFMA (half the VALU work of the relu form).  Other shapes ignore the
 * workspace and run dsa_indexer_fwd.
 * Precision (both forms, fp8): each score is within 1e-5 * k_scale * sum_h |w_h q_scale_h| (|q_h| . |k|)
 * of the exact value on the dequantised operands (the fp32 rounding bound of the dot products
 * and the head sum; measured <= 1.8e-6 of it at S = 4096 .. 131072 with signed head weights).
 * Relative to max_t |score| a row whose head weights cancel can show larger deviations
 * (about 9e-5 measured on early causal rows with N(0,1) weights).
 *   workspace        device scratch of at least dsa_indexer_fwd_workspace_size() bytes
 *                    (NULL: dsa_indexer_fwd's kernels)
 * dsa_indexer_fwd_workspace_size returns 0 where the split does not apply.
 */
int64_t dsa_indexer_fwd_workspace_size(int64_t batch, int64_t s_q, int64_t n_heads, int64_t head_dim, int dtype);
int dsa_indexer_fwd_ws(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                       float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                       int64_t head_dim, int64_t ld_scores, int64_t q_offset, int64_t cmp_ratio, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * dsa_indexer_fwd_ws without a workspace and without any allocation.  No counterpart in the
 * reference: this entry point is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The linear-split
 * pieces live in a static 32 MiB device array of the library (one per GPU, held until the
 * process ends), enough for dsa_indexer_fwd_noalloc_max_rows() = 63550 query rows
 * (batch * s_q) per call; more rows are rejected with DSA_ERR_INVALID_ARG (split them over
 * several calls).  Same arguments, results and kernels as dsa_indexer_fwd_ws; shapes the
 * split does not apply to run dsa_indexer_fwd's kernels.  Every call on a GPU uses that GPU's
 * one array, so calls that overlap on one GPU (concurrent streams or threads) race; calls on
 * one stream are ordered and safe.  Nothing in the array needs clearing between calls.
 * (While dsa_kernel_timing is enabled, every launch also creates two HIP events; it is off
 * by default.)
 */
int64_t dsa_indexer_fwd_noalloc_max_rows(void);
int dsa_indexer_fwd_noalloc(const void* q, const float* q_scale, const void* k, const float* k_scale,
                            const float* w, float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k,
                            int64_t n_heads, int64_t head_dim, int64_t ld_scores, int64_t q_offset,
                            int64_t cmp_ratio, void* stream);

/*
 * Per-row top-k of fp32 scores (reference: DSV32_SDPA.forward topk,
 * models/deepseek_v32/model.py:389-395; LiCompute, models/deepseek_v4/model.py:653-655).
 * Row (b, s) considers candidates t < min(s_k, (s + q_offset + 1) / cmp_ratio) whose score is
 * not NaN; it keeps the first k of a stable descending order by (score, lower index) with
 * -0.0 == +0.0.  indices[b, s, :] receive the chosen t + index_offset in ascending t order,
 * padded with -1; values (optional) the matching scores, -inf in padded slots.
 *   scores  [B, S, ld_scores] fp32; indices [B, S, k] int32; values [B, S, k] fp32 or NULL.
 * k <= 4096.
 */
int dsa_topk(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q, int64_t s_k,
             int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio, int64_t index_offset,
             void* stream);
/*
 * dsa_topk with a workspace (dsa_topk_workspace_size() bytes, 16-byte aligned; 0 bytes when
 * s_k <= 16384): rows longer than 16384 keys are read once into per-row candidate lists -
 * every key at or above a threshold estimated from a sample of the row, which at least k
 * keys reach, in index order - and selected from those; a row whose list would miss a key
 * or overflow is selected from its scores as dsa_topk does.  Same contract and results as
 * dsa_topk (bit for bit).  No counterpart in the reference (its top-k is fused into the
 * closed indexer op); the fused lightning indexer uses it for its long rows.
 */
int64_t dsa_topk_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t k);
int dsa_topk_ws(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q, int64_t s_k,
                int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio, int64_t index_offset,
                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The fused lightning indexer (reference: npu_lightning_indexer, ops/aclnn/lightning_indexer/
 * binding.cpp:14-31, as called by converters/kernels/dsa.py:217-226): the scores of
 * dsa_indexer_fwd_ws followed by dsa_topk, with the fp32 score rows kept in `workspace`
 * instead of a caller-visible buffer.  Same arguments and results as those two calls
 * (indices [B, S, k] int32 ascending with -1 padding, values [B, S, k] fp32 or NULL), with
 * ld_scores = s_k.  The score kernels leave the key spans past every query's causal
 * frontier unwritten and the top-k reads only each row's valid prefix, so the masked part
 * of the score matrix costs no memory traffic.
 * workspace: 256-byte aligned; dsa_lightning_indexer_workspace_size(.., max_rows) bytes
 * process max_rows query rows per pass (every row of every batch at once when max_rows >= S;
 * smaller workspaces run batch by batch in row chunks).  Calls on one stream may share it.
 */
int64_t dsa_lightning_indexer_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                                             int64_t head_dim, int dtype, int64_t max_rows);
int dsa_lightning_indexer(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                          int32_t* indices, float* values, int dtype, int64_t batch, int64_t s_q, int64_t s_k,
                          int64_t n_heads, int64_t head_dim, int64_t topk, int64_t q_offset, int64_t cmp_ratio,
                          int64_t index_offset, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Gathered sparse MLA attention forward (reference: npu_sparse_flash_attention with
 * attention_mode=2, converters/kernels/dsa.py:238-253; torch-native semantics
 * models/deepseek_v32/model.py:391-404).
 *   q        [B, S, H, D_qk]   (D_qk = latent D_v + rope)
 *   kv       [B, S_kv, D_qk]   one shared latent KV head; v = kv[..., :D_v]
 *   indices  [B, S, K] int32; slot j of row s is used iff 0 <= idx <= s + q_offset and idx < S_kv
 *   out      [B, S, H, D_v]
 *   softmax_max [B, S, H] fp32: max_j scale*q.k_j (natural-log units), -inf if no valid slot
 *   softmax_sum [B, S, H] fp32: sum_j exp(scale*q.k_j - softmax_max)
 * dtype DSA_BF16: MFMA path (requires D_v = 512 and D_qk = 576, the DeepSeek-V3.2 latent +
 * rope rows, or D_qk = 512, the rope-less DeepSeek-V4 rows where v = the whole row);
 * DSA_F32: exact fp32 path.
 */
int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices, void* out, float* softmax_max,
                       float* softmax_sum, int dtype, int64_t batch, int64_t s_q, int64_t s_kv, int64_t n_heads,
                       int64_t d_qk, int64_t d_v, int64_t topk, float scale, int64_t q_offset, void* stream);

/*
 * Backward of dsa_sparse_mla_fwd (reference: SparseAttnSharedKV.backward,
 * converters/kernels/npu_smla.py:303-348 -> sparse_attn_sharedkv/binding.cpp:62-88).
 *   dq        [B, S, H, D_qk]  same dtype as q (written)
 *   dkv_accum [B, S_kv, D_qk]  fp32, ACCUMULATED into (caller zeroes it); latent alias:
 *             dkv[:, :D_v] = dK_nope + dV, dkv[:, D_v:] = dK_rope
 *   mass      [B, S, K] fp32 or NULL: if given, also written with the head-summed attention
 *             probability at each slot (what dsa_attn_mass computes), taken from the P this
 *             backward recomputes anyway; bf16 path only (the A5 reference's
 *             sparse_flash_mla_grad returns the same quantity, converters/kernels/npu_smla.py:540-568)
 *   workspace  device scratch of workspace_bytes (dsa_sparse_mla_bwd_workspace_size() gives the
 *              default; a smaller one processes query rows in more chunks); fp32 dtype needs none
 * The bf16 path needs D_qk = 576 or 512, D_v = 512, H <= 128.  dKV is reduced per key through a
 * key-major CSR of the bf16 per-(row, slot) contributions, summed in fp32 in a fixed order
 * (no float atomics), so the same inputs and workspace size give the same dKV bit for bit;
 * another workspace size (another row chunking) changes the summation order.  The fp32
 * path scatters with fp32 atomics and is reproducible to rounding only.
 */
int64_t dsa_sparse_mla_bwd_workspace_size(int64_t batch, int64_t s_q, int64_t s_kv, int64_t n_heads,
                                          int64_t d_qk, int64_t topk);
int dsa_sparse_mla_bwd(const void* q, const void* kv, const int32_t* indices, const void* out, const void* dout,
                       const float* softmax_max, const float* softmax_sum, void* dq, float* dkv_accum, float* mass,
                       void* workspace, int64_t workspace_bytes, int dtype, int64_t batch, int64_t s_q,
                       int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                       int64_t q_offset, void* stream);

/*
 * dsa_sparse_mla_fwd / dsa_sparse_mla_bwd with the DeepSeek-V4 per-head attention sink folded
 * in (reference: SparseAttention.forward's attn_sink, models/deepseek_v4/model.py:573-623,
 * passed as `sinks` to npu_sparse_attn_shared_kv{,_grad}, converters/kernels/npu_smla.py:351-400).
 * The forward's epilogue does what dsa_attn_sink_fold does after the plain forward: out is
 * normalised by s2 = l e^(m - m2) + e^(sink - m2), m2 = max(m, sink[h]), and (m2, s2) are written
 * as the statistics (a row with no valid slot gets out = 0, (sink[h], 1)).  The backward takes
 * those statistics and also adds to dsink_accum[h] (fp32, caller zeroes it) the sink's gradient
 * - sum over rows of e^(sink - m2) / s2 * sum_d dout * out, from the delta pass it already makes.
 *   sinks [H] fp32 (required; NULL is an error)
 * Same shapes, dtypes, workspace and limits as the entry points without the sink.
 */
int dsa_sparse_mla_fwd_sink(const void* q, const void* kv, const int32_t* indices, const float* sinks, void* out,
                            float* softmax_max, float* softmax_sum, int dtype, int64_t batch, int64_t s_q,
                            int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                            int64_t q_offset, void* stream);
int dsa_sparse_mla_bwd_sink(const void* q, const void* kv, const int32_t* indices, const void* out,
                            const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                            float* dkv_accum, float* mass, const float* sinks, float* dsink_accum, void* workspace,
                            int64_t workspace_bytes, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                            int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale, int64_t q_offset,
                            void* stream);
/*
 * dsa_sparse_mla_bwd / dsa_sparse_mla_bwd_sink in one entry (sinks = NULL: no sink) that can
 * reduce dKV with a prebuilt pair CSR (dsa_pair_csr_build from the same indices, s_kv and
 * q_offset; NULL = build one).  The CSR is used when the workspace holds every query row in
 * one chunk and ignored otherwise.  No counterpart in the reference's op (see
 * dsa_pair_csr_build).
 */
int dsa_sparse_mla_bwd_ex(const void* q, const void* kv, const int32_t* indices, const void* out, const void* dout,
                          const float* softmax_max, const float* softmax_sum, void* dq, float* dkv_accum, float* mass,
                          const float* sinks, float* dsink_accum, const void* pair_csr, int64_t pair_csr_bytes,
                          void* workspace, int64_t workspace_bytes, int dtype, int64_t batch, int64_t s_q,
                          int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                          int64_t q_offset, void* stream);

/*
 * Head-summed attention probability at each selected slot (reference: get_attn_scores,
 * models/deepseek_v32/model.py:285-306, gathered/zeroed at :410-413):
 *   mass[b, s, j] = sum_h exp(scale*q[b,s,h].kv[idx_j] - lse[b,s,h]),  0 for unused slots,
 * with lse = softmax_max + log(softmax_sum) from dsa_sparse_mla_fwd.  bf16 needs D_qk = 576 or
 * 512 (the rope-less DeepSeek-V4 rows); fp32 takes any D_qk.
 */
int dsa_attn_mass(const void* q, const void* kv, const int32_t* indices, const float* softmax_max,
                  const float* softmax_sum, float* mass, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                  int64_t n_heads, int64_t d_qk, int64_t topk, float scale, int64_t q_offset, void* stream);

/*
 * Indexer KL loss and its gradients (reference: DSAIndexerLoss.forward,
 * models/common/dsa_indexer_loss.py:138-160, as fused by
 * npu_sparse_lightning_indexer_grad_kl_loss, converters/kernels/dsa.py:159-183).
 * Per row (b,s): I_j = sum_h w[h] relu(q_idx[h].k_idx[idx_j]) over used slots, target
 * t_j = mass_j / Z with Z = sum_j mass_j, row loss
 * Z * sum_{t_j > 0} t_j (log max(t_j, eps) - log_softmax(I)_j) * loss_scale
 * (rows with Z <= eps use a zero score vector and get no gradient, as the reference does).
 *   q_idx [B,S,H_I,D_I] bf16, k_idx [B,S_k,D_I] bf16, w [B,S,H_I] fp32, mass [B,S,K] fp32
 *   dq_idx [B,S,H_I,D_I] fp32 (written), dk_idx_accum [B,S_k,D_I] fp32 (ACCUMULATED),
 *   dw [B,S,H_I] fp32 (written), loss_rows [B,S] fp32 (written; the op's loss is their sum)
 * grad_scale multiplies every gradient (the upstream gradient of the summed loss), times
 * *grad_scale_dev when that device fp32 scalar is given (so a caller holding the upstream
 * gradient on the device needs no host round trip; NULL = 1).
 * H_I = 64, D_I = 128 run on MFMA with a workspace of
 * dsa_indexer_kl_grad_workspace_size() bytes; other shapes use an exact fp32 kernel.
 */
int64_t dsa_indexer_kl_grad_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                                           int64_t head_dim, int64_t topk);
int dsa_indexer_kl_grad(const void* q_idx, const void* k_idx, const float* w, const int32_t* indices,
                        const float* mass, float* dq_idx, float* dk_idx_accum, float* dw, float* loss_rows,
                        void* workspace, int64_t workspace_bytes, int64_t batch, int64_t s_q, int64_t s_k,
                        int64_t n_heads, int64_t head_dim, int64_t topk, int64_t q_offset, float loss_scale,
                        float eps, float grad_scale, const float* grad_scale_dev, void* stream);
/*
 * dsa_indexer_kl_grad with two optional extras (NULL = without them):
 *   softmax_out [B,S,K] fp32 (written): the indexer's softmax over the slots, exp(I_j -
 *     logsumexp of the row's usable I) at usable slots and 0 at the others (reference: the
 *     softmax_out of cann_ops_transformer's sparse_lightning_indexer_kl_loss_grad,
 *     converters/kernels/npu_smla.py:584-602, which _compute_li_loss :405-420 logs);
 *   pair_csr / pair_csr_bytes: a CSR built by dsa_pair_csr_build from the same indices,
 *     s_k and q_offset (the caller guarantees it), reduced with instead of building one; used
 *     when the workspace holds every query row in one chunk, ignored otherwise.  No
 *     counterpart in the reference's op: it lets the attention backward and this op share
 *     one key-major pair list per step.
 */
int dsa_indexer_kl_grad_ex(const void* q_idx, const void* k_idx, const float* w, const int32_t* indices,
                           const float* mass, float* dq_idx, float* dk_idx_accum, float* dw, float* loss_rows,
                           float* softmax_out, const void* pair_csr, int64_t pair_csr_bytes, void* workspace,
                           int64_t workspace_bytes, int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                           int64_t head_dim, int64_t topk, int64_t q_offset, float loss_scale, float eps,
                           float grad_scale, const float* grad_scale_dev, void* stream);

/*
 * Key-major CSR of the usable (query row, slot) pairs of an index tensor (no counterpart in
 * the reference: the closed CANN ops scatter with atomics).  indices [B,S,K] int32; slot j of
 * row s is usable iff 0 <= idx < s_k and idx <= s + q_offset.  The buffer (256-byte aligned,
 * dsa_pair_csr_size() bytes) holds, per batch element, the pair list sorted by key (rows in
 * order within each key) with its key pointers and segment table; dsa_sparse_mla_bwd_ex and
 * dsa_indexer_kl_grad_ex reduce their per-pair contribution rows with it, so the attention
 * backward's dKV and the indexer loss's dK_index, which use the same indices, build it once.
 */
int64_t dsa_pair_csr_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t topk);
/* query rows per chunk that a workspace of workspace_bytes gives dsa_sparse_mla_bwd{,_ex}
 * (bf16 path) / dsa_indexer_kl_grad{,_ex} (H_I = 64, D_I = 128); s_q means one chunk, where a
 * prebuilt pair CSR is used; 0 = the workspace is too small */
int64_t dsa_sparse_mla_bwd_chunk_rows(int64_t batch, int64_t s_q, int64_t s_kv, int64_t d_qk, int64_t topk,
                                      int64_t workspace_bytes);
int64_t dsa_indexer_kl_grad_chunk_rows(int64_t batch, int64_t s_q, int64_t s_k, int64_t topk,
                                       int64_t workspace_bytes);
int dsa_pair_csr_build(const int32_t* indices, int64_t batch, int64_t s_q, int64_t s_k, int64_t topk,
                       int64_t q_offset, void* csr, int64_t csr_bytes, void* stream);

/*
 * Block KV compressor (reference: Compressor._forward_bsnd + overlap_transform,
 * models/deepseek_v4/model.py:174-221).
 *   kv, score [B, S, coff*D] fp32 (coff = 2 with overlap, else 1); ape [ratio, coff*D] fp32
 *   out [B, S/ratio, D]: fp32 pooled values, or, with norm_weight != NULL,
 *   RMSNorm(bf16(pooled)) * norm_weight written as bf16 (out_dtype selects f32/bf16 output).
 * RoPE epilogue (model.py:218-220), with rope_cs != NULL: the last rope_dim features of the
 * stored row (bf16-rounded first when out is bf16) are rotated in interleaved pairs
 * (2i, 2i+1) by cs[pos][i] = (cos, sin), rope_cs fp32 [n_pos, rope_dim/2, 2] (torch's
 * view_as_real of freqs_cis), pos = the block's first token position: positions[b*S + c*ratio]
 * (int32 [B*S]) or c*ratio when positions is NULL; rows at positions outside the table are
 * not rotated.  rope_dim a multiple of 4, <= D.
 */
int dsa_compressor_fwd(const float* kv, const float* score, const float* ape, const float* norm_weight, void* out,
                       int out_dtype, int64_t batch, int64_t s, int64_t d, int64_t ratio, int overlap,
                       float norm_eps, const float* rope_cs, int64_t n_pos, int64_t rope_dim,
                       const int32_t* positions, void* stream);

/*
 * Indexer input producer (reference: Indexer.forward, models/deepseek_v32/model.py:264-282 with
 * rotate_activation :196-221; models/deepseek_v4/model.py:343-357): per row of D = 128 bf16
 * features (x [rows, heads, 128], one row per query head or key),
 *   1. RoPE of features [rope_start, rope_start + rope_dim) in fp32, rounded to bf16: pairs
 *      (rope_start + 2i, +1) when interleaved (V4), (rope_start + i, rope_start + i + rope_dim/2)
 *      otherwise (V3.2's blocked layout), rotated by cs[pos][i]; rope_cs fp32
 *      [n_pos, rope_dim/2, 2]; pos = positions[row] (int32 [rows]) or
 *      pos_offset + row % seq_len; rows at positions outside the table are not rotated;
 *      rope_dim = 0 skips the step;
 *   2. with hadamard != 0: y = bf16(bf16(H x) * 128^-0.5), H the Sylvester Hadamard matrix;
 *   3. y written as bf16 [rows, heads, 128] (y != NULL) and/or its fp8-e4m3fn per-row
 *      quantisation q8 [rows, heads, 128] with scale [rows, heads] fp32 (the rule of
 *      dsa_quantize_fp8_rows).
 */
int dsa_indexer_prep(const void* x, void* y, uint8_t* q8, float* scale, int64_t rows, int64_t heads, int64_t d,
                     int64_t seq_len, const float* rope_cs, int64_t n_pos, const int32_t* positions,
                     int64_t pos_offset, int64_t rope_dim, int64_t rope_start, int interleaved, int hadamard,
                     void* stream);

/*
 * Per-row fp8-e4m3fn quantisation of indexer operands (q_I rows [.., H_I, D_I], k_I rows).
 *   x [rows, d] bf16 or fp32 (in_dtype), q [rows, d] e4m3fn bytes, scale [rows] fp32:
 *   scale = max(amax|x_row| / 448, 1e-12), q = e4m3fn(x / scale) rounded to nearest even,
 *   magnitudes that round above 448 -> NaN; byte-identical to torch's float8_e4m3fn cast of
 *   the same quotient.  d <= 2048 (DSA_ERR_UNSUPPORTED beyond).
 */
int dsa_quantize_fp8_rows(const void* x, int in_dtype, uint8_t* q, float* scale, int64_t rows, int64_t d,
                          void* stream);

/*
 * Attention sink (DeepSeek-V4): a per-head logit with no value in every row's softmax.
 * dsa_attn_sink_fold, after dsa_sparse_mla_fwd over the row's keys: with m, l the row's
 * softmax_max / softmax_sum, m2 = max(m, sink[h]), a = l e^(m - m2), s2 = a + e^(sink - m2);
 * out[row, h, :] *= a / s2 in place and (softmax_max, softmax_sum) <- (m2, s2), which is
 * what dsa_sparse_mla_bwd then needs.  dsa_attn_sink_grad adds to dsink[h] (fp32, caller
 * zeroes it) - sum over rows of e^(sink - m2) / s2 * sum_d dout * out.
 *   out / dout [rows, n_heads, d_v] in dtype (bf16 or fp32), statistics [rows, n_heads].
 */
int dsa_attn_sink_fold(void* out, float* softmax_max, float* softmax_sum, const float* sinks, int dtype,
                       int64_t rows, int64_t n_heads, int64_t d_v, void* stream);
int dsa_attn_sink_grad(const void* out, const void* dout, const float* softmax_max, const float* softmax_sum,
                       const float* sinks, float* dsink, int dtype, int64_t rows, int64_t n_heads, int64_t d_v,
                       void* stream);

/*
 * Block KV compressor over a packed varlen ("TND") batch (reference: Compressor._forward_tnd,
 * models/deepseek_v4/model.py:223-274).  Block c pools the ratio tokens starting at
 * block_starts[c] (device int64 [n_blocks], each in [0, n_tokens - ratio]; a start outside
 * that range yields a zero row); with overlap its first ratio slots are the previous listed
 * block's first D features when c > 0 and positions[block_starts[c]] >= ratio (device int32
 * [n_tokens] request-local positions).
 *   kv, score [n_tokens, coff*D] fp32; out [n_blocks, D] as in dsa_compressor_fwd; the RoPE
 *   epilogue rotates block c at positions[block_starts[c]] (model.py:266-273).
 */
int dsa_compressor_fwd_tnd(const float* kv, const float* score, const float* ape, const float* norm_weight,
                           void* out, int out_dtype, int64_t n_tokens, int64_t d, int64_t ratio, int overlap,
                           const int64_t* block_starts, int64_t n_blocks, const int32_t* positions, float norm_eps,
                           const float* rope_cs, int64_t n_pos, int64_t rope_dim, void* stream);

/*
 * MLA weight absorption (reference: models/deepseek_v32/model.py:520-535, the einsum
 * q_nope . w_uk before the attention, and :574-575, the output . w_uv_t after it):
 *   c[t, h, 0:n] = sum_k a[t, h, k] * wt[h, :, k]   (bf16 in, fp32 accumulation, bf16 out)
 *   c[t, h, n:n + append_width] = append[t, h, 0:append_width]   (append != NULL)
 *   a [tokens, heads, lda], wt [heads, n, k] (the weight transposed: row = output column),
 *   c [tokens, heads, ldc], append [tokens, heads, ld_append]; (k, n) = (128, 512) or (512, 128).
 * Forward of the query absorb: a = q_nope, wt = w_uk^T, append = q_pe, c = q [.., 576];
 * of the output absorb: a = attention output, wt = w_uv; their input gradients are the
 * other shape with the weight's transpose.
 */
int dsa_mla_absorb(const void* a, int64_t lda, const void* wt, void* c, int64_t ldc, const void* append,
                   int64_t ld_append, int64_t append_width, int64_t tokens, int64_t heads, int64_t k, int64_t n,
                   void* stream);

/*
 * Packed varlen ("TND") metadata built on the device (reference: build_smla_attention_masks,
 * models/deepseek_v4/tnd.py:97-164, which reads its lengths back to the host with .item()).
 * positions [n] int32 or int64 (pos_dtype_bytes 4 / 8), packed tokens in row-major order, -1
 * for padding after the last valid token.  A request starts at every position 0 and at the
 * first token; a ratio-r block starts at token t when positions[t] % r == 0 and the valid
 * token t + r - 1 has position positions[t] + r - 1.  ratios: device int32 [n_ratios]
 * (<= 4, each > 0).  Outputs, all device int32 (R = number of requests, known only on the
 * device):
 *   counts [4 + 2 n_ratios]: valid tokens, R, max request length, 1 if a valid token follows
 *          padding (invalid input), then per ratio (blocks, max compressed length);
 *   cu_q [n + 1] (entries 0..R), block_starts [n_ratios, n] (entries 0..blocks-1),
 *   cu_cmp [n_ratios, n + 1] (entries 0..R), residual [n_ratios, n] (entries 0..R-1).
 */
int dsa_tnd_metadata(const void* positions, int pos_dtype_bytes, int64_t n, const int* ratios, int64_t n_ratios,
                     int* counts, int* cu_q, int* block_starts, int* cu_cmp, int* residual, void* stream);

/*
 * Packed varlen ("TND") batches.  n_seq sequences are packed along the token axis:
 * sequence i owns query tokens [cu_seqlens_q[i], cu_seqlens_q[i+1]) and key tokens
 * [cu_seqlens_k[i], cu_seqlens_k[i+1]) of the packed tensors (the fixed-length layouts above
 * with B = 1 and S = total tokens).  cu_seqlens_* are HOST int32 arrays of n_seq + 1
 * non-decreasing entries starting at 0 (the launch schedule is decided on the host).
 * Index tensors hold sequence-local key positions (0 = the sequence's first key), -1 for
 * empty slots.  Within a sequence the causal rule is the fixed-length one aligned
 * bottom-right: q_offset_i = max(0, len_k_i - len_q_i) for token keys.  Each call runs the
 * fixed-length kernels once per non-empty sequence, in order, on `stream`, so the
 * workspace of one call serves every sequence.  A sequence with queries and no keys is an
 * error, except in the indexer, where its rows get no candidate (-1 padding).
 */

/* dsa_indexer_fwd + dsa_topk per sequence.  Keys may be compressed (cmp_ratio > 1):
 * then sequence i has cmp_ratio * len_k_i + cmp_residual_k[i] original key tokens
 * (cmp_residual_k: host int32 [n_seq] or NULL = 0) and, for sparse_mode 3,
 * q_offset_i = max(0, that count - len_q_i); sparse_mode 0 applies no causal rule.
 * scores_ws: device fp32 scratch of ws_bytes (>= 4 * the longest key sequence; a row chunk
 * of a sequence is scored into it at a time; for fp8 with H_I = 64 each chunk row also takes
 * dsa_indexer_fwd_workspace_size(1, 1, H_I, D_I, dtype) bytes of linear-split pieces, placed
 * after the chunk's scores at a 256-byte boundary, so add that per row plus 256).  indices [T_q, topk] int32, values
 * [T_q, topk] fp32 or NULL. */
int dsa_lightning_indexer_varlen(const void* q, const float* q_scale, const void* k, const float* k_scale,
                                 const float* w, int32_t* indices, float* values, float* scores_ws, int64_t ws_bytes,
                                 int dtype, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                 const int32_t* cmp_residual_k, int64_t n_seq, int64_t n_heads, int64_t head_dim,
                                 int64_t topk, int64_t cmp_ratio, int64_t sparse_mode, int64_t index_offset,
                                 void* stream);
int dsa_sparse_mla_fwd_varlen(const void* q, const void* kv, const int32_t* indices, void* out, float* softmax_max,
                              float* softmax_sum, int dtype, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv,
                              int64_t n_seq, int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                              void* stream);
/* largest per-sequence dsa_sparse_mla_bwd_workspace_size() of the batch */
int64_t dsa_sparse_mla_bwd_varlen_workspace_size(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv,
                                                 int64_t n_seq, int64_t n_heads, int64_t d_qk, int64_t topk);
int dsa_sparse_mla_bwd_varlen(const void* q, const void* kv, const int32_t* indices, const void* out,
                              const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                              float* dkv_accum, float* mass, void* workspace, int64_t workspace_bytes, int dtype,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv, int64_t n_seq,
                              int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale, void* stream);
int dsa_attn_mass_varlen(const void* q, const void* kv, const int32_t* indices, const float* softmax_max,
                         const float* softmax_sum, float* mass, int dtype, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_kv, int64_t n_seq, int64_t n_heads, int64_t d_qk, int64_t topk,
                         float scale, void* stream);
/* largest per-sequence dsa_indexer_kl_grad_workspace_size() of the batch */
int64_t dsa_indexer_kl_grad_varlen_workspace_size(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                                  int64_t n_seq, int64_t n_heads, int64_t head_dim, int64_t topk);
int dsa_indexer_kl_grad_varlen(const void* q_idx, const void* k_idx, const float* w, const int32_t* indices,
                               const float* mass, float* dq_idx, float* dk_idx_accum, float* dw, float* loss_rows,
                               void* workspace, int64_t workspace_bytes, const int32_t* cu_seqlens_q,
                               const int32_t* cu_seqlens_k, int64_t n_seq, int64_t n_heads, int64_t head_dim,
                               int64_t topk, float loss_scale, float eps, float grad_scale,
                               const float* grad_scale_dev, void* stream);

/*
 * Packed varlen batches with DEVICE cu_seqlens (no host copy of the lengths, so no host
 * synchronisation per batch).  Same contracts as the _varlen entry points above (reference:
 * npu_lightning_indexer / npu_sparse_flash_attention / npu_sparse_lightning_indexer_grad_kl_loss
 * with layout TND and actual_seq_lengths as tensors, ops/aclnn/lightning_indexer/binding.cpp:14,
 * converters/kernels/dsa.py:159-177, :238-253), except that the lengths are not validated on
 * the host: every window is clamped into the key tensor, and a sequence with queries and no
 * keys gives its rows no candidate instead of an error.
 */

/* Workspace of one dsa_lightning_indexer_tnd call whose row chunks hold up to max_rows rows
 * (0 if the shape has no tile kernel: D_I must be 128, H_I a multiple of 16 up to 128, bf16 or
 * fp8).  Per chunk: fp32 score rows of t_k (rounded up to 4) columns, the linear-split pieces
 * (fp8, H_I = 64), the top-k candidate lists (t_k > 16384) and the row geometry. */
int64_t dsa_lightning_indexer_tnd_workspace_size(int64_t t_q, int64_t t_k, int64_t n_heads, int64_t head_dim,
                                                 int dtype, int64_t topk, int64_t max_rows);
/* dsa_lightning_indexer_varlen with device cu_seqlens_q / cu_seqlens_k (int32 [n_seq + 1]) and
 * cmp_residual_k (device int32 [n_seq] or NULL): query rows are taken in chunks of as many
 * rows as the workspace holds; per chunk a geometry kernel reads each row's key window from
 * the device lengths, the persistent score kernels walk the (query group, key span) pairs
 * that hold work, and the top-k selects each row's window.  Indices are sequence-local (+
 * index_offset), -1 padded, bit-identical to dsa_lightning_indexer_varlen's. */
int dsa_lightning_indexer_tnd(const void* q, const float* q_scale, const void* k, const float* k_scale,
                              const float* w, int32_t* indices, float* values, int dtype,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              const int32_t* cmp_residual_k, int64_t n_seq, int64_t t_q, int64_t t_k,
                              int64_t n_heads, int64_t head_dim, int64_t topk, int64_t cmp_ratio, int64_t sparse_mode,
                              int64_t index_offset, void* workspace, int64_t workspace_bytes, void* stream);
/* Sequence-local slot indices [t_q, topk] -> global key rows (cu_seqlens_k[i] + v), keeping a
 * slot iff it passes the per-sequence causal rule of the _varlen attention entry points
 * (0 <= v < len_k_i, v <= s - cu_seqlens_q[i] + max(0, len_k_i - len_q_i)), else -1.  The
 * fixed-length attention, mass and indexer KL entry points then take the whole batch as one
 * [1, t_q] problem with q_offset >= t_k (no causal test): dsa_sparse_mla_fwd(_varlen)
 * results are bit-identical per row; dKV and dk_I sum the same contributions in another
 * fp32 grouping. */
int dsa_tnd_global_indices(const int32_t* indices, int32_t* out, const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int64_t n_seq, int64_t t_q, int64_t t_k, int64_t topk,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MI355X_H */
