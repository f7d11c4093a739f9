// Packed variable-length ("TND") batches: per-sequence schedules over the fixed-length
// entry points.
//
// A TND batch packs n_seq sequences along the token axis.  Sequence i owns query tokens
// [cu_q[i], cu_q[i+1]) and key tokens [cu_k[i], cu_k[i+1]); its index tensors hold
// sequence-local key positions.  Every tensor of a sequence is therefore one contiguous
// slice of the packed tensor, and the sequence is exactly a batch-1 call of the
// fixed-length kernels on those slices with the sequence's own causal offset.  The
// schedule walks the host copy of cu_seqlens and enqueues one such call per non-empty
// sequence on the caller's stream (in order, so per-call scratch is reused safely);
// sequences of up to 32K tokens fill the GPU on their own, which is what makes a host
// schedule cheaper than a device-side row-to-sequence search inside every kernel.
#include <algorithm>

#include "dsa_common.h"

namespace dsa {
namespace {

int64_t elem_bytes(int dtype) { return dtype == DSA_F32 ? 4 : dtype == DSA_BF16 ? 2 : 1; }

template <typename T>
T* at(T* base, int64_t bytes) {
  return base ? (T*)((char*)base + bytes) : nullptr;
}
template <typename T>
const T* at(const T* base, int64_t bytes) {
  return base ? (const T*)((const char*)base + bytes) : nullptr;
}

// cu_seqlens checks: n_seq + 1 non-decreasing entries starting at 0
int check_cu(const int32_t* cu, int64_t n_seq, const char* what, const char* name) {
  if (!cu) return set_error(DSA_ERR_INVALID_ARG, "%s: %s is null", what, name);
  if (cu[0] != 0) return set_error(DSA_ERR_INVALID_ARG, "%s: %s[0] must be 0 (got %d)", what, name, cu[0]);
  for (int64_t i = 0; i < n_seq; ++i)
    if (cu[i + 1] < cu[i])
      return set_error(DSA_ERR_INVALID_ARG, "%s: %s must be non-decreasing (entry %lld)", what, name,
                       (long long)(i + 1));
  return DSA_OK;
}

int check_seqs(const int32_t* cu_q, const int32_t* cu_k, int64_t n_seq, const char* what) {
  if (n_seq <= 0) return set_error(DSA_ERR_INVALID_ARG, "%s: n_seq must be positive", what);
  if (int rc = check_cu(cu_q, n_seq, what, "cu_seqlens_q")) return rc;
  if (int rc = check_cu(cu_k, n_seq, what, "cu_seqlens_k")) return rc;
  return DSA_OK;
}

// bottom-right causal offset of a sequence whose keys are tokens (compression ratio 1)
int64_t token_offset(int64_t len_q, int64_t len_k) { return std::max<int64_t>(0, len_k - len_q); }

int no_keys(const char* what, int64_t i, int64_t len_q) {
  return set_error(DSA_ERR_INVALID_ARG, "%s: sequence %lld has %lld query tokens and no keys", what, (long long)i,
                   (long long)len_q);
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_lightning_indexer_varlen(const void* q, const float* q_scale, const void* k,
                                            const float* k_scale, const float* w, int32_t* indices, float* values,
                                            float* scores_ws, int64_t ws_bytes, int dtype, const int32_t* cu_seqlens_q,
                                            const int32_t* cu_seqlens_k, const int32_t* cmp_residual_k, int64_t n_seq,
                                            int64_t n_heads, int64_t head_dim, int64_t topk, int64_t cmp_ratio,
                                            int64_t sparse_mode, int64_t index_offset, void* stream) {
  using namespace dsa;
  const char* what = "dsa_lightning_indexer_varlen";
  if (!q || !k || !w || !indices || !scores_ws) return set_error(DSA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (int rc = check_seqs(cu_seqlens_q, cu_seqlens_k, n_seq, what)) return rc;
  if (n_heads <= 0 || head_dim <= 0 || topk <= 0 || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "%s: bad sizes", what);
  if (sparse_mode != 0 && sparse_mode != 3)
    return set_error(DSA_ERR_UNSUPPORTED, "%s: sparse_mode %lld (0 or 3)", what, (long long)sparse_mode);
  const int64_t es = elem_bytes(dtype);
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t q0 = cu_seqlens_q[i], lq = cu_seqlens_q[i + 1] - q0;
    const int64_t k0 = cu_seqlens_k[i], lk = cu_seqlens_k[i + 1] - k0;
    if (lq == 0) continue;
    // original (uncompressed) key tokens of the sequence: whole blocks plus the residual
    const int64_t res = cmp_residual_k ? cmp_residual_k[i] : 0;
    if (res < 0) return set_error(DSA_ERR_INVALID_ARG, "%s: cmp_residual_k[%lld] < 0", what, (long long)i);
    const int64_t q_off = sparse_mode == 3 ? std::max<int64_t>(0, cmp_ratio * lk + res - lq) : (int64_t)1 << 40;
    // per chunk row: its fp32 scores, plus (fp8, H_I = 64) the linear-split pieces placed after
    // the chunk's scores at a 256-byte boundary, plus (rows longer than 16384 keys) the top-k
    // candidate list after those
    const int64_t lin_bytes = dsa_indexer_fwd_workspace_size(1, 1, n_heads, head_dim, dtype);
    const bool long_rows = lk > 16384;
    const int64_t cand_row = long_rows ? topk_cand_bytes(1, topk) - 256 : 0;
    const int64_t row_bytes = 4 * std::max<int64_t>(lk, 1) + lin_bytes + cand_row;
    const int64_t rows =
        std::min<int64_t>(lq, std::max<int64_t>(0, ws_bytes - (lin_bytes ? 256 : 0) - (long_rows ? 512 : 0)) /
                                  row_bytes);
    if (rows <= 0)
      return set_error(DSA_ERR_INVALID_ARG, "%s: score scratch of %lld bytes holds no row of sequence %lld", what,
                       (long long)ws_bytes, (long long)i);
    for (int64_t r0 = 0; r0 < lq; r0 += rows) {
      const int64_t nr = std::min(rows, lq - r0);
      const int64_t row = q0 + r0;
      void* lin_ws = lin_bytes ? (void*)((char*)scores_ws + (rows * 4 * lk + 255) / 256 * 256) : nullptr;
      void* cand_ws = long_rows ? (void*)((char*)scores_ws + (rows * 4 * lk + 255) / 256 * 256 +
                                          (rows * lin_bytes + 255) / 256 * 256)
                                : nullptr;
      if (lk > 0) {
        // (spans past every frontier stay unwritten: the top-k reads only valid prefixes)
        if (int rc = indexer_fwd(at(q, row * n_heads * head_dim * es), at(q_scale, row * n_heads * 4),
                                 at(k, k0 * head_dim * es), at(k_scale, k0 * 4), at(w, row * n_heads * 4), scores_ws,
                                 dtype, 1, nr, lk, n_heads, head_dim, lk, q_off + r0, cmp_ratio, lin_ws,
                                 nr * lin_bytes, stream, false))
          return rc;
      }
      // with no keys the selection sees no candidate and pads the rows with -1
      if (int rc = topk_rows(scores_ws, at(indices, row * topk * 4), at(values, row * topk * 4), 1, nr, lk, lk, topk,
                             q_off + r0, cmp_ratio, index_offset, cand_ws, stream))
        return rc;
    }
  }
  return DSA_OK;
}

extern "C" int dsa_sparse_mla_fwd_varlen(const void* q, const void* kv, const int32_t* indices, void* out,
                                         float* softmax_max, float* softmax_sum, int dtype,
                                         const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv, int64_t n_seq,
                                         int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                                         void* stream) {
  using namespace dsa;
  const char* what = "dsa_sparse_mla_fwd_varlen";
  if (int rc = check_seqs(cu_seqlens_q, cu_seqlens_kv, n_seq, what)) return rc;
  const int64_t es = elem_bytes(dtype);
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t q0 = cu_seqlens_q[i], lq = cu_seqlens_q[i + 1] - q0;
    const int64_t k0 = cu_seqlens_kv[i], lk = cu_seqlens_kv[i + 1] - k0;
    if (lq == 0) continue;
    if (lk == 0) return no_keys(what, i, lq);
    if (int rc = dsa_sparse_mla_fwd(at(q, q0 * n_heads * d_qk * es), at(kv, k0 * d_qk * es),
                                    at(indices, q0 * topk * 4), at(out, q0 * n_heads * d_v * es),
                                    at(softmax_max, q0 * n_heads * 4), at(softmax_sum, q0 * n_heads * 4), dtype, 1,
                                    lq, lk, n_heads, d_qk, d_v, topk, scale, token_offset(lq, lk), stream))
      return rc;
  }
  return DSA_OK;
}

extern "C" int64_t dsa_sparse_mla_bwd_varlen_workspace_size(const int32_t* cu_seqlens_q,
                                                            const int32_t* cu_seqlens_kv, int64_t n_seq,
                                                            int64_t n_heads, int64_t d_qk, int64_t topk) {
  if (!cu_seqlens_q || !cu_seqlens_kv || n_seq <= 0) return 0;
  int64_t ws = 0;
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t lq = cu_seqlens_q[i + 1] - cu_seqlens_q[i], lk = cu_seqlens_kv[i + 1] - cu_seqlens_kv[i];
    if (lq > 0 && lk > 0) ws = std::max(ws, dsa_sparse_mla_bwd_workspace_size(1, lq, lk, n_heads, d_qk, topk));
  }
  return ws;
}

extern "C" int dsa_sparse_mla_bwd_varlen(const void* q, const void* kv, const int32_t* indices, const void* out,
                                         const void* dout, const float* softmax_max, const float* softmax_sum,
                                         void* dq, float* dkv_accum, float* mass, void* workspace,
                                         int64_t workspace_bytes, int dtype, const int32_t* cu_seqlens_q,
                                         const int32_t* cu_seqlens_kv, int64_t n_seq, int64_t n_heads, int64_t d_qk,
                                         int64_t d_v, int64_t topk, float scale, void* stream) {
  using namespace dsa;
  const char* what = "dsa_sparse_mla_bwd_varlen";
  if (int rc = check_seqs(cu_seqlens_q, cu_seqlens_kv, n_seq, what)) return rc;
  const int64_t es = elem_bytes(dtype);
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t q0 = cu_seqlens_q[i], lq = cu_seqlens_q[i + 1] - q0;
    const int64_t k0 = cu_seqlens_kv[i], lk = cu_seqlens_kv[i + 1] - k0;
    if (lq == 0) continue;
    if (lk == 0) return no_keys(what, i, lq);
    const int64_t qb = q0 * n_heads * d_qk * es, ob = q0 * n_heads * d_v * es, hb = q0 * n_heads * 4;
    if (int rc = dsa_sparse_mla_bwd(at(q, qb), at(kv, k0 * d_qk * es), at(indices, q0 * topk * 4), at(out, ob),
                                    at(dout, ob), at(softmax_max, hb), at(softmax_sum, hb), at(dq, qb),
                                    at(dkv_accum, k0 * d_qk * 4), at(mass, q0 * topk * 4), workspace,
                                    workspace_bytes, dtype, 1, lq, lk, n_heads, d_qk, d_v, topk, scale,
                                    token_offset(lq, lk), stream))
      return rc;
  }
  return DSA_OK;
}

extern "C" int dsa_attn_mass_varlen(const void* q, const void* kv, const int32_t* indices, const float* softmax_max,
                                    const float* softmax_sum, float* mass, int dtype, const int32_t* cu_seqlens_q,
                                    const int32_t* cu_seqlens_kv, int64_t n_seq, int64_t n_heads, int64_t d_qk,
                                    int64_t topk, float scale, void* stream) {
  using namespace dsa;
  const char* what = "dsa_attn_mass_varlen";
  if (int rc = check_seqs(cu_seqlens_q, cu_seqlens_kv, n_seq, what)) return rc;
  const int64_t es = elem_bytes(dtype);
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t q0 = cu_seqlens_q[i], lq = cu_seqlens_q[i + 1] - q0;
    const int64_t k0 = cu_seqlens_kv[i], lk = cu_seqlens_kv[i + 1] - k0;
    if (lq == 0) continue;
    if (lk == 0) return no_keys(what, i, lq);
    const int64_t hb = q0 * n_heads * 4;
    if (int rc = dsa_attn_mass(at(q, q0 * n_heads * d_qk * es), at(kv, k0 * d_qk * es), at(indices, q0 * topk * 4),
                               at(softmax_max, hb), at(softmax_sum, hb), at(mass, q0 * topk * 4), dtype, 1, lq, lk,
                               n_heads, d_qk, topk, scale, token_offset(lq, lk), stream))
      return rc;
  }
  return DSA_OK;
}

extern "C" int64_t dsa_indexer_kl_grad_varlen_workspace_size(const int32_t* cu_seqlens_q,
                                                             const int32_t* cu_seqlens_k, int64_t n_seq,
                                                             int64_t n_heads, int64_t head_dim, int64_t topk) {
  if (!cu_seqlens_q || !cu_seqlens_k || n_seq <= 0) return 0;
  int64_t ws = 0;
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t lq = cu_seqlens_q[i + 1] - cu_seqlens_q[i], lk = cu_seqlens_k[i + 1] - cu_seqlens_k[i];
    if (lq > 0 && lk > 0) ws = std::max(ws, dsa_indexer_kl_grad_workspace_size(1, lq, lk, n_heads, head_dim, topk));
  }
  return ws;
}

extern "C" int dsa_indexer_kl_grad_varlen(const void* q_idx, const void* k_idx, const float* w,
                                          const int32_t* indices, const float* mass, float* dq_idx,
                                          float* dk_idx_accum, float* dw, float* loss_rows, void* workspace,
                                          int64_t workspace_bytes, const int32_t* cu_seqlens_q,
                                          const int32_t* cu_seqlens_k, int64_t n_seq, int64_t n_heads,
                                          int64_t head_dim, int64_t topk, float loss_scale, float eps,
                                          float grad_scale, const float* grad_scale_dev, void* stream) {
  using namespace dsa;
  const char* what = "dsa_indexer_kl_grad_varlen";
  if (int rc = check_seqs(cu_seqlens_q, cu_seqlens_k, n_seq, what)) return rc;
  const int64_t es = 2;  // bf16 q_idx / k_idx
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t q0 = cu_seqlens_q[i], lq = cu_seqlens_q[i + 1] - q0;
    const int64_t k0 = cu_seqlens_k[i], lk = cu_seqlens_k[i + 1] - k0;
    if (lq == 0) continue;
    if (lk == 0) return no_keys(what, i, lq);
    const int64_t hd = n_heads * head_dim;
    if (int rc = dsa_indexer_kl_grad(at(q_idx, q0 * hd * es), at(k_idx, k0 * head_dim * es), at(w, q0 * n_heads * 4),
                                     at(indices, q0 * topk * 4), at(mass, q0 * topk * 4), at(dq_idx, q0 * hd * 4),
                                     at(dk_idx_accum, k0 * head_dim * 4), at(dw, q0 * n_heads * 4),
                                     at(loss_rows, q0 * 4), workspace, workspace_bytes, 1, lq, lk, n_heads, head_dim,
                                     topk, token_offset(lq, lk), loss_scale, eps, grad_scale, grad_scale_dev,
                                     stream))
      return rc;
  }
  return DSA_OK;
}

// ----- packed batches with device cu_seqlens: one launch over all rows -----
// The attention, its mass and the indexer KL take a packed batch as one [1, T] problem when
// its slot indices are global key rows: row s of sequence i keeps local slot v iff
// 0 <= v < (its causal count under the per-sequence rule of the host schedule above:
// min(len_k, s - cu_q[i] + max(0, len_k - len_q) + 1)), as cu_k[i] + v, and -1 otherwise.
// Run with the causal test off (q_offset past every key), the fixed-length kernels then
// compute each row from exactly the rows the per-sequence launch would gather, in the same
// order; only the key-major reductions (dKV, dk_I) group their fp32 sums differently.
namespace dsa {
namespace {
__global__ void __launch_bounds__(256)
tnd_global_indices_kernel(const int32_t* __restrict__ idx, int32_t* __restrict__ out,
                          const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int n_seq, int t_q,
                          int t_k, int topk) {
  const int s = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (s >= t_q) return;  // whole waves
  int first, end;
  tnd_row_window(cu_q, cu_k, nullptr, n_seq, s, 1, true, t_k, first, end);
  const int n = end - first;
  const int32_t* src = idx + (int64_t)s * topk;
  int32_t* dst = out + (int64_t)s * topk;
  for (int j = lane; j < topk; j += 64) {
    const int v = src[j];
    dst[j] = (v >= 0 && v < n) ? first + v : -1;
  }
}
}  // namespace
}  // namespace dsa

extern "C" int dsa_tnd_global_indices(const int32_t* indices, int32_t* out, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, int64_t n_seq, int64_t t_q, int64_t t_k,
                                      int64_t topk, void* stream) {
  using namespace dsa;
  const char* what = "dsa_tnd_global_indices";
  if (!indices || !out || !cu_seqlens_q || !cu_seqlens_k) return set_error(DSA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (n_seq <= 0 || t_q < 0 || t_k < 0 || topk <= 0 || n_seq > 2147483646LL || t_q > 2147483647LL ||
      t_k > 2147483647LL || topk > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "%s: bad sizes", what);
  if (t_q == 0) return DSA_OK;
  hipStream_t st = (hipStream_t)stream;
  {
    const TimedLaunch tl("tnd_global_indices_kernel", st);
    tnd_global_indices_kernel<<<ceil_div(t_q, 4), 256, 0, st>>>(indices, out, cu_seqlens_q, cu_seqlens_k,
                                                                (int)n_seq, (int)t_q, (int)t_k, (int)topk);
  }
  return check_launch(what);
}
