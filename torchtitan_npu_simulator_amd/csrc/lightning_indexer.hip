// The fused lightning indexer of the reference's npu_lightning_indexer binding (BSND): index
// scores and the per-query top-k in one call, returning only the selected indices (and
// optionally their scores), with the fp32 score rows living in the caller's workspace
// (reference: ops/aclnn/lightning_indexer/binding.cpp:14-31, called from
// converters/kernels/dsa.py:159-175).
//
// Rows are processed in chunks of the workspace's capacity: all batches together when every
// row fits, else batch by batch.  Each chunk runs the score kernels with the spans past every
// query's causal frontier left unwritten and the top-k, which reads only each row's valid
// prefix, straight into the output rows.  The linear-split pieces of the fp8 H_I = 64 shape
// sit after the chunk's scores.
#include <algorithm>

#include "dsa_common.h"

namespace dsa {
namespace {

int64_t idx_elem_bytes(int dtype) { return dtype == DSA_F32 ? 4 : dtype == DSA_BF16 ? 2 : 1; }

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// long rows (more than 16384 keys) select through per-row candidate lists (k <= 4096)
int64_t cand_bytes(int64_t nb, int64_t rows, int64_t s_k) {
  return s_k > 16384 ? align256(topk_cand_bytes(nb * rows, 4096)) : 0;
}

// bytes of one chunk of `rows` query rows over `nb` batches: the score rows, the
// linear-split pieces, the top-k candidate lists
int64_t chunk_bytes(int64_t nb, int64_t rows, int64_t s_k, int64_t n_heads, int64_t head_dim, int dtype) {
  return align256(nb * rows * s_k * 4) + align256(dsa_indexer_fwd_workspace_size(nb, rows, n_heads, head_dim, dtype)) +
         cand_bytes(nb, rows, s_k);
}

}  // namespace
}  // namespace dsa

extern "C" int64_t dsa_lightning_indexer_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                                                        int64_t head_dim, int dtype, int64_t max_rows) {
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || max_rows <= 0) return 0;
  const int64_t rows = std::min(s_q, max_rows);
  return dsa::chunk_bytes(rows == s_q ? batch : 1, rows, s_k, n_heads, head_dim, dtype);
}

extern "C" int dsa_lightning_indexer(const void* q, const float* q_scale, const void* k, const float* k_scale,
                                     const float* w, int32_t* indices, float* values, int dtype, int64_t batch,
                                     int64_t s_q, int64_t s_k, int64_t n_heads, int64_t head_dim, int64_t topk,
                                     int64_t q_offset, int64_t cmp_ratio, int64_t index_offset, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  using namespace dsa;
  const char* what = "dsa_lightning_indexer";
  if (!q || !k || !w || !indices || !workspace) return set_error(DSA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || n_heads <= 0 || head_dim <= 0 || topk <= 0 || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "%s: bad sizes", what);
  if ((uintptr_t)workspace % 256) return set_error(DSA_ERR_INVALID_ARG, "%s: workspace must be 256-byte aligned", what);
  // all batches in one pass when every row fits, else batch by batch in row chunks
  int64_t nb = batch, rows = s_q;
  if (chunk_bytes(batch, s_q, s_k, n_heads, head_dim, dtype) > workspace_bytes) {
    nb = 1;
    int64_t lo = 0, hi = s_q;  // largest row count whose chunk fits
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (chunk_bytes(1, mid, s_k, n_heads, head_dim, dtype) <= workspace_bytes) lo = mid;
      else hi = mid - 1;
    }
    rows = lo;
    if (rows == 0)
      return set_error(DSA_ERR_INVALID_ARG, "%s: workspace of %lld bytes holds no query row (%lld needed)", what,
                       (long long)workspace_bytes, (long long)chunk_bytes(1, 1, s_k, n_heads, head_dim, dtype));
  }
  const int64_t es = idx_elem_bytes(dtype);
  float* scores = (float*)workspace;
  for (int64_t b0 = 0; b0 < batch; b0 += nb) {
    for (int64_t r0 = 0; r0 < s_q; r0 += rows) {
      const int64_t nr = std::min(rows, s_q - r0);
      const int64_t row = b0 * s_q + r0;  // first (batch, row) of the chunk
      const int64_t lin_bytes = dsa_indexer_fwd_workspace_size(nb, nr, n_heads, head_dim, dtype);
      void* lin_ws = lin_bytes ? (void*)((char*)workspace + align256(nb * nr * s_k * 4)) : nullptr;
      void* cand_ws = cand_bytes(nb, nr, s_k)
                          ? (void*)((char*)workspace + align256(nb * nr * s_k * 4) + align256(lin_bytes))
                          : nullptr;
      // (with one batch per pass the chunk's rows are contiguous in q, w and the outputs)
      const char* qc = (const char*)q + row * n_heads * head_dim * es;
      if (int rc = indexer_fwd(qc, q_scale ? q_scale + row * n_heads : nullptr,
                               (const char*)k + b0 * s_k * head_dim * es, k_scale ? k_scale + b0 * s_k : nullptr,
                               w + row * n_heads, scores, dtype, nb, nr, s_k, n_heads, head_dim, s_k, q_offset + r0,
                               cmp_ratio, lin_ws, lin_bytes, stream, false))
        return rc;
      if (int rc = topk_rows(scores, indices + row * topk, values ? values + row * topk : nullptr, nb, nr, s_k, s_k,
                             topk, q_offset + r0, cmp_ratio, index_offset, cand_ws, stream))
        return rc;
    }
  }
  return DSA_OK;
}
