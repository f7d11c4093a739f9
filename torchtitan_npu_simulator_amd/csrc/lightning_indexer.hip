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

// Geometry of rows [row0, row0 + rows) in the layout indexer_fwd_tnd reads, one thread per
// group of `gr` rows: [first: rows][end: rows][span start: G][work end: G][span count,
// then its exclusive prefix: G + 1].
__global__ void __launch_bounds__(256)
tnd_geometry_kernel(const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                    const int32_t* __restrict__ res, int n_seq, int64_t row0, int rows, int cmp_ratio, int causal,
                    int t_k, int gr, int span, int* __restrict__ geo) {
  const int G = (rows + gr - 1) / gr;
  const int grp = blockIdx.x * 256 + threadIdx.x;
  if (grp >= G) return;
  int lo = 0x7fffffff, hi = 0;
  for (int i = 0; i < gr; ++i) {
    const int r = grp * gr + i;
    if (r >= rows) break;
    int first, end;
    tnd_row_window(cu_q, cu_k, res, n_seq, row0 + r, cmp_ratio, causal != 0, t_k, first, end);
    geo[r] = first;
    geo[rows + r] = end;
    if (end > first) {
      lo = min(lo, first);
      hi = max(hi, end);
    }
  }
  const bool any = hi > 0 && lo < hi;
  geo[2 * rows + grp] = any ? lo : 0;
  geo[2 * rows + G + grp] = any ? hi : 0;
  geo[2 * rows + 2 * G + grp] = any ? (hi - lo + span - 1) / span : 0;
}

// exclusive prefix of the G span counts in place, the total at index G (one workgroup)
__global__ void __launch_bounds__(1024)
tnd_prefix_kernel(int* __restrict__ cnt, int G) {
  __shared__ int wsum[16];
  __shared__ int carry_sh;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (t == 0) carry_sh = 0;
  __syncthreads();
  for (int base = 0; base < G; base += 1024) {
    const int v = base + t < G ? cnt[base + t] : 0;
    int x = v;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = carry_sh;
    for (int w2 = 0; w2 < wave; ++w2) before += wsum[w2];
    if (base + t < G) cnt[base + t] = before + x - v;
    __syncthreads();
    if (t == 1023) carry_sh = before + x;
    __syncthreads();
  }
  if (t == 0) cnt[G] = carry_sh;
}

int64_t tnd_ld(int64_t t_k) { return (t_k + 3) / 4 * 4; }  // 16-byte aligned score rows

// bytes of one chunk of `rows` packed rows: scores, linear-split pieces, top-k candidate
// lists, geometry
int64_t tnd_chunk_bytes(int64_t rows, int64_t t_k, int64_t n_heads, int64_t head_dim, int dtype, int64_t topk,
                        int gr) {
  const int64_t groups = (rows + gr - 1) / gr;
  return align256(rows * tnd_ld(t_k) * 4) + align256(dsa_indexer_fwd_workspace_size(1, rows, n_heads, head_dim, dtype)) +
         (t_k > 16384 ? align256(topk_cand_bytes(rows, topk)) : 0) + align256(4 * (2 * rows + 3 * groups + 1));
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

extern "C" int64_t dsa_lightning_indexer_tnd_workspace_size(int64_t t_q, int64_t t_k, int64_t n_heads,
                                                            int64_t head_dim, int dtype, int64_t topk,
                                                            int64_t max_rows) {
  int gr = 0, sk = 0;
  if (t_q <= 0 || t_k <= 0 || topk <= 0 || max_rows <= 0 || !dsa::indexer_tnd_tiling(dtype, n_heads, head_dim, &gr, &sk))
    return 0;
  return dsa::tnd_chunk_bytes(std::min(t_q, max_rows), t_k, n_heads, head_dim, dtype, topk, gr);
}

extern "C" int dsa_lightning_indexer_tnd(const void* q, const float* q_scale, const void* k, const float* k_scale,
                                         const float* w, int32_t* indices, float* values, int dtype,
                                         const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                         const int32_t* cmp_residual_k, int64_t n_seq, int64_t t_q, int64_t t_k,
                                         int64_t n_heads, int64_t head_dim, int64_t topk, int64_t cmp_ratio,
                                         int64_t sparse_mode, int64_t index_offset, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  using namespace dsa;
  const char* what = "dsa_lightning_indexer_tnd";
  if (!q || !k || !w || !indices || !workspace || !cu_seqlens_q || !cu_seqlens_k)
    return set_error(DSA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (n_seq <= 0 || t_q <= 0 || t_k <= 0 || topk <= 0 || cmp_ratio <= 0 || n_seq > 2147483646LL ||
      t_q > 2147483647LL || t_k > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "%s: bad sizes", what);
  if (sparse_mode != 0 && sparse_mode != 3)
    return set_error(DSA_ERR_UNSUPPORTED, "%s: sparse_mode %lld (0 or 3)", what, (long long)sparse_mode);
  if ((uintptr_t)workspace % 256) return set_error(DSA_ERR_INVALID_ARG, "%s: workspace must be 256-byte aligned", what);
  int gr = 0, span = 0;
  if (!indexer_tnd_tiling(dtype, n_heads, head_dim, &gr, &span))
    return set_error(DSA_ERR_UNSUPPORTED, "%s: H_I=%lld, D_I=%lld, dtype %d has no tile kernel", what,
                     (long long)n_heads, (long long)head_dim, dtype);
  int64_t rows = t_q;  // largest chunk whose workspace fits
  if (tnd_chunk_bytes(rows, t_k, n_heads, head_dim, dtype, topk, gr) > workspace_bytes) {
    int64_t lo = 0, hi = t_q;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (tnd_chunk_bytes(mid, t_k, n_heads, head_dim, dtype, topk, gr) <= workspace_bytes) lo = mid;
      else hi = mid - 1;
    }
    rows = lo;
    if (rows == 0)
      return set_error(DSA_ERR_INVALID_ARG, "%s: workspace of %lld bytes holds no query row (%lld needed)", what,
                       (long long)workspace_bytes,
                       (long long)tnd_chunk_bytes(1, t_k, n_heads, head_dim, dtype, topk, gr));
  }
  hipStream_t st = (hipStream_t)stream;
  const int64_t es = idx_elem_bytes(dtype), ld = tnd_ld(t_k);
  for (int64_t r0 = 0; r0 < t_q; r0 += rows) {
    const int64_t nr = std::min(rows, t_q - r0);
    const int64_t groups = (nr + gr - 1) / gr;
    char* base = (char*)workspace;
    float* scores = (float*)base;
    base += align256(nr * ld * 4);
    const int64_t lin_bytes = dsa_indexer_fwd_workspace_size(1, nr, n_heads, head_dim, dtype);
    void* lin_ws = lin_bytes ? (void*)base : nullptr;
    base += align256(lin_bytes);
    void* cand_ws = nullptr;
    if (t_k > 16384) {
      cand_ws = base;
      base += align256(topk_cand_bytes(nr, topk));
    }
    int* geo = (int*)base;
    {
      const TimedLaunch tl("tnd_geometry_kernel", st);
      tnd_geometry_kernel<<<(unsigned)ceil_div(groups, 256), 256, 0, st>>>(
          cu_seqlens_q, cu_seqlens_k, cmp_residual_k, (int)n_seq, r0, (int)nr, (int)cmp_ratio, sparse_mode == 3 ? 1 : 0,
          (int)t_k, gr, span, geo);
      tnd_prefix_kernel<<<1, 1024, 0, st>>>(geo + 2 * nr + 2 * groups, (int)groups);
    }
    if (int rc = check_launch(what)) return rc;
    const char* qc = (const char*)q + r0 * n_heads * head_dim * es;
    if (int rc = indexer_fwd_tnd(qc, q_scale ? q_scale + r0 * n_heads : nullptr, k, k_scale, w + r0 * n_heads,
                                 scores, dtype, nr, t_k, n_heads, head_dim, ld, geo, groups, lin_ws, lin_bytes,
                                 stream))
      return rc;
    // each row's valid prefix is its window's length; its scores sit at columns [0, length)
    if (int rc = topk_rows(scores, indices + r0 * topk, values ? values + r0 * topk : nullptr, 1, nr, t_k, ld, topk,
                           0, 1, index_offset, cand_ws, stream, geo, nr))
      return rc;
  }
  return DSA_OK;
}
