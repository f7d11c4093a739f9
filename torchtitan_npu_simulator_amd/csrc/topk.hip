// Per-row top-k select by 8-bit radix select (4 passes, MSB first) on orderable uint32
// keys, followed by a stable compaction that emits the chosen indices in ascending order.
//
// Contract (bit-exact): row (b, s) considers t < n_valid = min(s_k, (s + q_offset + 1) /
// cmp_ratio) whose score is not NaN; it keeps the first k of a stable descending order by
// (score, lower index) with -0.0 == +0.0.  Ties at the threshold are broken by lower index
// because the compaction walks indices in order and admits equal keys until the quota is
// met.  One 256-thread workgroup per row; rows up to 16384 candidates are cached in LDS,
// longer rows are re-read from global (L2) on each pass.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kCacheMax = 16384;  // candidates cached in LDS (64 KiB)

__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0u;  // NaN: excluded (key 0 is below every real value's key)
  const uint32_t u = __float_as_uint(x + 0.0f);  // -0.0 -> +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// inclusive scan over 256 threads (Hillis-Steele in LDS); returns inclusive value
__device__ __forceinline__ uint32_t block_scan_incl(uint32_t v, uint32_t* buf) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {
    const uint32_t add = t >= off ? buf[t - off] : 0u;
    __syncthreads();
    buf[t] += add;
    __syncthreads();
  }
  const uint32_t r = buf[t];
  __syncthreads();
  return r;
}

template <bool kCached>
__global__ void __launch_bounds__(kThreads)
topk_kernel(const float* __restrict__ scores, int32_t* __restrict__ out_idx, float* __restrict__ out_val, int S,
            int s_k, int64_t ld, int k, int64_t q_offset, int cmp_ratio, int64_t index_offset) {
  extern __shared__ uint32_t cache[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan_buf[kThreads];
  __shared__ uint32_t sh_prefix, sh_mask, sh_remaining;

  const int s = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int64_t row = (int64_t)b * S + s;
  const float* src = scores + row * ld;
  int64_t nv64 = (s + q_offset + 1) / cmp_ratio;
  const int nv = (int)max((int64_t)0, min((int64_t)s_k, nv64));

  auto key_at = [&](int i) -> uint32_t { return kCached ? cache[i] : order_key(src[i]); };

  // candidates
  uint32_t cnt = 0;
  for (int i = t; i < nv; i += kThreads) {
    const uint32_t key = order_key(src[i]);
    if (kCached) cache[i] = key;
    cnt += key != 0u;
  }
  const uint32_t total = block_scan_incl(cnt, scan_buf);  // value at t is partial; take last
  if (t == kThreads - 1) sh_remaining = total;
  __syncthreads();
  const uint32_t n_cand = sh_remaining;
  __syncthreads();

  uint32_t thresh = 0u;  // keys > thresh are taken outright
  uint32_t need_eq = 0u; // keys == thresh taken, lowest indices first
  if (n_cand > (uint32_t)k) {
    if (t == 0) {
      sh_prefix = 0u;
      sh_mask = 0u;
      sh_remaining = (uint32_t)k;
    }
    __syncthreads();
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      hist[t] = 0u;
      __syncthreads();
      const uint32_t prefix = sh_prefix, mask = sh_mask;
      for (int i = t; i < nv; i += kThreads) {
        const uint32_t key = key_at(i);
        if (key != 0u && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      // suffix sums: suf[d] = sum_{e >= d} hist[e]; thread t handles bin d = 255 - t
      const uint32_t incl = block_scan_incl(hist[255 - t], scan_buf);  // sum over bins >= 255-t
      const uint32_t excl = incl - hist[255 - t];                      // bins > 255-t
      const uint32_t rem = sh_remaining;
      __syncthreads();
      if (excl < rem && incl >= rem) {  // exactly one bin satisfies this
        const uint32_t d = 255u - (uint32_t)t;
        sh_prefix = prefix | (d << shift);
        sh_mask = mask | (255u << shift);
        sh_remaining = rem - excl;
      }
      __syncthreads();
    }
    thresh = sh_prefix;
    need_eq = sh_remaining;
  }

  // stable compaction over contiguous per-thread segments, ascending index order
  const int seg = (nv + kThreads - 1) / kThreads;
  const int i0 = min(nv, t * seg), i1 = min(nv, i0 + seg);
  uint32_t c_gt = 0, c_eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = key_at(i);
    c_gt += key > thresh;
    c_eq += (key == thresh) && key != 0u;
  }
  const uint32_t eq_before = block_scan_incl(c_eq, scan_buf) - c_eq;
  const uint32_t eq_take = need_eq > eq_before ? min(c_eq, need_eq - eq_before) : 0u;
  const uint32_t mine = c_gt + eq_take;
  const uint32_t pos0 = block_scan_incl(mine, scan_buf) - mine;
  int32_t* oi = out_idx + row * k;
  float* ov = out_val ? out_val + row * k : nullptr;
  uint32_t pos = pos0, eq_seen = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = key_at(i);
    bool take = key > thresh;
    if (!take && key == thresh && key != 0u) {
      take = eq_seen < eq_take;
      ++eq_seen;
    }
    if (take) {
      oi[pos] = (int32_t)(i + index_offset);
      if (ov) ov[pos] = src[i];
      ++pos;
    }
  }
  const uint32_t taken = min(n_cand, (uint32_t)k);
  for (int j = (int)taken + t; j < k; j += kThreads) {
    oi[j] = -1;
    if (ov) ov[j] = -INFINITY;
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_topk(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q,
                        int64_t s_k, int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio,
                        int64_t index_offset, void* stream) {
  using namespace dsa;
  if (!scores || !indices) return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k < 0 || k <= 0 || k > 4096 || ld_scores < s_k || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: bad sizes (B=%lld S=%lld S_k=%lld ld=%lld k=%lld r=%lld)",
                     (long long)batch, (long long)s_q, (long long)s_k, (long long)ld_scores, (long long)k,
                     (long long)cmp_ratio);
  if (s_q > 2147483647LL || batch > 65535 || s_k > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)s_q, (unsigned)batch);
  if (s_k <= kCacheMax) {
    topk_kernel<true><<<grid, kThreads, (size_t)s_k * 4, st>>>(scores, indices, values, (int)s_q, (int)s_k,
                                                               ld_scores, (int)k, q_offset, (int)cmp_ratio,
                                                               index_offset);
  } else {
    topk_kernel<false><<<grid, kThreads, 0, st>>>(scores, indices, values, (int)s_q, (int)s_k, ld_scores, (int)k,
                                                  q_offset, (int)cmp_ratio, index_offset);
  }
  return check_launch("dsa_topk");
}
