// Packed varlen ("TND") metadata on the device: the request layout and compressed-block
// bookkeeping of a batch of token positions, with no host round trip.
//
// Input: positions [n] (int64, or int32) of the packed tokens in row-major order, -1 for
// padding (allowed only after the last valid token).  A request starts at every position 0
// and at the first token.  For each compression ratio r, a block starts at token t when
// positions[t] % r == 0 and token t + r - 1 exists inside the valid tokens with position
// positions[t] + r - 1 (the whole block lies in one request).
//
// Outputs (capacity n requests / blocks; the counts live on the device):
//   counts[0] = number of valid tokens, counts[1] = number of requests R,
//   counts[2] = max request length, counts[3] = 1 if a valid token follows padding (an
//   invalid batch), counts[4 + 2j] = blocks of ratio j, counts[5 + 2j] = max compressed
//   length of ratio j;
//   cu_q [n + 1]: request boundaries [0, ends..] (entries 0..R);
//   per ratio j: block_starts_j [n] (token indices, entries 0..blocks-1),
//   cu_cmp_j [n + 1] (compressed-row boundaries per request, entries 0..R) and
//   residual_j [n] (request length - r * its compressed length, entries 0..R-1).
//
// One workgroup of 1024 threads walks the tokens in chunks of 1024: a workgroup-wide
// prefix sum of the request-start flags and of each ratio's block-start flags turns every
// flag into its output slot, with running totals carried between chunks.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kT = 1024;
constexpr int kMaxRatios = 4;

// exclusive prefix sum over the workgroup of v (0/1 flags or small counts); returns the
// thread's exclusive sum and writes the total to *total
__device__ __forceinline__ int block_exclusive_scan(int v, int* sh, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  if (tid < 64) {
    int w = tid < kT / 64 ? sh[tid] : 0;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) {
      const int y = __shfl_up(w, d, 64);
      if (tid >= d) w += y;
    }
    if (tid < kT / 64) sh[16 + tid] = w;  // inclusive wave totals
  }
  __syncthreads();
  const int before = wave > 0 ? sh[16 + wave - 1] : 0;
  *total = sh[16 + kT / 64 - 1];
  __syncthreads();  // sh is reused by the next scan
  return before + x - v;
}

template <typename P>
__global__ void __launch_bounds__(kT)
tnd_meta_kernel(const P* __restrict__ pos, int64_t n, const int* __restrict__ ratios, int n_ratios,
                int* __restrict__ counts, int* __restrict__ cu_q, int* __restrict__ block_starts,
                int* __restrict__ cu_cmp, int* __restrict__ residual) {
  __shared__ int sh[32];
  __shared__ int s_nvalid, s_bad;
  const int tid = threadIdx.x;
  // pass 0: the valid prefix (count of positions >= 0; any valid token after padding is an error)
  int cnt = 0, first_pad = 0x7fffffff;
  for (int64_t t = tid; t < n; t += kT) {
    if (pos[t] >= 0) ++cnt;
    else first_pad = min(first_pad, (int)t);
  }
  if (tid == 0) {
    s_nvalid = 0;
    s_bad = 0x7fffffff;
  }
  __syncthreads();
  atomicAdd(&s_nvalid, cnt);
  atomicMin(&s_bad, first_pad);
  __syncthreads();
  const int nv = s_nvalid;
  const bool bad = s_bad < nv;  // padding before the last valid token
  int r_req = 0, r_blk[kMaxRatios] = {0, 0, 0, 0};
  int max_len = 0, max_cmp[kMaxRatios] = {0, 0, 0, 0};
  int prev_start = -1;  // (thread 0) start of the request still open at the chunk boundary
  (void)prev_start;
  for (int64_t c0 = 0; c0 < nv; c0 += kT) {
    const int t = (int)(c0 + tid);
    const bool valid = t < nv;
    const int64_t p = valid ? (int64_t)pos[t] : -1;
    const int st = valid && (t == 0 || p == 0);
    int tot;
    const int req = r_req + block_exclusive_scan(st, sh, &tot);
    if (st) cu_q[req] = t;
    for (int j = 0; j < n_ratios; ++j) {
      const int r = ratios[j];
      int bs = 0;
      if (valid && p % r == 0 && t + r - 1 < nv) bs = (int64_t)pos[t + r - 1] == p + r - 1;
      int totb;
      const int slot = r_blk[j] + block_exclusive_scan(bs, sh, &totb);
      if (bs) block_starts[(int64_t)j * n + slot] = t;
      if (st) cu_cmp[(int64_t)j * (n + 1) + req] = slot;  // blocks before this request's first token
      r_blk[j] += totb;
    }
    r_req += tot;
  }
  __syncthreads();
  // close the lists: cu_q[R] = nv, cu_cmp[R] = total blocks; then lengths and maxima
  if (tid == 0) {
    cu_q[r_req] = nv;
    for (int j = 0; j < n_ratios; ++j) cu_cmp[(int64_t)j * (n + 1) + r_req] = r_blk[j];
  }
  __syncthreads();
  for (int i = tid; i < r_req; i += kT) {
    const int len = cu_q[i + 1] - cu_q[i];
    max_len = max(max_len, len);
    for (int j = 0; j < n_ratios; ++j) {
      const int cl = cu_cmp[(int64_t)j * (n + 1) + i + 1] - cu_cmp[(int64_t)j * (n + 1) + i];
      residual[(int64_t)j * n + i] = len - ratios[j] * cl;
      max_cmp[j] = max(max_cmp[j], cl);
    }
  }
  if (tid == 0) {
    counts[0] = nv;
    counts[1] = r_req;
    counts[2] = 0;
    counts[3] = bad ? 1 : 0;
    for (int j = 0; j < n_ratios; ++j) {
      counts[4 + 2 * j] = r_blk[j];
      counts[5 + 2 * j] = 0;
    }
  }
  __syncthreads();
  atomicMax(&counts[2], max_len);
  for (int j = 0; j < n_ratios; ++j) atomicMax(&counts[5 + 2 * j], max_cmp[j]);
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_tnd_metadata(const void* positions, int pos_dtype_bytes, int64_t n, const int* ratios,
                                int64_t n_ratios, int* counts, int* cu_q, int* block_starts, int* cu_cmp,
                                int* residual, void* stream) {
  using namespace dsa;
  if (!positions || !counts || !cu_q || (n_ratios > 0 && (!ratios || !block_starts || !cu_cmp || !residual)))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_tnd_metadata: null pointer");
  if (n <= 0 || n > INT32_MAX - 1) return set_error(DSA_ERR_INVALID_ARG, "dsa_tnd_metadata: %lld tokens", (long long)n);
  if (n_ratios < 0 || n_ratios > kMaxRatios)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_tnd_metadata: at most %d compression ratios", kMaxRatios);
  if (pos_dtype_bytes != 4 && pos_dtype_bytes != 8)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_tnd_metadata: positions must be int32 or int64");
  hipStream_t st = (hipStream_t)stream;
  if (pos_dtype_bytes == 8)
    tnd_meta_kernel<int64_t><<<1, kT, 0, st>>>((const int64_t*)positions, n, ratios, (int)n_ratios, counts, cu_q,
                                               block_starts, cu_cmp, residual);
  else
    tnd_meta_kernel<int32_t><<<1, kT, 0, st>>>((const int32_t*)positions, n, ratios, (int)n_ratios, counts, cu_q,
                                               block_starts, cu_cmp, residual);
  return check_launch("dsa_tnd_metadata");
}
