// Key-major CSR of (query row, slot) pairs and the contribution reduction shared by the
// attention backward (dKV, 576 wide) and the indexer KL gradient (dK_index, 128 wide).
//
// The pairs of a query-row chunk are counted per key with LDS-privatised histograms
// (keys <= 16384; plain global atomics beyond), scanned into row_ptr, and placed by a
// second pass that reserves one contiguous range per (workgroup, key).  The reduction
// then gives every key a single owner that sums its pairs' bf16 contribution rows in
// fp32 and adds the result to the caller's accumulator with plain loads/stores, so no
// float atomics are issued.  Order within a key's list varies run to run, so fp32 sums
// may differ in the last bits between runs.
#pragma once
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kCsrRows = 16;     // query rows per counting workgroup
constexpr int kLdsKeys = 16384;  // keys privatised in LDS

__device__ __forceinline__ bool csr_slot_ok(int v, int s_kv, int64_t limit) {
  return v >= 0 && v < s_kv && (int64_t)v <= limit;
}

template <bool kFill>
__global__ void __launch_bounds__(256)
csr_count_kernel(const int32_t* __restrict__ idx, int* __restrict__ counts, int* __restrict__ cursor,
                 int* __restrict__ pairs, int S, int s_kv, int K, int64_t q_offset, int row0, int rows, int b) {
  extern __shared__ int hist[];
  const bool priv = s_kv <= kLdsKeys;
  const int r0 = blockIdx.x * kCsrRows;
  const int r1 = min(rows, r0 + kCsrRows);
  if (priv) {
    for (int j = threadIdx.x; j < s_kv; j += 256) hist[j] = 0;
    __syncthreads();
  }
  for (int lr = r0; lr < r1; ++lr) {
    const int tok = row0 + lr;
    const int32_t* ridx = idx + ((int64_t)b * S + tok) * K;
    const int64_t limit = tok + q_offset;
    for (int j = threadIdx.x; j < K; j += 256) {
      const int v = ridx[j];
      if (!csr_slot_ok(v, s_kv, limit)) continue;
      if (!kFill) {
        if (priv) atomicAdd(&hist[v], 1);
        else atomicAdd(&counts[v], 1);
      } else if (!priv) {
        const int pos = atomicAdd(&cursor[v], 1);
        pairs[pos] = lr * K + j;
      } else {
        atomicAdd(&hist[v], 1);
      }
    }
  }
  if (!priv) return;
  __syncthreads();
  if (!kFill) {
    for (int j = threadIdx.x; j < s_kv; j += 256)
      if (hist[j]) atomicAdd(&counts[j], hist[j]);
    return;
  }
  // fill: reserve this workgroup's range per key, then place pairs
  for (int j = threadIdx.x; j < s_kv; j += 256) {
    const int c = hist[j];
    hist[j] = c ? atomicAdd(&cursor[j], c) : 0;
  }
  __syncthreads();
  for (int lr = r0; lr < r1; ++lr) {
    const int tok = row0 + lr;
    const int32_t* ridx = idx + ((int64_t)b * S + tok) * K;
    const int64_t limit = tok + q_offset;
    for (int j = threadIdx.x; j < K; j += 256) {
      const int v = ridx[j];
      if (!csr_slot_ok(v, s_kv, limit)) continue;
      const int pos = atomicAdd(&hist[v], 1);
      pairs[pos] = lr * K + j;
    }
  }
}

__global__ void zero_i32_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// exclusive scan of counts -> row_ptr (s_kv + 1 entries) and cursor = row_ptr; one workgroup
__global__ void __launch_bounds__(1024) csr_scan_kernel(const int* __restrict__ counts, int* __restrict__ row_ptr,
                                                        int* __restrict__ cursor, int s_kv) {
  __shared__ int buf[1024];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < s_kv; base += 1024) {
    const int j = base + threadIdx.x;
    const int v = j < s_kv ? counts[j] : 0;
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int add = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
      __syncthreads();
      buf[threadIdx.x] += add;
      __syncthreads();
    }
    const int excl = carry + buf[threadIdx.x] - v;
    if (j < s_kv) {
      row_ptr[j] = excl;
      cursor[j] = excl;
    }
    __syncthreads();
    if (threadIdx.x == 1023) carry += buf[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) row_ptr[s_kv] = carry;
}

// acc[key] += sum over the key's pairs of bf16 contribution rows of kChunks 16-byte chunks.
// The key-sorted pair list is cut into segments of kSegPairs pairs, one wave each, so a
// key selected by thousands of rows (the causal prefix) is summed by many waves instead of
// one; seg_key[s] names the key holding pair s * kSegPairs.  A wave walks its segment in
// groups of 8 pairs (indices through scalar loads, all 8 rows loaded before any is summed)
// and flushes its partial sum whenever the key changes: with a plain read-add-write if the
// key lies wholly inside the segment (sole owner), else with fp32 atomic adds (only keys
// that straddle a segment boundary, at most two partial sums per segment).
// 576-wide rows (72 chunks): lane l owns chunk l, and chunk 64 + (l & 7) is loaded by every
// lane (one 128-byte line per instruction) and stored by lanes 0..7.  128-wide rows
// (16 chunks): lanes 16s .. 16s+15 own the row of pair 4g + s of each group of 4 (four
// streams), combined with two lane exchanges at the flush.
constexpr int kSegPairs = 256;

__device__ __forceinline__ void add_bf16x8(float (&acc)[8], const u32x4& v) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    acc[2 * r] += bf16_lo(v[r]);
    acc[2 * r + 1] += bf16_hi(v[r]);
  }
}
__device__ __forceinline__ void flush8(float* d, float (&acc)[8], bool sole) {
  if (sole) {
    float4* d4 = reinterpret_cast<float4*>(d);
    float4 x = d4[0], y = d4[1];
    x.x += acc[0]; x.y += acc[1]; x.z += acc[2]; x.w += acc[3];
    y.x += acc[4]; y.y += acc[5]; y.z += acc[6]; y.w += acc[7];
    d4[0] = x;
    d4[1] = y;
  } else {
#pragma unroll
    for (int r = 0; r < 8; ++r) atomicAdd(d + r, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) acc[r] = 0.f;
}

// seg_key[s] = the key k with row_ptr[k] <= s * kSegPairs < row_ptr[k + 1]
__global__ void __launch_bounds__(256)
csr_seg_key_kernel(const int* __restrict__ row_ptr, int* __restrict__ seg_key, int s_kv) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= s_kv) return;
  const int s0 = (row_ptr[k] + kSegPairs - 1) / kSegPairs, s1 = (row_ptr[k + 1] + kSegPairs - 1) / kSegPairs;
  for (int s = s0; s < s1; ++s) seg_key[s] = k;
}

template <int kChunks>
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const uint16_t* __restrict__ cbuf, const int* __restrict__ row_ptr, const int* __restrict__ pairs,
                  const int* __restrict__ seg_key, float* __restrict__ acc_out, int s_kv, int rows, int K, int b) {
  static_assert(kChunks == 72 || kChunks == 16, "row widths of the attention and indexer reductions");
  constexpr int kWidth = kChunks * 8;
  constexpr int kGroup = 8;
  const int seg = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n_pairs = row_ptr[s_kv];
  const int seg0 = seg * kSegPairs;
  if (seg0 >= n_pairs) return;
  const int seg1 = min(seg0 + kSegPairs, n_pairs);
  const uint16_t* cb = cbuf + (int64_t)b * rows * K * kWidth;
  float* dbase = acc_out + (int64_t)b * s_kv * kWidth;
  int k = seg_key[seg];
  int kbeg = row_ptr[k], kend = row_ptr[k + 1];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float acc2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // 72-chunk rows: chunk 64 + (lane & 7)
  const int stream = lane >> 4, c16 = lane & 15;               // 16-chunk rows
  auto flush = [&]() {
    const bool sole = kbeg >= seg0 && kend <= seg1;
    float* d = dbase + (int64_t)k * kWidth;
    if constexpr (kChunks == 72) {
      flush8(d + 8 * lane, acc, sole);
      if (lane < kChunks - 64) flush8(d + 512 + 8 * lane, acc2, sole);
      else
#pragma unroll
        for (int r = 0; r < 8; ++r) acc2[r] = 0.f;
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = xor32_sum(xor16_sum(acc[r]));
      if (lane < 16) flush8(d + 8 * c16, acc, sole);
      else
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[r] = 0.f;
    }
  };
  for (int p = seg0; p < seg1; p += kGroup) {
    int pr[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) pr[u] = pairs[min(p + u, seg1 - 1)];
    u32x4 v[kGroup], w[kGroup];
    if constexpr (kChunks == 72) {
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const uint16_t* row = cb + (int64_t)pr[u] * kWidth;
        v[u] = *reinterpret_cast<const u32x4*>(row + 8 * lane);
        w[u] = *reinterpret_cast<const u32x4*>(row + 512 + 8 * (lane & 7));
      }
    } else {
#pragma unroll
      for (int u = 0; u < kGroup / 4; ++u) {
        const int mine = stream == 0 ? pr[4 * u] : stream == 1 ? pr[4 * u + 1] : stream == 2 ? pr[4 * u + 2] : pr[4 * u + 3];
        v[u] = *reinterpret_cast<const u32x4*>(cb + (int64_t)mine * kWidth + 8 * c16);
      }
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int q = p + u;
      if (q >= seg1) break;
      while (q >= kend) {  // key change (keys without pairs are stepped over)
        if (kend > kbeg) flush();
        ++k;
        kbeg = kend;
        kend = row_ptr[k + 1];
      }
      if constexpr (kChunks == 72) {
        add_bf16x8(acc, v[u]);
        add_bf16x8(acc2, w[u]);
      } else {
        // four pairs per load group: stream s adds its row when q is pair 4 (u / 4) + s
        if (stream == (u & 3)) add_bf16x8(acc, v[u >> 2]);
      }
    }
  }
  flush();
}

// Bytes of the CSR workspace csr_reduce needs: counts, row_ptr, cursor (s_kv + 1 ints
// each) and the segment table (one int per kSegPairs pairs of the chunk).
inline int64_t csr_ws_bytes(int64_t s_kv, int64_t rows, int64_t K) {
  return (3 * (s_kv + 1) + (rows * K + kSegPairs - 1) / kSegPairs) * 4;
}

// Build the CSR for query rows [row0, row0 + rows) of batch element b and reduce the
// contribution rows cbuf[b][row][slot][8 * row_chunks] into acc_out[b][key][...].
// csr_ws holds csr_ws_bytes(s_kv, rows, K) bytes.
inline int csr_reduce(const int32_t* idx, const uint16_t* cbuf, float* acc_out, int* pairs, int* csr_ws, int S,
                      int s_kv, int K, int64_t q_offset, int row0, int rows, int b, int row_chunks, hipStream_t st) {
  int* counts = csr_ws;
  int* row_ptr = counts + (s_kv + 1);
  int* cursor = row_ptr + (s_kv + 1);
  int* seg_key = cursor + (s_kv + 1);
  const size_t hist_bytes = s_kv <= kLdsKeys ? (size_t)s_kv * 4 : 0;
  zero_i32_kernel<<<ceil_div(s_kv + 1, 256), 256, 0, st>>>(counts, s_kv + 1);
  const unsigned cgrid = ceil_div(rows, kCsrRows);
  csr_count_kernel<false><<<cgrid, 256, hist_bytes, st>>>(idx, counts, cursor, pairs, S, s_kv, K, q_offset, row0,
                                                          rows, b);
  csr_scan_kernel<<<1, 1024, 0, st>>>(counts, row_ptr, cursor, s_kv);
  csr_count_kernel<true><<<cgrid, 256, hist_bytes, st>>>(idx, counts, cursor, pairs, S, s_kv, K, q_offset, row0, rows,
                                                         b);
  csr_seg_key_kernel<<<ceil_div(s_kv, 256), 256, 0, st>>>(row_ptr, seg_key, s_kv);
  const unsigned rgrid = ceil_div(ceil_div((int64_t)rows * K, kSegPairs), 4);
  if (row_chunks == 72)
    dkv_reduce_kernel<72><<<rgrid, 256, 0, st>>>(cbuf, row_ptr, pairs, seg_key, acc_out, s_kv, rows, K, b);
  else if (row_chunks == 16)
    dkv_reduce_kernel<16><<<rgrid, 256, 0, st>>>(cbuf, row_ptr, pairs, seg_key, acc_out, s_kv, rows, K, b);
  else
    return set_error(DSA_ERR_UNSUPPORTED, "csr_reduce: row width %d chunks", row_chunks);
  return check_launch("csr_reduce");
}

}  // namespace
}  // namespace dsa
