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

// acc[key] += sum over the key's pairs of bf16 contribution rows (row_chunks x 8 values);
// 2 keys per workgroup, one thread per 16-byte chunk of the row
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const uint16_t* __restrict__ cbuf, const int* __restrict__ row_ptr, const int* __restrict__ pairs,
                  float* __restrict__ acc_out, int s_kv, int rows, int K, int b, int row_chunks) {
  const int key = blockIdx.x * 2 + (threadIdx.x >> 7);
  const int c = threadIdx.x & 127;
  if (key >= s_kv || c >= row_chunks) return;
  const int p0 = row_ptr[key], p1 = row_ptr[key + 1];
  if (p0 == p1) return;
  const int width = row_chunks * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint16_t* cb = cbuf + (int64_t)b * rows * K * width;
  int p = p0;
  for (; p + 4 <= p1; p += 4) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const u32x4*>(cb + (int64_t)pairs[p + u] * width + 8 * c);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[2 * r] += bf16_lo(v[u][r]);
        acc[2 * r + 1] += bf16_hi(v[u][r]);
      }
  }
  for (; p < p1; ++p) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(cb + (int64_t)pairs[p] * width + 8 * c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[2 * r] += bf16_lo(v[r]);
      acc[2 * r + 1] += bf16_hi(v[r]);
    }
  }
  float* d = acc_out + ((int64_t)b * s_kv + key) * width + 8 * c;
#pragma unroll
  for (int r = 0; r < 8; ++r) d[r] += acc[r];
}

// Build the CSR for query rows [row0, row0 + rows) of batch element b and reduce the
// contribution rows cbuf[b][row][slot][8 * row_chunks] into acc_out[b][key][...].
// csr_ws holds counts, row_ptr and cursor (3 x (s_kv + 1) ints).
inline int csr_reduce(const int32_t* idx, const uint16_t* cbuf, float* acc_out, int* pairs, int* csr_ws, int S,
                      int s_kv, int K, int64_t q_offset, int row0, int rows, int b, int row_chunks, hipStream_t st) {
  int* counts = csr_ws;
  int* row_ptr = counts + (s_kv + 1);
  int* cursor = row_ptr + (s_kv + 1);
  const size_t hist_bytes = s_kv <= kLdsKeys ? (size_t)s_kv * 4 : 0;
  zero_i32_kernel<<<ceil_div(s_kv + 1, 256), 256, 0, st>>>(counts, s_kv + 1);
  const unsigned cgrid = ceil_div(rows, kCsrRows);
  csr_count_kernel<false><<<cgrid, 256, hist_bytes, st>>>(idx, counts, cursor, pairs, S, s_kv, K, q_offset, row0,
                                                          rows, b);
  csr_scan_kernel<<<1, 1024, 0, st>>>(counts, row_ptr, cursor, s_kv);
  csr_count_kernel<true><<<cgrid, 256, hist_bytes, st>>>(idx, counts, cursor, pairs, S, s_kv, K, q_offset, row0, rows,
                                                         b);
  dkv_reduce_kernel<<<ceil_div(s_kv, 2), 256, 0, st>>>(cbuf, row_ptr, pairs, acc_out, s_kv, rows, K, b, row_chunks);
  return check_launch("csr_reduce");
}

}  // namespace
}  // namespace dsa
