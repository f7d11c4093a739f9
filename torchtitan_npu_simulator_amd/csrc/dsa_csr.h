// Key-major CSR of (query row, slot) pairs and the contribution reduction shared by the
// attention backward (dKV, 576 wide) and the indexer KL gradient (dK_index, 128 wide).
//
// The pairs of a query-row chunk are counted per key with LDS-privatised histograms (one
// workgroup per block of query rows and 16384-key range, the ranges of one row block
// adjacent in launch order so they share its index rows in L2) stored as a [row block][key]
// count table; a two-level column scan of that table gives every (row block, key) its
// offset inside the key's list, a scan of the key totals gives row_ptr, and a second pass
// places each row block's pairs at row_ptr + its offset, row by row.  No global atomics are
// issued, and the order of a key's list is the same in every run (rows in order within each
// span of up to 2048 slots; only a key repeated inside one row has its entries for that row
// placed in either order, which top-k output never has).
// The row block grows with the key count (about four pairs per key and workgroup), which
// keeps the count table about the size of the pair list.  The reduction then gives every
// key a single owner that sums its pairs' bf16 contribution rows in fp32 and adds the
// result to the caller's accumulator with plain loads/stores; a key whose list straddles
// reduction segments has each segment's partial sum stored apart and added, in segment
// order, by a fix-up pass.  No float atomics are issued and every sum is taken in a fixed
// order, so the accumulator's result is the same bit for bit in every run.
#pragma once
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kCsrRowsMin = 16;   // query rows per counting workgroup: at least
constexpr int kCsrRowsMax = 512;  // and at most
constexpr int kCsrRowBatch = 8;   // index rows loaded together
constexpr int kLdsKeys = 16384;  // keys privatised in LDS
constexpr int kColChunk = 32;    // row blocks per chunk of the count table's column scan

// query rows per counting workgroup: about four pairs per key of a range
inline int csr_rows_per_wg(int64_t s_kv, int64_t K) {
  const int64_t want = 4 * s_kv / (K > 0 ? K : 1);
  return (int)(want < kCsrRowsMin ? kCsrRowsMin : want > kCsrRowsMax ? kCsrRowsMax : want);
}

__device__ __forceinline__ bool csr_slot_ok(int v, int s_kv, int64_t limit) {
  return v >= 0 && v < s_kv && (int64_t)v <= limit;
}

// Calls f(key - key0, pair) for every valid slot of query rows [r0, r1) whose key lies in
// [key0, key0 + nkeys); the index rows of kCsrRowBatch rows are loaded before any is used.
// kOrdered: a workgroup barrier after each row's calls, so the calls of row r all come
// before those of row r + 1 (every thread of the workgroup must call this).
template <bool kVec, bool kOrdered = false, typename F>
__device__ __forceinline__ void csr_for_pairs(const int32_t* __restrict__ idx, int S, int s_kv, int K, int64_t q_offset,
                                              int row0, int r0, int r1, int b, int key0, int nkeys, F&& f) {
  constexpr int kPer = kVec ? 2 : 8;  // loads per row and chunk (int4 or int)
  constexpr int kW = kVec ? 4 : 1;
  const int t = threadIdx.x;
  for (int lr0 = r0; lr0 < r1; lr0 += kCsrRowBatch) {
    for (int j0 = 0; j0 < K; j0 += 256 * kPer * kW) {
      int v[kCsrRowBatch][kPer][kW];
#pragma unroll
      for (int a = 0; a < kCsrRowBatch; ++a) {
        const int lr = min(lr0 + a, r1 - 1);
        const int32_t* ridx = idx + ((int64_t)b * S + row0 + lr) * K;
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int j = j0 + kW * (t + 256 * u);
          if constexpr (kVec) {
            const int4 w = *reinterpret_cast<const int4*>(ridx + min(j, K - 4));
            v[a][u][0] = w.x, v[a][u][1] = w.y, v[a][u][2] = w.z, v[a][u][3] = w.w;
          } else {
            v[a][u][0] = ridx[min(j, K - 1)];
          }
        }
      }
#pragma unroll
      for (int a = 0; a < kCsrRowBatch; ++a) {
        const int lr = lr0 + a;
        if (lr >= r1) break;  // (uniform over the workgroup)
        const int64_t limit = (int64_t)(row0 + lr) + q_offset;
#pragma unroll
        for (int u = 0; u < kPer; ++u)
#pragma unroll
          for (int e = 0; e < kW; ++e) {
            const int j = j0 + kW * (t + 256 * u) + e;
            const int key = v[a][u][e];
            if (j < K && csr_slot_ok(key, s_kv, limit) && (unsigned)(key - key0) < (unsigned)nkeys)
              f(key - key0, lr * K + j);
          }
        if constexpr (kOrdered) __syncthreads();
      }
    }
  }
}

// Count pass (kFill = false): table[rb][key] = the number of pairs of row block rb with
// that key, for every key of the workgroup's range (zeros included), plain stores.
// Fill pass: a key's pairs of row block rb start at row_ptr[key] + chunk_off[rb / kColChunk]
// [key] + table[rb][key] (the table then holding offsets inside the column chunk) and are
// placed row by row.
template <bool kFill, bool kVec>
__global__ void __launch_bounds__(256)
csr_count_kernel(const int32_t* __restrict__ idx, int* __restrict__ table, const int* __restrict__ chunk_off,
                 const int* __restrict__ row_ptr, int* __restrict__ pairs, int S, int s_kv, int K, int64_t q_offset,
                 int row0, int rows, int b, int n_ranges, int rows_per_wg, int* __restrict__ dup_flag) {
  extern __shared__ int hist[];
  // dup_flag (when given): the count pass clears it; the fill then runs only if the staged
  // fill before it raised it
  if (dup_flag) {
    if (!kFill) {
      if (blockIdx.x == 0 && threadIdx.x == 0) *dup_flag = 0;
    } else if (*dup_flag == 0) {
      return;
    }
  }
  const int rb = blockIdx.x / n_ranges, kr = blockIdx.x - rb * n_ranges;
  const int key0 = kr * kLdsKeys, nkeys = min(kLdsKeys, s_kv - key0);
  const int r0 = rb * rows_per_wg;
  const int r1 = min(rows, r0 + rows_per_wg);
  int* trow = table + (int64_t)rb * s_kv + key0;
  if (!kFill) {
    for (int j = threadIdx.x; j < nkeys; j += 256) hist[j] = 0;
    __syncthreads();
    csr_for_pairs<kVec>(idx, S, s_kv, K, q_offset, row0, r0, r1, b, key0, nkeys,
                        [&](int u, int) { atomicAdd(&hist[u], 1); });
    __syncthreads();
    for (int j = threadIdx.x; j < nkeys; j += 256) trow[j] = hist[j];
    return;
  }
  const int* coff = chunk_off + (int64_t)(rb / kColChunk) * s_kv + key0;
  // The column scan left table[rb][key] = the pairs of the row blocks before rb in its chunk of
  // kColChunk, so where rb + 1 lies in the same chunk, table[rb + 1][key] - table[rb][key] is
  // rb's own count: a row block with no pair in this key range places nothing here and skips
  // the walk over its index rows (a packed batch on global key rows keeps each row's keys in
  // its own sequence; causal rows keep theirs below the row).  The last row block of a chunk
  // always walks.
  const int n_rb = (int)gridDim.x / n_ranges;
  const bool next_in_chunk = (rb + 1) % kColChunk != 0 && rb + 1 < n_rb;
  int any = next_in_chunk ? 0 : 1;
  for (int j = threadIdx.x; j < nkeys; j += 256) {
    const int c = trow[j];
    hist[j] = row_ptr[key0 + j] + coff[j] + c;
    if (next_in_chunk) any |= trow[s_kv + j] - c;
  }
  if (!__syncthreads_or(any)) return;
  csr_for_pairs<kVec, true>(idx, S, s_kv, K, q_offset, row0, r0, r1, b, key0, nkeys,
                            [&](int u, int pair) { pairs[atomicAdd(&hist[u], 1)] = pair; });
}

// Staged fill (key spaces of at most kFillKeys * kFillRangesMax keys): workgroup = kFillRB
// consecutive row blocks of the count pass x a kFillKeys-key range.  A key's pairs from those
// row blocks are contiguous in its list (row blocks in order, rows in order within each),
// starting at row_ptr[key] + chunk_off[rb0 / kColChunk][key] + table[rb0][key].  They are
// staged per key in LDS one aligned 8-pair (32-byte) sector of the list at a time, and a
// sector whose pairs are all this workgroup's leaves as one 32-byte write once its last pair
// is placed; the first sector of a key's run (shared with the run before it) and its last
// open sector go out pair by pair.  Scattered 4-byte stores would each leave L2 as a 32-byte
// write: the lines of a list are evicted before the neighbouring runs reach them.  Each row's
// positions are handed out (LDS atomics) and its pairs staged, then (after a barrier) its
// completed sectors are written, then (after another) the next row may reuse their slots.
// That needs each key at most once per row, which top-k output is; a workgroup that meets a
// key twice in one row raises *dup_flag, and the unstaged fill (csr_count_kernel<true>, which
// runs after this one only when the flag is set) redoes the whole list.
constexpr int kFillKeys = 3584;
constexpr int kFillRangesMax = 4;
constexpr int kFillRB = 4;          // count-pass row blocks per fill workgroup
constexpr int kFillThreads = 512;

template <bool kVec>
__global__ void __launch_bounds__(kFillThreads)
csr_fill_staged_kernel(const int32_t* __restrict__ idx, const int* __restrict__ table,
                       const int* __restrict__ chunk_off, const int* __restrict__ row_ptr, int* __restrict__ pairs,
                       int* __restrict__ dup_flag, int S, int s_kv, int K, int64_t q_offset, int row0, int rows, int b,
                       int n_franges, int rows_per_rb, int n_rb) {
  __shared__ int cur[kFillKeys];             // next list position of each key of the range
  __shared__ int first[kFillKeys];           // the workgroup's first list position of each key
  __shared__ int4 stg[kFillKeys][2];         // the open sector of each key (pair at position & 7)
  __shared__ int seen[kFillKeys];            // the last row (within the workgroup) that placed the key
  __shared__ int dup;
  // the n_franges workgroups of one row group read the same index rows: they run on one XCD
  // (workgroups go to the 8 XCDs round-robin by id), in consecutive dispatch slots, so the
  // rows come from that XCD's L2 after the first read.  Group g runs on XCD g % 8; the grid
  // holds 8 * n_franges * ceil(groups / 8) workgroups and the surplus ones return.
  const int xcd = (int)blockIdx.x % 8, slot = (int)blockIdx.x / 8;
  const int grp = xcd + 8 * (slot / n_franges), kr = slot % n_franges;
  const int rb0 = grp * kFillRB;
  if (rb0 >= n_rb) return;
  const int key0 = kr * kFillKeys, nkeys = min(kFillKeys, s_kv - key0);
  const int r0 = rb0 * rows_per_rb, r1 = min(rows, min(rb0 + kFillRB, n_rb) * rows_per_rb);
  const int t = threadIdx.x;
  {
    const int* trow = table + (int64_t)rb0 * s_kv + key0;
    const int* coff = chunk_off + (int64_t)(rb0 / kColChunk) * s_kv + key0;
    for (int j = t; j < nkeys; j += kFillThreads) {
      const int p0 = row_ptr[key0 + j] + coff[j] + trow[j];
      cur[j] = p0;
      first[j] = p0;
      seen[j] = -1;
    }
    if (t == 0) dup = 0;
  }
  __syncthreads();
  int* const stg_i = reinterpret_cast<int*>(&stg[0][0]);
  constexpr int kW = kVec ? 4 : 1;
  constexpr int kPer = (2048 + kFillThreads * kW - 1) / (kFillThreads * kW);  // loads per row and chunk
  constexpr int kP = kPer * kW;                                                // pairs per thread and row
  for (int lr0 = r0; lr0 < r1; lr0 += kCsrRowBatch) {
    for (int j0 = 0; j0 < K; j0 += kFillThreads * kPer * kW) {
      int v[kCsrRowBatch][kPer][kW];
#pragma unroll
      for (int a = 0; a < kCsrRowBatch; ++a) {
        const int lr = min(lr0 + a, r1 - 1);
        const int32_t* ridx = idx + ((int64_t)b * S + row0 + lr) * K;
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int j = j0 + kW * (t + kFillThreads * u);
          if constexpr (kVec) {
            const int4 w = *reinterpret_cast<const int4*>(ridx + min(j, K - 4));
            v[a][u][0] = w.x, v[a][u][1] = w.y, v[a][u][2] = w.z, v[a][u][3] = w.w;
          } else {
            v[a][u][0] = ridx[min(j, K - 1)];
          }
        }
      }
#pragma unroll
      for (int a = 0; a < kCsrRowBatch; ++a) {
        const int lr = lr0 + a;
        if (lr >= r1) break;  // (uniform over the workgroup)
        const int64_t limit = (int64_t)(row0 + lr) + q_offset;
        const int tag = lr;
        int dk[kP], dp[kP];  // key and position of each pair that completed a sector (else -1)
#pragma unroll
        for (int u = 0; u < kPer; ++u)
#pragma unroll
          for (int e = 0; e < kW; ++e) {
            const int j = j0 + kW * (t + kFillThreads * u) + e;
            const int key = v[a][u][e];
            dk[kW * u + e] = -1;
            if (j < K && csr_slot_ok(key, s_kv, limit) && (unsigned)(key - key0) < (unsigned)nkeys) {
              const int k = key - key0;
              if (atomicExch(&seen[k], tag) == tag) dup = 1;
              const int pos = atomicAdd(&cur[k], 1);
              stg_i[8 * k + (pos & 7)] = lr * K + j;
              if ((pos & 7) == 7) {
                dk[kW * u + e] = k;
                dp[kW * u + e] = pos;
              }
            }
          }
        __syncthreads();  // the row's pairs are staged
        if (dup) {  // (workgroup-uniform) a key twice in one row: the unstaged fill takes over
          if (t == 0) *dup_flag = 1;
          return;
        }
#pragma unroll
        for (int i = 0; i < kP; ++i) {
          const int k = dk[i];
          if (k < 0) continue;
          const int base = dp[i] - 7;
          if (base >= first[k]) {
            int4* dst = reinterpret_cast<int4*>(pairs + base);
            dst[0] = stg[k][0];
            dst[1] = stg[k][1];
          } else {
            for (int q = first[k]; q <= dp[i]; ++q) pairs[q] = stg_i[8 * k + (q & 7)];
          }
        }
        __syncthreads();  // the written sectors' slots may be restaged by the next row
      }
    }
  }
  // each key's open sector: its positions [max(first, end & ~7), end)
  for (int k = t; k < nkeys; k += kFillThreads) {
    const int e = cur[k];
    if ((e & 7) == 0) continue;
    for (int q = max(first[k], e & ~7); q < e; ++q) pairs[q] = stg_i[8 * k + (q & 7)];
  }
}

template <bool kFill>
void launch_csr_count(bool vec, unsigned grid, size_t lds, hipStream_t st, const int32_t* idx, int* table,
                      const int* chunk_off, const int* row_ptr, int* pairs, int S, int s_kv, int K, int64_t q_offset,
                      int row0, int rows, int b, int n_ranges, int rows_per_wg, int* dup_flag) {
  const TimedLaunch tl(kFill ? (dup_flag ? "csr_count_kernel<fill, repair>" : "csr_count_kernel<fill>")
                             : "csr_count_kernel<count>",
                       st);
  if (vec)
    csr_count_kernel<kFill, true><<<grid, 256, lds, st>>>(idx, table, chunk_off, row_ptr, pairs, S, s_kv, K,
                                                          q_offset, row0, rows, b, n_ranges, rows_per_wg, dup_flag);
  else
    csr_count_kernel<kFill, false><<<grid, 256, lds, st>>>(idx, table, chunk_off, row_ptr, pairs, S, s_kv, K,
                                                           q_offset, row0, rows, b, n_ranges, rows_per_wg, dup_flag);
}

// Column scan of the count table, first level: within each chunk of kColChunk row blocks,
// table[rb][key] <- exclusive prefix over the chunk's earlier row blocks, and
// chunk_off[c][key] <- the chunk's total.  One thread per (key, chunk); its loads are
// issued together.
__global__ void __launch_bounds__(256)
csr_colscan_kernel(int* __restrict__ table, int* __restrict__ chunk_off, int s_kv, int n_rb) {
  const int key = blockIdx.x * 256 + threadIdx.x;
  const int c = blockIdx.y;
  if (key >= s_kv) return;
  const int rb0 = c * kColChunk, n = min(kColChunk, n_rb - rb0);
  int* col = table + (int64_t)rb0 * s_kv + key;
  int v[kColChunk];
#pragma unroll
  for (int i = 0; i < kColChunk; ++i) v[i] = i < n ? col[(int64_t)i * s_kv] : 0;
  int run = 0;
#pragma unroll
  for (int i = 0; i < kColChunk; ++i) {
    if (i < n) col[(int64_t)i * s_kv] = run;
    run += v[i];
  }
  chunk_off[(int64_t)c * s_kv + key] = run;
}

// Second level: chunk_off[c][key] <- exclusive prefix over the earlier chunks, and
// counts[key] <- the key's total.  One thread per key.
__global__ void __launch_bounds__(256)
csr_chunkscan_kernel(int* __restrict__ chunk_off, int* __restrict__ counts, int s_kv, int n_chunks) {
  const int key = blockIdx.x * 256 + threadIdx.x;
  if (key >= s_kv) return;
  int run = 0;
  for (int c0 = 0; c0 < n_chunks; c0 += 16) {
    int v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = c0 + i < n_chunks ? chunk_off[(int64_t)(c0 + i) * s_kv + key] : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (c0 + i < n_chunks) chunk_off[(int64_t)(c0 + i) * s_kv + key] = run;
      run += v[i];
    }
  }
  counts[key] = run;
}

// exclusive scan of counts -> row_ptr (s_kv + 1 entries) and cursor = row_ptr; one
// workgroup over tiles of 1024 x 32 counts: thread t loads its 32 consecutive counts of
// the tile at once (int4 loads), the 1024 segment sums are scanned (wave scans + the 16
// wave totals), and each thread writes its segment's prefixes; a carry crosses tiles.
constexpr int kScanPer = 32;
__global__ void __launch_bounds__(1024) csr_scan_kernel(const int* __restrict__ counts, int* __restrict__ row_ptr,
                                                        int* __restrict__ cursor, int s_kv) {
  __shared__ int wsum[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool vec = ((uintptr_t)counts % 16) == 0;
  int carry = 0;
  for (int base = 0; base < s_kv; base += 1024 * kScanPer) {
    const int j0 = base + kScanPer * t;
    int v[kScanPer];
    if (vec && j0 + kScanPer <= s_kv) {
#pragma unroll
      for (int u = 0; u < kScanPer / 4; ++u) {
        const int4 w = *reinterpret_cast<const int4*>(counts + j0 + 4 * u);
        v[4 * u] = w.x, v[4 * u + 1] = w.y, v[4 * u + 2] = w.z, v[4 * u + 3] = w.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kScanPer; ++u) v[u] = j0 + u < s_kv ? counts[j0 + u] : 0;
    }
    int sum = 0;
#pragma unroll
    for (int u = 0; u < kScanPer; ++u) sum += v[u];
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int run = carry + incl - sum;
    int tile_total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      if (w < wave) run += wsum[w];
      tile_total += wsum[w];
    }
#pragma unroll
    for (int u = 0; u < kScanPer; ++u) {
      if (j0 + u < s_kv) {
        row_ptr[j0 + u] = run;
        if (cursor) cursor[j0 + u] = run;
      }
      run += v[u];
    }
    carry += tile_total;
    __syncthreads();  // wsum is rewritten by the next tile
  }
  if (t == 0) row_ptr[s_kv] = carry;
}

// acc[key] += sum over the key's pairs of bf16 contribution rows of kChunks 16-byte chunks.
// The key-sorted pair list is cut into segments of kSegPairs pairs, one wave each, so a
// key selected by thousands of rows (the causal prefix) is summed by many waves instead of
// one; seg_key[s] names the key holding pair s * kSegPairs.  A wave walks its segment in
// groups of 8 pairs (indices through scalar loads, all 8 rows loaded before any is summed)
// and flushes its partial sum whenever the key changes: with a plain read-add-write if the
// key lies wholly inside the segment (sole owner), else into the segment's partial-sum slot
// (only keys that straddle a segment boundary, at most two per segment), which the fix-up
// pass adds in segment order.  The contribution rows are read once and never again, so
// they are loaded non-temporally (nt), which keeps them from displacing the accumulator
// and the pair list in the caches (≈6 % faster on the 576-wide rows).
// 576-wide rows (72 chunks): lane l owns chunk l, and chunk 64 + (l & 7) is loaded by every
// lane (one 128-byte line per instruction) and stored by lanes 0..7; 512-wide rows (64
// chunks): lane l owns chunk l.  128-wide rows
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
// sole owner: d += acc (read-add-write); a straddling key's segment partial: d = acc
__device__ __forceinline__ void flush8(float* d, float (&acc)[8], bool sole) {
  float4* d4 = reinterpret_cast<float4*>(d);
  float4 x = make_float4(acc[0], acc[1], acc[2], acc[3]), y = make_float4(acc[4], acc[5], acc[6], acc[7]);
  if (sole) {
    const float4 a = d4[0], c = d4[1];
    x.x += a.x; x.y += a.y; x.z += a.z; x.w += a.w;
    y.x += c.x; y.y += c.y; y.z += c.z; y.w += c.w;
  }
  d4[0] = x;
  d4[1] = y;
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
                  const int* __restrict__ seg_key, float* __restrict__ acc_out, float* __restrict__ part, int s_kv,
                  int rows, int K, int b) {
  static_assert(kChunks == 72 || kChunks == 64 || kChunks == 16, "row widths of the attention and indexer reductions");
  constexpr int kWidth = kChunks * 8;
  constexpr int kGroup = kChunks == 16 ? 16 : 8;  // pairs per load group (16-chunk rows: four per load)
  const int seg = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n_pairs = row_ptr[s_kv];
  const int seg0 = seg * kSegPairs;
  if (seg0 >= n_pairs) return;
  const int seg1 = min(seg0 + kSegPairs, n_pairs);
  const uint16_t* cb = cbuf + (int64_t)b * rows * K * kWidth;
  float* dbase = acc_out + (int64_t)b * s_kv * kWidth;
  int k = seg_key[seg];
  const int k_first = k;
  int kbeg = row_ptr[k], kend = row_ptr[k + 1];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float acc2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // 72-chunk rows: chunk 64 + (lane & 7)
  const int stream = lane >> 4, c16 = lane & 15;               // 16-chunk rows
  auto flush = [&]() {
    // a straddling key is the segment's first key (partial slot 0) or its last (slot 1)
    const bool sole = kbeg >= seg0 && kend <= seg1;
    float* d = sole ? dbase + (int64_t)k * kWidth : part + ((int64_t)seg * 2 + (k == k_first ? 0 : 1)) * kWidth;
    if constexpr (kChunks >= 64) {
      flush8(d + 8 * lane, acc, sole);
      if constexpr (kChunks == 72) {
        if (lane < kChunks - 64) flush8(d + 512 + 8 * lane, acc2, sole);
        else
#pragma unroll
          for (int r = 0; r < 8; ++r) acc2[r] = 0.f;
      }
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
    if constexpr (kChunks >= 64) {
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const uint16_t* row = cb + (int64_t)pr[u] * kWidth;
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + 8 * lane));
        if constexpr (kChunks == 72) w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + 512 + 8 * (lane & 7)));
      }
    } else {
#pragma unroll
      for (int u = 0; u < kGroup / 4; ++u) {
        const int mine = stream == 0 ? pr[4 * u] : stream == 1 ? pr[4 * u + 1] : stream == 2 ? pr[4 * u + 2] : pr[4 * u + 3];
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cb + (int64_t)mine * kWidth + 8 * c16));
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
      if constexpr (kChunks >= 64) {
        add_bf16x8(acc, v[u]);
        if constexpr (kChunks == 72) add_bf16x8(acc2, w[u]);
      } else {
        // four pairs per load group: stream s adds its row when q is pair 4 (u / 4) + s
        if (stream == (u & 3)) add_bf16x8(acc, v[u >> 2]);
      }
    }
  }
  flush();
}

// A straddling key: acc_out[k] += its segments' partial sums, in segment order (partial slot
// 0 where k is the segment's first key, else slot 1).  One wave per key.
template <int kWidth>
__global__ void __launch_bounds__(256)
csr_partial_fixup_kernel(const int* __restrict__ row_ptr, const int* __restrict__ seg_key,
                         const float* __restrict__ part, float* __restrict__ acc_out, int s_kv, int b) {
  const int k = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (k >= s_kv) return;
  const int kbeg = row_ptr[k], kend = row_ptr[k + 1];
  if (kend <= kbeg) return;
  const int s0 = kbeg / kSegPairs, s1 = (kend - 1) / kSegPairs;
  if (s0 == s1) return;  // inside one segment: its owner added it
  constexpr int kPer = kWidth / 64;
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
  for (int sg = s0; sg <= s1; ++sg) {
    const float* src = part + ((int64_t)sg * 2 + (seg_key[sg] == k ? 0 : 1)) * kWidth;
#pragma unroll
    for (int i = 0; i < kPer; ++i) acc[i] += src[lane + 64 * i];
  }
  float* d = acc_out + ((int64_t)b * s_kv + k) * kWidth;
#pragma unroll
  for (int i = 0; i < kPer; ++i) d[lane + 64 * i] += acc[i];
}

// Bytes of the CSR workspace csr_reduce needs for contribution rows of `width` floats:
// counts and row_ptr (s_kv + 1 ints each), the segment table (one int per kSegPairs pairs
// of the chunk), the [row block][key] count table, the [column chunk][key] chunk offsets
// and two partial-sum rows per segment (at a 16-byte boundary).
inline int64_t csr_ws_ints(int64_t s_kv, int64_t rows, int64_t K) {
  const int64_t n_rb = (rows + csr_rows_per_wg(s_kv, K) - 1) / csr_rows_per_wg(s_kv, K);
  const int64_t n_chunks = (n_rb + kColChunk - 1) / kColChunk;
  const int64_t n_seg = (rows * K + kSegPairs - 1) / kSegPairs;
  return (2 * (s_kv + 1) + n_seg + (n_rb + n_chunks) * s_kv + 3) / 4 * 4 + 4;  // (+4: the fill's dup flag last)
}
inline int64_t csr_part_bytes(int64_t rows, int64_t K, int64_t width) {
  return (rows * K + kSegPairs - 1) / kSegPairs * 2 * width * 4;
}
inline int64_t csr_ws_bytes(int64_t s_kv, int64_t rows, int64_t K, int64_t width) {
  return csr_ws_ints(s_kv, rows, K) * 4 + csr_part_bytes(rows, K, width);
}

// A built CSR: the key-sorted pair list with its key pointers and segment table.
struct CsrView {
  const int* pairs;
  const int* row_ptr;
  const int* seg_key;
};

// Build the CSR of query rows [row0, row0 + rows) of batch element b: `pairs` holds
// rows * K ints, csr_ws csr_ws_ints(s_kv, rows, K) ints.
inline int csr_build(const int32_t* idx, int* pairs, int* csr_ws, int S, int s_kv, int K, int64_t q_offset, int row0,
                     int rows, int b, hipStream_t st, CsrView* view) {
  const int rows_per_wg = csr_rows_per_wg(s_kv, K);
  const int64_t n_rb = ceil_div(rows, rows_per_wg);
  const int64_t n_chunks = ceil_div(n_rb, kColChunk);
  int* counts = csr_ws;
  int* row_ptr = counts + (s_kv + 1);
  int* seg_key = row_ptr + (s_kv + 1);
  const int64_t n_seg = ceil_div((int64_t)rows * K, kSegPairs);
  int* table = seg_key + n_seg;
  int* chunk_off = table + n_rb * s_kv;
  const int n_ranges = (int)ceil_div(s_kv, kLdsKeys);
  const size_t hist_bytes = (size_t)(s_kv < kLdsKeys ? s_kv : kLdsKeys) * 4;
  const int64_t cgrid = n_rb * (int64_t)n_ranges;
  if (cgrid > 2147483647LL || n_chunks > 65535)
    return set_error(DSA_ERR_INVALID_ARG, "csr_reduce: too many rows x keys");
  const int64_t row_base = (int64_t)b * S + row0;  // int4 loads need 16-byte aligned index rows
  const bool vec = K % 4 == 0 && ((uintptr_t)(idx + row_base * K) % 16) == 0;
  const int n_franges = (int)ceil_div(s_kv, kFillKeys);
  const bool staged = n_franges <= kFillRangesMax;
  int* dup_flag = staged ? csr_ws + csr_ws_ints(s_kv, rows, K) - 1 : nullptr;
  launch_csr_count<false>(vec, (unsigned)cgrid, hist_bytes, st, idx, table, nullptr, nullptr, pairs, S, s_kv, K,
                          q_offset, row0, rows, b, n_ranges, rows_per_wg, dup_flag);
  {
    const TimedLaunch tl("csr_colscan_kernel", st);
    csr_colscan_kernel<<<dim3((unsigned)ceil_div(s_kv, 256), (unsigned)n_chunks), 256, 0, st>>>(table, chunk_off,
                                                                                                 s_kv, (int)n_rb);
  }
  {
    const TimedLaunch tl("csr_chunkscan_kernel", st);
    csr_chunkscan_kernel<<<(unsigned)ceil_div(s_kv, 256), 256, 0, st>>>(chunk_off, counts, s_kv, (int)n_chunks);
  }
  {
    const TimedLaunch tl("csr_scan_kernel", st);
    csr_scan_kernel<<<1, 1024, 0, st>>>(counts, row_ptr, nullptr, s_kv);
  }
  if (staged) {
    const unsigned fgrid = (unsigned)(8 * n_franges * ceil_div(ceil_div(n_rb, kFillRB), 8));
    {
      const TimedLaunch tl("csr_fill_staged_kernel", st);
      if (vec)
        csr_fill_staged_kernel<true><<<fgrid, kFillThreads, 0, st>>>(idx, table, chunk_off, row_ptr, pairs, dup_flag, S,
                                                                    s_kv, K, q_offset, row0, rows, b, n_franges,
                                                                    rows_per_wg, (int)n_rb);
      else
        csr_fill_staged_kernel<false><<<fgrid, kFillThreads, 0, st>>>(idx, table, chunk_off, row_ptr, pairs, dup_flag,
                                                                     S, s_kv, K, q_offset, row0, rows, b, n_franges,
                                                                     rows_per_wg, (int)n_rb);
    }
    // (returns at once unless a key repeated inside a row made the staged fill give up)
    launch_csr_count<true>(vec, (unsigned)cgrid, hist_bytes, st, idx, table, chunk_off, row_ptr, pairs, S, s_kv, K,
                           q_offset, row0, rows, b, n_ranges, rows_per_wg, dup_flag);
  } else {
    launch_csr_count<true>(vec, (unsigned)cgrid, hist_bytes, st, idx, table, chunk_off, row_ptr, pairs, S, s_kv, K,
                           q_offset, row0, rows, b, n_ranges, rows_per_wg, nullptr);
  }
  {
    const TimedLaunch tl("csr_seg_key_kernel", st);
    csr_seg_key_kernel<<<ceil_div(s_kv, 256), 256, 0, st>>>(row_ptr, seg_key, s_kv);
  }
  view->pairs = pairs;
  view->row_ptr = row_ptr;
  view->seg_key = seg_key;
  return check_launch("csr_reduce(build)");
}

// Reduce the contribution rows cbuf[b][row][slot][8 * row_chunks] of the rows a built CSR
// covers into acc_out[b][key][...]; `part` holds csr_part_bytes(rows, K, 8 * row_chunks).
inline int csr_reduce_built(const CsrView& v, const uint16_t* cbuf, float* acc_out, float* part, int s_kv, int rows,
                            int K, int b, int row_chunks, hipStream_t st) {
  const unsigned rgrid = ceil_div(ceil_div((int64_t)rows * K, kSegPairs), 4);
  const TimedLaunch tl(row_chunks == 72   ? "dkv_reduce_kernel<72>"
                       : row_chunks == 64 ? "dkv_reduce_kernel<64>"
                                          : "dkv_reduce_kernel<16>",
                       st);
  if (row_chunks == 72)
    dkv_reduce_kernel<72><<<rgrid, 256, 0, st>>>(cbuf, v.row_ptr, v.pairs, v.seg_key, acc_out, part, s_kv, rows, K, b);
  else if (row_chunks == 64)
    dkv_reduce_kernel<64><<<rgrid, 256, 0, st>>>(cbuf, v.row_ptr, v.pairs, v.seg_key, acc_out, part, s_kv, rows, K, b);
  else if (row_chunks == 16)
    dkv_reduce_kernel<16><<<rgrid, 256, 0, st>>>(cbuf, v.row_ptr, v.pairs, v.seg_key, acc_out, part, s_kv, rows, K, b);
  else
    return set_error(DSA_ERR_UNSUPPORTED, "csr_reduce: row width %d chunks", row_chunks);
  if (int rc = check_launch("csr_reduce")) return rc;
  {
    const TimedLaunch tl2("csr_partial_fixup_kernel", st);
    const unsigned fgrid = (unsigned)ceil_div(s_kv, 4);
    if (row_chunks == 72)
      csr_partial_fixup_kernel<576><<<fgrid, 256, 0, st>>>(v.row_ptr, v.seg_key, part, acc_out, s_kv, b);
    else if (row_chunks == 64)
      csr_partial_fixup_kernel<512><<<fgrid, 256, 0, st>>>(v.row_ptr, v.seg_key, part, acc_out, s_kv, b);
    else
      csr_partial_fixup_kernel<128><<<fgrid, 256, 0, st>>>(v.row_ptr, v.seg_key, part, acc_out, s_kv, b);
  }
  return check_launch("csr_reduce(fix-up)");
}

// Build the CSR for query rows [row0, row0 + rows) of batch element b and reduce the
// contribution rows cbuf[b][row][slot][8 * row_chunks] into acc_out[b][key][...].
// csr_ws holds csr_ws_bytes(s_kv, rows, K) bytes.
inline int csr_reduce(const int32_t* idx, const uint16_t* cbuf, float* acc_out, int* pairs, int* csr_ws, int S,
                      int s_kv, int K, int64_t q_offset, int row0, int rows, int b, int row_chunks, hipStream_t st) {
  if (s_kv <= 0 || rows <= 0) return DSA_OK;  // no pairs: the accumulator keeps its contents
  CsrView v;
  if (int rc = csr_build(idx, pairs, csr_ws, S, s_kv, K, q_offset, row0, rows, b, st, &v)) return rc;
  float* part = reinterpret_cast<float*>(csr_ws + csr_ws_ints(s_kv, rows, K));
  return csr_reduce_built(v, cbuf, acc_out, part, s_kv, rows, K, b, row_chunks, st);
}

// A prebuilt CSR of every query row of every batch element, shared by the reductions of one
// index tensor (the attention backward's dKV and the indexer KL op's dK_index): per batch
// element, rows * K pair ints then csr_ws_ints of key pointers, segment table and the build's
// scratch tables.
inline int64_t pair_csr_batch_ints(int64_t s_kv, int64_t rows, int64_t K) {
  return (rows * K + 3) / 4 * 4 + csr_ws_ints(s_kv, rows, K);
}
inline int64_t pair_csr_bytes_of(int64_t batch, int64_t s_q, int64_t s_kv, int64_t K) {
  return batch * pair_csr_batch_ints(s_kv, s_q, K) * 4;
}
inline CsrView pair_csr_view(const void* csr, int64_t s_kv, int64_t rows, int64_t K, int b) {
  const int* base = reinterpret_cast<const int*>(csr) + (int64_t)b * pair_csr_batch_ints(s_kv, rows, K);
  const int* ws = base + (rows * K + 3) / 4 * 4;
  CsrView v;
  v.pairs = base;
  v.row_ptr = ws + (s_kv + 1);
  v.seg_key = ws + 2 * (s_kv + 1);
  return v;
}

}  // namespace
}  // namespace dsa
