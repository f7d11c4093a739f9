// Per-row top-k select: radix select on orderable uint32 keys with range-adaptive 11-bit
// digits, followed by a stable compaction that emits the chosen indices in ascending order.
//
// Contract (bit-exact): row (b, s) considers t < n_valid = min(s_k, (s + q_offset + 1) /
// cmp_ratio) whose score is not NaN; it keeps the first k of a stable descending order by
// (score, lower index) with -0.0 == +0.0.  Only the valid prefix of a row is read.
//
// One 256-thread workgroup per row.  A row is read in segments of 1024·kR scores: thread t
// holds float4 chunks j = 0..kR-1 at positions 4(t + 256 j), so a segment is one coalesced
// sweep and index order is (segment, j, thread, element).  The scores become order keys
// once, as they are loaded; rows of one segment stay in registers for every pass, longer
// rows are re-read per pass (from L2 / MALL).  A chunk that starts past the row's valid
// prefix (causal rows) is skipped by the whole workgroup, in every pass.
//   (a row with at most k valid positions takes every candidate: no pass)
//   pass 0   count of candidates, min and max key
//   pass 1.. histogram of the next 11 bits of (key - min) below the current bin; the bin
//            holding the k-th largest key becomes the new prefix.  Digits start at the
//            highest set bit of (max - min), so clustered scores (all of one exponent)
//            spread over the bins from the first pass on.  Stops when the bin's keys are
//            exactly the remaining quota or the bin is a single key value.
//   compact  key > T is taken; key == T is taken for the first need_eq such keys in index
//            order.  Output position = (#taken-above before it) + min(#equal before it,
//            need_eq), from wave ballots and per-(wave, chunk) totals (the key == T ballots
//            only when the threshold has ties).
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kDigitBits = 11;
constexpr int kBins = 1 << kDigitBits;
constexpr int kBinsPerThread = kBins / kThreads;

__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0u;  // NaN (and masked positions): not a candidate; key 0 is below every real key
  const uint32_t u = __float_as_uint(x + 0.0f);  // -0.0 -> +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// the least float f with order_key(f) >= T, for 1 <= T <= order_key(+inf): order_key(x) >= T
// iff x >= f (IEEE compare: NaN never passes, -0 and +0 compare equal as their keys do)
__device__ __forceinline__ float key_floor(uint32_t T) {
  if (T <= 0x007fffffu) return -INFINITY;  // every real key (order_key(-inf) = 0x007fffff) reaches T
  return __uint_as_float((T & 0x80000000u) ? (T & 0x7fffffffu) : ~T);
}

__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, (uint32_t)__shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, (uint32_t)__shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_scan_incl_u(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}
// number of set bits of `mask` in lanes below this one
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// kMode: 0 every row from its scores; 1 rows from the candidate list of topk_cand_kernel
// (cand_cnt[row] >= 0; other rows are left to mode 2), which holds every key at or above a
// threshold that at least k keys reach, in index order; 2 only the rows whose candidate
// list was not usable (cand_cnt[row] < 0), from their scores
template <int kR, bool kSingle, bool kVec, int kMode = 0>
__global__ void __launch_bounds__(kThreads)
topk_kernel(const float* __restrict__ scores, int32_t* __restrict__ out_idx, float* __restrict__ out_val, int S,
            int s_k, int64_t ld, int k, int64_t q_offset, int cmp_ratio, int64_t index_offset,
            const uint2* __restrict__ cand = nullptr, const int* __restrict__ cand_cnt = nullptr, int cap = 0,
            const int* __restrict__ win = nullptr, int64_t win_rows = 0) {
  static_assert(kMode != 1 || kSingle, "a candidate list is one segment");
  constexpr int kSeg = kThreads * 4 * kR;
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t red[3][kWaves];
  __shared__ uint32_t tot[2][kR][kWaves];  // per-(chunk, wave) counts of key > T and key == T
  __shared__ uint32_t sh_bin[3];

  // rows are dispatched last-first: under the causal rule the later rows hold the longest
  // valid prefixes, so the slowest workgroups start first instead of forming the tail
  const int s = S - 1 - (int)blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t row = (int64_t)b * S + s;
  const float* src = scores + row * ld;
  const int64_t nv64 = win ? (int64_t)(win[win_rows + row] - win[row]) : (s + q_offset + 1) / cmp_ratio;
  int nv = (int)max((int64_t)0, min((int64_t)s_k, nv64));
  const uint2* crow = kMode == 1 ? cand + row * (int64_t)cap : nullptr;
  if constexpr (kMode == 1) {
    const int c = cand_cnt[row];
    if (c < 0) return;  // (left to the fallback launch)
    nv = c;             // candidates, in index order
  } else if constexpr (kMode == 2) {
    if (cand_cnt[row] >= 0) return;
  }
  const int nseg = kSingle ? 1 : (nv + kSeg - 1) / kSeg;
  const int s_k4 = s_k & ~3;  // scores [0, s_k4) are covered by whole float4 loads

  // chunk j of segment sg covers positions [sg kSeg + 1024 j, +1024): it holds a valid
  // position iff it starts below nv (workgroup-uniform), so chunks past the row's valid
  // prefix are neither loaded nor examined
  auto live = [&](int sg, int j) { return sg * kSeg + kThreads * 4 * j < nv; };
  // order keys of the thread's scores; positions past the valid prefix and NaN scores are
  // key 0 (not candidates)
  uint32_t key[kR][4];
  // (candidate lists: each candidate's position in the row, read with its key so that the
  // output pass issues no load under its per-lane branches)
  uint32_t cpos[kMode == 1 ? kR : 1][4];
  // Every load of a segment is issued before any key is formed and no load sits under a
  // lane-dependent branch, so a wave has all of them in flight at once (a branch per lane
  // would make the compiler wait for each load before the next); chunks past the valid
  // prefix are skipped under a workgroup-uniform branch.  Lanes at or past nv read a clamped
  // in-row position that their key then ignores.
  // (the lambdas are forced inline: called from several loops, an out-of-line copy would take
  // `key` by reference and put it in scratch memory)
  auto load_seg = [&](int sg) __attribute__((always_inline)) {
    if constexpr (kMode == 1) {  // candidates: the score's bits as stored, then its key
      const int last = max(nv - 1, 0);
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        const int base = sg * kSeg + 4 * (t + kThreads * j);
        if (live(sg, j)) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint2 cv = crow[min(base + e, last)];
            key[j][e] = cv.x;
            cpos[j][e] = cv.y;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kR; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) key[j][e] = order_key(__uint_as_float(key[j][e]));
      }
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        const int base = sg * kSeg + 4 * (t + kThreads * j);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (base + e >= nv) key[j][e] = 0u;
      }
      return;
    }
    float x[kR][4];
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int base = sg * kSeg + 4 * (t + kThreads * j);
      if (!live(sg, j)) continue;
      if constexpr (kVec) {
        // a lane with base < s_k4 has base <= s_k4 - 4 (both multiples of 4): it reads its own
        // four scores; lanes past s_k4 read in-row scores that are masked or replaced below
        const float4 v = *reinterpret_cast<const float4*>(src + min(base, s_k4 - 4));
        x[j][0] = v.x;
        x[j][1] = v.y;
        x[j][2] = v.z;
        x[j][3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[j][e] = src[min(base + e, nv - 1)];
      }
    }
    if (kVec && nv > s_k4) {  // (row-uniform) a valid prefix reaching into the ragged tail
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        const int base = sg * kSeg + 4 * (t + kThreads * j);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (base + e >= s_k4 && base + e < nv) x[j][e] = src[base + e];
      }
    }
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int base = sg * kSeg + 4 * (t + kThreads * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) key[j][e] = base + e < nv ? order_key(x[j][e]) : 0u;
    }
  };

  int32_t* oi = out_idx + row * k;
  float* ov = out_val ? out_val + row * k : nullptr;
  if (nv == 0) {
    for (int j = t; j < k; j += kThreads) {
      oi[j] = -1;
      if (ov) ov[j] = -INFINITY;
    }
    return;
  }

  // ---- a row with at most k valid positions: every candidate, no pass ----
  uint32_t T = 0u, need_eq = 0u;  // (T = 0, need_eq = 0: every candidate, key > 0)
  if (nv <= k) {
    if (kSingle) load_seg(0);
  } else {
    // ---- pass 0: candidates, min and max key ----
    uint32_t cnt = 0, kmin = 0xffffffffu, kmax = 0u;
    for (int sg = 0; sg < nseg; ++sg) {
      load_seg(sg);
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        if (!live(sg, j)) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kv = key[j][e];
          cnt += kv != 0u;
          kmin = min(kmin, kv ? kv : 0xffffffffu);
          kmax = max(kmax, kv);
        }
      }
    }
    cnt = wave_sum_u(cnt);
    kmin = wave_min_u(kmin);
    kmax = wave_max_u(kmax);
    if (lane == 0) {
      red[0][wave] = cnt;
      red[1][wave] = kmin;
      red[2][wave] = kmax;
    }
    __syncthreads();
    uint32_t n_cand = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      n_cand += red[0][w];
      kmin = min(kmin, red[1][w]);
      kmax = max(kmax, red[2][w]);
    }

    // ---- threshold: take key > T, and key == T for the first need_eq in index order ----
    if (n_cand > (uint32_t)k) {
      const uint32_t range = kmax - kmin;
      int sh = range ? 32 - __clz(range) : 0;  // the current bin is rel = key - kmin in [lo, lo + 2^sh)
      uint32_t lo = 0u, rem = (uint32_t)k;
      bool whole_bin = false;
      while (sh > 0) {
        const int nsh = max(sh - kDigitBits, 0);
        const int nb = 1 << (sh - nsh);
        for (int i = t; i < nb; i += kThreads) hist[i] = 0u;
        __syncthreads();
        // a candidate is in the bin iff key - (kmin + lo) <= span in 32-bit arithmetic: keys
        // below the bin, key 0 (not a candidate) included, wrap to at least 2^32 - (kmin + lo),
        // which the span never reaches once it is clamped to 2^32 - 1 - (kmin + lo); the clamp
        // drops no candidate (candidate keys are at most order_key(+inf) = 0xff800000)
        const uint32_t base_key = kmin + lo;
        const uint32_t span = min(sh >= 32 ? 0xffffffffu : (1u << sh) - 1u, 0xffffffffu - base_key);
        for (int sg = 0; sg < nseg; ++sg) {
          if (!kSingle) load_seg(sg);
#pragma unroll
          for (int j = 0; j < kR; ++j) {
            if (!live(sg, j)) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t d = key[j][e] - base_key;
              if (d <= span) atomicAdd(&hist[d >> nsh], 1u);
            }
          }
        }
        __syncthreads();
        // thread t sums bins [nb - 8(t+1), nb - 8t) (from the top); exclusive scan in thread
        // order = keys in bins above its range
        const int hi = nb - kBinsPerThread * t;
        uint32_t c[kBinsPerThread], my = 0;
#pragma unroll
        for (int i = 0; i < kBinsPerThread; ++i) {
          const int bin = hi - 1 - i;
          c[i] = bin >= 0 ? hist[bin] : 0u;
          my += c[i];
        }
        const uint32_t incl = wave_scan_incl_u(my, lane);
        if (lane == 63) red[0][wave] = incl;
        __syncthreads();
        uint32_t above = incl - my;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
          if (w < wave) above += red[0][w];
        if (above < rem && rem <= above + my) {  // exactly one thread
#pragma unroll
          for (int i = 0; i < kBinsPerThread; ++i) {
            if (above < rem && rem <= above + c[i]) {
              sh_bin[0] = (uint32_t)(hi - 1 - i);
              sh_bin[1] = above;
              sh_bin[2] = c[i];
            }
            above += c[i];
          }
        }
        __syncthreads();
        const uint32_t bin = sh_bin[0], n_above = sh_bin[1], n_bin = sh_bin[2];
        lo += bin << nsh;
        rem -= n_above;
        sh = nsh;
        if (n_bin == rem) {
          whole_bin = true;
          break;
        }
        __syncthreads();  // sh_bin and red are rewritten by the next pass
      }
      if (whole_bin) {
        T = kmin + lo - 1u;  // lo >= 1 here: lo == 0 would take every candidate (n_cand == k)
        need_eq = 0u;
      } else {
        T = kmin + lo;
        need_eq = rem;
      }
    }
  }

  // ---- compaction in index order ----
  // (no tie at the threshold, the usual case: key > T alone decides, one ballot per score,
  // in a code path of its own so that it holds no tie state)
  auto compact = [&](auto ties_c) __attribute__((always_inline)) {
    constexpr bool kTies = decltype(ties_c)::value;
    uint32_t gt_base = 0, eq_base = 0;
    for (int sg = 0; sg < nseg; ++sg) {
      if (!kSingle) load_seg(sg);
      // per chunk j: lanes-below counts (< 256: 8 bits, four chunks per word) and this lane's
      // flag bits (4 bits, eight chunks per word), packed so that the compaction holds few
      // registers besides the keys
      constexpr int kW8 = (kR + 3) / 4, kW4 = (kR + 7) / 8;
      uint32_t pg[kW8], pe[kW8], mg[kW4], me[kW4];
#pragma unroll
      for (int i = 0; i < kW8; ++i) pg[i] = pe[i] = 0u;
#pragma unroll
      for (int i = 0; i < kW4; ++i) mg[i] = me[i] = 0u;
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        if (!live(sg, j)) continue;
        uint32_t below_g = 0, below_e = 0, wg = 0, we = 0, fg = 0, fe = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kv = key[j][e];
          const bool g = kv > T;
          const uint64_t bg = __ballot(g);
          below_g += lanes_below(bg);
          wg += (uint32_t)__popcll(bg);
          fg |= (uint32_t)g << e;
          if constexpr (kTies) {
            const bool q = kv == T && kv != 0u;
            const uint64_t bq = __ballot(q);
            below_e += lanes_below(bq);
            we += (uint32_t)__popcll(bq);
            fe |= (uint32_t)q << e;
          }
        }
        pg[j >> 2] |= below_g << (8 * (j & 3));
        pe[j >> 2] |= below_e << (8 * (j & 3));
        mg[j >> 3] |= fg << (4 * (j & 7));
        me[j >> 3] |= fe << (4 * (j & 7));
        if (lane == 0) {
          tot[0][j][wave] = wg;
          tot[1][j][wave] = we;
        }
      }
      __syncthreads();
      uint32_t run_g = gt_base, run_e = eq_base;  // counts before chunk j of this segment
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        if (!live(sg, j)) continue;
        uint32_t bg = run_g + ((pg[j >> 2] >> (8 * (j & 3))) & 0xffu), be = run_e + ((pe[j >> 2] >> (8 * (j & 3))) & 0xffu);
        const uint32_t fgj = mg[j >> 3] >> (4 * (j & 7)), fej = me[j >> 3] >> (4 * (j & 7));
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const uint32_t tg = tot[0][j][w], te = kTies ? tot[1][j][w] : 0u;
          if (w < wave) {
            bg += tg;
            be += te;
          }
          run_g += tg;
          run_e += te;
        }
        const int base = sg * kSeg + 4 * (t + kThreads * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool g = (fgj >> e) & 1u, q = kTies && ((fej >> e) & 1u);
          const bool take = g || (q && be < need_eq);
          const uint32_t pos = bg + (kTies ? min(be, need_eq) : 0u);
          if (take && pos < (uint32_t)k) {  // (always < k: the threshold admits at most k)
            int at = base + e;  // position in the row
            if constexpr (kMode == 1) at = (int)cpos[j][e];
            oi[pos] = (int32_t)(at + index_offset);
            if (ov) ov[pos] = src[at];  // (the score as given: -0.0 keeps its sign)
          }
          bg += g;
          be += q;
        }
      }
      gt_base = run_g;
      eq_base = run_e;
      if (!kSingle) __syncthreads();  // tot is rewritten by the next segment
    }
    // positions written (workgroup-uniform: the totals cover every wave)
    return gt_base + (kTies ? min(eq_base, need_eq) : 0u);
  };
  const uint32_t taken = min(need_eq != 0u ? compact(std::true_type{}) : compact(std::false_type{}), (uint32_t)k);
  for (int j = (int)taken + t; j < k; j += kThreads) {
    oi[j] = -1;
    if (ov) ov[j] = -INFINITY;
  }
}

// Long rows, candidate pass (one read of the row): a threshold T estimated from a sample of
// kCandChunks chunks of 1024 scores spread over the row's valid prefix, so that about
// 1.35 k keys of the row are expected to reach it, then every key >= T is written with its
// position to the row's candidate list (capacity cap), in index order (wave ballots and
// per-(wave, chunk) totals, as the top-k compaction).  cand_cnt[row] = the list's length
// when it holds at least k keys (or every candidate of the row) and fits, else -1: then
// the list may miss a top-k key and the row is selected from its scores instead.  With at
// least k keys >= T, the k-th largest key is >= T, so every key the top-k takes (ties at
// the threshold included) is in the list, in the same relative order.
constexpr int kCandChunks = 8;

template <bool kVec>
__global__ void __launch_bounds__(kThreads)
topk_cand_kernel(const float* __restrict__ scores, uint2* __restrict__ cand, int* __restrict__ cand_cnt, int cap,
                 int S, int s_k, int64_t ld, int k, int64_t q_offset, int cmp_ratio,
                 const int* __restrict__ win = nullptr, int64_t win_rows = 0) {
  constexpr int kR = 8, kSeg = kThreads * 4 * kR;  // 8192-score segments
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t red[3][kWaves];
  __shared__ uint32_t tot[kR][kWaves];
  __shared__ uint32_t sh_bin[2];

  const int s = S - 1 - (int)blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t row = (int64_t)b * S + s;
  const float* src = scores + row * ld;
  const int64_t nv64 = win ? (int64_t)(win[win_rows + row] - win[row]) : (s + q_offset + 1) / cmp_ratio;
  const int nv = (int)max((int64_t)0, min((int64_t)s_k, nv64));
  const int s_k4 = s_k & ~3;
  uint2* crow = cand + row * (int64_t)cap;

  // Loads as in topk_kernel: issued with no lane-dependent branch (so a wave keeps all of a
  // segment's loads in flight), at addresses clamped into the row; keys are formed after the
  // loads, and positions at or past the valid prefix, which may be unwritten, and NaN scores
  // are key 0 (not candidates).  The main pass covers positions [0, nm); with float4 rows the
  // at most three positions of a ragged tail [s_k4, nv) are appended after it (they are the
  // row's last positions).
  const int nm = kVec ? min(nv, s_k4) : nv;
  const int last = max(nm - 1, 0);
  auto load4 = [&](int base, bool lv, float (&x)[4]) __attribute__((always_inline)) {
    if constexpr (kVec) {  // (a lane with base < s_k4 has base <= s_k4 - 4: its own four scores)
      const float4 v = *reinterpret_cast<const float4*>(src + min(lv ? base : 4 * t, s_k4 - 4));
      x[0] = v.x;
      x[1] = v.y;
      x[2] = v.z;
      x[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = src[min(base + e, last)];
    }
  };
  auto keys4 = [&](int base, const float (&x)[4], uint32_t (&kk)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) kk[e] = base + e < nm ? order_key(x[e]) : 0u;
  };

  uint32_t T = 1u;  // every candidate (key > 0) when the row fits the list
  if (nv > cap) {
    // ---- threshold from the sample ----
    const int nchunk = nv >> 10;  // whole 1024-score chunks (>= 4: nv > cap >= 4096)
    uint32_t sk[kCandChunks][4];
    uint32_t ns = 0, kmin = 0xffffffffu, kmax = 0u;
    {
      float xs[kCandChunks][4];
#pragma unroll
      for (int j = 0; j < kCandChunks; ++j) load4(((j * nchunk) / kCandChunks) * 1024 + 4 * t, true, xs[j]);
#pragma unroll
      for (int j = 0; j < kCandChunks; ++j) keys4(((j * nchunk) / kCandChunks) * 1024 + 4 * t, xs[j], sk[j]);
    }
#pragma unroll
    for (int j = 0; j < kCandChunks; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ns += sk[j][e] != 0u;
        kmin = min(kmin, sk[j][e] ? sk[j][e] : 0xffffffffu);
        kmax = max(kmax, sk[j][e]);
      }
    }
    for (int i = t; i < kBins; i += kThreads) hist[i] = 0u;
    ns = wave_sum_u(ns);
    kmin = wave_min_u(kmin);
    kmax = wave_max_u(kmax);
    if (lane == 0) {
      red[0][wave] = ns;
      red[1][wave] = kmin;
      red[2][wave] = kmax;
    }
    __syncthreads();
    ns = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      ns += red[0][w];
      kmin = min(kmin, red[1][w]);
      kmax = max(kmax, red[2][w]);
    }
    if (ns > 0) {
      // sampled keys expected at or above T: 1.35 k of the row's nv, scaled to the sample
      const float want = 1.35f * (float)k * (float)ns / (float)nv + 8.f;
      const uint32_t target = (uint32_t)min((float)ns, want);
      // T is the target-th largest sampled key, rounded down to a digit of two histogram
      // levels over the sampled keys' range (as the radix passes: 2^11 bins from the top, then
      // 2^11 sub-bins of the bin that holds it), so that the count of row keys >= T follows the
      // sample's quantile and not the width of one coarse bin
      const uint32_t range = kmax - kmin;
      const int sh = range ? 32 - __clz(range) : 0;
      uint32_t lo = 0u, rem = target;
      for (int level = 0, cur = sh; level < 2 && cur > 0; ++level) {
        const int nsh = max(cur - kDigitBits, 0);
        const uint32_t base_key = kmin + lo;
        const uint32_t span = (cur >= 32 ? 0xffffffffu : (1u << cur) - 1u);
        if (level > 0) {
          for (int i = t; i < kBins; i += kThreads) hist[i] = 0u;
          __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < kCandChunks; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t d = sk[j][e] - base_key;  // keys below the bin (key 0 too) wrap past span
            if (sk[j][e] && d <= span) atomicAdd(&hist[d >> nsh], 1u);
          }
        __syncthreads();
        // the bin holding the rem-th largest key in range, from the top
        const int hi = kBins - kBinsPerThread * t;
        uint32_t c[kBinsPerThread], my = 0;
#pragma unroll
        for (int i = 0; i < kBinsPerThread; ++i) {
          c[i] = hist[hi - 1 - i];
          my += c[i];
        }
        const uint32_t incl = wave_scan_incl_u(my, lane);
        __syncthreads();  // (red is rewritten)
        if (lane == 63) red[0][wave] = incl;
        __syncthreads();
        uint32_t above = incl - my;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
          if (w < wave) above += red[0][w];
        if (above < rem && rem <= above + my) {  // exactly one thread
#pragma unroll
          for (int i = 0; i < kBinsPerThread; ++i) {
            if (above < rem && rem <= above + c[i]) {
              sh_bin[0] = (uint32_t)(hi - 1 - i);
              sh_bin[1] = above;
            }
            above += c[i];
          }
        }
        __syncthreads();
        lo += sh_bin[0] << nsh;
        rem -= sh_bin[1];
        cur = nsh;
        __syncthreads();  // (sh_bin and hist are rewritten by the next level)
      }
      T = kmin + lo;
    }
  }

  // ---- every key >= T with its position, in index order ----
  // (one segment's loads in flight per workgroup; the other resident workgroups of the CU
  // cover its ballots, barriers and list writes)
  const int nseg = (nm + kSeg - 1) / kSeg;
  auto load_seg = [&](int sg, float (&xx)[kR][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kR; ++j)
      load4(sg * kSeg + 4 * (t + kThreads * j), sg * kSeg + kThreads * 4 * j < nm, xx[j]);
  };
  // candidates are compared as floats (x >= Tf iff order_key(x) >= T) and stored as the
  // score's bits with the position; the selection over the list forms their keys
  const float Tf = key_floor(T);
  uint32_t run = 0;  // candidates before the current segment
  // (kFull: a segment with no position past nm, the test is the compare alone)
  auto compact_seg = [&](int sg, const float (&xx)[kR][4], auto full_c) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_c)::value;
    auto cand = [&](int j, int e) __attribute__((always_inline)) {
      return xx[j][e] >= Tf && (kFull || sg * kSeg + 4 * (t + kThreads * j) + e < nm);
    };
    uint32_t below[kR];
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      below[j] = 0u;
      if (sg * kSeg + kThreads * 4 * j >= nm) continue;  // (workgroup-uniform)
      uint32_t wt = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t bg = __ballot(cand(j, e));
        below[j] += lanes_below(bg);
        wt += (uint32_t)__popcll(bg);
      }
      if (lane == 0) tot[j][wave] = wt;
    }
    __syncthreads();
    uint32_t run_j = run;
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      if (sg * kSeg + kThreads * 4 * j >= nm) break;  // (workgroup-uniform)
      uint32_t pos = run_j + below[j];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const uint32_t tw = tot[j][w];
        if (w < wave) pos += tw;
        run_j += tw;
      }
      const int base = sg * kSeg + 4 * (t + kThreads * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (cand(j, e)) {
          if (pos < (uint32_t)cap) crow[pos] = make_uint2(__float_as_uint(xx[j][e]), (uint32_t)(base + e));
          ++pos;
        }
      }
    }
    run = run_j;
    __syncthreads();  // (tot is rewritten by the next segment)
  };
  for (int sg = 0; sg < nseg; ++sg) {
    float xx[kR][4];
    load_seg(sg, xx);
    if ((sg + 1) * kSeg <= nm)  // (workgroup-uniform)
      compact_seg(sg, xx, std::true_type{});
    else
      compact_seg(sg, xx, std::false_type{});
  }
  if (kVec && nv > nm && wave == 0) {  // (row-uniform) the ragged tail, in index order
    const int p = nm + lane;
    const float x = src[min(p, nv - 1)];
    const bool g = p < nv && x >= Tf;
    const uint64_t bg = __ballot(g);
    const uint32_t pos = run + lanes_below(bg);
    if (g && pos < (uint32_t)cap) crow[pos] = make_uint2(__float_as_uint(x), (uint32_t)p);
    run += (uint32_t)__popcll(bg);
  }
  if (t == 0) cand_cnt[row] = (nv <= cap || (run >= (uint32_t)k && run <= (uint32_t)cap)) ? (int)run : -1;
}

template <int kR, bool kSingle>
void launch_topk(bool vec, dim3 grid, hipStream_t st, const float* scores, int32_t* indices, float* values, int S,
                 int s_k, int64_t ld, int k, int64_t q_offset, int cmp_ratio, int64_t index_offset, const int* win,
                 int64_t win_rows) {
  const TimedLaunch tl("topk_kernel", st);
  if (vec)
    topk_kernel<kR, kSingle, true><<<grid, kThreads, 0, st>>>(scores, indices, values, S, s_k, ld, k, q_offset,
                                                              cmp_ratio, index_offset, nullptr, nullptr, 0, win,
                                                              win_rows);
  else
    topk_kernel<kR, kSingle, false><<<grid, kThreads, 0, st>>>(scores, indices, values, S, s_k, ld, k, q_offset,
                                                               cmp_ratio, index_offset, nullptr, nullptr, 0, win,
                                                               win_rows);
}

}  // namespace
}  // namespace dsa

namespace dsa {
// candidate list capacity for long rows: twice k, in whole 1024-key chunks of the selection
// (4096 covers k <= 2048, 8192 every k the entry points take)
int topk_cand_cap(int64_t k) { return k <= 2048 ? 4096 : 8192; }
int64_t topk_cand_bytes(int64_t rows, int64_t k) { return rows * (int64_t)topk_cand_cap(k) * 8 + rows * 4 + 256; }

// Long rows (s_k > 16384) with a candidate workspace of topk_cand_bytes(batch * s_q, k):
// candidate pass, selection over the candidate lists, the fallback rows from their scores.
int topk_long_cand(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q, int64_t s_k,
                   int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio, int64_t index_offset,
                   void* cand_ws, hipStream_t st, const int* win, int64_t win_rows) {
  const int cap = topk_cand_cap(k);
  uint2* cand = (uint2*)cand_ws;
  int* cnt = (int*)((char*)cand_ws + batch * s_q * (int64_t)cap * 8);
  dim3 grid((unsigned)s_q, (unsigned)batch);
  const bool vec = s_k >= 4 && (ld_scores % 4) == 0 && ((uintptr_t)scores % 16) == 0;
  const int S = (int)s_q, n = (int)s_k, kk = (int)k, r = (int)cmp_ratio;
  {
    const TimedLaunch tl("topk_cand_kernel", st);
    if (vec)
      topk_cand_kernel<true><<<grid, kThreads, 0, st>>>(scores, cand, cnt, cap, S, n, ld_scores, kk, q_offset, r,
                                                        win, win_rows);
    else
      topk_cand_kernel<false><<<grid, kThreads, 0, st>>>(scores, cand, cnt, cap, S, n, ld_scores, kk, q_offset, r,
                                                         win, win_rows);
  }
  {
    const TimedLaunch tl("topk_kernel<cand>", st);
    if (cap == 4096)
      topk_kernel<4, true, false, 1><<<grid, kThreads, 0, st>>>(scores, indices, values, S, n, ld_scores, kk,
                                                                q_offset, r, index_offset, cand, cnt, cap, win,
                                                                win_rows);
    else
      topk_kernel<8, true, false, 1><<<grid, kThreads, 0, st>>>(scores, indices, values, S, n, ld_scores, kk,
                                                                q_offset, r, index_offset, cand, cnt, cap, win,
                                                                win_rows);
  }
  {
    const TimedLaunch tl("topk_kernel<fallback>", st);
    if (vec)
      topk_kernel<8, false, true, 2><<<grid, kThreads, 0, st>>>(scores, indices, values, S, n, ld_scores, kk,
                                                                q_offset, r, index_offset, cand, cnt, cap, win,
                                                                win_rows);
    else
      topk_kernel<8, false, false, 2><<<grid, kThreads, 0, st>>>(scores, indices, values, S, n, ld_scores, kk,
                                                                 q_offset, r, index_offset, cand, cnt, cap, win,
                                                                 win_rows);
  }
  return check_launch("dsa_topk(candidates)");
}
}  // namespace dsa

extern "C" int dsa_topk(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q,
                        int64_t s_k, int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio,
                        int64_t index_offset, void* stream) {
  return dsa::topk_rows(scores, indices, values, batch, s_q, s_k, ld_scores, k, q_offset, cmp_ratio, index_offset,
                        nullptr, stream);
}

extern "C" int64_t dsa_topk_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t k) {
  if (batch <= 0 || s_q <= 0 || k <= 0 || s_k <= 16384) return 0;
  return dsa::topk_cand_bytes(batch * s_q, k);
}

extern "C" int dsa_topk_ws(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q,
                           int64_t s_k, int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio,
                           int64_t index_offset, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace dsa;
  const int64_t need = dsa_topk_workspace_size(batch, s_q, s_k, k);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk_ws: workspace of %lld bytes, %lld needed",
                     (long long)workspace_bytes, (long long)need);
  if (need > 0 && (uintptr_t)workspace % 16)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk_ws: workspace must be 16-byte aligned");
  return topk_rows(scores, indices, values, batch, s_q, s_k, ld_scores, k, q_offset, cmp_ratio, index_offset,
                   need > 0 ? workspace : nullptr, stream);
}

namespace dsa {
int topk_rows(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q, int64_t s_k,
              int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio, int64_t index_offset, void* cand_ws,
              void* stream, const int* win, int64_t win_rows) {
  if (!scores || !indices) return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k < 0 || k <= 0 || k > 4096 || ld_scores < s_k || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: bad sizes (B=%lld S=%lld S_k=%lld ld=%lld k=%lld r=%lld)",
                     (long long)batch, (long long)s_q, (long long)s_k, (long long)ld_scores, (long long)k,
                     (long long)cmp_ratio);
  if (s_q > 2147483647LL || batch > 65535 || s_k > 2147483647LL - 16384)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)s_q, (unsigned)batch);
  // float4 loads need 16-byte aligned rows and at least one whole float4 per row
  const bool vec = s_k >= 4 && (ld_scores % 4) == 0 && ((uintptr_t)scores % 16) == 0;
  const int S = (int)s_q, n = (int)s_k, kk = (int)k, r = (int)cmp_ratio;
  if (s_k <= 8192)
    launch_topk<8, true>(vec, grid, st, scores, indices, values, S, n, ld_scores, kk, q_offset, r, index_offset, win,
                         win_rows);
  else if (s_k <= 16384)
    launch_topk<16, true>(vec, grid, st, scores, indices, values, S, n, ld_scores, kk, q_offset, r, index_offset, win,
                          win_rows);
  else if (cand_ws)  // long rows: one read into candidate lists, selection over those
    return topk_long_cand(scores, indices, values, batch, s_q, s_k, ld_scores, k, q_offset, cmp_ratio, index_offset,
                          cand_ws, st, win, win_rows);
  else  // long rows: 8192-score segments re-read per pass; 61 VGPRs, seven waves per SIMD in flight
    launch_topk<8, false>(vec, grid, st, scores, indices, values, S, n, ld_scores, kk, q_offset, r, index_offset, win,
                          win_rows);
  return check_launch("dsa_topk");
}
}  // namespace dsa
