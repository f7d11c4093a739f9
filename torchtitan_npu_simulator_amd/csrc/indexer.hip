// Lightning-indexer scores on MFMA (bf16 or OCP fp8-e4m3 inputs, fp32 accumulation):
//   I[s, t] = ks[t] * sum_h (w[s,h] * qs[s,h]) * relu(q[s,h,:] . k[t,:])      (t valid)
//   I[s, t] = -inf                                                       (t invalid)
// (relu(c x) = c relu(x) for the positive per-token scales, so the quantise-then-
// dequantise product of the reference folds into the head weights and one key scale.)
#include <mutex>

#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kD = 128;            // indexer head dim on the MFMA path
constexpr int kThreads = 256;

// Workgroup = (4 waves x kQw queries) x a span of kSub key tiles.  Each wave keeps its
// queries' heads as MFMA A operands in VGPRs for the whole span (one read of Q per span,
// not per key tile), and the span's key tiles stream through two LDS buffers: tile i+1 is
// DMA'd (inline-asm global_load_lds; the keys sit in L2) while tile i is computed.  Per
// 16-key B tile read out of LDS:
//   bf16: 4 x v_mfma_f32_16x16x32_bf16 per (16-head tile, 16-key tile)
//   fp8 : 1 x v_mfma_scale_f32_16x16x128_f8f6f4 (scales 0 = identity)
// The 16x16 C tile (lane: key = l%16, heads 4(l/16)..+3) gets relu * w in registers, is
// summed over the head tiles in-lane and over the 4 lane groups with two lane swaps; a
// tile's scores are staged in LDS and written as whole rows.  Key ranges past every
// query's causal frontier are written as -inf without any MFMA, or left unwritten for
// consumers that read only each row's valid prefix (the fused indexer + top-k).
//
// Linear split (kLin, fp8 with two queries per wave): relu(x) = (x + |x|) / 2, so
//   sum_h c_h relu(x_h) = sum_h (c_h/2) |x_h| + u . k,   u = sum_h (c_h/2) q_h   (x_h = q_h . k)
// The |x| sum is one fma per C value (abs source modifier) instead of a max and an fma, which
// halves the VALU work that bounds this kernel.  u . k runs on the MFMA: u comes from a
// per-query pre-pass as kLinPieces fp8 pieces with power-of-two scales (u = sum_p 2^-e_p P_p
// to about 2^-18 of max|u|), held as the rows of one more A tile per query pair (rows 0-3:
// the pair's first query, rows 8-11: the second, the rest zero), so each 16-key tile costs
// 9 MFMAs per two queries instead of 8.
constexpr int kLinPieces = 4;
constexpr int64_t kLinRowBytes = kLinPieces * kD + kLinPieces * 4;  // pieces + their scales
template <bool kFp8, int kHeadTiles>
struct IdxTile {
  static constexpr int kQw = kFp8 ? (8 / kHeadTiles > 0 ? 8 / kHeadTiles : 1) : (4 / kHeadTiles > 0 ? 4 / kHeadTiles : 1);
  static constexpr int kQ = 4 * kQw;                      // queries per workgroup
  static constexpr int kRowBytes = kD * (kFp8 ? 1 : 2);   // 128 or 256
  static constexpr int kKeys = 32768 / kRowBytes;         // keys per LDS tile (32 KB)
  static constexpr int kSub = 4;                          // key tiles per workgroup
  static constexpr int kSpan = kKeys * kSub;              // keys per workgroup
  static constexpr int kCpr = kRowBytes / 16;             // 16-byte chunks per key row
  static constexpr int kTileBytes = kKeys * kRowBytes;
  static constexpr int kDmaPerWave = kTileBytes / 1024 / 4;
  static constexpr int kRegsPerTile = kFp8 ? 8 : 16;      // A/B dwords per lane per 16-row tile
  static constexpr int kStoreIters = (kQ * kKeys / 4 + kThreads - 1) / kThreads;  // float4 per thread
};
// key-row chunk swizzle: fp8 rows (128 B) alternate bank halves, so the 8 rows of one
// parity take distinct chunks; bf16 rows (256 B) all start on bank 0, 16 rows distinct
template <bool kFp8>
__device__ __forceinline__ int idx_swz(int r) { return kFp8 ? ((r >> 1) & 7) : (r & 15); }

// scores[rows s0.., keys t_lo..t_hi) = -inf (float4 stores where aligned)
__device__ __forceinline__ void fill_neg_inf(float* __restrict__ scores, int64_t row0, int nrows, int64_t ld,
                                             int t_lo, int t_hi, int tid) {
  if (t_hi <= t_lo) return;
  const int n4 = (t_hi - t_lo + 3) >> 2;
  const float4 m4 = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  for (int i = tid; i < nrows * n4; i += kThreads) {
    const int r = i / n4, c = i - r * n4;
    const int t = t_lo + 4 * c;
    float* dst = scores + (row0 + r) * ld + t;
    if (t + 4 <= t_hi && (((uintptr_t)dst) & 15) == 0) {
      *reinterpret_cast<float4*>(dst) = m4;
    } else {
      for (int e = 0; e < 4 && t + e < t_hi; ++e) dst[e] = -INFINITY;
    }
  }
}

// four e4m3fn bytes -> fp32 by the packed hardware conversion (OCP e4m3 on gfx950, the
// format the f8f6f4 MFMA reads)
__device__ __forceinline__ void fp8x4_to_f32(uint32_t v, float (&f)[4]) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false), hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}

// Pre-pass of the linear split, one wave per query row r:
//   u[r, :] = sum_h 0.5 * (w[r,h] * q_scale[r,h]) * q[r,h,:]
// lane l reads 16-byte pieces of heads 8i + l/8 (i < H/8), dims 16(l%8)..+15, and the eight
// lanes of one dim range are summed by lane exchanges.  Then kLinPieces greedy pieces:
// 2^e_p makes max|res_p| fit e4m3 (<= 448), P_p = e4m3(2^e_p res_p) by the hardware
// conversion, res_{p+1} = res_p - 2^-e_p P_p with P_p read back by the same hardware (so the
// residual is exact for whatever rounding the conversion applies); lane group p (= l/8)
// stores piece p.
// pieces [rows][kLinPieces][kD] bytes, then scales [rows][kLinPieces] fp32 (= 2^-e_p).
template <int H>
__global__ void __launch_bounds__(kThreads)
indexer_lin_pieces_kernel(const uint8_t* __restrict__ q, const float* __restrict__ q_scale,
                          const float* __restrict__ w, uint8_t* __restrict__ pieces, float* __restrict__ pscale,
                          int64_t nrows) {
  const int64_t r = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= nrows) return;  // whole waves
  const int lane = threadIdx.x & 63, grp = lane >> 3, d0 = 16 * (lane & 7);
  static_assert(H % 8 == 0, "eight heads per wave step");
  constexpr int kSteps = H / 8;
  float c[kSteps];
  u32x4 x[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {  // every load of the row issued at once
    const int64_t hr = r * H + 8 * i + grp;
    c[i] = w[hr] * (q_scale ? q_scale[hr] : 1.f);
    x[i] = *reinterpret_cast<const u32x4*>(q + hr * kD + d0);
  }
  float u[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) u[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    const float ci = 0.5f * c[i];
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) {
      float f[4];
      fp8x4_to_f32(x[i][d4], f);
#pragma unroll
      for (int e = 0; e < 4; ++e) u[4 * d4 + e] = fmaf(ci, f[e], u[4 * d4 + e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    u[e] += __shfl_xor(u[e], 8);
    u[e] += __shfl_xor(u[e], 16);
    u[e] += __shfl_xor(u[e], 32);
  }
  for (int p = 0; p < kLinPieces; ++p) {
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(u[e]));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));
    int ex = 0;
    if (m > 0.f && m <= 3.4028235e38f) {
      int E;
      const float f = frexpf(m, &E);  // m = f 2^E, f in [0.5, 1); 448 = 0.875 * 2^9
      ex = min((f <= 0.875f ? 9 : 8) - E, 126);
    }
    const float up = ldexpf(1.f, ex), down = ldexpf(1.f, -ex);  // exact powers of two
    u32x4 pk;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) {
      int v = __builtin_amdgcn_cvt_pk_fp8_f32(u[4 * d4] * up, u[4 * d4 + 1] * up, 0, false);
      v = __builtin_amdgcn_cvt_pk_fp8_f32(u[4 * d4 + 2] * up, u[4 * d4 + 3] * up, v, true);
      pk[d4] = (uint32_t)v;
      float f[4];
      fp8x4_to_f32(pk[d4], f);
#pragma unroll
      for (int e = 0; e < 4; ++e) u[4 * d4 + e] -= f[e] * down;
    }
    if (grp == p) *reinterpret_cast<u32x4*>(pieces + (r * kLinPieces + p) * kD + d0) = pk;
    if (lane == 0) pscale[r * kLinPieces + p] = down;
  }
}

// kTnd: packed rows whose key windows come from the device (row geometry of a packed batch,
// see tnd_layout): ``tnd`` holds, for the S rows of the call, each row's first valid key
// [S] and the end of its window [S], then per query group (kQ rows) the first key of its
// spans [ngroups], the end of its work [ngroups] and the exclusive prefix of its span
// counts [ngroups + 1].  The workgroups are persistent: each walks (group, span) items
// blockIdx.x, blockIdx.x + gridDim.x, ... up to the total, so the launch needs no host copy
// of the geometry.  A row's score for key t goes to column t - (its first key): row s holds
// its window's scores in [0, end - first), every other column is left unwritten.
template <bool kFp8, int kHeadTiles, bool kLin, bool kTnd = false>
__global__ void __launch_bounds__(kThreads, 2)
indexer_tile_kernel(const uint8_t* __restrict__ q, const float* __restrict__ q_scale, const uint8_t* __restrict__ k,
                    const float* __restrict__ k_scale, const float* __restrict__ w, float* __restrict__ scores,
                    int S, int s_k, int64_t ld, int64_t q_offset, int cmp_ratio,
                    const uint8_t* __restrict__ lin_pieces, const float* __restrict__ lin_scale, int fill_masked,
                    const int* __restrict__ tnd = nullptr, int ngroups = 0) {
  using T = IdxTile<kFp8, kHeadTiles>;
  static_assert(!kLin || (kFp8 && T::kQw == 2), "the linear split pairs two fp8 queries per wave");
  constexpr int H = kHeadTiles * 16;
  constexpr int kQw = T::kQw;
  constexpr int kK = T::kKeys;
  __shared__ u32x4 ktile[2][T::kTileBytes / 16];
  __shared__ float stage[T::kQ + 1][kK];  // + a spare row for duplicate lanes
  __shared__ float ksc[2][kK];
  __shared__ int nv_rows[T::kQ];
  __shared__ int kl_rows[kTnd ? T::kQ : 1];
  const int b = blockIdx.z;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int n_items = kTnd ? tnd[2 * S + 3 * ngroups] : 1;
  for (int item = kTnd ? (int)blockIdx.x : 0; item < n_items; item += kTnd ? (int)gridDim.x : 1) {
  int qg = blockIdx.x, t0 = blockIdx.y * T::kSpan, grp_end = 0;
  if constexpr (kTnd) {  // the item's group: the last one whose prefix is <= item
    const int* pfx = tnd + 2 * S + 2 * ngroups;
    int lo = 0, hi = ngroups - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pfx[mid] <= item) lo = mid;
      else hi = mid - 1;
    }
    qg = lo;
    t0 = tnd[2 * S + qg] + (item - pfx[qg]) * T::kSpan;
    grp_end = tnd[2 * S + ngroups + qg];
  }
  const int s0 = qg * T::kQ;
  const int t_end = min(s_k, t0 + T::kSpan);
  const int nrows = min(T::kQ, S - s0);

  // causal frontier: key t is valid for query s iff t < nvalid(s) (monotone in s)
  auto nvalid = [&](int s) -> int {
    const int64_t v = (s + q_offset + 1) / cmp_ratio;
    return (int)max((int64_t)0, min((int64_t)s_k, v));
  };
  const int nv_max = kTnd ? grp_end : nvalid(s0 + nrows - 1);  // last (largest) frontier of the workgroup
  const int t_work = min(t_end, nv_max);      // keys below t_work need MFMA work
  const int64_t q_row0 = (int64_t)b * S;

  if (t_work <= t0) {  // the whole key span lies past every query's frontier
    if (fill_masked) fill_neg_inf(scores, q_row0 + s0, nrows, ld, t0, t_end, tid);
    continue;
  }
  const int nsub = (t_work - t0 + kK - 1) / kK;  // key tiles with work

  // ---- key tile DMA: rows (row r, chunk c at c ^ idx_swz(r)) and key scales ----
  const uint8_t* kb_g = k + ((int64_t)b * s_k) * T::kRowBytes;
  const float* ks_g = k_scale ? k_scale + (int64_t)b * s_k : nullptr;
  auto issue_tile = [&](int sub, int buf) {
    const int tb = t0 + sub * kK;
#pragma unroll
    for (int i = 0; i < T::kDmaPerWave; ++i) {
      const int J = wave + 4 * i;
      const int p = J * 64 + lane;
      const int row = p / T::kCpr, pos = p - row * T::kCpr;
      const int key = min(tb + row, s_k - 1);
      dma16_to_lds(kb_g, (uint32_t)key * T::kRowBytes + 16 * (pos ^ idx_swz<kFp8>(row)),
                   (uint32_t)(uintptr_t)&ktile[buf][J * 64]);
    }
    if (ks_g && 64 * wave < kK)
      dma4_to_lds(ks_g, 4u * (uint32_t)min(tb + 64 * wave + lane, s_k - 1), (uint32_t)(uintptr_t)&ksc[buf][64 * wave]);
  };
  issue_tile(0, 0);
  if (!ks_g) {
    for (int i = tid; i < 2 * kK; i += kThreads) (&ksc[0][0])[i] = 1.f;
  }

  // ---- A operands (queries) and folded head weights, while the DMA is in flight ----
  const int qa = s0 + wave * kQw;
  uint32_t qa_reg[kQw][kHeadTiles][T::kRegsPerTile];
  float wv[kQw][kHeadTiles][4];
#pragma unroll
  for (int j = 0; j < kQw; ++j) {
    const int s = min(qa + j, S - 1);
    const int64_t qrow = (q_row0 + s) * H;
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
      const int head = ht * 16 + col;
      const uint8_t* src = q + (qrow + head) * kD * (kFp8 ? 1 : 2);
      if constexpr (kFp8) {  // lane holds k = 32g .. 32g+31
        const u32x4* p = reinterpret_cast<const u32x4*>(src + 32 * g);
        const u32x4 x0 = p[0], x1 = p[1];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          qa_reg[j][ht][r] = x0[r];
          qa_reg[j][ht][4 + r] = x1[r];
        }
      } else {  // step c: lane holds k = 32c + 8g .. +7
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(src + (32 * c + 8 * g) * 2);
#pragma unroll
          for (int r = 0; r < 4; ++r) qa_reg[j][ht][4 * c + r] = x[r];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int hr = ht * 16 + 4 * g + r;  // C row (head) held by this lane
        const float sc = q_scale ? q_scale[qrow + hr] : 1.f;
        wv[j][ht][r] = w[qrow + hr] * sc * (kLin ? 0.5f : 1.f);
      }
    }
  }
  // linear-split A tile (lane: row col, k = 32g..32g+31): rows 0-3 pieces of query qa,
  // rows 8-11 of query qa + 1; C rows 4g..4g+3 get the pieces' scales (g = 0: qa, g = 2:
  // qa + 1, odd g: zero rows)
  uint32_t la_reg[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float ls[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (kLin) {
    if ((col & 4) == 0) {
      const int s = min(qa + (col >> 3), S - 1);
      const u32x4* p = reinterpret_cast<const u32x4*>(lin_pieces + ((q_row0 + s) * kLinPieces + (col & 3)) * kD + 32 * g);
      const u32x4 x0 = p[0], x1 = p[1];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        la_reg[r] = x0[r];
        la_reg[4 + r] = x1[r];
      }
    }
    if ((g & 1) == 0) {
      const int s = min(qa + (g >> 1), S - 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) ls[r] = lin_scale[(q_row0 + s) * kLinPieces + r];
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) asm volatile("" : "+v"(la_reg[r]));
#pragma unroll
    for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(ls[r]));
  }
  // the operands are forced ready here: a compiler-inserted wait for them inside the tile
  // loop would also wait for the next tile's DMA
#pragma unroll
  for (int j = 0; j < kQw; ++j)
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
#pragma unroll
      for (int r = 0; r < T::kRegsPerTile; ++r) asm volatile("" : "+v"(qa_reg[j][ht][r]));
#pragma unroll
      for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(wv[j][ht][r]));
    }
  if (tid < T::kQ) {
    if constexpr (kTnd) {  // the row's window [first key, end)
      kl_rows[tid] = s0 + tid < S ? tnd[s0 + tid] : 0;
      nv_rows[tid] = s0 + tid < S ? tnd[S + s0 + tid] : 0;
    } else {
      nv_rows[tid] = s0 + tid < S ? nvalid(s0 + tid) : 0;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's tile-0 DMA landed
  __syncthreads();

  for (int sub = 0; sub < nsub; ++sub) {
    const int buf = sub & 1;
    const int tb = t0 + sub * kK;
    // the other buffer was last read before the previous iteration's barriers
    if (sub + 1 < nsub) issue_tile(sub + 1, buf ^ 1);

    // ---- 16-key tiles of this key tile, one software pipeline over (tile, query) items:
    // the MFMAs of the next item (the next query, or query 0 of the next 16-key tile,
    // whose B operand is read from LDS a tile ahead) are issued before the relu * w
    // reduction of the current item reads its results ----
    const lds_char* kt_b = lds_bytes(&ktile[buf][0]);
    const int ntiles = (min(kK, t_work - tb) + 15) >> 4;
    auto read_b = [&](int kt, uint32_t (&kb)[T::kRegsPerTile]) {
      const int row = 16 * kt + col;  // B operand row (key) of this lane
      if constexpr (kFp8) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const u32x4 x = lds_read16(kt_b + row * T::kRowBytes + 16 * ((2 * g + h2) ^ idx_swz<kFp8>(row)));
#pragma unroll
          for (int r = 0; r < 4; ++r) kb[4 * h2 + r] = x[r];
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 x = lds_read16(kt_b + row * T::kRowBytes + 16 * ((4 * c + g) ^ idx_swz<kFp8>(row)));
#pragma unroll
          for (int r = 0; r < 4; ++r) kb[4 * c + r] = x[r];
        }
      }
    };
    auto mfma_q = [&](int j, const uint32_t (&kb)[T::kRegsPerTile], f32x4 (&c)[kHeadTiles]) {
#pragma unroll
      for (int ht = 0; ht < kHeadTiles; ++ht) {
        c[ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if constexpr (kFp8) {
          i32x8 av, bv;
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            av[r] = (int)qa_reg[j][ht][r];
            bv[r] = (int)kb[r];
          }
          c[ht] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c[ht], 0, 0, 0, 0, 0, 0);
        } else {
#pragma unroll
          for (int c4i = 0; c4i < 4; ++c4i) {
            u32x4 av, bv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              av[r] = qa_reg[j][ht][4 * c4i + r];
              bv[r] = kb[4 * c4i + r];
            }
            c[ht] = mfma16x16x32(as_bf16x8(av), as_bf16x8(bv), c[ht]);
          }
        }
      }
    };
    auto mfma_lin = [&](const uint32_t (&kb)[T::kRegsPerTile], f32x4& c) {
      if constexpr (kLin) {
        i32x8 av, bv;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          av[r] = (int)la_reg[r];
          bv[r] = (int)kb[r];
        }
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
      }
    };
    // relu * w partial sum of item (kt, j) over this lane's 16 C values (kLin: |x| * w / 2)
    auto partial = [&](int j, const f32x4 (&c)[kHeadTiles]) -> float {
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int ht = 0; ht < kHeadTiles; ++ht)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          if constexpr (kLin) {
            p0 = fmaf(wv[j][ht][r], fabsf(c[ht][r]), p0);
            p1 = fmaf(wv[j][ht][r + 1], fabsf(c[ht][r + 1]), p1);
          } else {
            p0 = fmaf(wv[j][ht][r], relu_bits(c[ht][r]), p0);
            p1 = fmaf(wv[j][ht][r + 1], relu_bits(c[ht][r + 1]), p1);
          }
        }
      return p0 + p1;
    };
    // one 16-key tile: kQw items, each item's reduction behind the next item's MFMAs; raw
    // head sums are staged (key scale and causal mask are applied when the rows are stored)
    f32x4 cq[2][kHeadTiles];
    // B operands are read kAhead tiles before their first MFMA: two for fp8 (8 registers a
    // tile; three register sets rotate), one for bf16 (16 registers a tile, two sets)
    constexpr int kAhead = kFp8 ? 2 : 1;
    auto tile = [&](int kt, const uint32_t (&kb_cur)[T::kRegsPerTile], const uint32_t (&kb_nxt)[T::kRegsPerTile],
                    uint32_t (&kb_load)[T::kRegsPerTile], const f32x4& cl_cur, f32x4& cl_nxt) {
      read_b(min(kt + kAhead, ntiles - 1), kb_load);  // (the last tiles re-read the last one)
      float pe = 0.f;
#pragma unroll
      for (int j = 0; j < kQw; ++j) {
        // item (kt, j) is in cq[j & 1] (kQw is even, or 1 with the copy below)
        if (j + 1 < kQw) {
          mfma_q(j + 1, kb_cur, cq[(j + 1) & 1]);
        } else {
          mfma_q(0, kb_nxt, cq[(j + 1) & 1]);
          mfma_lin(kb_nxt, cl_nxt);
        }
        const float pj = partial(j, cq[j & 1]);
        if constexpr (kQw == 1) {
          const float v = xor32_sum(xor16_sum(pj));
          if (g == 0) stage[wave][16 * kt + col] = v;
        } else if ((j & 1) == 0) {
          pe = pj;
        } else {
          // queries j-1 and j together: a 32-lane swap leaves query j-1's sums over lane
          // groups {g, g^2} in lanes 0-31 and query j's in lanes 32-63; a 16-lane swap
          // completes both (lane groups 0,1 hold query j-1, groups 2,3 query j)
          const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(pe), __float_as_uint(pj), false, false);
          float h = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
          if constexpr (kLin)  // u . k of this lane group's query (zero in odd groups)
            h += cl_cur[0] * ls[0] + cl_cur[1] * ls[1] + cl_cur[2] * ls[2] + cl_cur[3] * ls[3];
          const float v = xor16_sum(h);
          // lane groups 1 and 3 hold copies: they write the spare row (no branch, so the
          // tile stays one scheduling region)
          stage[(g & 1) ? T::kQ : wave * kQw + j - 1 + (g >> 1)][16 * kt + col] = v;
        }
      }
      if constexpr (kQw == 1) {  // one query: the next tile's item went to cq[1]
#pragma unroll
        for (int ht = 0; ht < kHeadTiles; ++ht) cq[0][ht] = cq[1][ht];
      }
      if constexpr (kFp8) {
        // each MFMA followed by VALU work of the reductions (left to itself the scheduler
        // issues a tile's first item as one run of MFMAs)
#pragma unroll
        for (int i = 0; i < kQw * kHeadTiles + (kLin ? 1 : 0); ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
        }
      }
    };
    uint32_t kb_a[T::kRegsPerTile], kb_b[T::kRegsPerTile], kb_c[kAhead > 1 ? T::kRegsPerTile : 1];
    f32x4 cl_a = (f32x4){0.f, 0.f, 0.f, 0.f}, cl_b = cl_a, cl_c = cl_a;
    read_b(0, kb_a);
    if constexpr (kAhead > 1) read_b(min(1, ntiles - 1), kb_b);
    mfma_q(0, kb_a, cq[0]);
    mfma_lin(kb_a, cl_a);
    if constexpr (kAhead > 1) {
      for (int kt = 0; kt < ntiles; kt += 3) {  // three tiles per trip: the B registers rotate
        tile(kt, kb_a, kb_b, kb_c, cl_a, cl_b);
        if (kt + 1 < ntiles) tile(kt + 1, kb_b, kb_c, kb_a, cl_b, cl_c);
        if (kt + 2 < ntiles) tile(kt + 2, kb_c, kb_a, kb_b, cl_c, cl_a);
      }
    } else {
      for (int kt = 0; kt < ntiles; kt += 2) {  // two tiles per trip: the B registers alternate
        tile(kt, kb_a, kb_b, kb_b, cl_a, cl_b);
        if (kt + 1 < ntiles) tile(kt + 1, kb_b, kb_a, kb_a, cl_b, cl_a);
      }
    }
    __syncthreads();  // the tile's scores are staged

    // ---- scores out: whole rows; keys past t_work are -inf (beyond every frontier) ----
    float4 v[T::kStoreIters];
#pragma unroll
    for (int it = 0; it < T::kStoreIters; ++it) {
      const int i = tid + kThreads * it;
      const int qi = min(i / (kK / 4), T::kQ - 1), kk = 4 * (i % (kK / 4));
      // key t of row qi is valid iff t < nv_rows[qi] (<= t_work: staged keys past it are
      // never read)
      const int lim = nv_rows[qi] - tb - kk;
      const float4 x = *reinterpret_cast<const float4*>(&stage[qi][kk]);
      const float4 sc = *reinterpret_cast<const float4*>(&ksc[buf][kk]);
      v[it].x = 0 < lim ? x.x * sc.x : -INFINITY;
      v[it].y = 1 < lim ? x.y * sc.y : -INFINITY;
      v[it].z = 2 < lim ? x.z * sc.z : -INFINITY;
      v[it].w = 3 < lim ? x.w * sc.w : -INFINITY;
    }
    // next tile landed (this wave's DMA; the stores issued one iteration ago are long
    // done), and every wave has read the stage
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int it = 0; it < T::kStoreIters; ++it) {
      const int i = tid + kThreads * it;
      if (i >= T::kQ * (kK / 4)) break;
      const int qi = i / (kK / 4), kk = 4 * (i % (kK / 4));
      const int t = tb + kk;
      if (qi >= nrows || t >= t_end) continue;
      if constexpr (kTnd) {  // keys of the row's window only, at column key - first key
        const int kl = kl_rows[qi], end = nv_rows[qi];
        float* rowp = scores + (q_row0 + s0 + qi) * ld;
        const float vv[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t + e >= kl && t + e < end) rowp[t + e - kl] = vv[e];
        continue;
      }
      float* dst = scores + (q_row0 + s0 + qi) * ld + t;
      if (t + 4 <= t_end && (((uintptr_t)dst) & 15) == 0) {
        *reinterpret_cast<float4*>(dst) = v[it];
      } else {
        const float vv[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
        for (int e = 0; e < 4 && t + e < t_end; ++e) dst[e] = vv[e];
      }
    }
  }
  // key tiles of the span past every frontier
  if (fill_masked) fill_neg_inf(scores, q_row0 + s0, nrows, ld, t0 + nsub * kK, t_end, tid);
  if constexpr (kTnd) __syncthreads();  // the next item rewrites the row windows and tiles
  }
}

// Generic path (any H, D; fp32 arithmetic): one thread per (query, key).
template <typename T>
__device__ __forceinline__ float ldx(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldx<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldx<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f(p[i]); }
__device__ __forceinline__ float fp8_to_f(uint8_t v) {
  const int sgn = v >> 7, e = (v >> 3) & 15, m = v & 7;
  float r;
  if (e == 0) r = ldexpf((float)m / 8.f, -6);
  else if (e == 15 && m == 7) r = __int_as_float(0x7fc00000);
  else r = ldexpf(1.f + (float)m / 8.f, e - 7);
  return sgn ? -r : r;
}
template <>
__device__ __forceinline__ float ldx<uint8_t>(const uint8_t* p, int64_t i) { return fp8_to_f(p[i]); }

template <typename T>
__global__ void __launch_bounds__(256)
indexer_generic_kernel(const T* __restrict__ q, const float* __restrict__ q_scale, const T* __restrict__ k,
                       const float* __restrict__ k_scale, const float* __restrict__ w, float* __restrict__ scores,
                       int S, int s_k, int H, int D, int64_t ld, int64_t q_offset, int cmp_ratio) {
  const int s = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= s_k) return;
  const int64_t qrow = (int64_t)b * S + s;
  const int64_t v = (s + q_offset + 1) / cmp_ratio;
  const int nv = (int)max((int64_t)0, min((int64_t)s_k, v));
  float out = -INFINITY;
  if (t < nv) {
    const int64_t krow = (int64_t)b * s_k + t;
    float acc = 0.f;
    for (int h = 0; h < H; ++h) {
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(ldx(q, (qrow * H + h) * D + d), ldx(k, krow * D + d), dot);
      const float sc = q_scale ? q_scale[qrow * H + h] : 1.f;
      acc = fmaf(w[qrow * H + h] * sc, fmaxf(dot, 0.f), acc);
    }
    out = acc * (k_scale ? k_scale[krow] : 1.f);
  }
  scores[qrow * ld + t] = out;
}

// the linear split applies to the fp8 H_I = 64, D_I = 128 tile kernel (two queries per wave)
bool lin_split_shape(int dtype, int64_t n_heads, int64_t head_dim) {
  return dtype == DSA_FP8_E4M3 && n_heads == 64 && head_dim == kD;
}

}  // namespace

int indexer_fwd(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                int64_t head_dim, int64_t ld_scores, int64_t q_offset, int64_t cmp_ratio, void* workspace,
                int64_t workspace_bytes, void* stream, bool fill_masked) {
  const int fm = fill_masked ? 1 : 0;
  if (!q || !k || !w || !scores) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || n_heads <= 0 || head_dim <= 0 || ld_scores < s_k || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: bad sizes");
  if (s_q > 2147483647LL || batch > 65535 || s_k > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  const bool mfma_shape = head_dim == kD && n_heads % 16 == 0 && n_heads <= 128 && dtype != DSA_F32;
  // the tile kernels address key rows of one batch with 32-bit byte offsets
  const int64_t key_row_bytes = head_dim * (dtype == DSA_FP8_E4M3 ? 1 : 2);
  if (mfma_shape && s_k > (int64_t)(0xffffffffu / key_row_bytes))
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: %lld keys exceed the tile kernels' 32-bit key offsets "
                     "(at most %lld keys of %lld bytes)", (long long)s_k,
                     (long long)(0xffffffffu / key_row_bytes), (long long)key_row_bytes);
  if (workspace && lin_split_shape(dtype, n_heads, head_dim)) {
    const int64_t rows = batch * s_q;
    if (workspace_bytes < rows * kLinRowBytes)
      return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd_ws: workspace of %lld bytes, %lld needed",
                       (long long)workspace_bytes, (long long)(rows * kLinRowBytes));
    uint8_t* pieces = (uint8_t*)workspace;
    float* pscale = (float*)(pieces + rows * kLinPieces * kD);
    const uint8_t* qp = (const uint8_t*)q;
    {
      const TimedLaunch tl("indexer_lin_pieces_kernel<64>", st);
      indexer_lin_pieces_kernel<64><<<(unsigned)ceil_div(rows, kThreads / 64), kThreads, 0, st>>>(qp, q_scale, w,
                                                                                                 pieces, pscale, rows);
    }
    using Tl = IdxTile<true, 4>;
    dim3 grid(ceil_div(s_q, Tl::kQ), ceil_div(s_k, Tl::kSpan), (unsigned)batch);
    const TimedLaunch tl("indexer_tile_kernel<fp8, 4, split>", st);
    indexer_tile_kernel<true, 4, true><<<grid, kThreads, 0, st>>>(qp, q_scale, (const uint8_t*)k, k_scale, w, scores,
                                                                  (int)s_q, (int)s_k, ld_scores, q_offset,
                                                                  (int)cmp_ratio, pieces, pscale, fm);
    return check_launch("dsa_indexer_fwd_ws(mfma, linear split)");
  }
  if (mfma_shape) {
    const uint8_t* qp = (const uint8_t*)q;
    const uint8_t* kp = (const uint8_t*)k;
#define DSA_IDX_LAUNCH(FP8, HT)                                                                                   \
  do {                                                                                                             \
    using Tl = IdxTile<FP8, HT>;                                                                                   \
    dim3 grid(ceil_div(s_q, Tl::kQ), ceil_div(s_k, Tl::kSpan), (unsigned)batch);                                          \
    const TimedLaunch tl("indexer_tile_kernel", st);                                                               \
    indexer_tile_kernel<FP8, HT, false><<<grid, kThreads, 0, st>>>(qp, q_scale, kp, k_scale, w, scores, (int)s_q,      \
                                                                   (int)s_k, ld_scores, q_offset, (int)cmp_ratio,   \
                                                                   nullptr, nullptr, fm);                          \
  } while (0)
    const int ht = (int)(n_heads / 16);
    if (dtype == DSA_FP8_E4M3) {
      switch (ht) {
        case 1: DSA_IDX_LAUNCH(true, 1); break;
        case 2: DSA_IDX_LAUNCH(true, 2); break;
        case 4: DSA_IDX_LAUNCH(true, 4); break;
        case 8: DSA_IDX_LAUNCH(true, 8); break;
        default: return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: H_I=%lld", (long long)n_heads);
      }
    } else if (dtype == DSA_BF16) {
      switch (ht) {
        case 1: DSA_IDX_LAUNCH(false, 1); break;
        case 2: DSA_IDX_LAUNCH(false, 2); break;
        case 4: DSA_IDX_LAUNCH(false, 4); break;
        case 8: DSA_IDX_LAUNCH(false, 8); break;
        default: return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: H_I=%lld", (long long)n_heads);
      }
    } else {
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: dtype %d", dtype);
    }
#undef DSA_IDX_LAUNCH
    return check_launch("dsa_indexer_fwd(mfma)");
  }
  dim3 grid(ceil_div(s_k, 256), (unsigned)s_q, (unsigned)batch);
  if (s_q > 65535) return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: generic path needs S <= 65535");
  switch (dtype) {
    case DSA_F32:
      indexer_generic_kernel<float><<<grid, 256, 0, st>>>((const float*)q, q_scale, (const float*)k, k_scale, w,
                                                          scores, (int)s_q, (int)s_k, (int)n_heads, (int)head_dim,
                                                          ld_scores, q_offset, (int)cmp_ratio);
      break;
    case DSA_BF16:
      indexer_generic_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)q, q_scale, (const uint16_t*)k,
                                                             k_scale, w, scores, (int)s_q, (int)s_k, (int)n_heads,
                                                             (int)head_dim, ld_scores, q_offset, (int)cmp_ratio);
      break;
    case DSA_FP8_E4M3:
      indexer_generic_kernel<uint8_t><<<grid, 256, 0, st>>>((const uint8_t*)q, q_scale, (const uint8_t*)k, k_scale,
                                                            w, scores, (int)s_q, (int)s_k, (int)n_heads,
                                                            (int)head_dim, ld_scores, q_offset, (int)cmp_ratio);
      break;
    default:
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_fwd: dtype %d", dtype);
  }
  return check_launch("dsa_indexer_fwd(generic)");
}

// ----- packed rows with device geometry -----
bool indexer_tnd_tiling(int dtype, int64_t n_heads, int64_t head_dim, int* group_rows, int* span_keys) {
  if (head_dim != kD || n_heads % 16 != 0 || n_heads > 128 || (dtype != DSA_FP8_E4M3 && dtype != DSA_BF16))
    return false;
  const int ht = (int)(n_heads / 16);
  const bool fp8 = dtype == DSA_FP8_E4M3;
  // IdxTile<fp8, ht>: kQ = 4 * kQw, kSpan = 4 * (32768 / row bytes)
  const int qw = fp8 ? (8 / ht > 0 ? 8 / ht : 1) : (4 / ht > 0 ? 4 / ht : 1);
  *group_rows = 4 * qw;
  *span_keys = 4 * (32768 / (kD * (fp8 ? 1 : 2)));
  return true;
}

namespace {
// persistent workgroups of the packed-row launches: two per CU (the tile kernels' occupancy)
int tnd_workgroups(hipStream_t st) {
  static int cus[64] = {};
  int dev = 0;
  if (hipStreamGetDevice(st, &dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return 2 * cus[dev];
}
}  // namespace

int indexer_fwd_tnd(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                    float* scores, int dtype, int64_t rows, int64_t s_k, int64_t n_heads, int64_t head_dim,
                    int64_t ld_scores, const int* tnd, int64_t ngroups, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  const char* what = "dsa_lightning_indexer_tnd";
  int gr = 0, sk = 0;
  if (!indexer_tnd_tiling(dtype, n_heads, head_dim, &gr, &sk))
    return set_error(DSA_ERR_UNSUPPORTED, "%s: H_I=%lld, D_I=%lld, dtype %d has no tile kernel (H_I a multiple of 16 "
                     "up to 128, D_I 128, bf16 or fp8)", what, (long long)n_heads, (long long)head_dim, dtype);
  if (!q || !k || !w || !scores || !tnd) return set_error(DSA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (rows <= 0 || s_k <= 0 || ld_scores < s_k || rows > 2147483647LL || s_k > 2147483647LL ||
      ngroups != (rows + gr - 1) / gr)
    return set_error(DSA_ERR_INVALID_ARG, "%s: bad sizes", what);
  const int64_t key_row_bytes = head_dim * (dtype == DSA_FP8_E4M3 ? 1 : 2);
  if (s_k > (int64_t)(0xffffffffu / key_row_bytes))
    return set_error(DSA_ERR_UNSUPPORTED, "%s: %lld keys exceed the tile kernels' 32-bit key offsets", what,
                     (long long)s_k);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)tnd_workgroups(st), 1, 1);
  const uint8_t* qp = (const uint8_t*)q;
  const uint8_t* kp = (const uint8_t*)k;
  const int S = (int)rows, n = (int)s_k, G = (int)ngroups;
  if (lin_split_shape(dtype, n_heads, head_dim)) {
    if (!workspace || workspace_bytes < rows * kLinRowBytes)
      return set_error(DSA_ERR_INVALID_ARG, "%s: workspace of %lld bytes, %lld needed for the linear split", what,
                       (long long)workspace_bytes, (long long)(rows * kLinRowBytes));
    uint8_t* pieces = (uint8_t*)workspace;
    float* pscale = (float*)(pieces + rows * kLinPieces * kD);
    {
      const TimedLaunch tl("indexer_lin_pieces_kernel<64>", st);
      indexer_lin_pieces_kernel<64><<<(unsigned)ceil_div(rows, kThreads / 64), kThreads, 0, st>>>(qp, q_scale, w,
                                                                                                 pieces, pscale, rows);
    }
    const TimedLaunch tl("indexer_tile_kernel<fp8, 4, split, tnd>", st);
    indexer_tile_kernel<true, 4, true, true><<<grid, kThreads, 0, st>>>(qp, q_scale, kp, k_scale, w, scores, S, n,
                                                                        ld_scores, 0, 1, pieces, pscale, 0, tnd, G);
    return check_launch("dsa_lightning_indexer_tnd(linear split)");
  }
#define DSA_IDX_TND(FP8, HT)                                                                                      \
  do {                                                                                                             \
    const TimedLaunch tl("indexer_tile_kernel<tnd>", st);                                                          \
    indexer_tile_kernel<FP8, HT, false, true><<<grid, kThreads, 0, st>>>(qp, q_scale, kp, k_scale, w, scores, S, n, \
                                                                         ld_scores, 0, 1, nullptr, nullptr, 0, tnd, \
                                                                         G);                                       \
  } while (0)
  const bool fp8 = dtype == DSA_FP8_E4M3;
  switch ((int)(n_heads / 16) * 2 + (fp8 ? 1 : 0)) {
    case 2: DSA_IDX_TND(false, 1); break;
    case 3: DSA_IDX_TND(true, 1); break;
    case 4: DSA_IDX_TND(false, 2); break;
    case 5: DSA_IDX_TND(true, 2); break;
    case 8: DSA_IDX_TND(false, 4); break;
    case 9: DSA_IDX_TND(true, 4); break;
    case 16: DSA_IDX_TND(false, 8); break;
    case 17: DSA_IDX_TND(true, 8); break;
    default: return set_error(DSA_ERR_UNSUPPORTED, "%s: H_I=%lld", what, (long long)n_heads);
  }
#undef DSA_IDX_TND
  return check_launch("dsa_lightning_indexer_tnd");
}

}  // namespace dsa

extern "C" int dsa_indexer_fwd(const void* q, const float* q_scale, const void* k, const float* k_scale,
                               const float* w, float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k,
                               int64_t n_heads, int64_t head_dim, int64_t ld_scores, int64_t q_offset,
                               int64_t cmp_ratio, void* stream) {
  return dsa::indexer_fwd(q, q_scale, k, k_scale, w, scores, dtype, batch, s_q, s_k, n_heads, head_dim, ld_scores,
                          q_offset, cmp_ratio, nullptr, 0, stream, true);
}

extern "C" int64_t dsa_indexer_fwd_workspace_size(int64_t batch, int64_t s_q, int64_t n_heads, int64_t head_dim,
                                                  int dtype) {
  if (batch <= 0 || s_q <= 0 || !dsa::lin_split_shape(dtype, n_heads, head_dim)) return 0;
  return batch * s_q * dsa::kLinRowBytes;
}

extern "C" int dsa_indexer_fwd_ws(const void* q, const float* q_scale, const void* k, const float* k_scale,
                                  const float* w, float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k,
                                  int64_t n_heads, int64_t head_dim, int64_t ld_scores, int64_t q_offset,
                                  int64_t cmp_ratio, void* workspace, int64_t workspace_bytes, void* stream) {
  return dsa::indexer_fwd(q, q_scale, k, k_scale, w, scores, dtype, batch, s_q, s_k, n_heads, head_dim, ld_scores,
                          q_offset, cmp_ratio, workspace, workspace_bytes, stream, true);
}

// ----- the entry point that allocates nothing -----
// Scratch of dsa_indexer_fwd_noalloc: the linear-split pieces of up to kNoAllocRows query rows,
// in device memory that the code object carries (each GPU the library runs on holds its own
// copy until the process ends).  Host code never passes `scratch` itself to a kernel: its
// host-side name is not a device address.  The device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static constexpr int64_t kNoAllocScratchBytes = 32ll << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace dsa {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (looked up on first use).
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(DSA_ERR_LAUNCH, "dsa_indexer_fwd_noalloc: cannot tell the stream's device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return set_error(DSA_ERR_LAUNCH, "dsa_indexer_fwd_noalloc: hipGetDevice");
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return set_error(DSA_ERR_LAUNCH, "dsa_indexer_fwd_noalloc: hipSetDevice(%d)", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return set_error(DSA_ERR_LAUNCH, "dsa_indexer_fwd_noalloc: hipGetSymbolAddress(scratch): %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DSA_OK;
}
}  // namespace
}  // namespace dsa

extern "C" int64_t dsa_indexer_fwd_noalloc_max_rows(void) { return kNoAllocScratchBytes / dsa::kLinRowBytes; }

extern "C" int dsa_indexer_fwd_noalloc(const void* q, const float* q_scale, const void* k, const float* k_scale,
                                       const float* w, float* scores, int dtype, int64_t batch, int64_t s_q,
                                       int64_t s_k, int64_t n_heads, int64_t head_dim, int64_t ld_scores,
                                       int64_t q_offset, int64_t cmp_ratio, void* stream) {
  if (!dsa::lin_split_shape(dtype, n_heads, head_dim))  // no scratch on these shapes
    return dsa::indexer_fwd(q, q_scale, k, k_scale, w, scores, dtype, batch, s_q, s_k, n_heads, head_dim,
                            ld_scores, q_offset, cmp_ratio, nullptr, 0, stream, true);
  if (batch <= 0 || s_q <= 0) return dsa::set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd_noalloc: bad sizes");
  const int64_t max_rows = dsa_indexer_fwd_noalloc_max_rows();
  if (batch > max_rows || s_q > max_rows / batch)
    return dsa::set_error(DSA_ERR_INVALID_ARG,
                          "dsa_indexer_fwd_noalloc: %lld query rows exceed the static scratch (%lld rows of %lld "
                          "bytes); split the rows over several calls or use dsa_indexer_fwd_ws",
                          (long long)(batch * s_q), (long long)max_rows, (long long)dsa::kLinRowBytes);
  void* ws = nullptr;
  const int rc = dsa::noalloc_scratch((hipStream_t)stream, &ws);
  if (rc != DSA_OK) return rc;
  return dsa::indexer_fwd(q, q_scale, k, k_scale, w, scores, dtype, batch, s_q, s_k, n_heads, head_dim, ld_scores,
                          q_offset, cmp_ratio, ws, batch * s_q * dsa::kLinRowBytes, stream, true);
}
