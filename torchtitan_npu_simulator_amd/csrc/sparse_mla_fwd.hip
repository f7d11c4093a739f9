// Gathered sparse MLA attention forward for gfx950.
//
// One workgroup = one query token x up to 128 heads, 8 waves.  The token's selected
// latent-KV rows (576 bf16 = 1152 B each) are gathered in blocks of 32 into an LDS tile
// that all heads share, so each row crosses HBM/L2 once per token, not once per head.
// Wave w owns head group g = w & 3 (32 heads) and half h = w >> 2:
//   * QK: S^T[32 keys x 32 heads] partial over its half of the contraction (latent
//     columns 256h..256h+255 from VGPRs plus rope columns 512+32h..+31 from LDS) with
//     v_mfma_f32_32x32x16_bf16; the two halves swap partial S through LDS and add.
//   * softmax per head in the exp2 domain against a reference max fixed by the first
//     valid block: no per-block O rescale (P may reach 2^64, well inside the fp32/bf16
//     exponent range).  A row whose later logits outgrow that headroom is flagged with a
//     negative softmax_sum and recomputed exactly by the fixup pass.
//   * PV: O^T[256 dv of half h x 32 heads] += V^T . P^T, V read with ds_read_tr16_b64
//     straight from the row-major K tile (k_nope == v), so no transposed copy exists.
// Per-wave state: 128 AGPRs of O, 16 of S, ~64 VGPRs of Q: two waves fit per SIMD.
// The next block's rows are DMA'd straight into the other LDS buffer (global_load_lds,
// 16 B per lane) while the current block computes.
#include "dsa_common.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kRowChunks = kDqk / 8;           // 16-byte chunks per KV row (72)
constexpr int kRowBytes = kRowChunks * 16;     // 1152
constexpr int kBN = 32;                        // keys per block
constexpr int kTileChunks = kBN * kRowChunks;  // 2304
constexpr int kTileBytes = kTileChunks * 16;   // 36864
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kTileInstr = kTileChunks / 64;   // 36 wave-wide DMA instructions per tile
constexpr int kHeadsPerWG = 128;
constexpr int kQSteps = 16;                    // 16-column MFMA steps of latent Q per wave
constexpr float kHeadroom = 64.0f;             // log2 units of P above the reference max
constexpr int64_t kMaxGatherRows = (int64_t)UINT32_MAX / kRowBytes - 1;  // 32-bit byte offsets into kv
constexpr int kQBatch = 3;                     // LDS A-operand loads issued ahead of their MFMAs
constexpr int kVBatch = 2;                     // transposed V reads issued ahead of their MFMAs

__device__ __forceinline__ bool slot_ok(int v, int s_kv, int64_t limit) {
  return v >= 0 && v < s_kv && (int64_t)v <= limit;
}

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// ---- gathered tile loader shared by the forward and mass kernels ----
// A block tile is kBN rows x 72 16-byte chunks, filled by 36 wave-wide DMA instructions
// (global_load_lds, 16 B per lane): instruction J covers tile positions [64J, 64J+64),
// position p = row*72 + (chunk ^ swz8(row)), and wave w issues J = w, w+8, ...
// The slot indices reach a 4-entry LDS ring two blocks ahead of their DMA: wave 0 loads
// block b+3's indices into a register while block b computes and stores them into the
// ring one block later, so neither an index round trip nor a register spill sits in
// front of a gather (a spill reload would wait for every DMA in flight).
constexpr int kLoadsPerWave = (kTileInstr + kWaves - 1) / kWaves;  // 5
constexpr int kIdxRing = 4;

__device__ __forceinline__ int opaque(int x) {
  // keeps lane-derived addressing inside the loop (recomputed, not hoisted and spilled)
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ void issue_block(const uint16_t* kvb, u32x4* tile_buf, uint32_t* vmask_slot,
                                            const int* sidx, int blk, int K, uint32_t lim, int wave, int lane_in) {
  // a slot is usable when its index is in [0, lim] (lim = min(causal limit, S_kv - 1);
  // negative indices wrap to large unsigned values) and it lies before K
  const int rows_left = K - blk * kBN;
  const int lane = opaque(lane_in);
  const char* base = reinterpret_cast<const char*>(kvb);
  uint32_t raw[kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int J = min(wave + kWaves * i, kTileInstr - 1);
    raw[i] = (uint32_t)sidx[(J * 64 + lane) / kRowChunks];
  }
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int J = wave + kWaves * i;
    if (J < kTileInstr) {
      const int p = J * 64 + lane;
      const int row = p / kRowChunks, pos = p - row * kRowChunks;
      const bool ok = raw[i] <= lim && row < rows_left;
      const uint32_t off = (ok ? raw[i] : 0u) * (uint32_t)kRowBytes + (uint32_t)((pos ^ swz8(row)) * 16);
      __builtin_amdgcn_global_load_lds((const void*)(base + off),
                                       (__attribute__((address_space(3))) void*)&tile_buf[J * 64], 16, 0, 0);
    }
  }
  if (wave == 0) {
    const bool ok = lane < kBN && lane < rows_left && (uint32_t)sidx[lane & (kBN - 1)] <= lim;
    const uint64_t bal = __ballot(ok);
    if (lane == 0) *vmask_slot = (uint32_t)bal;
  }
}

// Index pipeline state of wave 0: the indices of block `blk` (lane < kBN), clamped to K.
__device__ __forceinline__ int load_block_idx(const int32_t* ridx, int K, int blk, int lane) {
  return ridx[min(blk * kBN + (lane & (kBN - 1)), K - 1)];
}

// Prologue: ring entries 0 and 1 hold blocks 0 and 1, `pending` holds block 2.
__device__ __forceinline__ void idx_ring_init(int (*sidx)[kBN], const int32_t* ridx, int K, int nblk, int wave,
                                              int lane, int& pending) {
  if (wave == 0) {
    const int i0 = load_block_idx(ridx, K, 0, lane);
    const int i1 = load_block_idx(ridx, K, 1, lane);
    if (lane < kBN) {
      sidx[0][lane] = i0;
      sidx[1][lane] = i1;
    }
    if (nblk > 2) pending = load_block_idx(ridx, K, 2, lane);
  }
}

// Iteration blk (after issuing block blk+1 from ring entry (blk+1)&3): store block blk+2
// into the ring and start loading block blk+3.  The barrier that ends the iteration makes
// the entry visible and the waitcnt before it lands `pending`.
__device__ __forceinline__ void idx_ring_advance(int (*sidx)[kBN], const int32_t* ridx, int K, int nblk, int blk,
                                                 int wave, int lane, int& pending) {
  if (wave == 0 && blk + 2 < nblk) {
    if (lane < kBN) sidx[(blk + 2) & (kIdxRing - 1)][lane] = pending;
    if (blk + 3 < nblk) pending = load_block_idx(ridx, K, blk + 3, lane);
  }
}

__global__ void __launch_bounds__(kThreads, 1)
sparse_mla_fwd_bf16_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv,
                           const int32_t* __restrict__ idx, uint16_t* __restrict__ out, float* __restrict__ smax,
                           float* __restrict__ ssum, int S, int s_kv, int H, int K, float scale_log2,
                           int64_t q_offset) {
  __shared__ u32x4 tile[2][kTileChunks];
  __shared__ u32x4 qpe[kHeadsPerWG][(kDqk - kDv) / 8];  // [head][16 B chunk] of q[:, 512:576]
  __shared__ f32x4 xs[kWaves][4][64];                   // partial S exchange, [wave][r/4][lane]
  __shared__ uint32_t vmask[2];
  __shared__ int sidx[kIdxRing][kBN];
  __shared__ int last_slot;

  const int tok = blockIdx.x;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, n = lane & 31, hh = lane >> 5;
  const int grp = wave & 3, half = wave >> 2;
  const int head = blockIdx.y * kHeadsPerWG + grp * 32 + n;
  const bool head_ok = head < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const int64_t lim64 = min(limit, (int64_t)s_kv - 1);  // largest usable key index
  const uint32_t lim = lim64 < 0 ? 0u : (uint32_t)lim64;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kDqk;
  const int64_t out_row = row_id * H + head;

  // ---- how many slot blocks hold a valid key (trailing -1 padding is skipped) ----
  if (tid == 0) last_slot = -1;
  __syncthreads();
  {
    int last = -1;
    for (int j = tid; j < K; j += kThreads)
      if (slot_ok(ridx[j], s_kv, limit)) last = j;
    if (last >= 0) atomicMax(&last_slot, last);
  }
  __syncthreads();
  const int nblk = (last_slot + kBN) / kBN;  // 0 when no valid slot
  if (nblk == 0) {
    if (head_ok) {
      uint32_t* o32 = reinterpret_cast<uint32_t*>(out + out_row * kDv) + half * (kDv / 4);
      for (int i = hh; i < kDv / 4; i += 2) o32[i] = 0u;
      if (half == 0 && hh == 0) {
        smax[out_row] = -INFINITY;
        ssum[out_row] = 0.f;
      }
    }
    return;
  }

  // ---- Q: latent columns 256*half .. +255 into VGPRs (qr[c] = q[256h + 16c + 8hh .. +8]);
  // the rope columns of all heads into LDS ----
  u32x4 qr[kQSteps];
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + out_row * kDqk);
#pragma unroll
    for (int c = 0; c < kQSteps; ++c)
      qr[c] = head_ok ? qh[32 * half + 2 * c + hh] : (u32x4){0u, 0u, 0u, 0u};
    if (half == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int ch = 2 * c + hh;  // 0..7
        qpe[grp * 32 + n][ch ^ (n & 7)] = head_ok ? qh[2 * (kDv / 16) + ch] : (u32x4){0u, 0u, 0u, 0u};
      }
    }
  }

  // ---- LDS byte offsets ----
  // QK A operand: key row n, chunk (32h + 2c + hh) ^ swz8(n) for latent step c; with
  // c = 4k + c' the XOR only touches the low 3 bits, so offset = qk_off[c'] + 128 k.
  const uint32_t tile_base = (uint32_t)(uintptr_t)(&tile[0][0]);
  const int xsw = swz8(n);
  uint32_t qk_off[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) qk_off[c4] = n * kRowBytes + 512 * half + 16 * ((2 * c4 + hh) ^ xsw);
  // rope steps: chunk 64 + 4h + 2c + hh (c = 0, 1)
  uint32_t pe_off[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) pe_off[c] = n * kRowBytes + 16 * ((64 + 4 * half + 2 * c + hh) ^ xsw);
  // Transposed V reads: 16-lane group G = lane/16 covers dv sub-half (G & 1) and k-half hh;
  // source lane s16 supplies key row 16c + 4hh + s16/4 (+8 for the second read) and dv
  // columns 256h + 32t + 16(G&1) + 4(s16%4) .. +3 -> chunk (32h + 4t + cl) ^ swz.
  // With t = 2u + t0: tr_off[t0] + 128 u (+ 18432 c, + 9216 for the second read).
  const int s16 = lane & 15;
  const int tr_row0 = 4 * hh + (s16 >> 2);
  const int tr_swz = swz8(tr_row0);
  const int tr_cl = 2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1);
  uint32_t tr_off[2];
#pragma unroll
  for (int t0 = 0; t0 < 2; ++t0)
    tr_off[t0] = tr_row0 * kRowBytes + 512 * half + 16 * ((4 * t0 + tr_cl) ^ tr_swz) + 8 * (s16 & 1);

  f32x16 o[kDv / 64];
#pragma unroll
  for (int t = 0; t < kDv / 64; ++t) o[t] = (f32x16){0};
  float m_ref = -INFINITY, m_true = -INFINITY, lsum = 0.f;
  bool clamped = false;

  int pending = 0;
  idx_ring_init(sidx, ridx, K, nblk, wave, lane, pending);
  __syncthreads();
  issue_block(kvb, tile[0], &vmask[0], sidx[0], 0, K, lim, wave, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    if (blk + 1 < nblk)
      issue_block(kvb, tile[buf ^ 1], &vmask[buf ^ 1], sidx[(blk + 1) & (kIdxRing - 1)], blk + 1, K, lim, wave, lane);
    idx_ring_advance(sidx, ridx, K, nblk, blk, wave, lane, pending);
    const uint32_t tb = tile_base + buf * kTileBytes;

    // ---- partial S^T over this wave's half of the contraction ----
    // A operands (key rows) are fetched from LDS in batches ahead of their MFMAs; the
    // sched_barrier keeps a batch together so its LDS latency overlaps the previous
    // batch's MFMAs.  B operands are the Q registers (rope steps: LDS).
    f32x16 s = (f32x16){0};
#pragma unroll
    for (int cb = 0; cb < kQSteps + 2; cb += kQBatch) {
      u32x4 a[kQBatch];
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) {
        const int c = cb + u;
        if (c < kQSteps) a[u] = *(const lds_u32x4*)(uintptr_t)(tb + qk_off[c & 3] + 128 * (c >> 2));
        else if (c < kQSteps + 2) a[u] = *(const lds_u32x4*)(uintptr_t)(tb + pe_off[c - kQSteps]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) {
        const int c = cb + u;
        if (c < kQSteps) {
          s = mfma32x32x16(as_bf16x8(a[u]), as_bf16x8(qr[c]), s);
        } else if (c < kQSteps + 2) {
          const u32x4 bq = qpe[grp * 32 + n][(4 * half + 2 * (c - kQSteps) + hh) ^ (n & 7)];
          s = mfma32x32x16(as_bf16x8(a[u]), as_bf16x8(bq), s);
        }
      }
    }
    // ---- swap partial S with the other half of the pair ----
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      xs[wave][r4][lane] = (f32x4){s[4 * r4], s[4 * r4 + 1], s[4 * r4 + 2], s[4 * r4 + 3]};
    __syncthreads();
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 other = xs[wave ^ 4][r4][lane];
      s[4 * r4] += other[0];
      s[4 * r4 + 1] += other[1];
      s[4 * r4 + 2] += other[2];
      s[4 * r4 + 3] += other[3];
    }

    // ---- mask, scale, block max (lane holds keys 8(r/4) + 4hh + r%4 of head n) ----
    const uint32_t vm = vmask[buf];
    float rmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * hh + (r & 3);
      const float x = ((vm >> key) & 1u) ? s[r] * scale_log2 : -INFINITY;
      s[r] = x;
      rmax = fmaxf(rmax, x);
    }
    rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
    // (a block with no valid slot leaves every s at -inf and contributes exact zeros)
    m_true = fmaxf(m_true, rmax);
    if (m_ref == -INFINITY) m_ref = rmax;  // first block with a valid key fixes the reference
    clamped |= rmax > m_ref + kHeadroom;
    float psum = 0.f;
    u32x4 pb0, pb1;
#pragma unroll
    for (int r = 0; r < 8; r += 2) {
      float pp[4];
      const int rr[4] = {r, r + 1, r + 8, r + 9};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float x = s[rr[u]];
        pp[u] = x == -INFINITY ? 0.f : exp2f(fminf(x - m_ref, kHeadroom));
      }
      psum += (pp[0] + pp[1]) + (pp[2] + pp[3]);
      pb0[r >> 1] = pack_bf16x2(pp[0], pp[1]);
      pb1[r >> 1] = pack_bf16x2(pp[2], pp[3]);
    }
    lsum += psum;

    // ---- O^T += V^T . P^T : 8 dv tiles x two 16-key steps, V read one step ahead ----
    auto read_v = [&](int c, int t) -> u32x4 {
      const uint32_t a1 = tb + tr_off[t & 1] + 128 * (t >> 1) + 18432 * c;
      const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a1));
      const i16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a1 + 9216));
      u32x4 av;
      av[0] = (uint32_t)(uint16_t)v1[0] | ((uint32_t)(uint16_t)v1[1] << 16);
      av[1] = (uint32_t)(uint16_t)v1[2] | ((uint32_t)(uint16_t)v1[3] << 16);
      av[2] = (uint32_t)(uint16_t)v2[0] | ((uint32_t)(uint16_t)v2[1] << 16);
      av[3] = (uint32_t)(uint16_t)v2[2] | ((uint32_t)(uint16_t)v2[3] << 16);
      return av;
    };
    {
      constexpr int kT = kDv / 64;
#pragma unroll
      for (int sb = 0; sb < 2 * kT; sb += kVBatch) {
        u32x4 av[kVBatch];
#pragma unroll
        for (int u = 0; u < kVBatch; ++u) av[u] = read_v((sb + u) / kT, (sb + u) % kT);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kVBatch; ++u) {
          const int c = (sb + u) / kT, t = (sb + u) % kT;
          o[t] = mfma32x32x16(as_bf16x8(av[u]), as_bf16x8(c == 0 ? pb0 : pb1), o[t]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA into buf^1 has landed
    __syncthreads();
  }

  // ---- epilogue: lane (head n, hh) holds dv = 256h + 64t + 8i + 4hh + j ----
  lsum += __shfl_xor(lsum, 32, 64);
  if (!head_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint2* orow = reinterpret_cast<uint2*>(out + out_row * kDv + 256 * half);
#pragma unroll
  for (int t = 0; t < kDv / 64; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dv = 32 * t + 8 * i + 4 * hh;
      uint2 w;
      w.x = pack_bf16x2(o[t][4 * i + 0] * inv, o[t][4 * i + 1] * inv);
      w.y = pack_bf16x2(o[t][4 * i + 2] * inv, o[t][4 * i + 3] * inv);
      orow[dv / 4] = w;
    }
  }
  if (half == 0 && hh == 0) {
    smax[out_row] = m_true * kLn2;
    // a negative sum marks a row whose logits outgrew the headroom; the fixup pass redoes it
    ssum[out_row] = clamped ? -1.f : lsum * exp2f(m_ref - m_true);
  }
}

// Head-summed softmax mass at the selected slots (target of the indexer KL loss):
//   mass[s, j] = sum_h exp2(S[h, j] * scale * log2e - lse2[h]),  lse2 from softmax_max/sum.
// Same token-per-workgroup gather and pair-split QK as the forward (8 waves, 128 heads);
// each wave sums P over its 32 heads with a 5-step butterfly (16 shuffles), the four head
// groups are added in LDS and one 128-byte row segment is stored per block.
__global__ void __launch_bounds__(kThreads, 1)
attn_mass_bf16_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv,
                      const int32_t* __restrict__ idx, const float* __restrict__ smax, const float* __restrict__ ssum,
                      float* __restrict__ mass, int S, int s_kv, int H, int K, float scale_log2, int64_t q_offset) {
  __shared__ u32x4 tile[2][kTileChunks];
  __shared__ u32x4 qpe[kHeadsPerWG][(kDqk - kDv) / 8];
  __shared__ f32x4 xs[kWaves][4][64];
  __shared__ float macc[2][kBN];
  __shared__ uint32_t vmask[2];
  __shared__ int sidx[kIdxRing][kBN];
  __shared__ int last_slot;

  const int tok = blockIdx.x, b = blockIdx.z, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, n = lane & 31, hh = lane >> 5;
  const int grp = wave & 3, half = wave >> 2;
  const int head = blockIdx.y * kHeadsPerWG + grp * 32 + n;
  const bool head_ok = head < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const int64_t lim64 = min(limit, (int64_t)s_kv - 1);  // largest usable key index
  const uint32_t lim = lim64 < 0 ? 0u : (uint32_t)lim64;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kDqk;
  const int64_t hrow = row_id * H + (head_ok ? head : 0);
  float* mrow = mass + row_id * K;

  if (tid == 0) last_slot = -1;
  if (tid < 2 * kBN) macc[tid / kBN][tid % kBN] = 0.f;
  __syncthreads();
  {
    int last = -1;
    for (int j = tid; j < K; j += kThreads)
      if (slot_ok(ridx[j], s_kv, limit)) last = j;
    if (last >= 0) atomicMax(&last_slot, last);
  }
  __syncthreads();
  const int nblk = (last_slot + kBN) / kBN;
  if (blockIdx.y == 0)  // slots past the last usable block are zero
    for (int j = nblk * kBN + tid; j < K; j += kThreads) mrow[j] = 0.f;
  if (nblk == 0) return;

  float lse2;
  {
    const float sm = head_ok ? ssum[hrow] : 0.f;
    lse2 = sm > 0.f ? (smax[hrow] + logf(sm)) * kLog2e : INFINITY;
  }
  u32x4 qr[kQSteps];
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + hrow * kDqk);
#pragma unroll
    for (int c = 0; c < kQSteps; ++c)
      qr[c] = head_ok ? qh[32 * half + 2 * c + hh] : (u32x4){0u, 0u, 0u, 0u};
    if (half == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int ch = 2 * c + hh;
        qpe[grp * 32 + n][ch ^ (n & 7)] = head_ok ? qh[2 * (kDv / 16) + ch] : (u32x4){0u, 0u, 0u, 0u};
      }
    }
  }
  const uint32_t tile_base = (uint32_t)(uintptr_t)(&tile[0][0]);
  const int xsw = swz8(n);
  uint32_t qk_off[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) qk_off[c4] = n * kRowBytes + 512 * half + 16 * ((2 * c4 + hh) ^ xsw);
  uint32_t pe_off[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) pe_off[c] = n * kRowBytes + 16 * ((64 + 4 * half + 2 * c + hh) ^ xsw);

  int pending = 0;
  idx_ring_init(sidx, ridx, K, nblk, wave, lane, pending);
  __syncthreads();
  issue_block(kvb, tile[0], &vmask[0], sidx[0], 0, K, lim, wave, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    if (blk + 1 < nblk)
      issue_block(kvb, tile[buf ^ 1], &vmask[buf ^ 1], sidx[(blk + 1) & (kIdxRing - 1)], blk + 1, K, lim, wave, lane);
    idx_ring_advance(sidx, ridx, K, nblk, blk, wave, lane, pending);
    const uint32_t tb = tile_base + buf * kTileBytes;
    // operands fetched in batches of 6 ahead of their MFMAs (sched_barrier keeps each batch
    // together so its LDS latency overlaps the previous batch's MFMAs)
    f32x16 s = (f32x16){0};
#pragma unroll
    for (int cb = 0; cb < kQSteps + 2; cb += 6) {
      u32x4 a[6], bq[6];
#pragma unroll
      for (int u = 0; u < 6; ++u) {
        const int c = cb + u;
        if (c < kQSteps) {
          a[u] = *(const lds_u32x4*)(uintptr_t)(tb + qk_off[c & 3] + 128 * (c >> 2));
          bq[u] = qr[c];
        } else {
          a[u] = *(const lds_u32x4*)(uintptr_t)(tb + pe_off[c - kQSteps]);
          bq[u] = qpe[grp * 32 + n][(4 * half + 2 * (c - kQSteps) + hh) ^ (n & 7)];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 6; ++u) s = mfma32x32x16(as_bf16x8(a[u]), as_bf16x8(bq[u]), s);
    }
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      xs[wave][r4][lane] = (f32x4){s[4 * r4], s[4 * r4 + 1], s[4 * r4 + 2], s[4 * r4 + 3]};
    __syncthreads();
    if (half == 0) {
      const uint32_t vm = vmask[buf];
      float v[16];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 other = xs[wave ^ 4][r4][lane];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * r4 + u;
          const int key = 8 * (r >> 2) + 4 * hh + (r & 3);
          const float x = s[r] + other[u];
          v[r] = ((vm >> key) & 1u) ? exp2f(x * scale_log2 - lse2) : 0.f;
        }
      }
      // butterfly over the 32 head lanes of this half-wave: after the steps on lane bits
      // 4,3,2,1 lane l holds the partial for value (l >> 1) & 15; bit 0 completes the sum
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int lb = 4 - st, m = 1 << lb;
        const bool up = (lane >> lb) & 1;
        const int nh = 8 >> st;  // values kept after this step
#pragma unroll
        for (int j = 0; j < nh; ++j) {
          const float send = up ? v[j] : v[j + nh];
          const float keep = up ? v[j + nh] : v[j];
          v[j] = keep + __shfl_xor(send, m, 64);
        }
      }
      const float tot = v[0] + __shfl_xor(v[0], 1, 64);
      if ((lane & 1) == 0) {
        const int r = (lane >> 1) & 15;
        const int key = 8 * (r >> 2) + 4 * hh + (r & 3);
        atomicAdd(&macc[buf][key], tot);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid < kBN) {
      const int slot = blk * kBN + tid;
      if (slot < K) {
        if (gridDim.y == 1) mrow[slot] = macc[buf][tid];
        else atomicAdd(&mrow[slot], macc[buf][tid]);
      }
      macc[buf][tid] = 0.f;
    }
  }
}

__device__ __forceinline__ float ld_elem(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float ld_elem(const uint16_t* p, int64_t i) { return bf16_to_f(p[i]); }
__device__ __forceinline__ void st_elem(float* p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st_elem(uint16_t* p, int64_t i, float v) { p[i] = f_to_bf16(v); }

// Exact path (any D, fp32 arithmetic): one workgroup per (token, head).  Serves fp32
// inputs and, in fixup mode (one workgroup per token, heads looped), recomputes the rows
// the MFMA kernel flagged with a negative softmax_sum.  Scores are staged in dynamic LDS.
template <typename T>
__global__ void __launch_bounds__(256)
sparse_mla_fwd_exact_kernel(const T* __restrict__ q, const T* __restrict__ kv, const int32_t* __restrict__ idx,
                            T* __restrict__ out, float* __restrict__ smax, float* __restrict__ ssum, int S,
                            int s_kv, int H, int K, int dqk, int dv, float scale, int64_t q_offset, int fixup) {
  extern __shared__ float sc[];
  __shared__ float red[256];
  const int tok = blockIdx.x, b = blockIdx.z, tid = threadIdx.x;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const T* kvb = kv + (int64_t)b * s_kv * dqk;
  const int64_t limit = tok + q_offset;
  const int h0 = fixup ? 0 : (int)blockIdx.y, h1 = fixup ? H : h0 + 1;
  for (int head = h0; head < h1; ++head) {
    const int64_t hr = row_id * H + head;
    if (fixup && !(ssum[hr] < 0.f)) continue;  // block-uniform
    const T* qh = q + hr * dqk;
    float lmax = -INFINITY;
    for (int j = tid; j < K; j += 256) {
      const int v = ridx[j];
      float x = -INFINITY;
      if (slot_ok(v, s_kv, limit)) {
        const T* kr = kvb + (int64_t)v * dqk;
        float acc = 0.f;
        for (int d = 0; d < dqk; ++d) acc = fmaf(ld_elem(qh, d), ld_elem(kr, d), acc);
        x = acc * scale;
      }
      sc[j] = x;
      lmax = fmaxf(lmax, x);
    }
    red[tid] = lmax;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
      __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    float lsum = 0.f;
    for (int j = tid; j < K; j += 256) {
      const float e = (m == -INFINITY) ? 0.f : expf(sc[j] - m);
      sc[j] = e;
      lsum += e;
    }
    red[tid] = lsum;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if (tid < st) red[tid] += red[tid + st];
      __syncthreads();
    }
    const float l = red[0];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T* orow = out + hr * dv;
    for (int d = tid; d < dv; d += 256) {
      float acc = 0.f;
      for (int j = 0; j < K; ++j) {
        const float e = sc[j];
        if (e != 0.f) acc = fmaf(e, ld_elem(kvb, (int64_t)ridx[j] * dqk + d), acc);
      }
      st_elem(orow, d, acc * inv);
    }
    __syncthreads();  // sc / red reused by the next head
    if (tid == 0) {
      smax[hr] = m;
      ssum[hr] = l;
    }
  }
}

// exact fp32 mass: one workgroup per token, thread per slot, heads looped
__global__ void __launch_bounds__(256)
attn_mass_f32_kernel(const float* __restrict__ q, const float* __restrict__ kv, const int32_t* __restrict__ idx,
                     const float* __restrict__ smax, const float* __restrict__ ssum, float* __restrict__ mass, int S,
                     int s_kv, int H, int K, int dqk, float scale, int64_t q_offset) {
  const int tok = blockIdx.x, b = blockIdx.z;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const float* kvb = kv + (int64_t)b * s_kv * dqk;
  for (int j = threadIdx.x; j < K; j += 256) {
    const int v = ridx[j];
    float acc = 0.f;
    if (slot_ok(v, s_kv, tok + q_offset)) {
      const float* kr = kvb + (int64_t)v * dqk;
      for (int h = 0; h < H; ++h) {
        const int64_t hr = row_id * H + h;
        const float sm = ssum[hr];
        if (!(sm > 0.f)) continue;
        const float* qh = q + hr * dqk;
        float dot = 0.f;
        for (int d = 0; d < dqk; ++d) dot = fmaf(qh[d], kr[d], dot);
        acc += expf(dot * scale - smax[hr] - logf(sm));
      }
    }
    mass[row_id * K + j] = acc;
  }
}

}  // namespace

}  // namespace dsa

extern "C" int dsa_attn_mass(const void* q, const void* kv, const int32_t* indices, const float* softmax_max,
                             const float* softmax_sum, float* mass, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                             int64_t n_heads, int64_t d_qk, int64_t topk, float scale, int64_t q_offset,
                             void* stream) {
  using namespace dsa;
  if (!q || !kv || !indices || !softmax_max || !softmax_sum || !mass)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_mass: null pointer");
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || n_heads <= 0 || topk <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_mass: bad sizes");
  if (s_q > 2147483647LL || batch > 65535 || s_kv > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_mass: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DSA_BF16) {
    if (d_qk != kDqk) return set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: bf16 path needs d_qk=576");
    if (s_kv > kMaxGatherRows) return set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: S_kv > %lld", (long long)kMaxGatherRows);
    const unsigned hgroups = ceil_div(n_heads, kHeadsPerWG);
    if (hgroups > 1) {  // partial sums from several head groups accumulate into a zeroed buffer
      if (hipMemsetAsync(mass, 0, (size_t)(batch * s_q * topk) * 4, st) != hipSuccess)
        return set_error(DSA_ERR_LAUNCH, "dsa_attn_mass: memset failed");
    }
    dim3 grid((unsigned)s_q, hgroups, (unsigned)batch);
    attn_mass_bf16_kernel<<<grid, kThreads, 0, st>>>((const uint16_t*)q, (const uint16_t*)kv, indices, softmax_max,
                                                     softmax_sum, mass, (int)s_q, (int)s_kv, (int)n_heads, (int)topk,
                                                     scale * kLog2e, q_offset);
    return check_launch("dsa_attn_mass(bf16)");
  }
  if (dtype == DSA_F32) {
    if (n_heads > 65535) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_mass: sizes out of range");
    dim3 grid((unsigned)s_q, 1, (unsigned)batch);
    attn_mass_f32_kernel<<<grid, 256, 0, st>>>((const float*)q, (const float*)kv, indices, softmax_max, softmax_sum,
                                               mass, (int)s_q, (int)s_kv, (int)n_heads, (int)topk, (int)d_qk, scale,
                                               q_offset);
    return check_launch("dsa_attn_mass(f32)");
  }
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: dtype %d", dtype);
}

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices, void* out, float* softmax_max,
                                  float* softmax_sum, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                                  int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                                  int64_t q_offset, void* stream) {
  using namespace dsa;
  if (!q || !kv || !indices || !out || !softmax_max || !softmax_sum)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_fwd: null pointer");
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || n_heads <= 0 || topk <= 0 || d_v <= 0 || d_qk < d_v)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_fwd: bad sizes (B=%lld S=%lld S_kv=%lld H=%lld K=%lld)",
                     (long long)batch, (long long)s_q, (long long)s_kv, (long long)n_heads, (long long)topk);
  if (s_q > 65535 * 64 || batch > 65535 || s_kv > INT32_MAX || topk > (1 << 20))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_fwd: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  if (topk * 4 > 64 * 1024)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: topk <= 16384 supported (got %lld)", (long long)topk);
  const size_t sc_bytes = (size_t)topk * sizeof(float);
  if (dtype == DSA_BF16) {
    if (d_qk != kDqk || d_v != kDv)
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: bf16 path needs d_qk=576, d_v=512 (got %lld/%lld)",
                       (long long)d_qk, (long long)d_v);
    if (s_kv > kMaxGatherRows)
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: S_kv > %lld", (long long)kMaxGatherRows);
    dim3 grid((unsigned)s_q, ceil_div(n_heads, kHeadsPerWG), (unsigned)batch);
    sparse_mla_fwd_bf16_kernel<<<grid, kThreads, 0, st>>>(
        (const uint16_t*)q, (const uint16_t*)kv, indices, (uint16_t*)out, softmax_max, softmax_sum, (int)s_q,
        (int)s_kv, (int)n_heads, (int)topk, scale * kLog2e, q_offset);
    if (int rc = check_launch("dsa_sparse_mla_fwd(bf16)")) return rc;
    dim3 fgrid((unsigned)s_q, 1, (unsigned)batch);
    sparse_mla_fwd_exact_kernel<uint16_t><<<fgrid, 256, sc_bytes, st>>>(
        (const uint16_t*)q, (const uint16_t*)kv, indices, (uint16_t*)out, softmax_max, softmax_sum, (int)s_q,
        (int)s_kv, (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset, 1);
    return check_launch("dsa_sparse_mla_fwd(bf16 fixup)");
  }
  if (dtype == DSA_F32) {
    dim3 grid((unsigned)s_q, (unsigned)n_heads, (unsigned)batch);
    sparse_mla_fwd_exact_kernel<float><<<grid, 256, sc_bytes, st>>>(
        (const float*)q, (const float*)kv, indices, (float*)out, softmax_max, softmax_sum, (int)s_q, (int)s_kv,
        (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset, 0);
    return check_launch("dsa_sparse_mla_fwd(f32)");
  }
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: dtype %d not supported", dtype);
}
