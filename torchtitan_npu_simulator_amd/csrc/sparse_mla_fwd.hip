// Gathered sparse MLA attention forward for gfx950.
//
// One workgroup = one query token x up to 128 heads, 4 waves (one per SIMD, each with the
// whole 512-register file).  The token's selected latent-KV rows (576 bf16 = 1152 B each)
// are gathered in blocks of 32 by DMA (global_load_lds) into a swizzled, triple-buffered
// LDS tile shared by all heads, so each row crosses L2 once per token.  Wave w owns heads
// 32w .. 32w+31 on v_mfma_f32_32x32x16_bf16 (one accumulation chain issues at full rate):
//   * QK: S^T[32 keys x 32 heads] over 36 k-steps of 16 columns; latent Q of the wave's
//     heads stays in 128 VGPRs for the whole token, rope Q in LDS; K rows are the A
//     operand, read one batch ahead of their MFMAs;
//   * softmax per head in the exp2 domain against a reference max fixed by the first
//     valid block: no per-block O rescale (P may reach 2^64, well inside the fp32/bf16
//     exponent range).  A row whose later logits outgrow that headroom is flagged with a
//     negative softmax_sum and recomputed exactly by the fixup pass;
//   * PV: O^T[512 dv x 32 heads] += V^T . P^T in 16 dv tiles, V read transposed by
//     ds_read_b64_tr_b16 straight from the row-major K tile (k_nope == v); the key order
//     inside the k dimension is the S^T accumulator order on both operands, so P is packed
//     from the softmax registers directly.  O (256 fp32 per lane) lives in the
//     accumulation registers.
// LDS traffic per token and block is 4 waves x (QK + PV) tile reads; one barrier per
// block, for the tile hand-off.
#include "dsa_common.h"
#include "dsa_gather.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kBN = 32;                        // keys per block
constexpr float kHeadroom = 64.0f;             // log2 units of P above the reference max
constexpr int kFwdWaves = 4;
constexpr int kFwdThreads = kFwdWaves * 64;
constexpr int kFwdHeads = 32 * kFwdWaves;      // heads per workgroup
constexpr int kLatSteps = kDv / 16;            // 32 latent k-steps (Q in registers)



template <int kD>  // row width of Q and KV: 576 (latent + rope) or 512 (no rope)
__global__ void __launch_bounds__(kFwdThreads, 1)
sparse_mla_fwd_bf16_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv,
                           const int32_t* __restrict__ idx, uint16_t* __restrict__ out, float* __restrict__ smax,
                           float* __restrict__ ssum, int S, int s_kv, int H, int K, float scale_log2,
                           int64_t q_offset, const float* __restrict__ sinks) {
  using Gather = RowGather<kFwdWaves, kD>;
  using Geo = GatherGeomT<kD>;
  constexpr int kPer = Gather::kMaxPerWave;
  constexpr int kTC = Geo::kTileChunks, kRB = Geo::kRowBytes;
  constexpr int kKS = kD / 16;                // MFMA k-steps of S^T (36 | 32)
  constexpr bool kRope = kKS > kLatSteps;     // the rope columns 512..575 exist
  __shared__ u32x4 tile[3][kTC];
  __shared__ u32x4 qpe[kRope ? kFwdHeads : 1][8];  // rope Q, [head][16 B chunk ^ ((head >> 1) & 7)]
  __shared__ int sidx[GatherGeom::kRing][Gather::kRingInts];
  __shared__ int sh_last;

  const int tok = blockIdx.x, b = blockIdx.z, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 31, h = lane >> 5;  // MFMA column (head / key row) and k half
  const int hl = wave * 32 + n;           // head within the workgroup
  const int head = blockIdx.y * kFwdHeads + hl;
  const bool hok = head < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int64_t orow = row_id * H + (hok ? head : 0);
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kD;

  // the row's slot indices (block count), the index ring entries of blocks 0..2 (wave 0,
  // DMA) and the row's Q are requested together; the block count waits only for the indices
  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) Gather::issue_idx(ridx, K, i, sidx[i], lane);  // clamped to slot K-1
  }
  // ---- Q: latent qb[s] = q[16s + 8h .. +8] of head `head` (B operand of S^T = K Q^T for
  // k-step s) in VGPRs; the rope columns go to LDS below ----
  // (unconditional loads, orow points at head 0 for absent heads: a load under a branch
  // would make the compiler wait for every load before the block count; absent heads are
  // zeroed after it)
  u32x4 qb[kLatSteps], qr[4];
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + orow * kD);
#pragma unroll
    for (int s = 0; s < kLatSteps; ++s) qb[s] = qh[2 * s + h];
#pragma unroll
    for (int j = 0; j < 4; ++j) qr[j] = kRope ? qh[64 + 4 * h + j] : (u32x4){0u, 0u, 0u, 0u};  // rope chunks 64 + 4h ..
  }
  const int nblk = count_row_blocks(ridx, K, s_kv, limit, vidx, &sh_last);
  if (nblk == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring DMA has landed before the LDS is released
    if (hok) {
      uint32_t* o32 = reinterpret_cast<uint32_t*>(out + orow * kDv);
      for (int i = h; i < kDv / 2; i += 2) o32[i] = 0u;
      if (h == 0) {  // (with a sink the row's only logit is the sink's)
        smax[orow] = sinks ? sinks[head] : -INFINITY;
        ssum[orow] = sinks ? 1.f : 0.f;
      }
    }
    return;
  }
  const uint32_t lim = gather_limit(limit, s_kv);

  if (!hok) {
#pragma unroll
    for (int s = 0; s < kLatSteps; ++s) qb[s] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) qr[j] = (u32x4){0u, 0u, 0u, 0u};
  }
  if constexpr (kRope) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // rope chunks 64..71: lane h writes 4h .. 4h+3
      const int ch = 4 * h + j;
      qpe[hl][ch ^ ((hl >> 1) & 7)] = qr[j];
    }
  }
#pragma unroll
  for (int s = 0; s < kLatSteps; ++s) asm volatile("" : "+v"(qb[s]));  // landed before any DMA

  // ---- LDS byte offsets ----
  // A operand of S^T, k-step s: key row n, chunk (2s + h) ^ swz_kv(n); with s = 4u + s0 the
  // XOR only touches bits 0..2 of 8u + 2s0 + h, so offset = ka_off[s0] + 128 u.
  uint32_t ka_off[4];
#pragma unroll
  for (int s0 = 0; s0 < 4; ++s0) ka_off[s0] = n * kRB + 16 * ((2 * s0 + h) ^ swz_kv(n));
  // rope B operand, step 32 + e: head row hl, chunk (2e + h) ^ ((hl >> 1) & 7)
  const lds_char* qpe_b = lds_bytes(&qpe[0][0]);
  // Transposed V reads for O^T[32 dv x 32 heads] += V^T . P^T, dv tile dt, key step kk:
  // lane group G = lane / 16 covers dv 16 (G & 1) .. +15 and k half h = G >> 1; source lane
  // c = lane % 16 supplies key row 16kk + 8x + 4h + c/4 (read x = 0, 1) and dv columns
  // 32dt + 16 (G & 1) + 4 (c % 4) .. +3, so result lane gets 4 consecutive keys of one dv
  // column.  k-slot 8h + t <-> key 16kk + 8 (t / 4) + 4h + t % 4 on both operands (the rows
  // the S^T accumulator holds for this lane).  swz_kv of those rows does not depend on kk,
  // and with dt = 2u + d0: offset = tr_off[x][d0] + 16 kk rows + 128 u.
  uint32_t tr_off[2][2];
  {
    const int c = lane & 15, G = lane >> 4;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int r = 8 * x + 4 * h + (c >> 2);
#pragma unroll
      for (int d0 = 0; d0 < 2; ++d0) {
        const int ch = 4 * d0 + 2 * (G & 1) + ((c & 3) >> 1);
        tr_off[x][d0] = r * kRB + 16 * (ch ^ swz_kv(r)) + 8 * (c & 1);
      }
    }
  }

  f32x16 o[kDv / 32];  // O^T tile dt: lane holds dv 32dt + 8j + 4h + i (i = 0..3) of its head
#pragma unroll
  for (int t = 0; t < kDv / 32; ++t) o[t] = (f32x16){0.f};
  float m_ref = -INFINITY, m_true = -INFINITY, lsum = 0.f;
  bool clamped = false;

  // ---- pipeline ----
  // iteration blk: QK(blk) on tile blk % 3 while block blk+1's rows are DMA'd into tile
  // (blk+1) % 3 (one instruction per QK batch), then softmax(blk) interleaved with PV(blk-1)
  // on tile (blk-1) % 3, whose P (bp_prev) was made one iteration earlier.  The iteration
  // ends with its DMAs landed (vmcnt 0) and one barrier, so a gather has about one block
  // time to arrive.  Block validity bits travel in SGPRs.
  const typename Gather::PackedLanes gl = Gather::packed_lanes(wave, lane);
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // ring entries 0..2 landed
  __syncthreads();                                                  // publishes them and qpe
  for (int i = tid; i < kTC; i += kFwdThreads) tile[2][i] = (u32x4){0u, 0u, 0u, 0u};
  uint32_t vm_cur = Gather::ring_valid(sidx[0], lane, lim, K);
#pragma unroll
  for (int i = 0; i < kPer; ++i) Gather::issue_slot(kvb, &tile[0][0], i, wave, Gather::ring_slot(sidx[0], i, gl), gl, lim, K);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  constexpr int kQBatch = 4;                  // k-steps per QK batch
  constexpr int kQB = kKS / kQBatch;          // 9 | 8 QK batches
  static_assert(kQB >= kPer, "one row DMA per QK batch");
  static_assert(kLatSteps % kQBatch == 0 && (kKS - kLatSteps == kQBatch || kKS == kLatSteps),
                "rope steps form the last QK batch");
  constexpr int kVB = kDv / 32;               // 16 PV batches (one dv tile, two key steps)
  u32x4 bp_prev[2] = {(u32x4){0u, 0u, 0u, 0u}, (u32x4){0u, 0u, 0u, 0u}};

  // S^T[32 keys x 32 heads] of block blk on v_mfma_f32_32x32x16_bf16 (one accumulator; the
  // 32x32 shape issues at full rate without independent chains).  Block blk+1's rows go out
  // meanwhile, one instruction per batch (ring entry `ring`, the slot value read a batch
  // ahead); its validity bits are returned.  Past the last block the ring entry is stale and
  // the rows land in a buffer nobody reads: every offset stays inside the KV tensor (a slot
  // is used only if it is <= lim, else row 0 is read).
  auto qk = [&](const lds_char* tb, u32x4* dst_tile, const int* ring, int rows_left, f32x16& sacc) {
    const uint32_t vm_n = Gather::ring_valid(ring, lane, lim, rows_left);
    uint32_t raw_next = Gather::ring_slot(ring, 0, gl);
    sacc = (f32x16){0.f};
    u32x4 a[2][kQBatch];
    u32x4 rope[kQBatch];
    auto read_a = [&](u32x4 (&dst)[kQBatch], int sb) {
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) dst[u] = lds_read16(tb + ka_off[u] + 128 * (sb / kQBatch));
    };
    read_a(a[0], 0);
    static_for<kQB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kQB) read_a(a[(nb + 1) & 1], (nb + 1) * kQBatch);
      if constexpr (kRope && (nb + 1) * kQBatch == kLatSteps) {  // rope B operands one batch ahead
#pragma unroll
        for (int e = 0; e < kQBatch; ++e) rope[e] = lds_read16(qpe_b + hl * 128 + 16 * ((2 * e + h) ^ ((hl >> 1) & 7)));
      }
      if constexpr (nb < kPer) {
        const uint32_t raw = raw_next;
        if constexpr (nb + 1 < kPer) raw_next = Gather::ring_slot(ring, nb + 1, gl);
        Gather::issue_slot(kvb, dst_tile, nb, wave, raw, gl, lim, rows_left);
      }
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) {
        constexpr int s0 = nb * kQBatch;
        const u32x4 bq = s0 < kLatSteps ? qb[(s0 + u) % kLatSteps] : rope[u];
        sacc = mfma32x32x16(as_bf16x8(a[nb & 1][u]), as_bf16x8(bq), sacc);
      }
      // the batch's LDS reads, address arithmetic and DMA are spread between its MFMAs:
      // with one accumulation chain the wave issues in order, so work placed after the
      // MFMAs would only overlap the last one
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);  // VALU / SALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // the row DMA
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    return vm_n;
  };

  // softmax of block blk (sacc, validity bits vm) into bp_new, interleaved batch by batch
  // with PV of block blk-1 (tile vb, P bp_prev; for blk = 0 a zeroed tile and P = 0).
  // Lane holds keys 8j + 4h + i (value 4j + i) of head `head`; the lane 32 apart holds
  // the other keys of the same head.
  auto read_v = [&](const lds_char* vb, u32x4 (&dst)[2], int dt) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const lds_char* base = vb + kk * 16 * kRB + 128 * (dt >> 1);
      dst[kk] = lds_read_tr_pair(base + tr_off[0][dt & 1], base + tr_off[1][dt & 1]);
    }
  };
  auto softmax_pv = [&](const lds_char* vb, const f32x16& sacc, uint32_t vm, u32x4 (&bp_new)[2]) {
    u32x4 av[2][2];  // [buffer][kk]
    read_v(vb, av[0], 0);
    const uint32_t vmh = vm >> (4 * h);  // bit 8j + i: key 8j + 4h + i
    float x[16], rmax;                     // masked logits, then P in place
    static_for<kVB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kVB) read_v(vb, av[(nb + 1) & 1], nb + 1);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) o[nb] = mfma32x32x16(as_bf16x8(av[nb & 1][kk]), as_bf16x8(bp_prev[kk]), o[nb]);
      // softmax work of this batch: masked logits and local max (0), cross-lane max and
      // reference update (1), exp2 of a quarter of the values (2..5), pack and sum (5)
      if constexpr (nb == 0) {
        rmax = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = 8 * (v >> 2) + (v & 3);
          x[v] = ((vmh >> key) & 1u) ? sacc[v] * scale_log2 : -INFINITY;
          rmax = fmaxf(rmax, x[v]);
        }
      } else if constexpr (nb == 1) {
        const float rm = xor32_max(rmax);
        // (a block with no valid slot leaves every x at -inf and contributes exact zeros)
        m_true = fmaxf(m_true, rm);
        if (m_ref == -INFINITY) m_ref = rm;  // first block with a valid key fixes the reference
        clamped |= rm > m_ref + kHeadroom;
        // while no key has been seen every x is -inf; subtracting 0 then keeps exp2 at 0
        rmax = m_ref == -INFINITY ? 0.f : m_ref;
      } else if constexpr (nb >= 2 && nb < 6) {
        constexpr int v0 = 4 * (nb - 2);
#pragma unroll
        for (int v = v0; v < v0 + 4; ++v) x[v] = __builtin_amdgcn_exp2f(fminf(x[v] - rmax, kHeadroom));
        // B operand P^T of key step kk = j / 2: k-slot 8h + t <-> value 4 (2kk + t / 4) + t % 4
        bp_new[v0 >> 3][(v0 & 4) >> 1] = pack_bf16x2(x[v0], x[v0 + 1]);
        bp_new[v0 >> 3][((v0 & 4) >> 1) + 1] = pack_bf16x2(x[v0 + 2], x[v0 + 3]);
        if constexpr (nb == 5) {
          float s4[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) s4[q4] = (x[4 * q4] + x[4 * q4 + 1]) + (x[4 * q4 + 2] + x[4 * q4 + 3]);
          lsum += (s4[0] + s4[1]) + (s4[2] + s4[3]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // PV of the last block
  auto pv_only = [&](const lds_char* vb) {
    u32x4 av[2][2];
    read_v(vb, av[0], 0);
    static_for<kVB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kVB) read_v(vb, av[(nb + 1) & 1], nb + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) o[nb] = mfma32x32x16(as_bf16x8(av[nb & 1][kk]), as_bf16x8(bp_prev[kk]), o[nb]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  for (int blk = 0; blk < nblk; ++blk) {
    if (wave == 0 && blk + 3 < nblk)
      Gather::issue_idx(ridx, K, blk + 3, sidx[(blk + 3) & (GatherGeom::kRing - 1)], lane);
    f32x16 sacc;
    // ring entry blk+1 landed during iteration blk-2 (or before the loop)
    const uint32_t vm_next = qk(lds_bytes(&tile[blk % 3][0]), &tile[(blk + 1) % 3][0],
                                sidx[(blk + 1) & (GatherGeom::kRing - 1)], K - (blk + 1) * kBN, sacc);
    u32x4 bp_new[2];
    softmax_pv(lds_bytes(&tile[(blk + 2) % 3][0]), sacc, vm_cur, bp_new);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // block blk+1 and ring entry blk+3 landed
    __syncthreads();
    vm_cur = vm_next;
    bp_prev[0] = bp_new[0];
    bp_prev[1] = bp_new[1];
  }
  pv_only(lds_bytes(&tile[(nblk - 1) % 3][0]));

  // ---- epilogue: lane holds dv = 32 dt + 8 j + 4 h + i of its head ----
  const float ls = xor32_sum(lsum);
  if (!hok) return;
  // a per-head sink (a logit with no value, natural-log units of the scaled score) joins
  // the row's denominator: O = acc / (ls + 2^(sink2 - m_ref)), and the row statistics
  // become (m2, s2) = (max(m, sink), sum e^(x - m2) + e^(sink - m2)); with no valid key
  // (m_ref = -inf) the sink term is +inf and O stays 0
  const float sk2 = sinks ? sinks[head] * kLog2e : -INFINITY;
  const float den = sinks ? ls + exp2f(sk2 - m_ref) : ls;
  const float inv = den > 0.f ? 1.f / den : 0.f;
  uint2* orp = reinterpret_cast<uint2*>(out + orow * kDv);
#pragma unroll
  for (int dt = 0; dt < kDv / 32; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 w;
      w.x = pack_bf16x2(o[dt][4 * j] * inv, o[dt][4 * j + 1] * inv);
      w.y = pack_bf16x2(o[dt][4 * j + 2] * inv, o[dt][4 * j + 3] * inv);
      orp[(32 * dt + 8 * j + 4 * h) / 4] = w;
    }
  if (h == 0) {
    const float l_true = ls > 0.f ? ls * exp2f(m_ref - m_true) : 0.f;  // sum at the true max
    float m_out = m_true, l_out = l_true;
    if (sinks) {
      m_out = fmaxf(m_true, sk2);
      l_out = (l_true > 0.f ? l_true * exp2f(m_true - m_out) : 0.f) + exp2f(sk2 - m_out);
    }
    smax[orow] = m_out * kLn2;
    // a negative sum marks a row whose logits outgrew the headroom; the fixup pass redoes it
    ssum[orow] = clamped ? -1.f : l_out;
  }
}

// Head-summed softmax mass at the selected slots (target of the indexer KL loss):
//   mass[s, j] = sum_h exp2(S[h, j] * scale * log2e - lse2[h]),  lse2 from softmax_max/sum.
// The forward's gather and QK pipeline without its PV half: one workgroup = one token x
// up to 128 heads on 4 waves (32 heads each, v_mfma_f32_32x32x16_bf16); S^T of block blk
// on tile blk & 1 while block blk+1's rows are DMA'd into the other tile (two tiles
// suffice: a block is not read after its QK).  The whole Q row of the wave's heads
// (latent and rope) stays in VGPRs, so the LDS holds little more than the two tiles and
// two workgroups share a CU.  Each wave sums P over its 32 heads (permlane16 swap, then
// DPP exchanges), the four waves' sums meet in LDS behind the block's barrier, and wave 0
// stores the block's 128-byte row segment at the start of the next iteration.
template <int kD>  // row width of Q and KV: 576 (latent + rope) or 512 (no rope)
__global__ void __launch_bounds__(kFwdThreads, 2)
attn_mass_bf16_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv,
                      const int32_t* __restrict__ idx, const float* __restrict__ smax, const float* __restrict__ ssum,
                      float* __restrict__ mass, int S, int s_kv, int H, int K, float scale_log2, int64_t q_offset) {
  using Gather = RowGather<kFwdWaves, kD>;
  using Geo = GatherGeomT<kD>;
  constexpr int kPer = Gather::kMaxPerWave;
  constexpr int kTC = Geo::kTileChunks, kRB = Geo::kRowBytes;
  constexpr int kKS = kD / 16;  // MFMA k-steps of S^T (36 | 32)
  __shared__ u32x4 tile[2][kTC];
  __shared__ int sidx[GatherGeom::kRing][Gather::kRingInts];
  __shared__ float part[2][kFwdWaves][kBN];  // [block parity][wave][key]: per-wave head sums
  __shared__ int sh_last;

  const int tok = blockIdx.x, b = blockIdx.z, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 31, h = lane >> 5;  // MFMA column (head / key row) and k half
  const int head = blockIdx.y * kFwdHeads + wave * 32 + n;
  const bool hok = head < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int64_t hrow = row_id * H + (hok ? head : 0);
  const int32_t* ridx = idx + row_id * K;
  float* mrow = mass + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kD;

  // the row's slot indices (block count), the ring entries of blocks 0..2 (wave 0, DMA),
  // the head's Q row and row statistics are requested together (unconditional loads from
  // head 0's row for absent heads, whose lse2 is then +inf)
  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) Gather::issue_idx(ridx, K, i, sidx[i], lane);  // clamped to slot K-1
  }
  u32x4 qb[kKS];  // qb[s] = q[16s + 8h .. +8] of head `head`: B operand of k-step s
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + hrow * kD);
#pragma unroll
    for (int s = 0; s < kKS; ++s) qb[s] = qh[2 * s + h];
  }
  const float mx = smax[hrow], sm = ssum[hrow];
  const int nblk = count_row_blocks(ridx, K, s_kv, limit, vidx, &sh_last);
  if (blockIdx.y == 0)  // slots past the last usable block hold no mass
    for (int j = nblk * kBN + tid; j < K; j += kFwdThreads) mrow[j] = 0.f;
  if (nblk == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring DMA has landed before the LDS is released
    return;
  }
  const uint32_t lim = gather_limit(limit, s_kv);
  const float lse2 = (hok && sm > 0.f) ? (mx + logf(sm)) * kLog2e : INFINITY;  // +inf -> P = 0
#pragma unroll
  for (int s = 0; s < kKS; ++s) asm volatile("" : "+v"(qb[s]));  // landed before any DMA

  // A operand of k-step s: key row n, chunk (2s + h) ^ swz_kv(n) = ka_off[s % 4] + 128 (s / 4)
  uint32_t ka_off[4];
#pragma unroll
  for (int s0 = 0; s0 < 4; ++s0) ka_off[s0] = n * kRB + 16 * ((2 * s0 + h) ^ swz_kv(n));

  const typename Gather::PackedLanes gl = Gather::packed_lanes(wave, lane);
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // ring entries 0..2 landed
  __syncthreads();
  uint32_t vm_cur = Gather::ring_valid(sidx[0], lane, lim, K);
#pragma unroll
  for (int i = 0; i < kPer; ++i) Gather::issue_slot(kvb, &tile[0][0], i, wave, Gather::ring_slot(sidx[0], i, gl), gl, lim, K);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  constexpr int kQBatch = 4;           // k-steps per QK batch
  constexpr int kQB = kKS / kQBatch;   // 9 | 8 QK batches
  static_assert(kQB >= kPer, "one row DMA per QK batch");

  // S^T[32 keys x 32 heads] of one block, with the next block's rows DMA'd one
  // instruction per batch (the forward's schedule); returns the next block's validity bits
  auto qk = [&](const lds_char* tb, u32x4* dst_tile, const int* ring, int rows_left, f32x16& sacc)
      __attribute__((always_inline)) {
    const uint32_t vm_n = Gather::ring_valid(ring, lane, lim, rows_left);
    uint32_t raw_next = Gather::ring_slot(ring, 0, gl);
    sacc = (f32x16){0.f};
    u32x4 a[2][kQBatch];
    auto read_a = [&](u32x4 (&dst)[kQBatch], int sb) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) dst[u] = lds_read16(tb + ka_off[u] + 128 * (sb / kQBatch));
    };
    read_a(a[0], 0);
    static_for<kQB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kQB) read_a(a[(nb + 1) & 1], (nb + 1) * kQBatch);
      if constexpr (nb < kPer) {
        const uint32_t raw = raw_next;
        if constexpr (nb + 1 < kPer) raw_next = Gather::ring_slot(ring, nb + 1, gl);
        Gather::issue_slot(kvb, dst_tile, nb, wave, raw, gl, lim, rows_left);
      }
#pragma unroll
      for (int u = 0; u < kQBatch; ++u)
        sacc = mfma32x32x16(as_bf16x8(a[nb & 1][u]), as_bf16x8(qb[nb * kQBatch + u]), sacc);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);  // VALU / SALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // the row DMA
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    return vm_n;
  };

  // P of one block summed over the wave's 32 heads into part[pb][wave][*].  Lane holds keys
  // 8j + 4h + i (value 4j + i) of head `head`; butterfly over the 32 head lanes: lane bits
  // 4..1 halve the 16 values (bit 4 by one permlane16 swap, bits 3..1 by DPP), bit 0
  // completes the sum, and lane l ends with value (l >> 1) & 15.  The halves are chosen by
  // bit masks (a select between two array elements would become an indexed read).
  auto block_mass = [&](const f32x16& sacc, uint32_t vm, int pb) __attribute__((always_inline)) {
    const uint32_t vmh = vm >> (4 * h);  // bit 8j + i: key 8j + 4h + i
    float pv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const bool ok = (vmh >> (8 * (v >> 2) + (v & 3))) & 1u;
      pv[v] = ok ? __builtin_amdgcn_exp2f(sacc[v] * scale_log2 - lse2) : 0.f;
    }
    const bool odd = (lane >> 4) & 1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // even rows keep value j, odd rows j + 8
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(pv[j]), __float_as_uint(pv[j + 8]), false, false);
      const float even_sum = pv[j] + __uint_as_float(r[1]), odd_sum = pv[j + 8] + __uint_as_float(r[0]);
      pv[j] = odd ? odd_sum : even_sum;
    }
    auto bstep = [&](auto mc, int nh) __attribute__((always_inline)) {
      constexpr int m = decltype(mc)::value;
      const uint32_t up = ((lane & m) != 0) ? 0xffffffffu : 0u;
#pragma unroll
      for (int j = 0; j < nh; ++j) {
        const uint32_t a = __float_as_uint(pv[j]), c = __float_as_uint(pv[j + nh]);
        const float send = __uint_as_float((a & up) | (c & ~up));
        const float keep = __uint_as_float((c & up) | (a & ~up));
        pv[j] = keep + lane_xor<m>(send);
      }
    };
    bstep(std::integral_constant<int, 8>{}, 4);
    bstep(std::integral_constant<int, 4>{}, 2);
    bstep(std::integral_constant<int, 2>{}, 1);
    const float tot = pv[0] + lane_xor<1>(pv[0]);
    if ((lane & 1) == 0) {
      const int r = (lane >> 1) & 15;
      part[pb][wave][8 * (r >> 2) + 4 * h + (r & 3)] = tot;
    }
  };

  // block fb's four wave sums -> global (its partials were published by the barrier that
  // ended its iteration); several head groups add into a zeroed row
  auto flush = [&](int fb) __attribute__((always_inline)) {
    if (wave == 0 && lane < kBN) {
      const int pb = fb & 1;
      const float t = (part[pb][0][lane] + part[pb][1][lane]) + (part[pb][2][lane] + part[pb][3][lane]);
      const int slot = fb * kBN + lane;
      if (slot < K) {
        if (gridDim.y == 1) mrow[slot] = t;
        else atomicAdd(&mrow[slot], t);
      }
    }
  };

  // iteration blk: the store of block blk-1, S^T of block blk on tile blk & 1 while block
  // blk+1's rows are DMA'd into the other tile, then P and the head sums of block blk; the
  // iteration ends with its DMAs landed and one barrier
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk > 0) flush(blk - 1);
    if (wave == 0 && blk + 3 < nblk)
      Gather::issue_idx(ridx, K, blk + 3, sidx[(blk + 3) & (GatherGeom::kRing - 1)], lane);
    f32x16 sacc;
    // ring entry blk+1 landed during iteration blk-2 (or before the loop)
    const uint32_t vm_next = qk(lds_bytes(&tile[blk & 1][0]), &tile[(blk + 1) & 1][0],
                                sidx[(blk + 1) & (GatherGeom::kRing - 1)], K - (blk + 1) * kBN, sacc);
    block_mass(sacc, vm_cur, blk & 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // block blk+1 and ring entry blk+3 landed
    __syncthreads();
    vm_cur = vm_next;
  }
  flush(nblk - 1);
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
                            int s_kv, int H, int K, int dqk, int dv, float scale, int64_t q_offset, int fixup,
                            const float* __restrict__ sinks) {
  extern __shared__ float sc[];
  __shared__ float red[256];
  const int tok = blockIdx.x, b = blockIdx.z, tid = threadIdx.x;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const T* kvb = kv + (int64_t)b * s_kv * dqk;
  const int64_t limit = tok + q_offset;
  const int h0 = fixup ? 0 : (int)blockIdx.y, h1 = fixup ? H : h0 + 1;
  if (fixup) {  // one parallel test of the row's flags: almost every row has none
    bool any = false;
    for (int hh = tid; hh < H; hh += 256) any |= ssum[row_id * H + hh] < 0.f;
    if (!__syncthreads_or(any)) return;
  }
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
    // per-head sink: O scaled by a / s2 with a = l e^(m - m2), s2 = a + e^(sink - m2)
    float m_out = m, l_out = l, fold = 1.f;
    if (sinks) {
      const float sk = sinks[head];
      m_out = fmaxf(m, sk);
      const float a = l > 0.f ? l * expf(m - m_out) : 0.f;
      l_out = a + expf(sk - m_out);
      fold = a / l_out;
    }
    const float inv = l > 0.f ? fold / l : 0.f;
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
      smax[hr] = m_out;
      ssum[hr] = l_out;
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
    if (d_qk != kDqk && d_qk != kDv)
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: bf16 path needs d_qk = 576 or 512 (got %lld)", (long long)d_qk);
    const int64_t max_rows = d_qk == kDqk ? GatherGeomT<kDqk>::kMaxRows : GatherGeomT<kDv>::kMaxRows;
    if (s_kv > max_rows) return set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: S_kv > %lld", (long long)max_rows);
    const unsigned hgroups = ceil_div(n_heads, kFwdHeads);
    if (hgroups > 1) {  // partial sums from several head groups accumulate into a zeroed buffer
      if (hipMemsetAsync(mass, 0, (size_t)(batch * s_q * topk) * 4, st) != hipSuccess)
        return set_error(DSA_ERR_LAUNCH, "dsa_attn_mass: memset failed");
    }
    dim3 grid((unsigned)s_q, hgroups, (unsigned)batch);
    auto kern = d_qk == kDqk ? attn_mass_bf16_kernel<kDqk> : attn_mass_bf16_kernel<kDv>;
    const TimedLaunch tl(d_qk == kDqk ? "attn_mass_bf16_kernel" : "attn_mass_bf16_kernel<512>", st);
    kern<<<grid, kFwdThreads, 0, st>>>((const uint16_t*)q, (const uint16_t*)kv, indices, softmax_max, softmax_sum, mass,
                                       (int)s_q, (int)s_kv, (int)n_heads, (int)topk, scale * kLog2e, q_offset);
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

namespace dsa {
static int sparse_mla_fwd_impl(const void* q, const void* kv, const int32_t* indices, const float* sinks, void* out,
                               float* softmax_max, float* softmax_sum, int dtype, int64_t batch, int64_t s_q,
                               int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                               int64_t q_offset, void* stream) {
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
    if ((d_qk != kDqk && d_qk != kDv) || d_v != kDv)
      return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: bf16 path needs d_qk = 576 or 512, d_v = 512 "
                       "(got %lld/%lld)", (long long)d_qk, (long long)d_v);
    const bool rope = d_qk == kDqk;
    const int64_t max_rows = rope ? GatherGeom::kMaxRows : GatherGeomT<kDv>::kMaxRows;
    if (s_kv > max_rows) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: S_kv > %lld", (long long)max_rows);
    dim3 grid((unsigned)s_q, ceil_div(n_heads, kFwdHeads), (unsigned)batch);
    {
      const TimedLaunch tl(rope ? "sparse_mla_fwd_bf16_kernel" : "sparse_mla_fwd_bf16_kernel<512>", st);
      if (rope)
        sparse_mla_fwd_bf16_kernel<kDqk><<<grid, kFwdThreads, 0, st>>>(
            (const uint16_t*)q, (const uint16_t*)kv, indices, (uint16_t*)out, softmax_max, softmax_sum, (int)s_q,
            (int)s_kv, (int)n_heads, (int)topk, scale * kLog2e, q_offset, sinks);
      else
        sparse_mla_fwd_bf16_kernel<kDv><<<grid, kFwdThreads, 0, st>>>(
            (const uint16_t*)q, (const uint16_t*)kv, indices, (uint16_t*)out, softmax_max, softmax_sum, (int)s_q,
            (int)s_kv, (int)n_heads, (int)topk, scale * kLog2e, q_offset, sinks);
    }
    if (int rc = check_launch("dsa_sparse_mla_fwd(bf16)")) return rc;
    dim3 fgrid((unsigned)s_q, 1, (unsigned)batch);
    const TimedLaunch tl("sparse_mla_fwd_exact_kernel<fixup>", st);
    sparse_mla_fwd_exact_kernel<uint16_t><<<fgrid, 256, sc_bytes, st>>>(
        (const uint16_t*)q, (const uint16_t*)kv, indices, (uint16_t*)out, softmax_max, softmax_sum, (int)s_q,
        (int)s_kv, (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset, 1, sinks);
    return check_launch("dsa_sparse_mla_fwd(bf16 fixup)");
  }
  if (dtype == DSA_F32) {
    dim3 grid((unsigned)s_q, (unsigned)n_heads, (unsigned)batch);
    const TimedLaunch tl("sparse_mla_fwd_exact_kernel<float>", st);
    sparse_mla_fwd_exact_kernel<float><<<grid, 256, sc_bytes, st>>>(
        (const float*)q, (const float*)kv, indices, (float*)out, softmax_max, softmax_sum, (int)s_q, (int)s_kv,
        (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset, 0, sinks);
    return check_launch("dsa_sparse_mla_fwd(f32)");
  }
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: dtype %d not supported", dtype);
}
}  // namespace dsa

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices, void* out, float* softmax_max,
                                  float* softmax_sum, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                                  int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                                  int64_t q_offset, void* stream) {
  return dsa::sparse_mla_fwd_impl(q, kv, indices, nullptr, out, softmax_max, softmax_sum, dtype, batch, s_q, s_kv,
                                  n_heads, d_qk, d_v, topk, scale, q_offset, stream);
}

extern "C" int dsa_sparse_mla_fwd_sink(const void* q, const void* kv, const int32_t* indices, const float* sinks,
                                       void* out, float* softmax_max, float* softmax_sum, int dtype, int64_t batch,
                                       int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v,
                                       int64_t topk, float scale, int64_t q_offset, void* stream) {
  if (!sinks) return dsa::set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_fwd_sink: null sinks");
  return dsa::sparse_mla_fwd_impl(q, kv, indices, sinks, out, softmax_max, softmax_sum, dtype, batch, s_q, s_kv,
                                  n_heads, d_qk, d_v, topk, scale, q_offset, stream);
}
