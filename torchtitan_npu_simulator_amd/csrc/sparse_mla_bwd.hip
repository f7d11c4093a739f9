// Gathered sparse MLA attention backward for gfx950, without float atomics.
//
// fp32 atomics on this part top out near 1.3 TB/s of payload (one dword per L2 channel
// per clock), far too slow for the dKV scatter-add (576 fp32 per (token, key) pair), so
// the backward reduces dKV through a key-major pass instead:
//
//   (delta) delta = rowsum(dO o O) per (token, head): formed by bwd_sdp_kernel from the O
//           rows it reads beside dO, or, with a per-head sink (whose gradient needs it for
//           every row), by bwd_delta_kernel in one streaming pass; the same fp32 sum either way.
//   (alpha) bwd_sdp_kernel, workgroup = token x 128 heads, 8 waves x 16 heads (the
//           forward's gather pipeline): S^T = K Q^T and dP^T = V dO^T on
//           v_mfma_f32_16x16x32_bf16 chains sharing every K operand read, P = exp2(S*scale*
//           log2e - lse2), dS = P (dP - delta); G[token][slot][128 hg + (0..63 | 64..127)] =
//           (dS * scale | P) in bf16 and the head-summed P (attention mass) per slot.
//           bwd_dqk_kernel, workgroup = token x 128 heads, 12 waves: dQ^T += K^T dS^T with
//           each wave owning d tiles for two 32-head groups (K read transposed, dS^T from
//           the G rows staged in LDS).
//   (beta)  bwd_contrib_kernel, workgroup = token, 12 waves (X slice in VGPRs, G streamed):
//           C[token][slot][0..576) = G[slot][0..256) . [Q_token ; dO_token]  (bf16 out),
//           the dKV contribution of one (token, slot) pair summed over all 128 heads.
//   (gamma) a CSR of (token, slot) pairs per key (LDS-privatised counting sort), then
//           dkv[key] += sum of its C rows in fp32, one owner per key (plain stores).
// Query rows are processed in chunks so the bf16 G / C scratch fits the caller's
// workspace.
#include <algorithm>

#include "dsa_common.h"
#include "dsa_csr.h"
#include "dsa_gather.h"

namespace dsa {
namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kBN = 32;
constexpr int kHG = 64;                       // heads per G head group (one 128-entry half of a G row)
constexpr int kGW = 256;                      // G row width: (dS | P) x 128 heads
constexpr int kHeadsMax = 128;
// G rows hold the slots of whole 32-key blocks (K rounded up), so every block's G stores
// are unconditional
__host__ __device__ __forceinline__ int64_t g_slots(int64_t K) { return (K + kBN - 1) / kBN * kBN; }

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;



// --------------------------------------------------------------------------------------
// (alpha-1) bwd_sdp_kernel: G and the attention mass of a token, all heads in one workgroup
//
// The forward's gather pipeline (block of 32 selected KV rows DMA'd into a swizzled LDS
// tile, double-buffered) with 8 waves x 16 heads, two waves per SIMD: wave w owns heads
// 16w .. 16w+15 on v_mfma_f32_16x16x32_bf16, S^T = K Q^T and dP^T = V dO^T as two 16-key
// halves each (four independent accumulation chains that share every K operand read;
// v = k_nope), so one wave's MFMAs run while the other waits on LDS, exponentials or the
// barrier.  Latent Q and dO of the wave's heads stay in AGPRs as B operands (lane (head c,
// group g) holds columns 32s + 8g .. +8 of k-step s), rope Q in LDS; A operands are the
// tile's K rows 16x + c, chunk 4s + g (swz_a16 keeps those reads conflict-free).  Lane
// (c, g) then holds keys 16x + 4g + r (r < 4) of head 16w + c: P = exp2(S*scale*log2e -
// lse2), dS = P (dP - delta); G = (dS * scale | P) is staged transposed in LDS (8-byte
// pieces of 4 slots) and leaves as whole 512-byte slot rows; the mass sums P over the 128
// heads (DPP butterfly over a wave's 16 head lanes, then the 8 waves).  No dQ here: with no
// dQ accumulators Q and dO of 16 heads fit beside two waves per SIMD.  Each K operand read
// serves 16 heads (twice the LDS reads of a 32-head wave), which the doubled wave count
// absorbs: b128 read throughput per CU grows with the waves issuing them.
// --------------------------------------------------------------------------------------
// piece swizzle of the 256-entry transposed stage (64-byte rows): the b64 writes of one
// piece by 16 consecutive head rows, and the flush's transposed reads (4 aligned rows x 4
// pieces per lane quarter), are conflict-free
__device__ __forceinline__ int g2_swz(int r) { return (r >> 1) & 7; }

constexpr int kSdpWaves = 8;

// kD: row width of Q and KV, 576 (latent + rope) or 512 (no rope).  kOwnDelta: delta =
// rowsum(dO o O) of each head is formed here from O (read beside dO, in dO's lane layout,
// then summed over the head's four lane groups) instead of read from dbuf
template <int kD, bool kOwnDelta>
__global__ void __launch_bounds__(64 * kSdpWaves, 1)
bwd_sdp_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv, const int32_t* __restrict__ idx,
                const uint16_t* __restrict__ dout, const uint16_t* __restrict__ out, const float* __restrict__ smax,
                const float* __restrict__ ssum, const float* __restrict__ dbuf, uint16_t* __restrict__ gbuf,
                float* __restrict__ mass, int S, int s_kv, int H, int K, float scale, int64_t q_offset, int row0) {
  constexpr int kW = kSdpWaves;
  using Gather = RowGather<kW, kD, true>;
  using Geo = GatherGeomT<kD>;
  constexpr int kPer = Gather::kMaxPerWave;
  constexpr int kLat = kDv / 32;     // 16 latent k-steps of 32 columns (dP has only these)
  constexpr int kSteps = kD / 32;    // 18 | 16
  constexpr int kRB = Geo::kRowBytes;
  constexpr bool kRope = kSteps > kLat;
  __shared__ u32x4 tile[2][Geo::kTileChunks];
  __shared__ u32x4 qpe[kRope ? kHeadsMax : 1][8];  // rope Q, [head][16 B chunk ^ ((head >> 1) & 7)]
  __shared__ uint2 gst[2][kGW][kBN / 4];  // [parity][G entry][piece of 4 slots ^ g2_swz(entry)]
  __shared__ float pst[2][kW][kBN];
  __shared__ int sidx[GatherGeom::kRing][Gather::kRingInts];
  __shared__ int sh_last;

  const int lr = blockIdx.x, tok = row0 + lr, b = blockIdx.z, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;  // MFMA column (head) and k group; A row c
  const int hl = wave * 16 + c;            // head (the workgroup holds all heads)
  const bool hok = hl < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int64_t hrow = row_id * H + (hok ? hl : 0);
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kD;
  uint16_t* grow = gbuf + ((int64_t)b * gridDim.x + lr) * (int64_t)g_slots(K) * kGW;
  float* mrow = mass ? mass + row_id * K : nullptr;

  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) Gather::issue_idx(ridx, K, i, sidx[i], lane);
  }
  // latent Q and dO of head hl: k-step s holds columns 32s + 8g .. +8; lane group g also
  // loads rope chunks 2g, 2g + 1 for the LDS copy (step kLat + j reads chunk 4j + g)
  u32x4 qb[kLat], db[kLat], qr[2];
  u32x4 ob[kOwnDelta ? kLat : 1];  // O in dO's layout (kOwnDelta)
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + hrow * kD);
    const u32x4* dh = reinterpret_cast<const u32x4*>(dout + hrow * kDv);
#pragma unroll
    for (int st = 0; st < kLat; ++st) qb[st] = qh[4 * st + g];
#pragma unroll
    for (int st = 0; st < kLat; ++st) db[st] = dh[4 * st + g];
#pragma unroll
    for (int j = 0; j < 2; ++j) qr[j] = kRope ? qh[64 + 2 * g + j] : (u32x4){0u, 0u, 0u, 0u};
    if constexpr (kOwnDelta) {
      const u32x4* oh = reinterpret_cast<const u32x4*>(out + hrow * kDv);
#pragma unroll
      for (int st = 0; st < kLat; ++st) ob[st] = oh[4 * st + g];
    }
  }
  const float mx = smax[hrow], sm = ssum[hrow];
  float dlt;
  if constexpr (!kOwnDelta) dlt = dbuf[((int64_t)b * gridDim.x + lr) * H + (hok ? hl : 0)];
  const int nblk = count_row_blocks(ridx, K, s_kv, limit, vidx, &sh_last);
  if (mrow)  // slots past the last usable block carry no mass
    for (int j = nblk * kBN + tid; j < K; j += 64 * kW) mrow[j] = 0.f;
  if (nblk == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring DMA has landed before the LDS is released
    return;
  }
  const uint32_t lim = gather_limit(limit, s_kv);
  if (!hok) {
#pragma unroll
    for (int st = 0; st < kLat; ++st) qb[st] = db[st] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 2; ++j) qr[j] = (u32x4){0u, 0u, 0u, 0u};
  }
  if constexpr (kRope) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // rope chunks 64..71: lane group g writes 2g, 2g + 1
      const int ch = 2 * g + j;
      qpe[hl][ch ^ ((hl >> 1) & 7)] = qr[j];
    }
  }
  const float lse2 = (hok && sm > 0.f) ? (mx + logf(sm)) * kLog2e : INFINITY;  // +inf -> P = 0
  if constexpr (kOwnDelta) {
    // The same fp32 sum as bwd_delta_kernel, bit for bit (so results do not depend on which
    // of the two formed delta): its lane l of a head sums 16-byte chunks l + 16 j (j = 0..3,
    // in order), which this lane group g holds for l = 4a + g as chunks 4 (a + 4j) + g; its
    // xor tree over l (8, 4, 2, 1) is a's two bits here, then g's across the lanes 32 and 16
    // apart (each step adds a value and its partner's, which commutes)
    static_assert(kLat == 16, "four chunks per lane of the delta pass");
    float sa[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          part += bf16_lo(db[a + 4 * j][r]) * bf16_lo(ob[a + 4 * j][r]) +
                  bf16_hi(db[a + 4 * j][r]) * bf16_hi(ob[a + 4 * j][r]);
      sa[a] = part;
    }
    dlt = xor16_sum(xor32_sum((sa[0] + sa[2]) + (sa[1] + sa[3])));
  }
  const float delta = hok ? dlt : 0.f;
  const float scale_log2 = scale * kLog2e;
  // landed before any DMA; held in AGPRs, which the MFMAs read directly as B operands
#pragma unroll
  for (int st = 0; st < kLat; ++st) asm volatile("" : "+a"(qb[st]), "+a"(db[st]));

  // A operand of half x, k-step s = 2u + s0: K row 16x + c, chunk (4s + g) = 8u + (4 s0 + g),
  // swizzled inside its group of 8 -> ka_off[x][s0] + 128 u
  uint32_t ka_off[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int s0 = 0; s0 < 2; ++s0) ka_off[x][s0] = (16 * x + c) * kRB + 16 * ((4 * s0 + g) ^ swz_a16(16 * x + c));
  // G entries of head hl: dS at 128 (hl / 64) + hl % 64, P 64 entries later
  const int e_ds = 128 * (hl >> 6) + (hl & 63), e_p = e_ds + 64;

  // G rows and mass of block fb from stage fb & 1 -> global, in three parts.  G part u:
  // slots 16u .. 16u+15; lane group (wave, G) takes entry octet oct = 4 wave + G; two
  // transposed reads give lane c the octet's 8 values of slot 16u + c.
  auto flush_part = [&](int fb, int part) {
    const int sb = fb & 1;
    if (part == 2) {
      if (mrow && tid < kBN && fb * kBN + tid < K)
        mrow[fb * kBN + tid] = ((pst[sb][0][tid] + pst[sb][1][tid]) + (pst[sb][2][tid] + pst[sb][3][tid])) +
                               ((pst[sb][4][tid] + pst[sb][5][tid]) + (pst[sb][6][tid] + pst[sb][7][tid]));
      return;
    }
    const int c16 = lane & 15;
    const lds_char* gb = lds_bytes(&gst[sb][0][0]);
    const int slot = fb * kBN + 16 * part + c16;
    const int oct = 4 * wave + (lane >> 4);
    const lds_char* a[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int row = 8 * oct + 4 * x + (c16 >> 2);
      const int piece = 4 * part + (c16 & 3);
      a[x] = gb + row * (kBN * 2) + 8 * (piece ^ g2_swz(row));
    }
    const u32x4 v = lds_read_tr_pair(a[0], a[1]);
    *reinterpret_cast<u32x4*>(grow + (int64_t)slot * kGW + 8 * oct) = v;  // (rows padded to whole blocks)
  };

  const typename Gather::PackedLanes gl = Gather::packed_lanes(wave, lane);
  const lds_char* qpe_b = lds_bytes(&qpe[0][0]);
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // ring entries 0..2 landed
  __syncthreads();                                                  // publishes them and qpe
  uint32_t vm_cur = Gather::ring_valid(sidx[0], lane, lim, K);
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    Gather::issue_slot(kvb, &tile[0][0], i, wave, Gather::ring_slot(sidx[0], i, gl), gl, lim, K);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  constexpr int kQBatch = 1;             // k-steps per batch
  constexpr int kQB = kSteps / kQBatch;  // 18 | 16 batches
  static_assert(kQB >= kPer, "one row DMA per batch");

  // P / dS / G staging / mass of block pb (S^T, dP^T halves sp, pp; validity vm), in pieces
  // spread over the next block's MFMA batches:
  //   0: P (8 values) and its stage,  1: dS and its stage,  3: mass butterfly + partial
  // value 4x + r of a lane: key 16x + 4g + r
  float pv[8];
  auto stage = [&](int sb, int e, const float (&src)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int pc = 4 * x + g;  // slots 16x + 4g .. +3
      gst[sb][e][pc ^ g2_swz(e)] = make_uint2(pack_bf16x2(src[4 * x], src[4 * x + 1]),
                                              pack_bf16x2(src[4 * x + 2], src[4 * x + 3]));
    }
  };
  auto pds_piece = [&](int piece, const f32x4 (&sp)[2], const f32x4 (&pp)[2], uint32_t vm, int pb) {
    const int sb = pb & 1;
    if (piece == 0) {
      if (vm == 0xffffffffu) {  // (wave-uniform) every key of the block is valid: no masking
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int r = 0; r < 4; ++r) pv[4 * x + r] = __builtin_amdgcn_exp2f(sp[x][r] * scale_log2 - lse2);
      } else {
        const uint32_t vmg = vm >> (4 * g);  // bit 16x + r: key 16x + 4g + r
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool ok = (vmg >> (16 * x + r)) & 1u;
            pv[4 * x + r] = ok ? __builtin_amdgcn_exp2f(sp[x][r] * scale_log2 - lse2) : 0.f;
          }
      }
      stage(sb, e_p, pv);
    } else if (piece == 1) {
      float dv[8];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int r = 0; r < 4; ++r) dv[4 * x + r] = pv[4 * x + r] * (pp[x][r] - delta) * scale;
      stage(sb, e_ds, dv);
    } else if (piece == 3) {
      // mass: butterfly over the 16 head lanes of a lane group (lane bits 3..1 halve the 8
      // values, bit 0 completes the sum); lane c ends with value (c >> 1) & 7.  The halves
      // are chosen by bit masks (a select between two array elements would become an
      // indexed read).
      auto bstep = [&](auto mc, int nh) {
        constexpr int m = decltype(mc)::value;
        const uint32_t up = ((lane & m) != 0) ? 0xffffffffu : 0u;
#pragma unroll
        for (int j = 0; j < nh; ++j) {
          const uint32_t a = __float_as_uint(pv[j]), bb = __float_as_uint(pv[j + nh]);
          const float send = __uint_as_float((a & up) | (bb & ~up));
          const float keep = __uint_as_float((bb & up) | (a & ~up));
          pv[j] = keep + lane_xor<m>(send);
        }
      };
      bstep(std::integral_constant<int, 8>{}, 4);
      bstep(std::integral_constant<int, 4>{}, 2);
      bstep(std::integral_constant<int, 2>{}, 1);
      const float tot = pv[0] + lane_xor<1>(pv[0]);
      if ((lane & 1) == 0) {
        const int v = (c >> 1) & 7;
        pst[sb][wave][16 * (v >> 2) + 4 * g + (v & 3)] = tot;
      }
    }
  };

  // iteration blk: S^T / dP^T of block blk on tile blk & 1 while block blk+1's rows are
  // DMA'd into the other tile, with P / dS / G / mass of block blk-1 and the G and mass
  // stores of block blk-2 spread over its MFMA batches; the iteration ends with its DMAs
  // landed and one barrier (which also publishes blk-1's stage for its flush).
  // (unrolled by two so that block blk's accumulators and block blk-1's alternate between
  // two register sets instead of being copied every block)
  f32x4 s_a[2], p_a[2], s_b[2], p_b[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) s_a[x] = p_a[x] = s_b[x] = p_b[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
  uint32_t vm_prev = 0u;
  auto block_iter = [&](int blk, f32x4 (&sacc)[2], f32x4 (&pacc)[2], const f32x4 (&sprev)[2],
                        const f32x4 (&pprev)[2]) {
    if (wave == 0 && blk + 3 < nblk)
      Gather::issue_idx(ridx, K, blk + 3, sidx[(blk + 3) & (GatherGeom::kRing - 1)], lane);
    const lds_char* tb = lds_bytes(&tile[blk & 1][0]);
    u32x4* dst_tile = &tile[(blk + 1) & 1][0];
    const int* ring = sidx[(blk + 1) & (GatherGeom::kRing - 1)];
    const int rows_left = K - (blk + 1) * kBN;
    const uint32_t vm_next = Gather::ring_valid(ring, lane, lim, rows_left);
    uint32_t raw_next = Gather::ring_slot(ring, 0, gl);
#pragma unroll
    for (int x = 0; x < 2; ++x) sacc[x] = pacc[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
    u32x4 a[2][kQBatch][2];  // [buffer][step of the batch][half]
    u32x4 rope[2];  // rope B operands of steps kLat, kLat + 1 (chunk 4j + g of the rope)
    auto read_a = [&](u32x4 (&dst)[kQBatch][2], int sb) {  // steps sb .. sb + kQBatch - 1
#pragma unroll
      for (int u = 0; u < kQBatch; ++u)
#pragma unroll
        for (int x = 0; x < 2; ++x) dst[u][x] = lds_read16(tb + ka_off[x][(sb + u) & 1] + 128 * ((sb + u) >> 1));
    };
    read_a(a[0], 0);
    static_for<kQB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      constexpr int s0 = nb * kQBatch;
      if constexpr (nb + 1 < kQB) read_a(a[(nb + 1) & 1], (nb + 1) * kQBatch);
      if constexpr (kRope && nb + 1 >= kLat && nb + 1 < kSteps) {  // rope B operand one batch ahead
        constexpr int j = nb + 1 - kLat;
        rope[j] = lds_read16(qpe_b + hl * 128 + 16 * ((4 * j + g) ^ ((hl >> 1) & 7)));
      }
      if constexpr (nb < kPer) {
        const uint32_t raw = raw_next;
        if constexpr (nb + 1 < kPer) raw_next = Gather::ring_slot(ring, nb + 1, gl);
        Gather::issue_slot(kvb, dst_tile, nb, wave, raw, gl, lim, rows_left);
      }
#pragma unroll
      for (int u = 0; u < kQBatch; ++u) {
        const u32x4 bq = s0 + u < kLat ? qb[(s0 + u) % kLat] : rope[(s0 + u - kLat) & 1];
#pragma unroll
        for (int x = 0; x < 2; ++x) sacc[x] = mfma16x16x32(as_bf16x8(a[nb & 1][u][x]), as_bf16x8(bq), sacc[x]);
        if constexpr (s0 < kLat) {
#pragma unroll
          for (int x = 0; x < 2; ++x)
            pacc[x] = mfma16x16x32(as_bf16x8(a[nb & 1][u][x]), as_bf16x8(db[s0 + u]), pacc[x]);
        }
      }
      // the pieces of block blk-1 and the flush of block blk-2 (after the block's last row
      // DMA) are spread over the block's MFMAs
      if constexpr (nb == 1 || nb == 4 || nb == 7) {
        if (blk > 0) pds_piece(nb == 1 ? 0 : nb == 4 ? 1 : 3, sprev, pprev, vm_prev, blk - 1);
      }
      if constexpr (nb >= kPer && (nb == 9 || nb == 11 || nb == 13)) {
        if (blk > 1) flush_part(blk - 2, (nb - 9) / 2);
      }
      static_for<(s0 < kLat ? 4 * kQBatch : 2 * kQBatch)>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
        __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);  // VALU / SALU
        __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // VMEM (row DMA, G stores)
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    // block blk-2's G and mass stores went out after the block's last row DMA; two store
    // instructions follow that DMA unconditionally (one per G part), so vmcnt(2) waits for
    // every DMA (they retire in order) but not for the stores
    if (blk > 1) {
      asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // block blk+1 and ring entry blk+3 landed
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    vm_prev = vm_cur;
    vm_cur = vm_next;
  };
  int blk = 0;
  for (; blk + 1 < nblk; blk += 2) {
    block_iter(blk, s_a, p_a, s_b, p_b);
    block_iter(blk + 1, s_b, p_b, s_a, p_a);
  }
  if (blk < nblk) block_iter(blk, s_a, p_a, s_b, p_b);
  // the last block's P / dS / G / mass, the stores of the one before, then its own stores
  const bool last_a = nblk & 1;
  f32x4 s_last[2], p_last[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    s_last[x] = last_a ? s_a[x] : s_b[x];
    p_last[x] = last_a ? p_a[x] : p_b[x];
  }
#pragma unroll
  for (int piece = 0; piece < 4; ++piece) pds_piece(piece, s_last, p_last, vm_prev, nblk - 1);  // (2: none)
  if (nblk > 1) {
    flush_part(nblk - 2, 0);
    flush_part(nblk - 2, 1);
    flush_part(nblk - 2, 2);
  }
  __syncthreads();
  flush_part(nblk - 1, 0);
  flush_part(nblk - 1, 1);
  flush_part(nblk - 1, 2);
}

// --------------------------------------------------------------------------------------
// (alpha-2) bwd_dqk_kernel: dQ = (dS * scale) K for a token, all heads in one workgroup
//
// The forward's P.V structure with P := the staged dS of bwd_sdp_kernel and V := the whole
// 576-column K row: dQ^T[32 d x 32 heads] += K^T dS^T on v_mfma_f32_32x32x16_bf16.  Twelve
// waves (three per SIMD; eight for 512-column rows): wave w owns the d tiles w % 6,
// w % 6 + 6, w % 6 + 12 (of 18; w % 4 + 4i of 16) for the two 32-head groups of half
// w / 6 (w / 4), so each K^T operand read from LDS feeds 4 MFMAs (2 head groups x 2 key
// steps) and the tile is read twice per workgroup instead of once per head group; dQ^T
// (3 x 2 x 16 fp32 per lane) stays in the accumulation registers.  The dS columns of each slot's G row (two 128-byte pieces) are
// DMA'd into a [slot][128 heads] tile (16-byte chunk c of slot r at c ^ 4 (r & 3)) and read
// back transposed with the forward's V^T lane pattern, so both operands share the k order.
// Keys that are not valid contribute 0.
// --------------------------------------------------------------------------------------
__device__ __forceinline__ int ds_swz(int r) { return 4 * (r & 3); }

template <int kD>  // row width of KV and dQ: 576 or 512
struct DqkShape {
  static constexpr int kDT = kD / 32;                 // 18 | 16 d tiles
  static constexpr int kPh = kD == 576 ? 6 : 4;       // d-tile owners per head half (18 = 6 x 3, 16 = 4 x 4)
  static constexpr int kWaves = 2 * kPh;              // 12 | 8 waves: three | two per SIMD
  static constexpr int kOwn = (kDT + kPh - 1) / kPh;  // d tiles per wave: 3 | 4
};

template <int kD>  // row width of KV and dQ: 576 or 512
__global__ void __launch_bounds__(DqkShape<kD>::kWaves * 64, 1)
bwd_dqk_kernel(const uint16_t* __restrict__ kv, const int32_t* __restrict__ idx, const uint16_t* __restrict__ gbuf,
               uint16_t* __restrict__ dq, int S, int s_kv, int H, int K, int64_t q_offset, int row0) {
  using Shape = DqkShape<kD>;
  constexpr int kWaves = Shape::kWaves, kPh = Shape::kPh;
  using Gather = RowGather<kWaves, kD>;
  using Geo = GatherGeomT<kD>;
  constexpr int kPer = Gather::kMaxPerWave;  // 3 | 4 row instructions per wave and block
  constexpr int kDT = Shape::kDT;
  constexpr int kOwn = Shape::kOwn;
  constexpr int kRB = Geo::kRowBytes;
  static_assert(kPer <= kOwn, "one row instruction per owned tile");
  static_assert(kWaves >= 8, "eight waves issue the dS tile DMA");
  __shared__ u32x4 tile[2][Geo::kTileChunks];
  __shared__ u32x4 dsl[2][kBN * 16];  // dS tile: [slot][16 chunks of 8 heads ^ ds_swz(slot)]
  __shared__ int sidx[GatherGeom::kRing][Gather::kRingInts];
  __shared__ int sh_last;

  const int lr = blockIdx.x, tok = row0 + lr, b = blockIdx.z, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wt = wave % kPh, hh2 = wave / kPh;  // d-tile owner, head half (groups 2 hh2, 2 hh2 + 1)
  const int n = lane & 31, h = lane >> 5;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kD;
  const uint16_t* grow = gbuf + ((int64_t)b * gridDim.x + lr) * (int64_t)g_slots(K) * kGW;

  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) Gather::issue_idx(ridx, K, i, sidx[i], lane);
  }
  const int nblk = count_row_blocks(ridx, K, s_kv, limit, vidx, &sh_last);
  if (nblk == 0) {  // no usable key: dQ = 0
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int i = tid; i < H * (kD / 2); i += kWaves * 64)
      reinterpret_cast<uint32_t*>(dq + row_id * H * kD)[i] = 0u;
    return;
  }
  const uint32_t lim = gather_limit(limit, s_kv);

  // K^T reads (A operand), as the forward's V^T reads: lane group G = lane / 16 covers d
  // 16 (G & 1) .. +15 and k half h = G >> 1; source lane c supplies key row 16kk + 8x + 4h
  // + c/4 and d columns 32dt + 16 (G & 1) + 4 (c % 4) .. +3; dt = 2u + d0 -> + 128 u.
  // dS^T reads (B operand) of head group g4: the same rows of the dS tile, heads 32 g4 +
  // 16 (G & 1) + 4 (c % 4) .. +3 (chunk 4 g4 + 2 (G & 1) + (c % 4) / 2); kk -> + 16 rows.
  uint32_t tr_off[2][2], ds_off[2][2];
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
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int dch = 4 * (2 * hh2 + gg) + 2 * (G & 1) + ((c & 3) >> 1);
        ds_off[gg][x] = r * 256 + 16 * (dch ^ ds_swz(r)) + 8 * (c & 1);
      }
    }
  }
  // dS tile DMA of block blk: instruction J (wave J) covers slots 4J .. 4J+3, lane ->
  // slot 4J + lane/16, stored chunk lane % 16 = source chunk (lane % 16) ^ ds_swz(slot);
  // source chunk c < 8: dS entries 8c .. (head group 0), else 128 + 8 (c - 8) (group 1)
  auto issue_ds = [&](int blk, int buf) {
    if (wave < 8) {  // (wave-uniform) eight instructions of 1 KB cover the 32 slots
      const int J = wave;
      const int r = 4 * J + (lane >> 4);
      const int c = (lane & 15) ^ ds_swz(r);
      const int eo = c < 8 ? 8 * c : 128 + 8 * (c - 8);
      // (G rows are padded to whole 32-slot blocks, and the score kernel writes exact zeros
      // at the padding slots past K, as at every unusable slot: no clamp to slot K - 1, whose
      // dS would otherwise stand in for them)
      const int slot = blk * kBN + r;
      dma16_to_lds(grow, (uint32_t)(slot * kGW + eo) * 2u, (uint32_t)(uintptr_t)&dsl[buf][J * 64]);
    }
  };

  f32x16 dqa[kOwn][2];
#pragma unroll
  for (int t = 0; t < kOwn; ++t)
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) dqa[t][gg] = (f32x16){0.f};

  const typename Gather::PackedLanes gl = Gather::packed_lanes(wave, lane);
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // ring entries 0..2 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    Gather::issue_slot(kvb, &tile[0][0], i, wave, Gather::ring_slot(sidx[0], i, gl), gl, lim, K);
  issue_ds(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    if (wave == 0 && blk + 3 < nblk)
      Gather::issue_idx(ridx, K, blk + 3, sidx[(blk + 3) & (GatherGeom::kRing - 1)], lane);
    const int buf = blk & 1;
    const lds_char* vb = lds_bytes(&tile[buf][0]);
    const lds_char* db = lds_bytes(&dsl[buf][0]);
    u32x4* dst_tile = &tile[buf ^ 1][0];
    const int* ring = sidx[(blk + 1) & (GatherGeom::kRing - 1)];
    const int rows_left = K - (blk + 1) * kBN;
    if (blk + 1 < nblk) issue_ds(blk + 1, buf ^ 1);
    auto read_kt = [&](u32x4 (&dst)[2], int dt) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const lds_char* base = vb + kk * 16 * kRB + 128 * (dt >> 1);
        dst[kk] = lds_read_tr_pair(base + tr_off[0][dt & 1], base + tr_off[1][dt & 1]);
      }
    };
    u32x4 av[2][2];
    read_kt(av[0], wt);
    // dS^T operands of the wave's two head groups.  No masking: the score kernel stores
    // dS = P (dP - delta) with P = 0 exactly at every unusable slot and absent head, and the
    // rows gathered for those slots (row 0) are finite, so they add exact zeros.
    u32x4 bs[2][2];
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        bs[gg][kk] = lds_read_tr_pair(db + ds_off[gg][0] + kk * 16 * 256, db + ds_off[gg][1] + kk * 16 * 256);
    uint32_t raw_next = Gather::ring_slot(ring, 0, gl);
    auto issue_rows = [&](auto tc) {  // one row instruction per tile
      constexpr int nb = decltype(tc)::value;
      if constexpr (nb < kPer) {
        const uint32_t raw = raw_next;
        if constexpr (nb + 1 < kPer) raw_next = Gather::ring_slot(ring, nb + 1, gl);
        Gather::issue_slot(kvb, dst_tile, nb, wave, raw, gl, lim, rows_left);
      }
    };
    static_for<kOwn>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      const int dt = wt + kPh * t;  // wave-uniform
      if (dt < kDT) {
        if (t + 1 < kOwn && dt + kPh < kDT) read_kt(av[(t + 1) & 1], dt + kPh);
        issue_rows(tc);  // block blk+1's rows
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
            dqa[t][gg] = mfma32x32x16(as_bf16x8(av[t & 1][kk]), as_bf16x8(bs[gg][kk]), dqa[t][gg]);
      } else {  // (waves with four tiles) the remaining row instructions
        issue_rows(tc);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // block blk+1 (rows, dS) and ring entry blk+3 landed
    __syncthreads();
  }

  // ---- epilogue: tile t, group gg: lane holds d = 32 dt + 8 j + 4 h + i of head
  // 32 (2 hh2 + gg) + n (dS was pre-scaled) ----
#pragma unroll
  for (int t = 0; t < kOwn; ++t) {
    const int dt = wt + kPh * t;
    if (dt >= kDT) break;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int hd = 32 * (2 * hh2 + gg) + n;
      if (hd >= H) continue;
      uint2* drow = reinterpret_cast<uint2*>(dq + (row_id * H + hd) * kD);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2 w;
        w.x = pack_bf16x2(dqa[t][gg][4 * j], dqa[t][gg][4 * j + 1]);
        w.y = pack_bf16x2(dqa[t][gg][4 * j + 2], dqa[t][gg][4 * j + 3]);
        drow[(32 * dt + 8 * j + 4 * h) / 4] = w;
      }
    }
  }
}

// --------------------------------------------------------------------------------------
// (beta) C[token][slot] = G[token][slot] . X_token,  X = [(Q, dO) per head group]
// rows of X: k = 128 hg + 64 type + i  ->  type 0: q[64hg + i], type 1: dout[64hg + i]
//
// One workgroup per token, 12 waves; the output columns form 16-column MFMA tiles (36 of
// a 576-wide row, 32 of a 512-wide one), three per wave at 576 columns (wave w: columns
// 48w .. 48w+47) and at 512 three for waves 0..7, two for waves 8..11 (8 tiles per SIMD
// either way).  Each wave keeps its slice of X transposed in VGPRs for the whole token (A
// operand of C^T = X^T G^T, 96 VGPRs).  G is streamed through a double-buffered LDS tile of
// 32 slots x 256 (DMA), so G, X and C each cross HBM exactly once.  The C rows of each
// 32-slot step are assembled in a double-buffered LDS stage (every wave adds its columns)
// and leave as whole 1152- (1024-) byte rows, 16 bytes per lane: the MFMA output layout
// alone would give 8-byte pieces scattered over 16 rows per store instruction.
// --------------------------------------------------------------------------------------
constexpr int kCW = 12;                     // waves
constexpr int kCThreads = kCW * 64;
constexpr int kCT = 32;                     // slots per G tile: one step (64 measured 1 % slower)
constexpr int kGTChunks = kCT * (kGW / 8);  // 1024 16-byte chunks (16 KB)
constexpr int kCS = 32;                     // slots per step (C stage rows)
constexpr int kXK = 64;                     // X rows staged per chunk while loading X
template <int kD>
struct ContribGeom {
  static constexpr int kRC = kD / 8;           // 16-byte chunks per C row (72 | 64)
  static constexpr int kStChunks = kCS * kRC;  // C stage: 2304 | 2048 chunks
  static constexpr int kXChunks = kXK * kRC;   // X staging: 4608 | 4096 chunks
  static constexpr int kNT = kD / 16;          // 16-column tiles (36 | 32)
  static constexpr int kFull = kNT - 2 * kCW;  // waves owning three tiles (12 | 8); the rest own two
  static_assert(kFull > 0 && kFull <= kCW, "two or three tiles per wave");
  static_assert(2 * kGTChunks + 2 * kStChunks >= kGTChunks + kXChunks, "X staging reuses the tile space after G tile 0");
  // first tile of wave w
  static __device__ __forceinline__ int tile0(int w) { return w < kFull ? 3 * w : 3 * kFull + 2 * (w - kFull); }
};

// C stage layout: row r (slot), 16-byte chunk c stored at c ^ ((r >> 1) & 7)
__device__ __forceinline__ int stage_swz(int r) { return (r >> 1) & 7; }

template <int kHGroups, int kD>
__global__ void __launch_bounds__(kCThreads, 1)
bwd_contrib_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ dout,
                   const int32_t* __restrict__ idx, const uint16_t* __restrict__ gbuf, uint16_t* __restrict__ cbuf,
                   int S, int s_kv, int H, int K, int64_t q_offset, int row0, int rows) {
  using CG = ContribGeom<kD>;
  constexpr int kRC = CG::kRC, kStChunks = CG::kStChunks, kXChunks = CG::kXChunks;
  constexpr int kKSteps = 4 * kHGroups;                // 32-row k steps of X (128 rows per head group)
  __shared__ u32x4 lds[2 * kGTChunks + 2 * kStChunks];  // X staging at start; then G tiles + C stages
  __shared__ int sh_last;

  const int lr = launch_row();  // local row in chunk
  const int tok = row0 + lr, b = blockIdx.y;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  const int nblk = count_row_blocks(ridx, K, s_kv, tok + q_offset, vidx, &sh_last);
  if (nblk == 0) return;
  const int nslots = min(K, nblk * kBN);
  const uint16_t* grow = gbuf + ((int64_t)b * rows + lr) * (int64_t)g_slots(K) * kGW;
  uint16_t* crow = cbuf + ((int64_t)b * rows + lr) * (int64_t)K * kD;
  const lds_char* lb = lds_bytes(&lds[0]);
  const int t0w = CG::tile0(wave);               // the wave's first 16-column tile
  const bool three = CG::kFull == kCW || wave < CG::kFull;  // (wave-uniform) it owns three tiles

  // ---- stream G tiles; per 32-slot step C^T[16 cols x 16 slots] = X^T . G^T on six tiles ----
  // G tile DMA: instruction J = wave + 12 i covers tile chunks [64J, 64J+64), chunk
  // p = slot*32 + (c ^ swz16(slot))
  lds_char* const gtile = lds_bytes(&lds[0]);
  lds_char* const stage = lds_bytes(&lds[2 * kGTChunks]);
  const int ntiles = (nslots + kCT - 1) / kCT;
  // (lane and thread indices pass through empty asm inside the loops so their derived
  // address arithmetic is recomputed there instead of being hoisted into registers that the
  // X slice needs)
  auto load_g = [&](int tl, int buf) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < (kGTChunks / 64 + kCW - 1) / kCW; ++i) {
      const int J = wave + kCW * i;
      if (J < kGTChunks / 64) {
        const int p = J * 64 + ln;
        const int slot = p >> 5, pos = p & 31;
        const int c = pos ^ swz16(slot);
        const int gs = min(tl * kCT + slot, K - 1);
        dma16_to_lds(grow, (uint32_t)(gs * kGW + c * 8) * 2u,
                     (uint32_t)(uintptr_t)&lds[buf * kGTChunks + J * 64]);
      }
    }
  };
  load_g(0, 0);

  // ---- X^T slice into VGPRs: xa[t][ks] = X[32 ks + 8g .. +8][16 (t0w + t) + col] ----
  // (rows of dO at the rope columns are zero, so every MFMA below runs unconditionally)
  // G tile 0 is requested first: its DMA lands in tile buffer 0 while X is staged through
  // the LDS after it.  X is staged in 2 * kHGroups chunks of 64 rows; every chunk's loads
  // are issued before the first is staged, so the chunks cost one memory round trip, not
  // one each.
  u32x4 xa[3][kKSteps];
  const int tr_row = 8 * g + (col >> 2);  // source row within a 32-row k step (+4 second read)
  constexpr int kXPer = (kXChunks + kCThreads - 1) / kCThreads;  // staged chunks per thread and X chunk
  u32x4 xraw[2 * kHGroups][kXPer];
#pragma unroll
  for (int kc = 0; kc < 2 * kHGroups; ++kc) {
    const int hgk = kc >> 1, type = kc & 1;
#pragma unroll
    for (int m = 0; m < kXPer; ++m) {
      // (no load under a lane-dependent branch, which would make the compiler wait for each
      // load before the next: addresses are clamped into the tensors and the chunks outside
      // them zeroed after the load)
      const int i = tid + kCThreads * m;
      const int ic = min(i, kXChunks - 1);
      const int row = ic / kRC, c = ic - row * kRC;
      const int head = hgk * kHG + row;
      const int64_t hrow = row_id * H + min(head, H - 1);
      const u32x4 v = type == 0 ? *reinterpret_cast<const u32x4*>(q + hrow * kD + c * 8)
                                : *reinterpret_cast<const u32x4*>(dout + hrow * kDv + min(c, kDv / 8 - 1) * 8);
      const bool ok = i < kXChunks && head < H && (type == 0 || c < kDv / 8);
      xraw[kc][m] = ok ? v : (u32x4){0u, 0u, 0u, 0u};
    }
  }
  u32x4* const xst = &lds[kGTChunks];  // X staging: after G tile 0
#pragma unroll
  for (int kc = 0; kc < 2 * kHGroups; ++kc) {
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kXPer; ++m) {
      const int i = tid + kCThreads * m;
      const int row = i / kRC, c = i - row * kRC;
      if (i < kXChunks) xst[row * kRC + (c ^ swz8(row))] = xraw[kc][m];
    }
    __syncthreads();
#pragma unroll
    for (int kl = 0; kl < 2; ++kl) {  // two 32-row k steps per staged chunk
      const int ks = 2 * kc + kl;
      const int r1 = 32 * kl + tr_row, r2 = r1 + 4;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const int c0 = 2 * min(t0w + t, CG::kNT - 1) + ((col & 3) >> 1);  // (a two-tile wave's third: unused)
        const lds_char* a1 = lb + 16 * (kGTChunks + r1 * kRC + (c0 ^ swz8(r1))) + 8 * (col & 1);
        const lds_char* a2 = lb + 16 * (kGTChunks + r2 * kRC + (c0 ^ swz8(r2))) + 8 * (col & 1);
        xa[t][ks] = lds_read_tr_pair(a1, a2);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) asm volatile("" : "+v"(xa[t][ks]));  // landed before the DMAs
  __syncthreads();

  // C-row store instructions a wave issues per step: one per 768-chunk slice of the stage
  // that holds any of its chunks (576 columns: 3 for every wave; 512: 3 for waves 0..7, 2
  // for waves 8..11)
  constexpr int kStSlices = (kStChunks + kCThreads - 1) / kCThreads;
  const bool last_slice = kStChunks % kCThreads == 0 || wave * 64 < kStChunks % kCThreads;
  // the C rows of step n leave the stage during step n+1's MFMAs (one slice of row stores
  // per two k-steps), so the stores overlap matrix work instead of following a barrier
  auto store_rows = [&](int m, int ps0, int pstep) __attribute__((always_inline)) {
    const lds_char* pst = stage + (pstep & 1) * (kStChunks * 16);
    int t_ = tid;
    asm volatile("" : "+v"(t_));
    const int i = t_ + kCThreads * m;
    const int r = i / kRC, c = i - r * kRC;
    if ((kStChunks % kCThreads == 0 || i < kStChunks) && ps0 + r < nslots) {
      const u32x4 v = lds_read16(pst + r * (kRC * 16) + 16 * (c ^ stage_swz(r)));
      // non-temporal: the rows are read back once, by the key-major reduction (with the
      // reduction's non-temporal loads this makes that pass ≈4 % faster and this one ≈0.7 %
      // slower)
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(crow + (int64_t)(ps0 + r) * kD + 8 * c));
    }
  };
  int step = 0;
  int prev_s0 = -1;  // first slot of the step whose rows wait in the stage (-1: none)
  for (int tl = 0; tl < ntiles; ++tl) {
    const int buf = tl & 1;
    // this wave's part of tile tl landed.  Its DMA was issued before the C-row stores that
    // tile tl-1's step issues, those of step tl-2 (none when tl-1 is step 0).  Every row of
    // a step before the last exists, so every store instruction of that step issues; vector
    // memory operations retire in issue order, so waiting until only those stores are
    // outstanding covers the DMA and leaves the stores in flight
    static_assert(kStSlices == 3 && kCT == kCS, "the counted waits below assume three stage slices, one step per tile");
    if (tl <= 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (last_slice) {
      asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    }
    __syncthreads();  // every wave's part landed; the other G buffer is free
    if (tl + 1 < ntiles) load_g(tl + 1, buf ^ 1);
    const lds_char* gb = gtile + buf * (kGTChunks * 16);
    for (int sh = 0; sh < kCT / kCS; ++sh, ++step) {
      const int s0 = tl * kCT + kCS * sh;  // first slot of the step
      if (s0 >= nslots) break;             // workgroup-uniform
      f32x4 acc[2][3];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int t = 0; t < 3; ++t) acc[h2][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
      const lds_char* gl[2];
      int sw[2];
      int cl = col;
      asm volatile("" : "+v"(cl));
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int sl = kCS * sh + 16 * h2 + cl;  // B operand row (slot) within the tile
        gl[h2] = gb + 16 * (sl * 32);
        sw[h2] = swz16(sl);
      }
      u32x4 bg[2][2];  // [buffer][h2]
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) bg[0][h2] = lds_read16(gl[h2] + 16 * (g ^ sw[h2]));
#pragma unroll
      for (int ks = 0; ks < kKSteps; ++ks) {
        if (ks + 1 < kKSteps) {
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) bg[(ks + 1) & 1][h2] = lds_read16(gl[h2] + 16 * ((4 * (ks + 1) + g) ^ sw[h2]));
        }
        // (the next k-step's reads stay ahead of this step's MFMAs; left to itself the
        // compiler issues each read just before its MFMA and waits for it there)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int t = 0; t < 2; ++t)
            acc[h2][t] = mfma16x16x32(as_bf16x8(xa[t][ks]), as_bf16x8(bg[ks & 1][h2]), acc[h2][t]);
        if (three) {
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
            acc[h2][2] = mfma16x16x32(as_bf16x8(xa[2][ks]), as_bf16x8(bg[ks & 1][h2]), acc[h2][2]);
        }
        if (prev_s0 >= 0) {  // slice m after k-step 2m + 1 (with four k-steps: the last two after the last)
#pragma unroll
          for (int m = 0; m < kStSlices; ++m)
            if (ks == min(2 * m + 1, kKSteps - 1)) store_rows(m, prev_s0, step - 1);
        }
      }
      // lane (slot 16 h2 + col, g) holds columns 16 (t0w + t) + 4g + r: 8 bytes at chunk
      // 2 (t0w + t) + g/2, half g & 1 of the stage row
      lds_char* stg = stage + (step & 1) * (kStChunks * 16);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int r = 16 * h2 + col;
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          if (t == 2 && !three) break;
          typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 w2 = {pack_bf16x2(acc[h2][t][0], acc[h2][t][1]), pack_bf16x2(acc[h2][t][2], acc[h2][t][3])};
          const int c = 2 * (t0w + t) + (g >> 1);
          *(__attribute__((address_space(3))) u32x2*)(stg + r * (kRC * 16) + 16 * (c ^ stage_swz(r)) + 8 * (g & 1)) = w2;
        }
      }
      __syncthreads();  // the step's C rows are complete in the stage
      prev_s0 = s0;
    }
  }
  // the last step's rows
  if (prev_s0 >= 0) {
#pragma unroll
    for (int m = 0; m < kStSlices; ++m) store_rows(m, prev_s0, step - 1);
  }
}

// --------------------------------------------------------------------------------------
// exact fp32 path (any D): one workgroup per (token, head); dkv by fp32 atomics
// --------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
bwd_exact_f32_kernel(const float* __restrict__ q, const float* __restrict__ kv, const int32_t* __restrict__ idx,
                     const float* __restrict__ out, const float* __restrict__ dout, const float* __restrict__ smax,
                     const float* __restrict__ ssum, float* __restrict__ dq, float* __restrict__ dkv, int S,
                     int s_kv, int H, int K, int dqk, int dv, float scale, int64_t q_offset,
                     const float* __restrict__ sinks, float* __restrict__ dsink) {
  extern __shared__ float ds[];  // K
  __shared__ float red[256];
  const int tok = blockIdx.x, head = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int64_t row_id = (int64_t)b * S + tok;
  const int64_t hr = row_id * H + head;
  const int32_t* ridx = idx + row_id * K;
  const float* qh = q + hr * dqk;
  const float* doh = dout + hr * dv;
  const float* kvb = kv + (int64_t)b * s_kv * dqk;
  const int64_t limit = tok + q_offset;
  float part = 0.f;
  for (int d = tid; d < dv; d += 256) part += doh[d] * out[hr * dv + d];
  red[tid] = part;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  const float delta = red[0];
  const float sm = ssum[hr];
  const float lse = sm > 0.f ? smax[hr] + logf(sm) : INFINITY;
  if (sinks && tid == 0) atomicAdd(&dsink[head], -expf(sinks[head] - lse) * delta);  // (one per token and head)
  __syncthreads();
  for (int j = tid; j < K; j += 256) {
    const int v = ridx[j];
    float g = 0.f;
    if (slot_ok(v, s_kv, limit)) {
      const float* kr = kvb + (int64_t)v * dqk;
      float s = 0.f, dp = 0.f;
      for (int d = 0; d < dqk; ++d) s = fmaf(qh[d], kr[d], s);
      for (int d = 0; d < dv; ++d) dp = fmaf(doh[d], kr[d], dp);
      const float p = expf(s * scale - lse);
      g = p * (dp - delta);
      // dV part (uses p) goes straight out; dK part below
      for (int d = 0; d < dv; ++d) atomicAdd(&dkv[((int64_t)b * s_kv + v) * dqk + d], p * doh[d]);
    }
    ds[j] = g;
  }
  __syncthreads();
  for (int d = tid; d < dqk; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < K; ++j) {
      const float g = ds[j];
      if (g == 0.f) continue;
      const int v = ridx[j];
      acc = fmaf(g, kvb[(int64_t)v * dqk + d], acc);
      atomicAdd(&dkv[((int64_t)b * s_kv + v) * dqk + d], scale * g * qh[d]);
    }
    dq[hr * dqk + d] = scale * acc;
  }
}

// delta[b][lr][h] = sum_d dO[row, h, d] * O[row, h, d] (fp32) for the chunk's rows: one
// 16-lane group per (row, head), 32 columns per lane (four 16-byte loads of each tensor).
// With a per-head sink it also writes pd[b][lr][h] = -p_sink delta, p_sink = e^(sink - m2) /
// s2 from the row statistics (which include the sink): the sink's gradient summed over rows.
__global__ void __launch_bounds__(256)
bwd_delta_kernel(const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, float* __restrict__ delta,
                 int64_t n, int S, int H, int row0, int rows, const float* __restrict__ sinks,
                 const float* __restrict__ smax, const float* __restrict__ ssum, float* __restrict__ pd) {
  const int64_t grp = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (b, lr, h) flattened, n of them
  const int l = threadIdx.x & 15;
  const int64_t g = grp < n ? grp : n - 1;
  const int64_t b = g / ((int64_t)rows * H), rem = g - b * rows * H;
  const int64_t hr = (b * S + row0 + rem / H) * H + rem % H;
  const u32x4* o4 = reinterpret_cast<const u32x4*>(out + hr * kDv);
  const u32x4* d4 = reinterpret_cast<const u32x4*>(dout + hr * kDv);
  u32x4 ov[4], dv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    ov[c] = o4[l + 16 * c];
    dv[c] = d4[l + 16 * c];
  }
  float part = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      part += bf16_lo(dv[c][r]) * bf16_lo(ov[c][r]) + bf16_hi(dv[c][r]) * bf16_hi(ov[c][r]);
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
  if (l == 0 && grp < n) {
    delta[g] = part;
    if (sinks) {
      const float ps = expf(sinks[rem % H] - smax[hr]) / ssum[hr];
      pd[g] = -ps * part;
    }
  }
}

// dsink[h] += sum over the chunk's rows of pd[row][h]: one workgroup per head
__global__ void __launch_bounds__(256)
sink_colsum_kernel(const float* __restrict__ pd, int64_t nrows, int H, float* __restrict__ dsink) {
  __shared__ float red[256];
  const int h = blockIdx.x, t = threadIdx.x;
  float acc = 0.f;
  for (int64_t r = t; r < nrows; r += 256) acc += pd[r * H + h];
  red[t] = acc;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (t < st) red[t] += red[t + st];
    __syncthreads();
  }
  if (t == 0) dsink[h] += red[0];
}

struct BwdPlan {
  int64_t rows;  // query rows per chunk
  int64_t g_bytes, c_bytes, pairs_bytes, csr_bytes, delta_bytes, total;  // (delta twice: delta and the sink part)
};

// Scratch per chunk: G and C (bf16, C rows `width` columns), the CSR pair list and
// offsets, and delta (fp32 per row and head).
BwdPlan plan_bwd(int64_t batch, int64_t s_q, int64_t s_kv, int64_t topk, int64_t budget, int64_t width) {
  BwdPlan p{};
  const int64_t per_row = batch * g_slots(topk) * kGW * 2 + batch * topk * (int64_t)(width * 2 + 4) +
                          2 * batch * kHeadsMax * 4 + topk * width / 32;  // (last: CSR segment partials)
  int64_t rows = s_q;
  if (budget > 0) rows = std::max<int64_t>(1, std::min<int64_t>(s_q, budget / per_row));
  p.rows = rows;
  p.g_bytes = batch * rows * g_slots(topk) * kGW * 2;
  p.c_bytes = batch * rows * topk * width * 2;
  p.pairs_bytes = rows * topk * 4;
  p.csr_bytes = csr_ws_bytes(s_kv, rows, topk, width);
  p.delta_bytes = batch * rows * kHeadsMax * 4;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  p.total = al(p.g_bytes) + al(p.c_bytes) + al(p.pairs_bytes) + al(p.csr_bytes) + 2 * al(p.delta_bytes);
  return p;
}

constexpr int64_t kDefaultBudget = 32LL << 30;  // scratch for the G / C chunks (C3 in one chunk)

}  // namespace
}  // namespace dsa

extern "C" int64_t dsa_sparse_mla_bwd_workspace_size(int64_t batch, int64_t s_q, int64_t s_kv, int64_t n_heads,
                                                     int64_t d_qk, int64_t topk) {
  (void)n_heads;
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || topk <= 0) return 0;
  const int64_t width = d_qk == dsa::kDv ? dsa::kDv : dsa::kDqk;  // C row width of the bf16 path
  return dsa::plan_bwd(batch, s_q, s_kv, topk, dsa::kDefaultBudget, width).total;
}

namespace dsa {
static int sparse_mla_bwd_impl(const void* q, const void* kv, const int32_t* indices, const void* out,
                               const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                               float* dkv_accum, float* mass, void* workspace, int64_t workspace_bytes, int dtype,
                               int64_t batch, int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v,
                               int64_t topk, float scale, int64_t q_offset, const float* sinks, float* dsink,
                               const void* csr, void* stream) {
  if (!q || !kv || !indices || !out || !dout || !softmax_max || !softmax_sum || !dq || !dkv_accum)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: null pointer");
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || n_heads <= 0 || topk <= 0 || d_v <= 0 || d_qk < d_v)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: bad sizes");
  if (s_q > 2147483647LL || s_kv > 2147483647LL || batch > 65535 || topk > (1 << 20))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DSA_F32) {
    if (mass) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: the fp32 path has no mass output "
                               "(use dsa_attn_mass)");
    if (topk * 4 > 64 * 1024) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: fp32 topk <= 16384");
    if (s_q > 2147483647LL || n_heads > 65535)
      return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: sizes out of range");
    dim3 grid((unsigned)s_q, (unsigned)n_heads, (unsigned)batch);
    {
      const TimedLaunch tl("bwd_exact_f32_kernel", st);
      bwd_exact_f32_kernel<<<grid, 256, topk * 4, st>>>(
          (const float*)q, (const float*)kv, indices, (const float*)out, (const float*)dout, softmax_max, softmax_sum,
          (float*)dq, dkv_accum, (int)s_q, (int)s_kv, (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset,
          sinks, dsink);
    }
    return check_launch("dsa_sparse_mla_bwd(f32)");
  }
  if (dtype != DSA_BF16) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: dtype %d", dtype);
  if ((d_qk != kDqk && d_qk != kDv) || d_v != kDv)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: bf16 path needs d_qk = 576 or 512, d_v = 512");
  if (n_heads > kHeadsMax) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: bf16 path needs H <= 128");
  const bool rope = d_qk == kDqk;
  const int64_t max_rows = rope ? GatherGeom::kMaxRows : GatherGeomT<kDv>::kMaxRows;
  if (s_kv > max_rows) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: S_kv > %lld", (long long)max_rows);
  if (!workspace) return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: workspace required");
  // choose the largest chunk whose scratch fits the given workspace
  BwdPlan plan = plan_bwd(batch, s_q, s_kv, topk, workspace_bytes, d_qk);
  while (plan.total > workspace_bytes && plan.rows > 1) plan = plan_bwd(batch, plan.rows - 1, s_kv, topk, 0, d_qk);
  if (plan.total > workspace_bytes)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: workspace of %lld bytes is too small",
                     (long long)workspace_bytes);
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  char* ws = (char*)workspace;
  uint16_t* gbuf = (uint16_t*)ws;
  uint16_t* cbuf = (uint16_t*)(ws + al(plan.g_bytes));
  int* pairs = (int*)(ws + al(plan.g_bytes) + al(plan.c_bytes));
  int* counts = (int*)(ws + al(plan.g_bytes) + al(plan.c_bytes) + al(plan.pairs_bytes));
  float* dbuf = (float*)(ws + al(plan.g_bytes) + al(plan.c_bytes) + al(plan.pairs_bytes) + al(plan.csr_bytes));
  float* pdbuf = (float*)((char*)dbuf + al(plan.delta_bytes));  // the sink's per-(row, head) gradient parts
  const unsigned hgroups = ceil_div(n_heads, kHG);

  for (int64_t r0 = 0; r0 < s_q; r0 += plan.rows) {
    const int rows = (int)std::min<int64_t>(plan.rows, s_q - r0);
    if (sinks) {
      const int64_t groups = batch * rows * n_heads;
      const TimedLaunch tl("bwd_delta_kernel", st);
      bwd_delta_kernel<<<(unsigned)((groups * 16 + 255) / 256), 256, 0, st>>>(
          (const uint16_t*)out, (const uint16_t*)dout, dbuf, groups, (int)s_q, (int)n_heads, (int)r0, rows, sinks,
          softmax_max, softmax_sum, pdbuf);
      if (int rc = check_launch("dsa_sparse_mla_bwd(delta)")) return rc;
    }
    if (sinks) {
      const TimedLaunch tl("sink_colsum_kernel", st);
      sink_colsum_kernel<<<(unsigned)n_heads, 256, 0, st>>>(pdbuf, batch * rows, (int)n_heads, dsink);
      if (int rc = check_launch("dsa_sparse_mla_bwd(sink)")) return rc;
    }
    dim3 ga((unsigned)rows, 1, (unsigned)batch);
    {
      const TimedLaunch tl(rope ? "bwd_sdp_kernel" : "bwd_sdp_kernel<512>", st);
      // with no sink, delta is formed inside (the sink's gradient needs the delta pass)
      auto* kern = sinks ? (rope ? bwd_sdp_kernel<kDqk, false> : bwd_sdp_kernel<kDv, false>)
                         : (rope ? bwd_sdp_kernel<kDqk, true> : bwd_sdp_kernel<kDv, true>);
      kern<<<ga, 64 * kSdpWaves, 0, st>>>((const uint16_t*)q, (const uint16_t*)kv, indices, (const uint16_t*)dout,
                                          (const uint16_t*)out, softmax_max, softmax_sum, dbuf, gbuf, mass, (int)s_q,
                                          (int)s_kv, (int)n_heads, (int)topk, scale, q_offset, (int)r0);
    }
    if (int rc = check_launch("dsa_sparse_mla_bwd(sdp)")) return rc;
    {
      const TimedLaunch tl(rope ? "bwd_dqk_kernel" : "bwd_dqk_kernel<512>", st);
      auto* kern = rope ? bwd_dqk_kernel<kDqk> : bwd_dqk_kernel<kDv>;
      const int threads = 64 * (rope ? DqkShape<kDqk>::kWaves : DqkShape<kDv>::kWaves);
      kern<<<ga, threads, 0, st>>>((const uint16_t*)kv, indices, gbuf, (uint16_t*)dq, (int)s_q, (int)s_kv,
                                   (int)n_heads, (int)topk, q_offset, (int)r0);
    }
    if (int rc = check_launch("dsa_sparse_mla_bwd(dq)")) return rc;
    dim3 gb((unsigned)rows, (unsigned)batch);
    {
      static const char* const names[2][2] = {{"bwd_contrib_kernel<1,512>", "bwd_contrib_kernel<2,512>"},
                                              {"bwd_contrib_kernel<1>", "bwd_contrib_kernel<2>"}};
      const TimedLaunch tl(names[rope][hgroups == 1 ? 0 : 1], st);
      auto* kern = rope ? (hgroups == 1 ? bwd_contrib_kernel<1, kDqk> : bwd_contrib_kernel<2, kDqk>)
                        : (hgroups == 1 ? bwd_contrib_kernel<1, kDv> : bwd_contrib_kernel<2, kDv>);
      kern<<<gb, kCThreads, 0, st>>>((const uint16_t*)q, (const uint16_t*)dout, indices, gbuf, cbuf, (int)s_q,
                                     (int)s_kv, (int)n_heads, (int)topk, q_offset, (int)r0, rows);
    }
    if (int rc = check_launch("dsa_sparse_mla_bwd(contrib)")) return rc;
    // a prebuilt CSR of every row serves a one-chunk plan; otherwise each chunk builds its own
    const bool prebuilt = csr && rows == s_q;
    for (int b = 0; b < (int)batch; ++b) {
      if (prebuilt) {
        float* part = reinterpret_cast<float*>(counts + csr_ws_ints(s_kv, rows, topk));
        if (int rc = csr_reduce_built(pair_csr_view(csr, s_kv, rows, topk, b), cbuf, dkv_accum, part, (int)s_kv, rows,
                                      (int)topk, b, (int)(d_qk / 8), st))
          return rc;
      } else if (int rc = csr_reduce(indices, cbuf, dkv_accum, pairs, counts, (int)s_q, (int)s_kv, (int)topk, q_offset,
                                     (int)r0, rows, b, (int)(d_qk / 8), st)) {
        return rc;
      }
    }
  }
  return DSA_OK;
}

// a prebuilt CSR's size against the call that wants to use it
static int check_pair_csr(const void* csr, int64_t csr_bytes, int64_t batch, int64_t s_q, int64_t s_kv, int64_t topk,
                          const char* what) {
  if (!csr) return DSA_OK;
  if (csr_bytes < pair_csr_bytes_of(batch, s_q, s_kv, topk))
    return set_error(DSA_ERR_INVALID_ARG, "%s: pair CSR of %lld bytes is too small", what, (long long)csr_bytes);
  return DSA_OK;
}
}  // namespace dsa

extern "C" int64_t dsa_sparse_mla_bwd_chunk_rows(int64_t batch, int64_t s_q, int64_t s_kv, int64_t d_qk,
                                                 int64_t topk, int64_t workspace_bytes) {
  using namespace dsa;
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || topk <= 0 || workspace_bytes <= 0) return 0;
  BwdPlan plan = plan_bwd(batch, s_q, s_kv, topk, workspace_bytes, d_qk);
  while (plan.total > workspace_bytes && plan.rows > 1) plan = plan_bwd(batch, plan.rows - 1, s_kv, topk, 0, d_qk);
  return plan.total > workspace_bytes ? 0 : plan.rows;
}

extern "C" int64_t dsa_pair_csr_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t topk) {
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || topk <= 0) return 0;
  return dsa::pair_csr_bytes_of(batch, s_q, s_k, topk);
}

extern "C" int dsa_pair_csr_build(const int32_t* indices, int64_t batch, int64_t s_q, int64_t s_k, int64_t topk,
                                  int64_t q_offset, void* csr, int64_t csr_bytes, void* stream) {
  using namespace dsa;
  if (!indices || !csr) return set_error(DSA_ERR_INVALID_ARG, "dsa_pair_csr_build: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || topk <= 0 || s_q > 2147483647LL || s_k > 2147483647LL || batch > 65535 ||
      topk > (1 << 20))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_pair_csr_build: bad sizes");
  if ((uintptr_t)csr % 256) return set_error(DSA_ERR_INVALID_ARG, "dsa_pair_csr_build: buffer must be 256-byte aligned");
  if (csr_bytes < pair_csr_bytes_of(batch, s_q, s_k, topk))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_pair_csr_build: buffer of %lld bytes, %lld needed", (long long)csr_bytes,
                     (long long)pair_csr_bytes_of(batch, s_q, s_k, topk));
  hipStream_t st = (hipStream_t)stream;
  for (int b = 0; b < (int)batch; ++b) {
    int* base = reinterpret_cast<int*>(csr) + (int64_t)b * pair_csr_batch_ints(s_k, s_q, topk);
    int* ws = base + (s_q * topk + 3) / 4 * 4;
    CsrView v;
    if (int rc = csr_build(indices, base, ws, (int)s_q, (int)s_k, (int)topk, q_offset, 0, (int)s_q, b, st, &v))
      return rc;
  }
  return DSA_OK;
}

namespace dsa {
}  // namespace dsa

extern "C" int dsa_sparse_mla_bwd(const void* q, const void* kv, const int32_t* indices, const void* out,
                                  const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                                  float* dkv_accum, float* mass, void* workspace, int64_t workspace_bytes, int dtype,
                                  int64_t batch,
                                  int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v,
                                  int64_t topk, float scale, int64_t q_offset, void* stream) {
  return dsa::sparse_mla_bwd_impl(q, kv, indices, out, dout, softmax_max, softmax_sum, dq, dkv_accum, mass, workspace,
                                  workspace_bytes, dtype, batch, s_q, s_kv, n_heads, d_qk, d_v, topk, scale, q_offset,
                                  nullptr, nullptr, nullptr, stream);
}

extern "C" int dsa_sparse_mla_bwd_sink(const void* q, const void* kv, const int32_t* indices, const void* out,
                                       const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                                       float* dkv_accum, float* mass, const float* sinks, float* dsink_accum,
                                       void* workspace, int64_t workspace_bytes, int dtype, int64_t batch,
                                       int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v,
                                       int64_t topk, float scale, int64_t q_offset, void* stream) {
  if (!sinks || !dsink_accum) return dsa::set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd_sink: null sinks / dsink");
  return dsa::sparse_mla_bwd_impl(q, kv, indices, out, dout, softmax_max, softmax_sum, dq, dkv_accum, mass, workspace,
                                  workspace_bytes, dtype, batch, s_q, s_kv, n_heads, d_qk, d_v, topk, scale, q_offset,
                                  sinks, dsink_accum, nullptr, stream);
}

extern "C" int dsa_sparse_mla_bwd_ex(const void* q, const void* kv, const int32_t* indices, const void* out,
                                     const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                                     float* dkv_accum, float* mass, const float* sinks, float* dsink_accum,
                                     const void* pair_csr, int64_t pair_csr_bytes, void* workspace,
                                     int64_t workspace_bytes, int dtype, int64_t batch, int64_t s_q, int64_t s_kv,
                                     int64_t n_heads, int64_t d_qk, int64_t d_v, int64_t topk, float scale,
                                     int64_t q_offset, void* stream) {
  if (sinks && !dsink_accum) return dsa::set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd_ex: sinks without dsink");
  if (int rc = dsa::check_pair_csr(pair_csr, pair_csr_bytes, batch, s_q, s_kv, topk, "dsa_sparse_mla_bwd_ex"))
    return rc;
  return dsa::sparse_mla_bwd_impl(q, kv, indices, out, dout, softmax_max, softmax_sum, dq, dkv_accum, mass, workspace,
                                  workspace_bytes, dtype, batch, s_q, s_kv, n_heads, d_qk, d_v, topk, scale, q_offset,
                                  sinks, sinks ? dsink_accum : nullptr, pair_csr, stream);
}

