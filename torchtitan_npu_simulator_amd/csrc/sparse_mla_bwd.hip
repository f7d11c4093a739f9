// Gathered sparse MLA attention backward for gfx950, without float atomics.
//
// fp32 atomics on this part top out near 1.3 TB/s of payload (one dword per L2 channel
// per clock), far too slow for the dKV scatter-add (576 fp32 per (token, key) pair), so
// the backward reduces dKV through a key-major pass instead:
//
//   (alpha) bwd_dq_kernel, workgroup = (token, 64-head group), 4 waves x 16 heads:
//           recompute [S ; dP] = [Q ; dO] K^T for the wave's 16 heads as ONE 32-row
//           v_mfma_f32_32x32x16_bf16 chain over the gathered KV tile (rows 0..15 the
//           heads' Q, rows 16..31 their dO; v = k_nope, so the first 512 columns serve both),
//           P = exp2(S*scale*log2e - lse2), dS = P (dP - delta); G[token][slot][128 hg +
//           (0..63 | 64..127)] = (dS * scale | P) in bf16 staged in LDS; dQ^T += K^T dS^T
//           (K read transposed with ds_read_tr16_b64, dS^T from the G stage) in AGPRs.
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
constexpr int kRowChunks = kDqk / 8;
constexpr int kRowBytes = kRowChunks * 16;
constexpr int kBN = 32;
constexpr int kTileChunks = kBN * kRowChunks;
constexpr int kTileBytes = kTileChunks * 16;
constexpr int kTileInstr = kTileChunks / 64;  // 36
constexpr int kHG = 64;                       // heads per alpha workgroup
constexpr int kGW = 256;                      // G row width: (dS | P) x 128 heads
constexpr int kHeadsMax = 128;

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ u32x4 tr_pair(uint32_t a1, uint32_t a2) {
  const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a1));
  const i16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a2));
  u32x4 av;
  av[0] = (uint32_t)(uint16_t)v1[0] | ((uint32_t)(uint16_t)v1[1] << 16);
  av[1] = (uint32_t)(uint16_t)v1[2] | ((uint32_t)(uint16_t)v1[3] << 16);
  av[2] = (uint32_t)(uint16_t)v2[0] | ((uint32_t)(uint16_t)v2[1] << 16);
  av[3] = (uint32_t)(uint16_t)v2[2] | ((uint32_t)(uint16_t)v2[3] << 16);
  return av;
}

// 8-byte piece swizzle of the slot-major G stage (256-byte rows, piece p of slot r at
// p ^ gs_swz(r)): injective over the 32 slots, so the 32 lanes writing one piece column
// hit 32 distinct bank pairs; bits 2..3 follow r & 3, so a transposed read of 4 slots x
// 4 pieces (4-aligned) covers 16 distinct pieces; a 16-lane read of a whole row is a
// permutation of the row.
__device__ __forceinline__ int gs_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3) | (((r >> 4) & 1) << 4); }

// --------------------------------------------------------------------------------------
// (alpha) dQ and G
// --------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 1)
bwd_dq_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kv, const int32_t* __restrict__ idx,
              const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, const float* __restrict__ smax,
              const float* __restrict__ ssum, const float* __restrict__ dbuf, uint16_t* __restrict__ dq,
              uint16_t* __restrict__ gbuf, float* __restrict__ mbase, int64_t m_hg_stride, int64_t m_b_stride,
              int m_row_base, int S, int s_kv, int H, int K, float scale, int64_t q_offset, int row0) {
  using Gather = RowGather<4>;
  __shared__ u32x4 tile[3][kTileChunks];
  // staged G of this head group, slot-major: [block parity][slot][8-byte piece of 4 entries
  // (dS heads 0..63 | P heads 0..63), at piece ^ gs_swz(slot)]
  __shared__ __attribute__((aligned(16))) uint2 gst[2][kBN][2 * kHG / 4];
  __shared__ float pst[2][4][kBN];          // per-wave head sums of P (attention mass)
  __shared__ float2 hstat[4][16];           // per wave and head: (delta, lse2)
  __shared__ int sidx[GatherGeom::kRing][Gather::kRingInts];
  __shared__ int sh_last;

  const int tok = row0 + blockIdx.x;  // row within the batch element
  const int hg = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int head = hg * kHG + wave * 16 + col;
  const bool head_ok = head < H;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kvb = kv + (int64_t)b * s_kv * kDqk;
  const int64_t hrow = row_id * H + (head_ok ? head : 0);
  // G rows of this chunk: [local row][slot][kGW]
  uint16_t* grow = gbuf + ((int64_t)b * gridDim.x + blockIdx.x) * (int64_t)K * kGW;

  // head-summed P of this head group for the row (mass; the host adds the head groups)
  float* mrow = mbase ? mbase + hg * m_hg_stride + b * m_b_stride + (int64_t)(m_row_base + blockIdx.x) * K : nullptr;

  // ---- prologue: the row's slot indices (block count), the index ring entries of blocks
  // 0..2 (wave 0, DMA), the per-head operands Q (B layout of S^T = K Q^T), dO (B layout
  // of dP^T = V dO^T), O and the row statistics are all requested before any is waited
  // for: the block count needs only the first loads, the operands land meanwhile ----
  int vidx[kIdxU];
  load_row_indices(ridx, K, vidx);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) Gather::issue_idx(ridx, K, i, sidx[i], lane);  // clamped to slot K-1
  }
  // A operand of [S ; dP] = [Q ; dO] K^T (32x32x16, k-step s = columns 16s .. 16s+15):
  // lane (row an, k half ah) holds columns 16s + 8ah .. +8 of row an: Q of head
  // 16 wave + an for an < 16, dO of head 16 wave + an - 16 otherwise (dO has no rope
  // columns: zero for s >= 32).  delta = rowsum(dO o O) comes from the pre-pass.
  // (unconditional loads, arow points at head 0 for absent heads: a load under a branch
  // would make the compiler wait for every load before the block count; absent heads are
  // zeroed after it)
  const int an = lane & 31, ah = lane >> 5;
  const bool a_is_q = an < 16;
  const int a_head = hg * kHG + wave * 16 + (an & 15);
  const bool a_ok = a_head < H;
  const int64_t arow = row_id * H + (a_ok ? a_head : 0);
  constexpr int kAS = kDqk / 16;  // 36 k-steps
  constexpr int kAL = kDv / 16;   // 32 of them cover the latent columns
  u32x4 aq[kAS];
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(q + arow * kDqk);
    const u32x4* dh = reinterpret_cast<const u32x4*>(dout + arow * kDv);
    const u32x4* src = a_is_q ? qh : dh;
#pragma unroll
    for (int st = 0; st < kAL; ++st) aq[st] = src[2 * st + ah];
#pragma unroll
    for (int st = kAL; st < kAS; ++st) aq[st] = qh[2 * st + ah];
  }
  const float mx = smax[arow], sm = ssum[arow];
  const float dlt = dbuf[((int64_t)b * gridDim.x + blockIdx.x) * H + (a_ok ? a_head : 0)];

  const int nblk = count_row_blocks(ridx, K, s_kv, limit, vidx, &sh_last);
  if (mrow)  // slots past the last usable block carry no mass
    for (int j = nblk * kBN + tid; j < K; j += 256) mrow[j] = 0.f;
  if (nblk == 0) {  // no usable key: dQ = 0 (G rows are never read)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring DMA has landed before the LDS is released
    if (head_ok) {
      uint32_t* d32 = reinterpret_cast<uint32_t*>(dq + hrow * kDqk);
      for (int i = g; i < kDqk / 2; i += 4) d32[i] = 0u;
    }
    return;
  }
  const uint32_t lim = gather_limit(limit, s_kv);

  if (!a_ok) {
#pragma unroll
    for (int st = 0; st < kAS; ++st) aq[st] = (u32x4){0u, 0u, 0u, 0u};
  }
  if (!a_is_q) {
#pragma unroll
    for (int st = kAL; st < kAS; ++st) aq[st] = (u32x4){0u, 0u, 0u, 0u};
  }
  // delta and lse2 of head 16 wave + an (rows an < 16) go through LDS to the lanes that
  // hold the head's S / dP values: lane (key an, ah) holds rows 8j + 4ah + i (j < 2: S,
  // j >= 2: dP of the same head), i.e. heads hw(v) = 8 (v >> 2) + 4 ah + (v & 3), v < 8
  float dl[8], l2[8];
  {
    const float lse2 = (a_ok && sm > 0.f) ? (mx + logf(sm)) * kLog2e : INFINITY;  // +inf -> P = 0
    if (a_is_q && ah == 0) hstat[wave][an] = make_float2(a_ok ? dlt : 0.f, lse2);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float2 st2 = hstat[wave][8 * (v >> 2) + 4 * ah + (v & 3)];  // written by this wave
      dl[v] = st2.x;
      l2[v] = st2.y;
    }
  }
  const float scale_log2 = scale * kLog2e;

  // LDS offsets.  B operand of [S ; dP] (key an, k half ah), k-step s: chunk (2s + ah) ^
  // swz_kv(an); with s = 4u + s0 the XOR touches only bits 0..2 -> kb_off[s0] + 128 u.
  uint32_t kb_off[4];
#pragma unroll
  for (int s0 = 0; s0 < 4; ++s0) kb_off[s0] = an * kRowBytes + 16 * ((2 * s0 + ah) ^ swz_kv(an));
  // Transposed K reads for dQ^T += K^T dS^T: group g, source lane col supplies key row
  // 4g + col/4 (+16 for the second read), d columns 16dt + 4(col%4) -> chunk 2dt + (col%4)/2.
  const int tr_row = 4 * g + (col >> 2);
  const int tr_x = swz_kv(tr_row);
  const int tr_c0 = (col & 3) >> 1;
  uint32_t tr_off[4];  // dt = 4u + d0 -> chunk (8u + 2 d0 + tr_c0) ^ tr_x = 8u + ((2 d0 + tr_c0) ^ tr_x)
#pragma unroll
  for (int d0 = 0; d0 < 4; ++d0) tr_off[d0] = tr_row * kRowBytes + 16 * ((2 * d0 + tr_c0) ^ tr_x) + 8 * (col & 1);

  f32x4 dqa[kDqk / 16];
#pragma unroll
  for (int t = 0; t < kDqk / 16; ++t) dqa[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // G and mass of block `fb` staged in gst/pst[fb & 1] -> global, in three parts so they
  // can be spread over the next block's dQ MFMAs (fb < 0: nothing is stored).  G part u:
  // slots 16u .. 16u+15, 16 lanes per slot row (16 bytes each, whole 256-byte rows).
  // Part 2: the head group's attention mass of the block's 32 slots.
  auto flush_part = [&](int fb, int part) {
    const int sb = fb & 1;
    if (part == 2) {
      if (mrow && fb >= 0 && tid < kBN && fb * kBN + tid < K)
        mrow[fb * kBN + tid] = (pst[sb][0][tid] + pst[sb][1][tid]) + (pst[sb][2][tid] + pst[sb][3][tid]);
      return;
    }
    const int i = tid + 256 * part, row = i >> 4, k = i & 15;
    const int p0 = (2 * k) ^ gs_swz(row);  // the pair (2k, 2k+1) stays one aligned 16-byte pair
    u32x4 v = *reinterpret_cast<const u32x4*>(&gst[sb][row][p0 & ~1]);
    if (p0 & 1) v = (u32x4){v[2], v[3], v[0], v[1]};
    const int slot = fb * kBN + row;
    if (fb >= 0 && slot < K)  // the row holds K slots only
      *reinterpret_cast<u32x4*>(grow + (int64_t)slot * kGW + 2 * kHG * hg + 8 * k) = v;
  };

  // the per-head operands must have arrived before the first DMA: a later wait for them
  // would also wait for every row DMA in flight
#pragma unroll
  for (int st = 0; st < kAS; ++st) asm volatile("" : "+v"(aq[st]));
#pragma unroll
  for (int v = 0; v < 8; ++v) asm volatile("" : "+v"(dl[v]), "+v"(l2[v]));

  // ---- pipeline (as in the forward) ----
  // iteration blk: [S ; dP] of block blk on tile blk % 3 while block blk+1's rows are
  // DMA'd into tile (blk+1) % 3 (one instruction per S/dP batch), then P / dS of blk
  // interleaved batch by batch with dQ of blk-1 on tile (blk-1) % 3 (its dS^T operand read
  // back from blk-1's G stage, which this wave wrote), G / mass staging of blk and the
  // stores of blk-1's.  The iteration ends with its DMAs landed (vmcnt 0) and one barrier.
  // Tile (blk-1) % 3 for blk = 0 is zeroed (dS^T = 0 there, and 0 * garbage could be NaN).
  constexpr int kPer = Gather::kMaxPerWave;
  const typename Gather::PackedLanes gl = Gather::packed_lanes(wave, lane);
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // ring entries 0..2 landed
  __syncthreads();
  for (int i = tid; i < kTileChunks; i += 256) tile[2][i] = (u32x4){0u, 0u, 0u, 0u};  // dQ of "block -1"
  uint32_t vm_cur = Gather::ring_valid(sidx[0], lane, lim, K);
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    Gather::issue_slot(kvb, &tile[0][0], i, wave, Gather::ring_slot(sidx[0], i, gl), gl, lim, K);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  constexpr int kSB = 4;                   // k-steps per S/dP batch
  constexpr int kSN = kAS / kSB;           // 9 batches
  static_assert(kSN >= kPer, "one row DMA per S/dP batch");
  constexpr int kDB = 4;                   // dQ tiles per batch
  constexpr int kDN = (kDqk / 16) / kDB;   // 9 batches

  // [S ; dP] of one block (one 32x32x16 accumulation chain, full rate); block blk+1's DMA
  // meanwhile (ring entry `ring`, slot value read a batch ahead); returns blk+1's validity
  // bits.  Past the last block the ring entry is stale and the rows land in a buffer nobody
  // reads: every offset stays inside the KV tensor.
  auto sdp = [&](const lds_char* tb, u32x4* dst_tile, const int* ring, int rows_left, f32x16& acc) -> uint32_t {
    const uint32_t vm_n = Gather::ring_valid(ring, lane, lim, rows_left);
    uint32_t raw_next = Gather::ring_slot(ring, 0, gl);
    acc = (f32x16){0.f};
    u32x4 kb[2][kSB];
    auto read_b = [&](u32x4 (&dst)[kSB], int sb) {
#pragma unroll
      for (int u = 0; u < kSB; ++u) dst[u] = lds_read16(tb + kb_off[u] + 128 * (sb / kSB));
    };
    read_b(kb[0], 0);
    static_for<kSN>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kSN) read_b(kb[(nb + 1) & 1], (nb + 1) * kSB);
      if constexpr (nb < kPer) {
        const uint32_t raw = raw_next;
        if constexpr (nb + 1 < kPer) raw_next = Gather::ring_slot(ring, nb + 1, gl);
        Gather::issue_slot(kvb, dst_tile, nb, wave, raw, gl, lim, rows_left);
      }
#pragma unroll
      for (int u = 0; u < kSB; ++u) acc = mfma32x32x16(as_bf16x8(aq[nb * kSB + u]), as_bf16x8(kb[nb & 1][u]), acc);
      // one accumulation chain issues in order: spread the batch's LDS reads, address
      // arithmetic and DMA between its MFMAs
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);  // VALU / SALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // the row DMA
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    return vm_n;
  };

  // Transposed K reads for dQ^T += K^T dS^T (tile vb)
  auto read_kt = [&](const lds_char* vb, u32x4 (&dst)[kDB], int db4) {
#pragma unroll
    for (int u = 0; u < kDB; ++u) {
      const int dt = db4 + u;
      const lds_char* a1 = vb + tr_off[dt & 3] + 128 * (dt >> 2);
      dst[u] = lds_read_tr_pair(a1, a1 + 16 * kRowBytes);
    }
  };

  // dQ^T operand B = dS^T * scale of block fb from its G stage (the wave's own entries):
  // lane (head col, g) takes slots 4g .. 4g+3 and 16 + 4g .. +3 (the k-slot order of the
  // transposed K reads) by two transposed reads; source lane c supplies slot row
  // 4g + c/4 (+16) and entries 16 wave + 4 (c % 4) .. +3
  auto read_bds = [&](int fb) -> u32x4 {
    const lds_char* gb = lds_bytes(&gst[fb & 1][0][0]);
    const int q = 4 * wave + (col & 3);
    const int r0 = 4 * g + (col >> 2), r1 = r0 + 16;
    return lds_read_tr_pair(gb + r0 * (2 * kHG * 2) + 8 * (q ^ gs_swz(r0)),
                            gb + r1 * (2 * kHG * 2) + 8 * (q ^ gs_swz(r1)));
  };

  // P / dS of block blk (acc, validity vm): G and mass staged for blk; interleaved with
  // dQ of block blk-1 (tile vb, dS^T from blk-1's G stage; nothing for blk = 0) and the
  // stores of blk-1
  auto pds_dq = [&](const lds_char* vb, const f32x16& acc, uint32_t vm, int blk, const u32x4& bds,
                    u32x4& bds_next) {
    u32x4 at[2][kDB];
    read_kt(vb, at[0], 0);
    const bool ok = (vm >> an) & 1u;
    const int sb = blk & 1;
    float pv[8], dsv[8];
    // G stage: lane (slot an, ah) writes its 8 heads' values as two 8-byte pieces: heads
    // 16 wave + 4 ah + (0..3) and 16 wave + 8 + 4 ah + (0..3); P entries follow the 64 dS
    auto stage = [&](const float (&val)[8], int piece0, float mul) {
      const int pa = piece0 + 4 * wave + ah, pb = pa + 2;
      gst[sb][an][pa ^ gs_swz(an)] = make_uint2(pack_bf16x2(val[0] * mul, val[1] * mul),
                                                pack_bf16x2(val[2] * mul, val[3] * mul));
      gst[sb][an][pb ^ gs_swz(an)] = make_uint2(pack_bf16x2(val[4] * mul, val[5] * mul),
                                                pack_bf16x2(val[6] * mul, val[7] * mul));
    };
    static_for<kDN>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kDN) read_kt(vb, at[(nb + 1) & 1], (nb + 1) * kDB);
#pragma unroll
      for (int u = 0; u < kDB; ++u)
        dqa[nb * kDB + u] = mfma16x16x32(as_bf16x8(at[nb & 1][u]), as_bf16x8(bds), dqa[nb * kDB + u]);
      if constexpr (nb == 0) {  // P and dS: value v < 8 is S of head hw(v) at key an, v + 8 its dP
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float p = ok ? __builtin_amdgcn_exp2f(acc[v] * scale_log2 - l2[v]) : 0.f;
          pv[v] = p;
          dsv[v] = p * (acc[v + 8] - dl[v]);
        }
      } else if constexpr (nb == 1) {
        stage(dsv, 0, scale);
      } else if constexpr (nb == 2) {
        stage(pv, kHG / 4, 1.f);
      } else if constexpr (nb == 4) {
        bds_next = read_bds(blk);  // written above by this wave; used by the next block's dQ
      } else if constexpr (nb == 3) {
        // attention mass: the lane's 8 heads, then the 8 of the lane 32 apart
        const float part = ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
        const float tot = xor32_sum(part);
        if (mrow && ah == 0) pst[sb][wave][an] = tot;
      } else if constexpr (nb >= 6) {
        flush_part(blk - 1, nb - 6);  // G (two parts) and mass of the previous block
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // dQ of the last block
  auto dq_only = [&](const lds_char* vb, const u32x4& bds) {
    u32x4 at[2][kDB];
    read_kt(vb, at[0], 0);
    static_for<kDN>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      if constexpr (nb + 1 < kDN) read_kt(vb, at[(nb + 1) & 1], (nb + 1) * kDB);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kDB; ++u)
        dqa[nb * kDB + u] = mfma16x16x32(as_bf16x8(at[nb & 1][u]), as_bf16x8(bds), dqa[nb * kDB + u]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  u32x4 bds_cur = (u32x4){0u, 0u, 0u, 0u};  // dS^T of block -1
  for (int blk = 0; blk < nblk; ++blk) {
    if (wave == 0 && blk + 3 < nblk)
      Gather::issue_idx(ridx, K, blk + 3, sidx[(blk + 3) & (GatherGeom::kRing - 1)], lane);
    f32x16 acc;
    // ring entry blk+1 landed during iteration blk-2 (or before the loop)
    const uint32_t vm_next = sdp(lds_bytes(&tile[blk % 3][0]), &tile[(blk + 1) % 3][0],
                                 sidx[(blk + 1) & (GatherGeom::kRing - 1)], K - (blk + 1) * kBN, acc);
    u32x4 bds_next;
    pds_dq(lds_bytes(&tile[(blk + 2) % 3][0]), acc, vm_cur, blk, bds_cur, bds_next);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // block blk+1 and ring entry blk+3 landed
    __syncthreads();
    vm_cur = vm_next;
    bds_cur = bds_next;
  }
  dq_only(lds_bytes(&tile[(nblk - 1) % 3][0]), bds_cur);
  // the last block's G and mass were staged before the loop's final barrier
  flush_part(nblk - 1, 0);
  flush_part(nblk - 1, 1);
  flush_part(nblk - 1, 2);

  // ---- dQ epilogue: lane (head col, g) holds d = 16 dt + 4 g + r (dS^T was pre-scaled) ----
  if (!head_ok) return;
  uint2* drow = reinterpret_cast<uint2*>(dq + hrow * kDqk);
#pragma unroll
  for (int dt = 0; dt < kDqk / 16; ++dt) {
    uint2 w;
    w.x = pack_bf16x2(dqa[dt][0], dqa[dt][1]);
    w.y = pack_bf16x2(dqa[dt][2], dqa[dt][3]);
    drow[(16 * dt + 4 * g) / 4] = w;
  }
}

// --------------------------------------------------------------------------------------
// (beta) C[token][slot] = G[token][slot] . X_token,  X = [(Q, dO) per head group]
// rows of X: k = 128 hg + 64 type + i  ->  type 0: q[64hg + i], type 1: dout[64hg + i]
//
// One workgroup per token, 12 waves; wave w owns the 48 output columns 48w .. 48w+47
// (three 16-column MFMA tiles) and keeps its slice of X transposed in VGPRs for the whole
// token (A operand of C^T = X^T G^T, 96 VGPRs).  G is streamed through a double-buffered
// LDS tile of 64 slots x 256 (DMA), so G, X and C each cross HBM exactly once.  The C rows
// of each 32-slot step are assembled in a double-buffered LDS stage (every wave adds its
// 48 columns) and leave as whole 1152-byte rows, 16 bytes per lane: the MFMA output layout
// alone would give 8-byte pieces scattered over 16 rows per store instruction.
// --------------------------------------------------------------------------------------
constexpr int kCW = 12;                     // waves
constexpr int kCThreads = kCW * 64;
constexpr int kCT = 64;                     // slots per G tile
constexpr int kGTChunks = kCT * (kGW / 8);  // 2048 16-byte chunks (32 KB)
constexpr int kCS = 32;                     // slots per step (C stage rows)
constexpr int kStChunks = kCS * kRowChunks; // 2304 chunks (36 KB)
constexpr int kXK = 64;                     // X rows staged per chunk while loading X
constexpr int kXChunks = kXK * kRowChunks;  // 4608 chunks (73.7 KB)
static_assert(2 * kGTChunks + 2 * kStChunks >= kXChunks, "X staging reuses the tile space");

// C stage layout: row r (slot), 16-byte chunk c stored at c ^ ((r >> 1) & 7)
__device__ __forceinline__ int stage_swz(int r) { return (r >> 1) & 7; }

template <int kHGroups>
__global__ void __launch_bounds__(kCThreads, 1)
bwd_contrib_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ dout,
                   const int32_t* __restrict__ idx, const uint16_t* __restrict__ gbuf, uint16_t* __restrict__ cbuf,
                   int S, int s_kv, int H, int K, int64_t q_offset, int row0, int rows) {
  constexpr int kKSteps = 4 * kHGroups;                // 32-row k steps of X (128 rows per head group)
  __shared__ u32x4 lds[2 * kGTChunks + 2 * kStChunks];  // X staging at start; then G tiles + C stages
  __shared__ int sh_last;

  const int lr = blockIdx.x;  // local row in chunk
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
  const uint16_t* grow = gbuf + ((int64_t)b * rows + lr) * (int64_t)K * kGW;
  uint16_t* crow = cbuf + ((int64_t)b * rows + lr) * (int64_t)K * kDqk;
  const lds_char* lb = lds_bytes(&lds[0]);

  // ---- X^T slice into VGPRs: xa[t][ks] = X[32 ks + 8g .. +8][48w + 16t + col] ----
  // (rows of dO at the rope columns are zero, so every MFMA below runs unconditionally)
  u32x4 xa[3][kKSteps];
  const int tr_row = 8 * g + (col >> 2);  // source row within a 32-row k step (+4 second read)
#pragma unroll
  for (int kc = 0; kc < 2 * kHGroups; ++kc) {
    __syncthreads();
    const int hgk = kc >> 1, type = kc & 1;
    for (int i = tid; i < kXChunks; i += kCThreads) {
      const int row = i / kRowChunks, c = i - row * kRowChunks;
      const int head = hgk * kHG + row;
      u32x4 v = (u32x4){0u, 0u, 0u, 0u};
      if (head < H) {
        if (type == 0) v = *reinterpret_cast<const u32x4*>(q + (row_id * H + head) * kDqk + c * 8);
        else if (c < kDv / 8) v = *reinterpret_cast<const u32x4*>(dout + (row_id * H + head) * kDv + c * 8);
      }
      lds[row * kRowChunks + (c ^ swz8(row))] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kl = 0; kl < 2; ++kl) {  // two 32-row k steps per staged chunk
      const int ks = 2 * kc + kl;
      const int r1 = 32 * kl + tr_row, r2 = r1 + 4;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const int c0 = (48 * wave + 16 * t) / 8 + ((col & 3) >> 1);
        const lds_char* a1 = lb + 16 * (r1 * kRowChunks + (c0 ^ swz8(r1))) + 8 * (col & 1);
        const lds_char* a2 = lb + 16 * (r2 * kRowChunks + (c0 ^ swz8(r2))) + 8 * (col & 1);
        xa[t][ks] = lds_read_tr_pair(a1, a2);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) asm volatile("" : "+v"(xa[t][ks]));  // landed before the DMAs
  __syncthreads();

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
  int step = 0;
  for (int tl = 0; tl < ntiles; ++tl) {
    const int buf = tl & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of tile tl (and its stores) done
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
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int t = 0; t < 3; ++t)
            acc[h2][t] = mfma16x16x32(as_bf16x8(xa[t][ks]), as_bf16x8(bg[ks & 1][h2]), acc[h2][t]);
      }
      // lane (slot 16 h2 + col, g) holds columns 48w + 16t + 4g + r: 8 bytes at chunk
      // 6w + 2t + g/2, half g & 1 of the stage row
      lds_char* stg = stage + (step & 1) * (kStChunks * 16);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int r = 16 * h2 + col;
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 w2 = {pack_bf16x2(acc[h2][t][0], acc[h2][t][1]), pack_bf16x2(acc[h2][t][2], acc[h2][t][3])};
          const int c = 6 * wave + 2 * t + (g >> 1);
          *(__attribute__((address_space(3))) u32x2*)(stg + r * (kRowChunks * 16) + 16 * (c ^ stage_swz(r)) + 8 * (g & 1)) = w2;
        }
      }
      __syncthreads();  // the step's C rows are complete in the stage
      // whole rows out: thread chunk i -> row i / 72, chunk i % 72
      int t_ = tid;
      asm volatile("" : "+v"(t_));
#pragma unroll
      for (int m = 0; m < kStChunks / kCThreads; ++m) {
        const int i = t_ + kCThreads * m;
        const int r = i / kRowChunks, c = i - r * kRowChunks;
        if (s0 + r < nslots) {
          const u32x4 v = lds_read16(stg + r * (kRowChunks * 16) + 16 * (c ^ stage_swz(r)));
          *reinterpret_cast<u32x4*>(crow + (int64_t)(s0 + r) * kDqk + 8 * c) = v;
        }
      }
    }
  }
}

// --------------------------------------------------------------------------------------
// exact fp32 path (any D): one workgroup per (token, head); dkv by fp32 atomics
// --------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
bwd_exact_f32_kernel(const float* __restrict__ q, const float* __restrict__ kv, const int32_t* __restrict__ idx,
                     const float* __restrict__ out, const float* __restrict__ dout, const float* __restrict__ smax,
                     const float* __restrict__ ssum, float* __restrict__ dq, float* __restrict__ dkv, int S,
                     int s_kv, int H, int K, int dqk, int dv, float scale, int64_t q_offset) {
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
// 16-lane group per (row, head), 32 columns per lane (four 16-byte loads of each tensor)
__global__ void __launch_bounds__(256)
bwd_delta_kernel(const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, float* __restrict__ delta,
                 int S, int H, int row0, int rows) {
  const int64_t grp = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (b, lr, h) flattened
  const int l = threadIdx.x & 15;
  const int64_t n = (int64_t)gridDim.y * rows * H;  // gridDim.y = batch
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
  if (l == 0 && grp < n) delta[g] = part;
}

struct BwdPlan {
  int64_t rows;  // query rows per chunk
  int64_t g_bytes, c_bytes, pairs_bytes, csr_bytes, mass_bytes, delta_bytes, total;
};

// Scratch per chunk: G and C (bf16), the CSR pair list and offsets, and the per-head-group
// mass partials (fp32, summed into the caller's mass after each chunk).
BwdPlan plan_bwd(int64_t batch, int64_t s_q, int64_t s_kv, int64_t topk, int64_t budget) {
  BwdPlan p{};
  const int64_t mass_groups = kHeadsMax / kHG;
  const int64_t per_row = batch * topk * (int64_t)(kGW * 2 + kDqk * 2 + 4 + 4 * mass_groups) + batch * kHeadsMax * 4;
  int64_t rows = s_q;
  if (budget > 0) rows = std::max<int64_t>(1, std::min<int64_t>(s_q, budget / per_row));
  p.rows = rows;
  p.g_bytes = batch * rows * topk * kGW * 2;
  p.c_bytes = batch * rows * topk * kDqk * 2;
  p.pairs_bytes = rows * topk * 4;
  p.csr_bytes = csr_ws_bytes(s_kv, rows, topk);
  p.mass_bytes = mass_groups * batch * rows * topk * 4;
  p.delta_bytes = batch * rows * kHeadsMax * 4;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  p.total = al(p.g_bytes) + al(p.c_bytes) + al(p.pairs_bytes) + al(p.csr_bytes) + al(p.mass_bytes) +
            al(p.delta_bytes);
  return p;
}

// mass[b, r0 + lr, :] = sum over head groups of the chunk's partials
__global__ void __launch_bounds__(256)
mass_combine_kernel(const float* __restrict__ part, float* __restrict__ mass, int groups, int64_t hg_stride,
                    int64_t row_elems, int S, int r0, int rows, int K) {
  const int64_t n = row_elems;  // batch * rows * K
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float acc = part[i];
    for (int hgi = 1; hgi < groups; ++hgi) acc += part[hgi * hg_stride + i];
    const int64_t b = i / ((int64_t)rows * K);
    const int64_t rem = i - b * (int64_t)rows * K;
    mass[(b * S + r0) * (int64_t)K + rem] = acc;
  }
}

constexpr int64_t kDefaultBudget = 32LL << 30;  // scratch for the G / C chunks (C3 in one chunk)

}  // namespace
}  // namespace dsa

extern "C" int64_t dsa_sparse_mla_bwd_workspace_size(int64_t batch, int64_t s_q, int64_t s_kv, int64_t n_heads,
                                                     int64_t d_qk, int64_t topk) {
  (void)n_heads;
  (void)d_qk;
  if (batch <= 0 || s_q <= 0 || s_kv <= 0 || topk <= 0) return 0;
  return dsa::plan_bwd(batch, s_q, s_kv, topk, dsa::kDefaultBudget).total;
}

extern "C" int dsa_sparse_mla_bwd(const void* q, const void* kv, const int32_t* indices, const void* out,
                                  const void* dout, const float* softmax_max, const float* softmax_sum, void* dq,
                                  float* dkv_accum, float* mass, void* workspace, int64_t workspace_bytes, int dtype,
                                  int64_t batch,
                                  int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t d_qk, int64_t d_v,
                                  int64_t topk, float scale, int64_t q_offset, void* stream) {
  using namespace dsa;
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
    bwd_exact_f32_kernel<<<grid, 256, topk * 4, st>>>(
        (const float*)q, (const float*)kv, indices, (const float*)out, (const float*)dout, softmax_max, softmax_sum,
        (float*)dq, dkv_accum, (int)s_q, (int)s_kv, (int)n_heads, (int)topk, (int)d_qk, (int)d_v, scale, q_offset);
    return check_launch("dsa_sparse_mla_bwd(f32)");
  }
  if (dtype != DSA_BF16) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: dtype %d", dtype);
  if (d_qk != kDqk || d_v != kDv)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: bf16 path needs d_qk=576, d_v=512");
  if (n_heads > kHeadsMax) return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: bf16 path needs H <= 128");
  if (s_kv > GatherGeom::kMaxRows)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: S_kv > %lld", (long long)GatherGeom::kMaxRows);
  if (!workspace) return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: workspace required");
  // choose the largest chunk whose scratch fits the given workspace
  BwdPlan plan = plan_bwd(batch, s_q, s_kv, topk, workspace_bytes);
  while (plan.total > workspace_bytes && plan.rows > 1) plan = plan_bwd(batch, plan.rows - 1, s_kv, topk, 0);
  if (plan.total > workspace_bytes)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_sparse_mla_bwd: workspace of %lld bytes is too small",
                     (long long)workspace_bytes);
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  char* ws = (char*)workspace;
  uint16_t* gbuf = (uint16_t*)ws;
  uint16_t* cbuf = (uint16_t*)(ws + al(plan.g_bytes));
  int* pairs = (int*)(ws + al(plan.g_bytes) + al(plan.c_bytes));
  int* counts = (int*)(ws + al(plan.g_bytes) + al(plan.c_bytes) + al(plan.pairs_bytes));
  float* mpart = (float*)(ws + al(plan.g_bytes) + al(plan.c_bytes) + al(plan.pairs_bytes) + al(plan.csr_bytes));
  float* dbuf = (float*)((char*)mpart + al(plan.mass_bytes));
  const unsigned hgroups = ceil_div(n_heads, kHG);

  for (int64_t r0 = 0; r0 < s_q; r0 += plan.rows) {
    const int rows = (int)std::min<int64_t>(plan.rows, s_q - r0);
    dim3 ga((unsigned)rows, hgroups, (unsigned)batch);
    // mass: one head group writes the caller's rows directly; several write partials
    float* mb = nullptr;
    int64_t m_hg = 0, m_b = 0;
    int m_row = 0;
    if (mass && hgroups == 1) {
      mb = mass;
      m_b = s_q * topk;
      m_row = (int)r0;
    } else if (mass) {
      mb = mpart;
      m_hg = batch * rows * topk;
      m_b = (int64_t)rows * topk;
    }
    {
      const int64_t groups = batch * rows * n_heads;
      bwd_delta_kernel<<<dim3((unsigned)((groups * 16 + 255) / 256), (unsigned)batch), 256, 0, st>>>(
          (const uint16_t*)out, (const uint16_t*)dout, dbuf, (int)s_q, (int)n_heads, (int)r0, rows);
      if (int rc = check_launch("dsa_sparse_mla_bwd(delta)")) return rc;
    }
    bwd_dq_kernel<<<ga, 256, 0, st>>>((const uint16_t*)q, (const uint16_t*)kv, indices, (const uint16_t*)out,
                                      (const uint16_t*)dout, softmax_max, softmax_sum, dbuf, (uint16_t*)dq, gbuf, mb,
                                      m_hg, m_b, m_row, (int)s_q, (int)s_kv, (int)n_heads, (int)topk, scale, q_offset,
                                      (int)r0);
    if (int rc = check_launch("dsa_sparse_mla_bwd(dq)")) return rc;
    if (mass && hgroups > 1) {
      const int64_t n = batch * rows * topk;
      const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 65535);
      mass_combine_kernel<<<blocks, 256, 0, st>>>(mpart, mass, (int)hgroups, m_hg, n, (int)s_q, (int)r0, rows,
                                                  (int)topk);
      if (int rc = check_launch("dsa_sparse_mla_bwd(mass)")) return rc;
    }
    dim3 gb((unsigned)rows, (unsigned)batch);
    if (hgroups == 1)
      bwd_contrib_kernel<1><<<gb, kCThreads, 0, st>>>((const uint16_t*)q, (const uint16_t*)dout, indices, gbuf, cbuf,
                                                      (int)s_q, (int)s_kv, (int)n_heads, (int)topk, q_offset, (int)r0,
                                                      rows);
    else
      bwd_contrib_kernel<2><<<gb, kCThreads, 0, st>>>((const uint16_t*)q, (const uint16_t*)dout, indices, gbuf, cbuf,
                                                      (int)s_q, (int)s_kv, (int)n_heads, (int)topk, q_offset, (int)r0,
                                                      rows);
    if (int rc = check_launch("dsa_sparse_mla_bwd(contrib)")) return rc;
    for (int b = 0; b < (int)batch; ++b)
      if (int rc = csr_reduce(indices, cbuf, dkv_accum, pairs, counts, (int)s_q, (int)s_kv, (int)topk, q_offset,
                              (int)r0, rows, b, kRowChunks, st))
        return rc;
  }
  return DSA_OK;
}
