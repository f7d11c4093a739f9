// Gathered KV-row pipeline shared by the sparse-attention kernels (gfx950).
//
// A block is kBN = 32 selected latent-KV rows of 576 bf16 (1152 B; 512 bf16 = 1024 B for
// the rope-less DeepSeek-V4 rows).  Its LDS tile holds the rows row-major with 16-byte chunk
// c of row r at chunk c ^ swz_kv(r), and is filled by 36 (32) wave-wide DMA instructions
// (global_load_lds, 16 B per lane): instruction J covers tile positions [64J, 64J+64),
// position p = r*72 + (c ^ swz_kv(r)) (r*64 + ...); wave w issues J = w, w + W, ...
// Unused slots (-1, past the causal limit, past K) load row 0 and are masked by the
// block's validity bits.
//
// Tiles are triple-buffered: while block b computes, block b+1 has landed or is landing
// and block b+2 is being issued, so a gather has two block times to arrive.  The slot
// indices reach a 4-entry LDS ring by DMA as well (wave 0, one dword per lane, issued for
// block b+3 just before block b+2's rows), so no index round trip precedes a gather and
// no register waits on a load inside the loop.
//
// Waiting: vector-memory loads retire in issue order, so "block b+1 and the indices of
// b+3 have landed" holds as soon as no more loads are outstanding than the rows of block
// b+2 that this wave issued after them.  Stores issued after those rows would only add
// to the count, so kernels issue their stores for block b-1 before block b+2's DMA.
// With no block b+2 in flight the wait is for everything (vmcnt 0).  The DMAs are inline
// assembly, so the compiler neither counts them nor waits on them; every wait is explicit.
#pragma once
#include "dsa_common.h"

namespace dsa {

typedef __attribute__((address_space(3))) u32x4 lds_u32x4_t;

// row width kDqkT: 576 (latent 512 + rope 64, DeepSeek-V3.2 MLA) or 512 (DeepSeek-V4 rows)
template <int kDqkT>
struct GatherGeomT {
  static constexpr int kDqk = kDqkT;
  static constexpr int kRowChunks = kDqk / 8;           // 72 | 64
  static constexpr int kRowBytes = kRowChunks * 16;     // 1152 | 1024
  static constexpr int kBN = 32;                        // rows per block
  static constexpr int kTileChunks = kBN * kRowChunks;  // 2304 | 2048 x 16 B
  static constexpr int kTileBytes = kTileChunks * 16;   // 36864 | 32768
  static constexpr int kTileInstr = kTileChunks / 64;   // 36 | 32 wave-wide DMA instructions
  static constexpr int kRing = 4;
  static constexpr int64_t kMaxRows = (int64_t)UINT32_MAX / kRowBytes - 1;  // 32-bit byte offsets
};
using GatherGeom = GatherGeomT<576>;

// slot value v of a row whose causal limit is `limit` is a usable key
__device__ __forceinline__ bool slot_ok(int v, int s_kv, int64_t limit) {
  return v >= 0 && v < s_kv && (int64_t)v <= limit;
}

// Number of 32-slot blocks up to the last usable slot of a row, in two parts so a kernel
// can request the row's indices together with its other prologue loads and test them
// later (one memory round trip): load_row_indices() issues each thread's first kIdxU
// index loads with no wait between them; count_row_blocks() tests them (a loop reads
// slots past kIdxU * blockDim.x) and reduces over the workgroup (needs sync).
constexpr int kIdxU = 8;
__device__ __forceinline__ void load_row_indices(const int32_t* ridx, int K, int (&v)[kIdxU]) {
#pragma unroll
  for (int u = 0; u < kIdxU; ++u) {
    const int j = (int)threadIdx.x + u * (int)blockDim.x;
    v[u] = j < K ? ridx[j] : -1;
  }
}
__device__ __forceinline__ int count_row_blocks(const int32_t* ridx, int K, int s_kv, int64_t limit,
                                                const int (&v)[kIdxU], int* sh_last) {
  if (threadIdx.x == 0) *sh_last = -1;
  int last = -1;
#pragma unroll
  for (int u = 0; u < kIdxU; ++u) {
    const int j = (int)threadIdx.x + u * (int)blockDim.x;
    if (j < K && slot_ok(v[u], s_kv, limit)) last = j;
  }
  for (int j = (int)threadIdx.x + kIdxU * (int)blockDim.x; j < K; j += blockDim.x)
    if (slot_ok(ridx[j], s_kv, limit)) last = j;
  __syncthreads();  // sh_last initialised
  if (last >= 0) atomicMax(sh_last, last);
  __syncthreads();
  const int n = (*sh_last + GatherGeom::kBN) / GatherGeom::kBN;
  __syncthreads();
  return n;
}

// usable-key limit of a row: slot value v is used iff (uint32)v <= lim
__device__ __forceinline__ uint32_t gather_limit(int64_t tok_limit, int s_kv) {
  const int64_t l = tok_limit < (int64_t)s_kv - 1 ? tok_limit : (int64_t)s_kv - 1;
  return l < 0 ? 0u : (uint32_t)l;
}

// kA16: tile chunks swizzled by swz_a16 (tiles read as 16x16x32 A operands) instead of swz_kv
template <int kWaves, int kDqkT = 576, bool kA16 = false>
struct RowGather {
  using G = GatherGeomT<kDqkT>;
  static constexpr int kMaxPerWave = (G::kTileInstr + kWaves - 1) / kWaves;
  static constexpr int kFullWaves = G::kTileInstr % kWaves == 0 ? kWaves : G::kTileInstr % kWaves;
  static constexpr int kRingInts = 64;  // one dword per lane; lanes 32..63 repeat 0..31

  // per-lane DMA geometry, computed once per workgroup: for the wave's i-th instruction
  // (J = wave + kWaves i) the tile row this lane loads and the swizzled byte offset of its
  // 16-byte chunk within the KV row
  struct Lanes {
    int row[kMaxPerWave];
    uint32_t cbyte[kMaxPerWave];
  };
  static __device__ __forceinline__ Lanes lanes(int wave, int lane) {
    Lanes L;
#pragma unroll
    for (int i = 0; i < kMaxPerWave; ++i) {
      const int J = min(wave + kWaves * i, G::kTileInstr - 1);
      const int p = J * 64 + lane;
      const int row = p / G::kRowChunks, pos = p - row * G::kRowChunks;
      L.row[i] = row;
      L.cbyte[i] = (uint32_t)((pos ^ (kA16 ? swz_a16(row) : swz_kv(row))) * 16);
    }
    return L;
  }

  // issue block `blk`'s row DMA into `tile` from ring entry `sidx`; wave 0 also writes the
  // block's validity bits.  `wave` must be wave-uniform (an SGPR value).
  static __device__ __forceinline__ void issue(const uint16_t* kvb, u32x4* tile, uint32_t* vmask_slot,
                                               const int* sidx, int blk, int K, uint32_t lim, int wave, int lane,
                                               const Lanes& L) {
    const int rows_left = K - blk * G::kBN;
    const char* base = reinterpret_cast<const char*>(kvb);
    uint32_t raw[kMaxPerWave];
#pragma unroll
    for (int i = 0; i < kMaxPerWave; ++i) raw[i] = (uint32_t)sidx[L.row[i]];
#pragma unroll
    for (int i = 0; i < kMaxPerWave; ++i) {
      const int J = wave + kWaves * i;
      if (J < G::kTileInstr) {
        const bool ok = raw[i] <= lim && L.row[i] < rows_left;
        const uint32_t off = (ok ? raw[i] : 0u) * (uint32_t)G::kRowBytes + L.cbyte[i];
        dma16_to_lds(base, off, (uint32_t)(uintptr_t)&tile[J * 64]);
      }
    }
    if (wave == 0) {
      const bool ok = lane < G::kBN && lane < rows_left && (uint32_t)sidx[lane & (G::kBN - 1)] <= lim;
      const uint64_t bal = __ballot(ok);
      if (lane == 0) *vmask_slot = (uint32_t)bal;
    }
  }

  // split form of issue(): prep() resolves the wave's row offsets (and wave 0's validity
  // bits) for block `blk`; issue_one(i) then sends the wave's i-th instruction, so a
  // kernel can spread the DMA over its compute instead of stalling on a burst
  static __device__ __forceinline__ void prep(uint32_t* vmask_slot, const int* sidx, int blk, int K, uint32_t lim,
                                              int wave, int lane, const Lanes& L, uint32_t (&off)[kMaxPerWave]) {
    const int rows_left = K - blk * G::kBN;
#pragma unroll
    for (int i = 0; i < kMaxPerWave; ++i) {
      const uint32_t raw = (uint32_t)sidx[L.row[i]];
      const bool ok = raw <= lim && L.row[i] < rows_left;
      off[i] = (ok ? raw : 0u) * (uint32_t)G::kRowBytes + L.cbyte[i];
    }
    if (wave == 0) {
      const bool ok = lane < G::kBN && lane < rows_left && (uint32_t)sidx[lane & (G::kBN - 1)] <= lim;
      const uint64_t bal = __ballot(ok);
      if (lane == 0) *vmask_slot = (uint32_t)bal;
    }
  }
  // register-light form for kernels that resolve each DMA instruction when they issue it
  // and keep a block's validity bits in SGPRs: the row geometry packed as
  // (row << 11) | chunk byte (16 bits, two instructions per VGPR)
  static constexpr int kPackedRegs = (kMaxPerWave + 1) / 2;
  struct PackedLanes {
    uint32_t rc[kPackedRegs];
  };
  static __device__ __forceinline__ PackedLanes packed_lanes(int wave, int lane) {
    const Lanes L = lanes(wave, lane);
    PackedLanes P;
#pragma unroll
    for (int k = 0; k < kPackedRegs; ++k) {
      const uint32_t lo = ((uint32_t)L.row[2 * k] << 11) | L.cbyte[2 * k];
      const uint32_t hi = 2 * k + 1 < kMaxPerWave ? (((uint32_t)L.row[2 * k + 1] << 11) | L.cbyte[2 * k + 1]) : 0u;
      P.rc[k] = lo | (hi << 16);
    }
    return P;
  }
  // the wave's i-th instruction straight from the ring: its slot value (read one batch
  // ahead by the caller, an LDS load), then the DMA
  typedef const __attribute__((address_space(3))) uint32_t lds_u32c;
  // (the packed word passes through an empty asm so the unpacking is not hoisted out of
  // the caller's loop, which would hold 2 kMaxPerWave unpacked values in registers)
  static __device__ __forceinline__ uint32_t unpack(const PackedLanes& P, int i) {
    uint32_t w = P.rc[i >> 1];
    asm volatile("" : "+v"(w));
    return (w >> (16 * (i & 1))) & 0xffffu;
  }
  static __device__ __forceinline__ uint32_t ring_slot(const int* ring, int i, const PackedLanes& P) {
    const uint32_t e = unpack(P, i);
    return *(lds_u32c*)(lds_bytes(const_cast<int*>(ring)) + ((e >> 11) << 2));
  }
  static __device__ __forceinline__ void issue_slot(const uint16_t* kvb, u32x4* tile, int i, int wave, uint32_t raw,
                                                    const PackedLanes& P, uint32_t lim, int rows_left) {
    static_assert(G::kRowBytes < (1 << 11) && G::kBN <= 32, "packed lane geometry");
    const int J = wave + kWaves * i;
    if constexpr (G::kTileInstr % kWaves != 0) {
      if (J >= G::kTileInstr) return;
    }
    const uint32_t e = unpack(P, i);
    const bool ok = raw <= lim && (int)(e >> 11) < rows_left;
    // row * 1152 as a 24-bit multiply (rows < 2^22 by kMaxRows)
    const uint32_t off = (ok ? __umul24(raw, (uint32_t)G::kRowBytes) : 0u) + (e & 0x7ffu);
    dma16_to_lds(kvb, off, (uint32_t)(uintptr_t)&tile[J * 64]);
  }
  // validity bits of a block (bit j = slot j usable), computed by every wave, wave-uniform
  static __device__ __forceinline__ uint32_t ring_valid(const int* ring, int lane, uint32_t lim, int rows_left) {
    const uint32_t v = *(lds_u32c*)(lds_bytes(const_cast<int*>(ring)) + ((lane & (G::kBN - 1)) << 2));
    const bool ok = lane < G::kBN && lane < rows_left && v <= lim;
    return (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)__ballot(ok));
  }

  static __device__ __forceinline__ void issue_one(const uint16_t* kvb, u32x4* tile, int i, int wave,
                                                   const uint32_t (&off)[kMaxPerWave]) {
    const int J = wave + kWaves * i;
    if (J < G::kTileInstr) dma16_to_lds(kvb, off[i], (uint32_t)(uintptr_t)&tile[J * 64]);
  }

  // wave 0: DMA the slot indices of block `blk` (clamped to K) into ring entry `ring`
  static __device__ __forceinline__ void issue_idx(const int32_t* ridx, int K, int blk, int* ring, int lane) {
    const int j = min(blk * G::kBN + (lane & (G::kBN - 1)), K - 1);
    dma4_to_lds(ridx, (uint32_t)j * 4u, (uint32_t)(uintptr_t)ring);
  }

  // prologue: indices of blocks 0..2 into ring entries 0..2 and landed, visible after the
  // caller's barrier
  static __device__ __forceinline__ void ring_init(int (*sidx)[kRingInts], const int32_t* ridx, int K, int nblk,
                                                   int wave, int lane) {
    if (wave == 0) {
      for (int i = 0; i < 3 && i < nblk; ++i) issue_idx(ridx, K, i, sidx[i], lane);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }

  // wait until block blk+1's rows (and the ring entry of blk+3) have landed; call at the
  // end of iteration blk, after which the caller's barrier publishes them
  static __device__ __forceinline__ void wait_next(bool rows2_in_flight, int wave) {
    if (!rows2_in_flight) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (kFullWaves == kWaves || wave < kFullWaves) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kMaxPerWave) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kMaxPerWave - 1) : "memory");
    }
  }
};

}  // namespace dsa
