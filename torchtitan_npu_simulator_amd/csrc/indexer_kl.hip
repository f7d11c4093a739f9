// Indexer KL loss and gradients at the selected keys (the fused op
// npu_sparse_lightning_indexer_grad_kl_loss of the reference).
//
// Per query row s (one workgroup, 4 waves, wave w owns index heads 16w..16w+15), over
// blocks of 64 selected slots whose key rows are DMA'd into a double-buffered LDS tile:
//   phase 1  I_j = sum_h w_h relu(q_h . k_{idx_j}): S = q k^T on v_mfma_f32_16x16x32_bf16 with
//            the waves splitting the slots and each holding q of all 64 heads, so I_j is
//            summed in-lane and across the lane groups of one wave; key rows go straight to
//            VGPRs three slot groups ahead (no LDS, no barrier)
//   phase 2  row statistics: softmax of I over usable slots, target t = mass / Z, the
//            row loss Z * sum_{t>0} t (log max(t, eps) - log_softmax(I)) * loss_scale and
//            g_j = dloss/dI_j = Z * loss_scale * grad_scale * (softmax_j * T - t_j)
//   phase 3  recompute S; E = g_j w_h [S > 0] staged in LDS as [slot][head] and
//            [head][slot]; dw_h = sum_j g_j relu(S);
//            dq^T[d x 16 heads] += k^T E^T (k read transposed with ds_read_tr16_b64);
//            dk^T[128 d x 16 slots of wave w] = q^T E over all 64 heads (q^T operands read
//            transposed from q staged in LDS once per row), written as bf16 whole rows
//            through a wave-private LDS stage and reduced per key by the shared CSR pass.
// LDS key rows (and q, staged once per row) use the swz_kl chunk swizzle: the b128 column
// reads of 16 rows and the transposed b64 reads are both conflict-free.
// A generic fp32 kernel (any H, D) handles shapes outside the MFMA tile.
#include <algorithm>

#include "dsa_common.h"
#include "dsa_csr.h"

namespace dsa {
namespace {

constexpr int kD = 128;
constexpr int kH = 64;
constexpr int kB = 64;           // slots per block
constexpr int kRowC = kD / 8;    // 16 chunks per key row
constexpr int kTileC = kB * kRowC;  // 1024 chunks (16 KB)
constexpr int kMaxK = 4096;

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef short i16x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool ok_slot(int v, int s_k, int64_t limit) {
  return v >= 0 && v < s_k && (int64_t)v <= limit;
}

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  const int t = threadIdx.x;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float o = __shfl_xor(v, m, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < 4; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(256, 2)
indexer_kl_mfma_kernel(const uint16_t* __restrict__ qi, const uint16_t* __restrict__ ki, const float* __restrict__ w,
                       const int32_t* __restrict__ idx, const float* __restrict__ mass, float* __restrict__ dq,
                       float* __restrict__ dw, float* __restrict__ loss_rows, uint16_t* __restrict__ ck, int S,
                       int s_k, int K, int64_t q_offset, float loss_scale, float eps, float grad_scale,
                       const float* __restrict__ grad_scale_dev, int row0, float* __restrict__ softmax_out) {
  __shared__ u32x4 kt[2][kTileC];           // gathered key rows [64][16 chunks], swizzled
  __shared__ u32x4 qs[kH * kRowC];          // q of the row [64 heads][16 chunks] (phase 3), swizzled
  extern __shared__ float iv[];             // I_j, then g_j: K rounded up to whole blocks
  __shared__ uint16_t es[kB][kH + 8];       // E as [slot][head]
  __shared__ uint16_t eh[kH][kB + 8];       // E as [head][slot]
  __shared__ float red[12];
  __shared__ int ring[4][kB];                 // slot indices of blocks b & 3
  __shared__ int sh_last;

  const int lr = blockIdx.x, b = blockIdx.y;
  const int tok = row0 + lr;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, g = lane >> 4;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const float* mrow = mass + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* kb = ki + (int64_t)b * s_k * kD;
  const int head_a = 16 * wave + col;  // A-operand row (head) of this lane
  // slots past the row's last usable one (the causal limit cuts early rows short) hold no
  // valid key: phases 1 and 3 stop at the block that holds it
  if (tid == 0) sh_last = -1;
  __syncthreads();
  {
    // (every index load issued before the first test: a loop of load-then-test waits for
    // each load in turn; slots past K re-read slot K - 1 and are not counted)
    int vs[kMaxK / 256];
#pragma unroll
    for (int u = 0; u < kMaxK / 256; ++u) vs[u] = ridx[min(tid + 256 * u, K - 1)];
    int last = -1;
#pragma unroll
    for (int u = 0; u < kMaxK / 256; ++u)
      if (tid + 256 * u < K && ok_slot(vs[u], s_k, limit)) last = tid + 256 * u;
    if (last >= 0) atomicMax(&sh_last, last);
  }
  __syncthreads();
  const int n_used = sh_last + 1;  // slots [0, n_used) hold every valid slot
  const int nblocks = (n_used + kB - 1) / kB;

  // the upstream gradient may live on the device (no host round trip for the caller)
  const float gsc = grad_scale_dev ? grad_scale * grad_scale_dev[0] : grad_scale;

  // Key-row gather, 64 rows x 256 B per block: 4 DMA instructions per wave, instruction
  // J = 4 wave + i covering tile chunks [64J, 64J+64) (row p / 16, chunk (p % 16) ^ swz_kl(row)).
  // The block's slot indices reach an LDS ring by DMA (wave 0, one dword per lane) two
  // blocks ahead, and every DMA is inline assembly (the compiler neither waits for it before
  // LDS reads nor counts it), so the only wait is the explicit one at the top of each block.
  auto load_idx = [&](int blk) {  // wave 0: indices of block blk into ring entry blk & 3
    if (wave == 0) {
      const int j = min(blk * kB + lane, K - 1);
      dma4_to_lds(ridx, (uint32_t)j * 4u, (uint32_t)(uintptr_t)&ring[blk & 3][0]);
    }
  };
  auto gather = [&](int blk, int buf) {
    // the four ring entries are read (and waited for) together before the first DMA: each
    // DMA's inline asm orders memory, so a read left between two of them is a round trip
    int vi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = ((wave * 4 + i) * 64 + lane) >> 4;
      vi[i] = ring[blk & 3][row];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(vi[i]));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int J = wave * 4 + i;
      const int p = J * 64 + lane;
      const int row = p >> 4, pos = p & 15;
      const int chunk = pos ^ swz_kl(row);
      const int slot = blk * kB + row;
      const int r = (slot < K && ok_slot(vi[i], s_k, limit)) ? vi[i] : 0;
      dma16_to_lds(kb, (uint32_t)r * (kD * 2) + chunk * 16, (uint32_t)(uintptr_t)&kt[buf][J * 64]);
    }
  };
  // prologue of a pass: ring entries 0 and 1, then block 0's rows
  auto start_pass = [&]() {
    load_idx(0);
    if (nblocks > 1) load_idx(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    gather(0, 0);
  };
  const uint32_t kt_base = (uint32_t)(uintptr_t)(&kt[0][0]);

  // ---------------- phase 1: index scores at the selected slots ----------------
  // Waves split the slots (wave w: slots 64 blk + 16 w + col) and hold q of all 64 heads as
  // A operands, so each I_j is complete inside one wave: no LDS, no barrier.  Slot
  // indices and the 256-byte key rows go straight to VGPRs by ordinary loads, three groups
  // ahead (lane (slot col, g) holds d chunks 32 c + 8 g .. +8 of its slot's key, the B
  // operand of S = q k^T).
  {
    u32x4 qall[4][kD / 32];  // q[16 ht + col][32 c + 8 g ..] (A operands, all heads)
    float wall[4][4];        // w[16 ht + 4 g + r] (C rows of this lane)
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      const u32x4* qh = reinterpret_cast<const u32x4*>(qi + (row_id * kH + 16 * ht + col) * kD);
#pragma unroll
      for (int c = 0; c < kD / 32; ++c) qall[ht][c] = qh[4 * c + g];
#pragma unroll
      for (int r = 0; r < 4; ++r) wall[ht][r] = w[row_id * kH + 16 * ht + 4 * g + r];
    }
    const int nsb = (n_used + 15) / 16;  // 16-slot groups up to the last usable slot
    auto slot_of = [&](int i) { return 16 * i + col; };  // group i = 4 blk + wave
    auto load_idx1 = [&](int i) -> int {
      const int sl = slot_of(i);
      return (i < nsb && sl < K) ? ridx[sl] : -1;
    };
    auto load_rows = [&](int v, u32x4 (&dst)[kD / 32]) {
      const int r = ok_slot(v, s_k, limit) ? v : 0;
      const u32x4* kr = reinterpret_cast<const u32x4*>(kb + (int64_t)r * kD);
#pragma unroll
      for (int c = 0; c < kD / 32; ++c) dst[c] = kr[4 * c + g];
    };
    // this wave's groups are i = wave, wave + 4, ...; key rows kDepth groups ahead, slot
    // indices one group further
    constexpr int kDepth = 3;
    u32x4 kq[kDepth][kD / 32];
    int vnext = load_idx1(wave + 4 * kDepth);
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_rows(load_idx1(wave + 4 * d), kq[d]);
    for (int i = wave; i < nsb; i += 4) {
      const int vn2 = load_idx1(i + 4 * (kDepth + 1));
      u32x4 knew[kD / 32];
      load_rows(vnext, knew);
      float part = 0.f;
#pragma unroll
      for (int ht = 0; ht < 4; ++ht) {
        f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kD / 32; ++c) acc = mfma16x16x32(as_bf16x8(qall[ht][c]), as_bf16x8(kq[0][c]), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) part = fmaf(wall[ht][r], relu_bits(acc[r]), part);
      }
      part = xor32_sum(xor16_sum(part));
      const int sl = slot_of(i);
      if (g == 0 && sl < K) iv[sl] = part;
#pragma unroll
      for (int d = 0; d + 1 < kDepth; ++d)
#pragma unroll
        for (int c = 0; c < kD / 32; ++c) kq[d][c] = kq[d + 1][c];
#pragma unroll
      for (int c = 0; c < kD / 32; ++c) kq[kDepth - 1][c] = knew[c];
      vnext = vn2;
    }
  }
  __syncthreads();

  // ---------------- phase 2: row statistics ----------------
  // each thread keeps its slots' validity, target mass and score in registers (one batch
  // of loads instead of a dependent load per pass); slot groups u with 256 u >= K are
  // skipped (workgroup-uniform).  Two block reductions: (max, sum of exp at that max, Z)
  // merged as running (max, sum) pairs, then (loss part, T).  exp and log use the hardware
  // base-2 instructions.
  constexpr int kPer = kMaxK / 256;
  float mv[kPer], xv[kPer];
  bool okv[kPer];
  // (the loads are unconditional, at slots clamped into the row, and their results selected
  // afterwards: under a lane-dependent branch the compiler waits for each load before the
  // next, one memory round trip per 256 slots)
  int vi[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {  // (groups past K re-read slot K - 1: cache hits, unused)
    const int jc = min(tid + 256 * u, K - 1);
    vi[u] = ridx[jc];
    mv[u] = mrow[jc];
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int j = tid + 256 * u;
    okv[u] = false;
    xv[u] = 0.f;
    if (256 * u < K) {
      okv[u] = j < K && ok_slot(vi[u], s_k, limit);
      mv[u] = j < K ? mv[u] : 0.f;
    } else {
      mv[u] = 0.f;
    }
  }
  float lmax = -INFINITY, zsum = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (256 * u >= K) continue;
    const int j = tid + 256 * u;
    xv[u] = j < K ? iv[j] : 0.f;
    if (okv[u]) {
      lmax = fmaxf(lmax, xv[u]);
      zsum += fmaxf(mv[u], 0.f);
    }
  }
  float esum = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (256 * u < K && okv[u]) esum += __builtin_amdgcn_exp2f((xv[u] - lmax) * kLog2e);
  // (max, sum) pairs: s_a e^(m_a - m) + s_b e^(m_b - m) at m = max(m_a, m_b); a side with
  // no valid slot has m = -inf, s = 0 and contributes 0
  auto merge = [](float& m, float& se, float mo, float so) {
    const float mn = fmaxf(m, mo);
    const float a = m == -INFINITY ? 0.f : se * __builtin_amdgcn_exp2f((m - mn) * kLog2e);
    const float b = mo == -INFINITY ? 0.f : so * __builtin_amdgcn_exp2f((mo - mn) * kLog2e);
    m = mn;
    se = a + b;
  };
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    const float mo = __shfl_xor(lmax, msk, 64), so = __shfl_xor(esum, msk, 64);
    merge(lmax, esum, mo, so);
    zsum += __shfl_xor(zsum, msk, 64);
  }
  if (lane == 0) {
    red[wave] = lmax;
    red[4 + wave] = esum;
    red[8 + wave] = zsum;
  }
  __syncthreads();
  float imax = red[0], E = red[4], Z = red[8];
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    merge(imax, E, red[i], red[4 + i]);
    Z += red[8 + i];
  }
  const bool valid_row = Z > eps;
  const float lse = imax + __builtin_amdgcn_logf(E) * kLn2;
  const float zc = fmaxf(Z, eps), rzc = 1.f / zc;
  const float ls_uniform = -__builtin_amdgcn_logf((float)K) * kLn2;
  float lpart = 0.f, tpos = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (256 * u >= K) continue;
    const float t = okv[u] ? fmaxf(mv[u], 0.f) * rzc : 0.f;
    if (t > 0.f) {
      const float ls = valid_row ? (xv[u] - lse) : ls_uniform;
      lpart += t * (__builtin_amdgcn_logf(fmaxf(t, eps)) * kLn2 - ls);
      tpos += t;
    }
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    lpart += __shfl_xor(lpart, msk, 64);
    tpos += __shfl_xor(tpos, msk, 64);
  }
  __syncthreads();  // red is rewritten
  if (lane == 0) {
    red[wave] = lpart;
    red[4 + wave] = tpos;
  }
  __syncthreads();
  const float lrow = (red[0] + red[1]) + (red[2] + red[3]);
  const float T = (red[4] + red[5]) + (red[6] + red[7]);
  if (tid == 0) loss_rows[row_id] = Z * lrow * loss_scale;
  const float gs = valid_row ? Z * loss_scale * gsc : 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (256 * u >= K) continue;
    const int j = tid + 256 * u;
    const float t = okv[u] ? fmaxf(mv[u], 0.f) * rzc : 0.f;
    const float sm = okv[u] ? __builtin_amdgcn_exp2f((xv[u] - lse) * kLog2e) : 0.f;
    if (j < K) {
      iv[j] = gs * (sm * T - t);
      if (softmax_out) softmax_out[row_id * K + j] = sm;  // the indexer's distribution over the slots
    }
  }

  // ---------------- phase 3: gradients ----------------
  // A = q [16 heads x 32 d] per step c: lane (head col, g) holds q[16 w + col][32c + 8g .. +8];
  // C layout of S = q k^T tiles: lane (slot col, g) holds heads 16w + 4g + r
  u32x4 qa[kD / 32];
  float wr[4];
  {
    const u32x4* qh = reinterpret_cast<const u32x4*>(qi + (row_id * kH + head_a) * kD);
#pragma unroll
    for (int c = 0; c < kD / 32; ++c) qa[c] = qh[4 * c + g];
#pragma unroll
    for (int r = 0; r < 4; ++r) wr[r] = w[row_id * kH + 16 * wave + 4 * g + r];
  }
  // these operands must have arrived before the first DMA: a wait for them inside the loop
  // would also wait for every row DMA in flight
#pragma unroll
  for (int c = 0; c < kD / 32; ++c) asm volatile("" : "+v"(qa[c]));
#pragma unroll
  for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(wr[r]));
  // S tiles (16 heads x 16 slots) of the block's four slot tiles: every operand read is
  // issued first, then the four accumulation chains run interleaved (the compiler would
  // otherwise issue each read just before its MFMA and wait for it there)
  auto s_tiles = [&](uint32_t tb, f32x4 (&sv)[4]) {
    u32x4 bk[4][kD / 32];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int row = 16 * st + col;
#pragma unroll
      for (int c = 0; c < kD / 32; ++c)
        bk[st][c] = *(const lds_u32x4*)(uintptr_t)(tb + 16 * (row * kRowC + ((4 * c + g) ^ swz_kl(row))));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 4; ++st) sv[st] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kD / 32; ++c)
#pragma unroll
      for (int st = 0; st < 4; ++st) sv[st] = mfma16x16x32(as_bf16x8(qa[c]), as_bf16x8(bk[st][c]), sv[st]);
  };
  f32x4 dqa[kD / 16];
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) dqa[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float dwp[4] = {0.f, 0.f, 0.f, 0.f};
  uint16_t* ckrow = ck + ((int64_t)b * gridDim.x + lr) * (int64_t)K * kD;
  // transposed key reads for dq^T += k^T E^T over a 32-slot k-step ks: group g, source lane
  // col supplies slot row 32 ks + 8g + col/4 (+4 second read), d columns 16dt + 4(col%4)
  const int tr_row = 8 * g + (col >> 2);
  if (gs != 0.f) {  // block-uniform
    // q^T for dk (A of 16x16x32 over heads): tile dt covers d = 16 dt + col, k-step ks
    // heads 32 ks + 8g .. +7; q [64 heads x 128 d] stays staged row-major in qs (swz_kl) for
    // the whole phase and is read transposed per block (source lane col supplies head row
    // 32 ks + 8g + col/4 (+4 second read), d columns 16 dt + 4 (col % 4)), which keeps 64
    // registers free for the S tiles' operand reads
    {  // (all four loads in flight before the first store)
      u32x4 qv[kH * kRowC / 256];
#pragma unroll
      for (int u = 0; u < kH * kRowC / 256; ++u) {
        const int i = tid + 256 * u, h = i >> 4, c = i & 15;
        qv[u] = *reinterpret_cast<const u32x4*>(qi + (row_id * kH + h) * kD + 8 * c);
      }
#pragma unroll
      for (int u = 0; u < kH * kRowC / 256; ++u) {
        const int i = tid + 256 * u, h = i >> 4, c = i & 15;
        qs[h * kRowC + (c ^ swz_kl(h))] = qv[u];
      }
    }
    const lds_char* qsb = lds_bytes(&qs[0]);
    auto read_qtr = [&](int dt, int ks) {
      const int r1 = 32 * ks + tr_row, r2 = r1 + 4;
      const int c0 = 2 * dt + ((col & 3) >> 1);
      return lds_read_tr_pair(qsb + 16 * (r1 * kRowC + (c0 ^ swz_kl(r1))) + 8 * (col & 1),
                              qsb + 16 * (r2 * kRowC + (c0 ^ swz_kl(r2))) + 8 * (col & 1));
    };
    start_pass();  // (its barrier also publishes qs)
    for (int blk = 0; blk < nblocks; ++blk) {
      const int buf = blk & 1;
      // tile[buf] and ring entry blk+1 landed.  Their DMAs were issued before the previous
      // block's four dk row stores (every slot of a block before the last exists, so all
      // four issue); vector memory operations retire in issue order, so waiting until only
      // those stores are outstanding covers the DMAs and leaves the stores in flight
      if (blk == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      }
      __syncthreads();  // es / eh free
      if (blk + 1 < nblocks) gather(blk + 1, buf ^ 1);
      if (blk + 2 < nblocks) load_idx(blk + 2);
      const uint32_t tb = kt_base + buf * (kTileC * 16);
      // g_j of the lane's four slots, read before the S tiles so that the reads overlap the
      // MFMAs (unconditional reads inside iv, slots past K select 0 afterwards)
      float gjv[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) gjv[st] = iv[blk * kB + 16 * st + col];  // (iv spans whole blocks)
      f32x4 sv[4];
      s_tiles(tb, sv);
      // E = g_j w_h [S > 0] in bf16: es[slot][head] takes the lane's four heads as one 8-byte
      // store; for eh[head][slot] the lanes of adjacent slots (col, col ^ 1) swap two values
      // so that each writes two whole dwords (slot pair, one head each)
      const bool odd = col & 1;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int sl = 16 * st + col;
        const int slot = blk * kB + sl;
        const float gj = slot < K ? gjv[st] : 0.f;
        float e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          e[r] = sv[st][r] > 0.f ? gj * wr[r] : 0.f;
          dwp[r] += gj * relu_bits(sv[st][r]);
        }
        const uint32_t p01 = pack_bf16x2(e[0], e[1]), p23 = pack_bf16x2(e[2], e[3]);
        *reinterpret_cast<uint2*>(&es[sl][16 * wave + 4 * g]) = make_uint2(p01, p23);
        const uint32_t recv = __float_as_uint(lane_xor<1>(__uint_as_float(odd ? p01 : p23)));
        // even lane: heads 4g, 4g+1 of slots (sl, sl+1); odd lane: heads 4g+2, 4g+3 of (sl-1, sl)
        const uint32_t da = odd ? ((recv & 0xffffu) | (p23 << 16)) : ((p01 & 0xffffu) | (recv << 16));
        const uint32_t db = odd ? ((recv >> 16) | (p23 & 0xffff0000u)) : ((p01 >> 16) | (recv & 0xffff0000u));
        const int ha = 16 * wave + 4 * g + (odd ? 2 : 0);
        *reinterpret_cast<uint32_t*>(&eh[ha][sl & ~1]) = da;
        *reinterpret_cast<uint32_t*>(&eh[ha + 1][sl & ~1]) = db;
      }
      __syncthreads();
      // dq^T[16 d x 16 heads] += k^T[16 d x 32 slots] E^T[32 slots x 16 heads], two k-steps
      // (per k-step all eight operand reads first, then the eight MFMAs)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4 eb = *reinterpret_cast<const u32x4*>(&eh[head_a][32 * ks + 8 * g]);
        const int r1 = 32 * ks + tr_row, r2 = r1 + 4;
        u32x4 av[kD / 16];
#pragma unroll
        for (int dt = 0; dt < kD / 16; ++dt) {
          const int c0 = 2 * dt + ((col & 3) >> 1);
          const uint32_t a1 = tb + 16 * (r1 * kRowC + (c0 ^ swz_kl(r1))) + 8 * (col & 1);
          const uint32_t a2 = tb + 16 * (r2 * kRowC + (c0 ^ swz_kl(r2))) + 8 * (col & 1);
          av[dt] = lds_read_tr_pair((const lds_char*)(uintptr_t)a1, (const lds_char*)(uintptr_t)a2);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = 0; dt < kD / 16; ++dt) dqa[dt] = mfma16x16x32(as_bf16x8(av[dt]), as_bf16x8(eb), dqa[dt]);
      }
      // dk^T[128 d x 16 slots of this wave] = q^T[d x 64 heads] . E[64 heads x slots 16w ..];
      // the wave's rows of es / eh are read by this wave only, so once its MFMA operands are
      // in registers they serve as its private stage: dk rows 0..7 in the es rows, 8..15 in
      // the eh rows, 256 B each with 16-byte chunk c at c ^ (row & 15), stored as whole rows
      {
        const int sl = 16 * wave + col;
        u32x4 eo[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) eo[ks] = *reinterpret_cast<const u32x4*>(&es[sl][32 * ks + 8 * g]);
        lds_char* stg[2] = {lds_bytes(&es[16 * wave][0]), lds_bytes(&eh[16 * wave][0])};
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // own es / eh reads done before reuse
        // lane (slot col, g) holds d = 16 dt + 4g + r: 8 bytes at chunk 2 dt + g / 2, half g & 1;
        // two halves of the d tiles keep the accumulators to 16 registers
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          u32x4 qt[kD / 32][2];  // the half's q^T operands, read before its MFMAs
#pragma unroll
          for (int d4 = 0; d4 < kD / 32; ++d4)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) qt[d4][ks] = read_qtr(4 * half + d4, ks);
          __builtin_amdgcn_sched_barrier(0);
          f32x4 c4[kD / 32];
#pragma unroll
          for (int d4 = 0; d4 < kD / 32; ++d4) {
            c4[d4] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) c4[d4] = mfma16x16x32(as_bf16x8(qt[d4][ks]), as_bf16x8(eo[ks]), c4[d4]);
          }
#pragma unroll
          for (int d4 = 0; d4 < kD / 32; ++d4) {
            const int dt = 4 * half + d4;
            const u32x2 wv = {pack_bf16x2(c4[d4][0], c4[d4][1]), pack_bf16x2(c4[d4][2], c4[d4][3])};
            const int c = 2 * dt + (g >> 1);
            *(__attribute__((address_space(3))) u32x2*)(stg[col >> 3] + (col & 7) * 256 + 16 * (c ^ col) + 8 * (g & 1)) = wv;
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int row = 4 * m + (lane >> 4), c = lane & 15;
          const u32x4 v = lds_read16(stg[row >> 3] + (row & 7) * 256 + 16 * (c ^ row));
          const int slot = blk * kB + 16 * wave + row;
          // (non-temporal: read back once, by the key-major reduction)
          if (slot < K) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(ckrow + (int64_t)slot * kD + 8 * c));
        }
      }
    }
  } else {  // zero contributions so the reduction can read every usable slot
    for (int i = tid; i < K * kRowC; i += 256) {
      const int slot = i >> 4, c = i & 15;
      *reinterpret_cast<u32x4*>(ckrow + (int64_t)slot * kD + 8 * c) = (u32x4){0u, 0u, 0u, 0u};
    }
  }
  // dw: lane (slot col, g) holds partials for heads 16w + 4g + r: sum over the 16 slot lanes
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = dwp[r];
    v += lane_xor<1>(v);
    v += lane_xor<2>(v);
    v += lane_xor<4>(v);
    v += lane_xor<8>(v);
    dwp[r] = v;
  }
  if (col == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r) dw[row_id * kH + 16 * wave + 4 * g + r] = dwp[r];
  // dq^T tile dt: lane (head col, g) holds d = 16 dt + 4g + r
  float* dqrow = dq + (row_id * kH + head_a) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 16; ++dt) *reinterpret_cast<f32x4*>(dqrow + 16 * dt + 4 * g) = dqa[dt];
}

// --------------------------------------------------------------------------------------
// generic fp32 path: one workgroup per row; dk by fp32 atomics (small shapes)
// --------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
indexer_kl_generic_kernel(const uint16_t* __restrict__ qi, const uint16_t* __restrict__ ki,
                          const float* __restrict__ w, const int32_t* __restrict__ idx,
                          const float* __restrict__ mass, float* __restrict__ dq, float* __restrict__ dk,
                          float* __restrict__ dw, float* __restrict__ loss_rows, int S, int s_k, int H, int D, int K,
                          int64_t q_offset, float loss_scale, float eps, float grad_scale,
                          const float* __restrict__ grad_scale_dev, float* __restrict__ softmax_out) {
  extern __shared__ float sh[];  // iv[K]
  __shared__ float red[4];
  const int tok = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int64_t row_id = (int64_t)b * S + tok;
  const int32_t* ridx = idx + row_id * K;
  const float* mrow = mass + row_id * K;
  const int64_t limit = tok + q_offset;
  const uint16_t* qrow = qi + row_id * H * D;
  const uint16_t* kb = ki + (int64_t)b * s_k * D;
  float* iv = sh;
  float lmax = -INFINITY, zsum = 0.f;
  for (int j = tid; j < K; j += 256) {
    const int v = ridx[j];
    float x = 0.f;
    if (ok_slot(v, s_k, limit)) {
      for (int h = 0; h < H; ++h) {
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot = fmaf(bf16_to_f(qrow[h * D + d]), bf16_to_f(kb[(int64_t)v * D + d]), dot);
        x = fmaf(w[row_id * H + h], fmaxf(dot, 0.f), x);
      }
      lmax = fmaxf(lmax, x);
      zsum += fmaxf(mrow[j], 0.f);
    }
    iv[j] = x;
  }
  const float imax = block_reduce(lmax, red, true);
  const float Z = block_reduce(zsum, red, false);
  float esum = 0.f;
  for (int j = tid; j < K; j += 256)
    if (ok_slot(ridx[j], s_k, limit)) esum += expf(iv[j] - imax);
  const float E = block_reduce(esum, red, false);
  const bool valid_row = Z > eps;
  const float lse = imax + logf(E);
  const float zc = fmaxf(Z, eps);
  float lpart = 0.f, tpos = 0.f;
  for (int j = tid; j < K; j += 256) {
    const bool ok = ok_slot(ridx[j], s_k, limit);
    const float t = ok ? fmaxf(mrow[j], 0.f) / zc : 0.f;
    if (t > 0.f) {
      const float ls = valid_row ? (iv[j] - lse) : -logf((float)K);
      lpart += t * (logf(fmaxf(t, eps)) - ls);
      tpos += t;
    }
  }
  const float lrow = block_reduce(lpart, red, false);
  const float T = block_reduce(tpos, red, false);
  if (tid == 0) loss_rows[row_id] = Z * lrow * loss_scale;
  const float gs = valid_row ? Z * loss_scale * (grad_scale_dev ? grad_scale * grad_scale_dev[0] : grad_scale) : 0.f;
  __syncthreads();
  for (int j = tid; j < K; j += 256) {
    const bool ok = ok_slot(ridx[j], s_k, limit);
    const float t = ok ? fmaxf(mrow[j], 0.f) / zc : 0.f;
    const float sm = ok ? expf(iv[j] - lse) : 0.f;
    iv[j] = gs * (sm * T - t);
    if (softmax_out) softmax_out[row_id * K + j] = sm;
  }
  __syncthreads();
  // dq[h][d], dw[h]: thread per (h, d); dk by atomics
  for (int hd = tid; hd < H * D; hd += 256) {
    const int h = hd / D, d = hd % D;
    float acc = 0.f, dwacc = 0.f;
    for (int j = 0; j < K; ++j) {
      const float gj = iv[j];
      if (gj == 0.f) continue;
      const int v = ridx[j];
      float dot = 0.f;
      for (int e = 0; e < D; ++e) dot = fmaf(bf16_to_f(qrow[h * D + e]), bf16_to_f(kb[(int64_t)v * D + e]), dot);
      if (dot > 0.f) {
        const float ew = gj * w[row_id * H + h];
        acc = fmaf(ew, bf16_to_f(kb[(int64_t)v * D + d]), acc);
        atomicAdd(&dk[((int64_t)b * s_k + v) * D + d], ew * bf16_to_f(qrow[h * D + d]));
        if (d == 0) dwacc += gj * dot;
      }
    }
    dq[(row_id * H + h) * D + d] = acc;
    if (d == 0) dw[row_id * H + h] = dwacc;
  }
}

struct KlPlan {
  int64_t rows, ck_bytes, pairs_bytes, csr_bytes, total;
};

KlPlan plan_kl(int64_t batch, int64_t rows, int64_t s_k, int64_t topk) {
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  KlPlan p{};
  p.rows = rows;
  p.ck_bytes = batch * rows * topk * kD * 2;
  p.pairs_bytes = rows * topk * 4;
  p.csr_bytes = csr_ws_bytes(s_k, rows, topk, 128);
  p.total = al(p.ck_bytes) + al(p.pairs_bytes) + al(p.csr_bytes);
  return p;
}

constexpr int64_t kKlBudget = 8LL << 30;

}  // namespace
}  // namespace dsa

extern "C" int64_t dsa_indexer_kl_grad_workspace_size(int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                                                      int64_t head_dim, int64_t topk) {
  using namespace dsa;
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || topk <= 0) return 0;
  if (!(n_heads == kH && head_dim == kD)) return 0;  // generic path needs no workspace
  const int64_t per_row = batch * topk * kD * 2 + topk * 4;
  const int64_t rows = std::max<int64_t>(1, std::min<int64_t>(s_q, kKlBudget / per_row));
  return plan_kl(batch, rows, s_k, topk).total;
}

extern "C" int64_t dsa_indexer_kl_grad_chunk_rows(int64_t batch, int64_t s_q, int64_t s_k, int64_t topk,
                                                  int64_t workspace_bytes) {
  using namespace dsa;
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || topk <= 0 || workspace_bytes <= 0) return 0;
  const int64_t per_row = batch * topk * kD * 2 + topk * 4;
  const int64_t rows = std::max<int64_t>(1, std::min<int64_t>(s_q, workspace_bytes / per_row));
  KlPlan plan = plan_kl(batch, rows, s_k, topk);
  while (plan.total > workspace_bytes && plan.rows > 1) plan = plan_kl(batch, plan.rows - 1, s_k, topk);
  return plan.total > workspace_bytes ? 0 : plan.rows;
}

extern "C" int dsa_indexer_kl_grad(const void* q_idx, const void* k_idx, const float* w, const int32_t* indices,
                                   const float* mass, float* dq_idx, float* dk_idx_accum, float* dw, float* loss_rows,
                                   void* workspace, int64_t workspace_bytes, int64_t batch, int64_t s_q, int64_t s_k,
                                   int64_t n_heads, int64_t head_dim, int64_t topk, int64_t q_offset,
                                   float loss_scale, float eps, float grad_scale, const float* grad_scale_dev,
                                   void* stream) {
  return dsa_indexer_kl_grad_ex(q_idx, k_idx, w, indices, mass, dq_idx, dk_idx_accum, dw, loss_rows, nullptr, nullptr,
                                0, workspace, workspace_bytes, batch, s_q, s_k, n_heads, head_dim, topk, q_offset,
                                loss_scale, eps, grad_scale, grad_scale_dev, stream);
}

extern "C" int dsa_indexer_kl_grad_ex(const void* q_idx, const void* k_idx, const float* w, const int32_t* indices,
                                      const float* mass, float* dq_idx, float* dk_idx_accum, float* dw,
                                      float* loss_rows, float* softmax_out, const void* pair_csr,
                                      int64_t pair_csr_bytes, void* workspace, int64_t workspace_bytes, int64_t batch,
                                      int64_t s_q, int64_t s_k, int64_t n_heads, int64_t head_dim, int64_t topk,
                                      int64_t q_offset, float loss_scale, float eps, float grad_scale,
                                      const float* grad_scale_dev, void* stream) {
  using namespace dsa;
  if (pair_csr && pair_csr_bytes < pair_csr_bytes_of(batch, s_q, s_k, topk))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad_ex: pair CSR of %lld bytes is too small",
                     (long long)pair_csr_bytes);
  if (!q_idx || !k_idx || !w || !indices || !mass || !dq_idx || !dk_idx_accum || !dw || !loss_rows)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || n_heads <= 0 || head_dim <= 0 || topk <= 0 || topk > kMaxK)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: bad sizes");
  if (s_q > 2147483647LL || batch > 65535 || s_k > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  if (!(n_heads == kH && head_dim == kD)) {
    if (s_q > 2147483647LL) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: sizes out of range");
    dim3 grid((unsigned)s_q, (unsigned)batch);
    const TimedLaunch tl("indexer_kl_generic_kernel", st);
    indexer_kl_generic_kernel<<<grid, 256, topk * 4, st>>>(
        (const uint16_t*)q_idx, (const uint16_t*)k_idx, w, indices, mass, dq_idx, dk_idx_accum, dw, loss_rows,
        (int)s_q, (int)s_k, (int)n_heads, (int)head_dim, (int)topk, q_offset, loss_scale, eps, grad_scale,
        grad_scale_dev, softmax_out);
    return check_launch("dsa_indexer_kl_grad(generic)");
  }
  if (!workspace) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: workspace required");
  const int64_t per_row = batch * topk * kD * 2 + topk * 4;
  int64_t rows = std::max<int64_t>(1, std::min<int64_t>(s_q, workspace_bytes / per_row));
  KlPlan plan = plan_kl(batch, rows, s_k, topk);
  while (plan.total > workspace_bytes && plan.rows > 1) plan = plan_kl(batch, plan.rows - 1, s_k, topk);
  if (plan.total > workspace_bytes)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_kl_grad: workspace of %lld bytes is too small",
                     (long long)workspace_bytes);
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  char* ws = (char*)workspace;
  uint16_t* ck = (uint16_t*)ws;
  int* pairs = (int*)(ws + al(plan.ck_bytes));
  int* csr = (int*)(ws + al(plan.ck_bytes) + al(plan.pairs_bytes));
  for (int64_t r0 = 0; r0 < s_q; r0 += plan.rows) {
    const int rows_c = (int)std::min<int64_t>(plan.rows, s_q - r0);
    dim3 grid((unsigned)rows_c, (unsigned)batch);
    {
      const TimedLaunch tl("indexer_kl_mfma_kernel", st);
      // iv: one float per slot of whole 64-slot blocks (dynamic LDS)
      const size_t iv_bytes = (size_t)((topk + kB - 1) / kB * kB) * sizeof(float);
      indexer_kl_mfma_kernel<<<grid, 256, iv_bytes, st>>>((const uint16_t*)q_idx, (const uint16_t*)k_idx, w, indices, mass,
                                                   dq_idx, dw, loss_rows, ck, (int)s_q, (int)s_k, (int)topk, q_offset,
                                                   loss_scale, eps, grad_scale, grad_scale_dev, (int)r0,
                                                   softmax_out);
    }
    if (int rc = check_launch("dsa_indexer_kl_grad(mfma)")) return rc;
    // a prebuilt CSR of every row (the one the attention backward reduced dKV with) serves a
    // one-chunk plan; otherwise each chunk builds its own
    const bool prebuilt = pair_csr && rows_c == s_q;
    for (int b = 0; b < (int)batch; ++b) {
      if (prebuilt) {
        float* part = reinterpret_cast<float*>(csr + csr_ws_ints(s_k, rows_c, topk));
        if (int rc = csr_reduce_built(pair_csr_view(pair_csr, s_k, rows_c, topk, b), ck, dk_idx_accum, part, (int)s_k,
                                      rows_c, (int)topk, b, kRowC, st))
          return rc;
      } else if (int rc = csr_reduce(indices, ck, dk_idx_accum, pairs, csr, (int)s_q, (int)s_k, (int)topk, q_offset,
                                     (int)r0, rows_c, b, kRowC, st)) {
        return rc;
      }
    }
  }
  return DSA_OK;
}
