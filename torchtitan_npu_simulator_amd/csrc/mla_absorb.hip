// MLA weight absorption, the per-head products around the absorbed attention
// (DeepSeek-V3.2 PreAttention / PostAttention, models/deepseek_v32/model.py:520-535, :574-575):
//   C[t, h, 0:N] = A[t, h, 0:K] . W[h]          (W = Wt[h]^T, Wt [H, N, K] row-major)
//   C[t, h, N:N+E] = E[t, h, 0:E]               (optional append: q_pe behind the absorbed q_nope)
// for (K, N) = (128, 512) (q_nope . w_uk, and the backward of the output projection) or
// (512, 128) (attention output . w_uv, and the backward of the query projection).
//
// Workgroup = one head x (8 waves x T 32-token tiles).  The head's Wt (N x K bf16, 128 KB)
// is staged once in LDS with 16-byte chunk c of row n at c ^ (n & 15) (conflict-free b128
// reads by 16 rows).  Per 32-token tile the wave computes C^T[32 n x 32 tokens] = Wt[n-tile]
// . A^T on v_mfma_f32_32x32x16_bf16 (A operand = 8 consecutive k of an Wt row from LDS, B
// operand = 8 consecutive k of a token's A row from global memory), fp32 accumulation, bf16
// output: lane (token, half) holds n = 8j + 4 half + i; a lane exchange between the two
// half-waves turns them into 16-byte stores.  Each Wt operand read from LDS feeds the
// wave's T token tiles (LDS traffic per MFMA / T):
//   (K, N) = (128, 512), T = 2: the tiles' A rows stay in VGPRs (8 k-steps x 2 tiles), the
//          16 n-tiles run in pairs (a whole 128-byte output line per iteration);
//   (K, N) = (512, 128), T = 2: the 4 n-tiles x 2 token tiles accumulate together while the
//          32 k-steps stream the A rows from global memory three steps ahead.
// Each workgroup stages its weight once and then walks token chunks; the waves share no
// state after the staging barrier.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int64_t kTargetWgs = 512;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int K, int N>
__device__ __forceinline__ void stage_wt(u32x4* ws, const uint16_t* __restrict__ wt, int h, int tid) {
  constexpr int kChunks = K / 8, kPer = N * kChunks / kThreads;
  static_assert(N * kChunks % kThreads == 0, "whole chunks per thread");
  const u32x4* wsrc = reinterpret_cast<const u32x4*>(wt + (int64_t)h * N * K);
  u32x4 v[kPer];  // every load in flight before the first LDS write
#pragma unroll
  for (int j = 0; j < kPer; ++j) v[j] = wsrc[tid + j * kThreads];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = tid + j * kThreads, n = i / kChunks, ch = i - n * kChunks;
    ws[n * kChunks + (ch ^ (n & 15))] = v[j];
  }
}

// store one 32x32 C^T tile: lane (token col, half) holds rows n = n0 + 8 j + 4 half + i.
// A v_permlane32_swap per j pair gives each lane 8 consecutive n: the lower half-wave
// n0 + 16 q .. + 7, the upper n0 + 16 q + 8 .. + 15, so every store is 16 bytes and a
// token's 32 bytes leave in one instruction.
__device__ __forceinline__ void store_tile(uint16_t* crow, int n0, int half, const f32x16& acc) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t x0 = pack_bf16x2(acc[8 * q], acc[8 * q + 1]), x1 = pack_bf16x2(acc[8 * q + 2], acc[8 * q + 3]);
    const uint32_t y0 = pack_bf16x2(acc[8 * q + 4], acc[8 * q + 5]), y1 = pack_bf16x2(acc[8 * q + 6], acc[8 * q + 7]);
    // (vdst, src) -> lower lanes (own vdst, upper partner's vdst), upper lanes (lower partner's src, own src)
    const auto r0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
    const auto r1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
    const u32x4 v = {r0[0], r1[0], r0[1], r1[1]};
    *reinterpret_cast<u32x4*>(crow + n0 + 16 * q + 8 * half) = v;
  }
}

__device__ __forceinline__ void append_cols(uint16_t* crow, const uint16_t* erow, int N, int app_w, int half) {
  for (int e = 8 * half; e < app_w; e += 16)
    *reinterpret_cast<u32x4*>(crow + N + e) = *reinterpret_cast<const u32x4*>(erow + e);
}

// (K, N) = (128, 512): the A rows of T token tiles stay in VGPRs; the n-tiles run in pairs,
// so each 128-byte line of a token's output is written whole within one iteration
__global__ void __launch_bounds__(kThreads, 1)
mla_absorb_q_kernel(const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ wt,
                    uint16_t* __restrict__ c, int64_t ldc, const uint16_t* __restrict__ app, int64_t ld_app,
                    int app_w, int64_t tokens, int heads) {
  constexpr int K = 128, N = 512, T = 2, kChunks = K / 8, kSteps = K / 16;
  __shared__ u32x4 ws[N * kChunks];  // 128 KB
  const int h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  stage_wt<K, N>(ws, wt, h, tid);
  __syncthreads();  // the only barrier: the waves run the chunks independently afterwards
  const lds_char* wl = lds_bytes(&ws[0]);
  for (int64_t t0 = ((int64_t)blockIdx.x * kWaves + wave) * (32 * T); t0 < tokens;
       t0 += (int64_t)gridDim.x * kWaves * (32 * T)) {
    int64_t row[T];
    bool ok[T];
    u32x4 bk[T][kSteps];
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const int64_t tok = t0 + 32 * u + col;
      ok[u] = tok < tokens;
      row[u] = (ok[u] ? tok : tokens - 1) * heads + h;
      const u32x4* arow = reinterpret_cast<const u32x4*>(a + row[u] * lda);
#pragma unroll
      for (int s = 0; s < kSteps; ++s) bk[u][s] = arow[2 * s + half];
    }
    // LDS address of chunk (2s + half) ^ (n & 15) of row n = 32 nt + col: lane term lo,
    // chunk (2s) ^ xm; kept opaque so that the compiler does not hoist every address
    uint32_t lo = 16u * (uint32_t)(col * kChunks);
    int xm = (col & 15) ^ half;
    asm volatile("" : "+v"(lo), "+v"(xm));
#pragma unroll 1
    for (int np = 0; np < N / 64; ++np) {
      f32x16 acc[2][T];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int u = 0; u < T; ++u)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[p][u][i] = 0.f;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const u32x4 av = lds_read16(wl + lo + 16 * ((64 * np + 32 * p) * kChunks + ((2 * s) ^ xm)));
#pragma unroll
          for (int u = 0; u < T; ++u) acc[p][u] = mfma32x32x16(as_bf16x8(av), as_bf16x8(bk[u][s]), acc[p][u]);
        }
      }
#pragma unroll
      for (int u = 0; u < T; ++u) {
        uint16_t* crow = c + row[u] * ldc;
        if (ok[u]) {
          store_tile(crow, 64 * np, half, acc[0][u]);
          store_tile(crow, 64 * np + 32, half, acc[1][u]);
        }
      }
    }
    if (app)
#pragma unroll
      for (int u = 0; u < T; ++u)
        if (ok[u]) append_cols(c + row[u] * ldc, app + row[u] * ld_app, N, app_w, half);
  }
}

// (K, N) = (512, 128): all n-tiles accumulate together, the A rows stream over the k-steps
__global__ void __launch_bounds__(kThreads, 1)
mla_absorb_o_kernel(const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ wt,
                    uint16_t* __restrict__ c, int64_t ldc, const uint16_t* __restrict__ app, int64_t ld_app,
                    int app_w, int64_t tokens, int heads) {
  constexpr int K = 512, N = 128, T = 2, kChunks = K / 8, kSteps = K / 16, kNT = N / 32, kAhead = 3;
  __shared__ u32x4 ws[N * kChunks];  // 128 KB
  const int h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  stage_wt<K, N>(ws, wt, h, tid);
  __syncthreads();  // the only barrier: the waves run the chunks independently afterwards
  const lds_char* wl = lds_bytes(&ws[0]);
  for (int64_t t0 = ((int64_t)blockIdx.x * kWaves + wave) * (32 * T); t0 < tokens;
       t0 += (int64_t)gridDim.x * kWaves * (32 * T)) {
    int64_t row[T];
    bool ok[T];
    const u32x4* arow[T];
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const int64_t tok = t0 + 32 * u + col;
      ok[u] = tok < tokens;
      row[u] = (ok[u] ? tok : tokens - 1) * heads + h;
      arow[u] = reinterpret_cast<const u32x4*>(a + row[u] * lda);
    }
    // B operands of k-steps s .. s + kAhead - 1 in a register ring
    u32x4 bk[kAhead][T];
#pragma unroll
    for (int s = 0; s < kAhead; ++s)
#pragma unroll
      for (int u = 0; u < T; ++u) bk[s][u] = arow[u][2 * s + half];
    // lane terms of the LDS addresses, opaque to the compiler so that it does not hoist the
    // 128 addresses of the k-loop out of the chunk loop (they would not fit in registers)
    uint32_t lo = 16u * (uint32_t)(col * kChunks);
    int xm = (col & 15) ^ half;
    asm volatile("" : "+v"(lo), "+v"(xm));
    f32x16 acc[kNT][T];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int u = 0; u < T; ++u)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[nt][u][i] = 0.f;
    static_for<kSteps>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      constexpr int slot = s % kAhead;
      // chunk (2s + half) ^ (n & 15) of row n = 32 nt + col; (n & 15) = (col & 15)
      const int sw = (16 * (s >> 3)) + ((2 * (s & 7)) ^ xm);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const u32x4 av = lds_read16(wl + lo + 16 * (32 * nt * kChunks + sw));
#pragma unroll
        for (int u = 0; u < T; ++u) acc[nt][u] = mfma32x32x16(as_bf16x8(av), as_bf16x8(bk[slot][u]), acc[nt][u]);
      }
      if constexpr (s + kAhead < kSteps) {
#pragma unroll
        for (int u = 0; u < T; ++u) bk[slot][u] = arow[u][2 * (s + kAhead) + half];
      }
    });
#pragma unroll
    for (int u = 0; u < T; ++u) {
      if (!ok[u]) continue;
      uint16_t* crow = c + row[u] * ldc;
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) store_tile(crow, 32 * nt, half, acc[nt][u]);
      if (app) append_cols(crow, app + row[u] * ld_app, N, app_w, half);
    }
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_mla_absorb(const void* a, int64_t lda, const void* wt, void* c, int64_t ldc, const void* append,
                              int64_t ld_append, int64_t append_width, int64_t tokens, int64_t heads, int64_t k,
                              int64_t n, void* stream) {
  using namespace dsa;
  if (!a || !wt || !c) return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: null pointer");
  if (tokens < 0 || heads <= 0 || heads > 65535) return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: bad sizes");
  const bool q_shape = k == 128 && n == 512, o_shape = k == 512 && n == 128;
  if (!q_shape && !o_shape)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_mla_absorb: (K, N) = (%lld, %lld); (128, 512) or (512, 128)",
                     (long long)k, (long long)n);
  if (lda < k || ldc < n + (append ? append_width : 0) || lda % 8 || ldc % 8 ||
      (append && (append_width <= 0 || append_width % 8 || ld_append < append_width || ld_append % 8)))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: leading dimensions (lda %lld, ldc %lld, append %lld/%lld; "
                     "multiples of 8 elements)", (long long)lda, (long long)ldc, (long long)append_width,
                     (long long)ld_append);
  if (((uintptr_t)a | (uintptr_t)wt | (uintptr_t)c) % 16 || (append && (uintptr_t)append % 16))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: operands must be 16-byte aligned");
  if (tokens == 0) return DSA_OK;
  // Each workgroup stages its head's weight once and then walks token chunks of
  // per_wg tokens gx apart: about kTargetWgs workgroups in all (every CU holds one).
  const int64_t per_wg = (int64_t)kWaves * 32 * 2;
  const int64_t chunks = (tokens + per_wg - 1) / per_wg;
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>(chunks, (kTargetWgs + heads - 1) / heads));
  dim3 grid((unsigned)gx, (unsigned)heads);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* ap = (const uint16_t*)a;
  const uint16_t* wp = (const uint16_t*)wt;
  const uint16_t* ep = (const uint16_t*)append;
  const TimedLaunch tl(q_shape ? "mla_absorb_q_kernel" : "mla_absorb_o_kernel", st);
  if (q_shape)
    mla_absorb_q_kernel<<<grid, kThreads, 0, st>>>(ap, lda, wp, (uint16_t*)c, ldc, ep, ld_append, (int)append_width,
                                                   tokens, (int)heads);
  else
    mla_absorb_o_kernel<<<grid, kThreads, 0, st>>>(ap, lda, wp, (uint16_t*)c, ldc, ep, ld_append, (int)append_width,
                                                   tokens, (int)heads);
  return check_launch("dsa_mla_absorb");
}
