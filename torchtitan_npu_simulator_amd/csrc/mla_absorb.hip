// MLA weight absorption, the per-head products around the absorbed attention
// (DeepSeek-V3.2 PreAttention / PostAttention, models/deepseek_v32/model.py:520-535, :574-575):
//   C[t, h, 0:N] = A[t, h, 0:K] . W[h]          (W = Wt[h]^T, Wt [H, N, K] row-major)
//   C[t, h, N:N+E] = E[t, h, 0:E]               (optional append: q_pe behind the absorbed q_nope)
// for (K, N) = (128, 512) (q_nope . w_uk, and the backward of the output projection) or
// (512, 128) (attention output . w_uv, and the backward of the query projection).
//
// Workgroup = one head x 256 tokens, 8 waves (wave w owns tokens 32w .. 32w+31).  The head's
// Wt (N x K bf16, 128 KB) is staged once in LDS with 16-byte chunk c of row n at
// c ^ (n & 15) (conflict-free b128 reads by 16 rows).  Per 32-token tile the wave computes
// C^T[32 n x 32 tokens] = Wt[n-tile] . A^T on v_mfma_f32_32x32x16_bf16: A operand = 8
// consecutive k of an Wt row from LDS, B operand = 8 consecutive k of a token's A row from
// global memory (held in VGPRs for the whole tile), fp32 accumulation, bf16 output: lane
// (token, half) holds n = 8j + 4 half + i and stores them as four 8-byte pieces.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTokensPerWg = 32 * kWaves;

template <int K, int N>
__global__ void __launch_bounds__(kThreads, 1)
mla_absorb_kernel(const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ wt,
                  uint16_t* __restrict__ c, int64_t ldc, const uint16_t* __restrict__ app, int64_t ld_app, int app_w,
                  int64_t tokens, int heads) {
  constexpr int kChunks = K / 8;        // 16-byte chunks per Wt row
  constexpr int kSteps = K / 16;        // MFMA k-steps
  constexpr int kNTiles = N / 32;
  __shared__ u32x4 ws[N * kChunks];     // 128 KB
  const int h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;

  // ---- stage Wt[h] (N rows of K) in LDS, swizzled ----
  const u32x4* wsrc = reinterpret_cast<const u32x4*>(wt + (int64_t)h * N * K);
  for (int i = tid; i < N * kChunks; i += kThreads) {
    const int n = i / kChunks, ch = i - n * kChunks;
    ws[n * kChunks + (ch ^ (n & 15))] = wsrc[i];
  }

  // ---- this wave's 32 tokens: B operands (A rows) into VGPRs ----
  const int64_t t0 = (int64_t)blockIdx.x * kTokensPerWg + 32 * wave;
  const int64_t tok = t0 + col;
  const bool tok_ok = tok < tokens;
  const int64_t row = (tok_ok ? tok : tokens - 1) * heads + h;  // (token, head) row
  u32x4 bk[kSteps];
  {
    const u32x4* arow = reinterpret_cast<const u32x4*>(a + row * lda);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) bk[s] = arow[2 * s + half];
  }
  __syncthreads();
  if (t0 >= tokens) return;  // whole wave past the end (after the barrier the others wait at)

  uint16_t* crow = c + row * ldc;
  const lds_char* wl = lds_bytes(&ws[0]);
#pragma unroll 1
  for (int nt = 0; nt < kNTiles; ++nt) {
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    const int n = 32 * nt + col;  // A-operand row of this lane
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int ch = 2 * s + half;
      const u32x4 av = lds_read16(wl + 16 * (n * kChunks + (ch ^ (n & 15))));
      acc = mfma32x32x16(as_bf16x8(av), as_bf16x8(bk[s]), acc);
    }
    if (tok_ok) {
      // lane (token col, half) holds C^T rows n = 32 nt + 8 j + 4 half + i, i = 0..3
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = {pack_bf16x2(acc[4 * j], acc[4 * j + 1]), pack_bf16x2(acc[4 * j + 2], acc[4 * j + 3])};
        *reinterpret_cast<u32x2*>(crow + 32 * nt + 8 * j + 4 * half) = v;
      }
    }
  }
  // ---- the appended columns (E = app_w bf16 per row, copied 8 bytes at a time) ----
  if (app && tok_ok) {
    const uint16_t* erow = app + row * ld_app;
    for (int e = 4 * half; e < app_w; e += 8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(crow + N + e) = *reinterpret_cast<const u32x2*>(erow + e);
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
  if (lda < k || ldc < n + (append ? append_width : 0) || lda % 8 || ldc % 4 ||
      (append && (append_width <= 0 || append_width % 4 || ld_append < append_width || ld_append % 4)))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: leading dimensions (lda %lld, ldc %lld, append %lld/%lld)",
                     (long long)lda, (long long)ldc, (long long)append_width, (long long)ld_append);
  if (((uintptr_t)a | (uintptr_t)wt) % 16 || (uintptr_t)c % 8 || (append && (uintptr_t)append % 8))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: misaligned operands");
  if (tokens == 0) return DSA_OK;
  const int64_t gx = (tokens + kTokensPerWg - 1) / kTokensPerWg;
  if (gx > INT32_MAX) return set_error(DSA_ERR_INVALID_ARG, "dsa_mla_absorb: too many tokens");
  dim3 grid((unsigned)gx, (unsigned)heads);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* ap = (const uint16_t*)a;
  const uint16_t* wp = (const uint16_t*)wt;
  const uint16_t* ep = (const uint16_t*)append;
  if (q_shape)
    mla_absorb_kernel<128, 512><<<grid, kThreads, 0, st>>>(ap, lda, wp, (uint16_t*)c, ldc, ep, ld_append,
                                                          (int)append_width, tokens, (int)heads);
  else
    mla_absorb_kernel<512, 128><<<grid, kThreads, 0, st>>>(ap, lda, wp, (uint16_t*)c, ldc, ep, ld_append,
                                                          (int)append_width, tokens, (int)heads);
  return check_launch("dsa_mla_absorb");
}
