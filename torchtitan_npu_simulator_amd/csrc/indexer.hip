// Lightning-indexer scores on MFMA (bf16 or OCP fp8-e4m3 inputs, fp32 accumulation):
//   I[s, t] = ks[t] * sum_h (w[s,h] * qs[s,h]) * relu(q[s,h,:] . k[t,:])      (t valid)
//   I[s, t] = -inf                                                       (t invalid)
// (relu(c x) = c relu(x) for the positive per-token scales, so the quantise-then-
// dequantise product of the reference folds into the head weights and one key scale.)
//
// Workgroup = 8 queries x 512 keys, 4 waves, 2 queries per wave.  A wave keeps its
// queries' 64 heads as MFMA A operands in VGPRs and streams 16-key B tiles straight from
// global memory (the whole key matrix is L2/MALL resident):
//   bf16: 4 x v_mfma_f32_16x16x32_bf16 per (16-head tile, 16-key tile)
//   fp8 : 1 x v_mfma_scale_f32_16x16x128_f8f6f4 (scales 0 = identity)
// The 16x16 C tile (lane: key = l%16, heads 4(l/16)..+3) gets relu * w in registers,
// is summed over the head tiles in-lane and over the 4 lane groups with two xor-shuffles.
// Causal tiles past a query block's frontier are written as -inf without any MFMA.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kD = 128;            // indexer head dim on the MFMA path
constexpr int kThreads = 256;
constexpr int kQPerWave = 2;
constexpr int kQPerWG = 4 * kQPerWave;  // 8
constexpr int kKeysPerWG = 512;

template <bool kFp8, int kHeadTiles>
__global__ void __launch_bounds__(kThreads)
indexer_mfma_kernel(const uint8_t* __restrict__ q, const float* __restrict__ q_scale, const uint8_t* __restrict__ k,
                    const float* __restrict__ k_scale, const float* __restrict__ w, float* __restrict__ scores,
                    int S, int s_k, int64_t ld, int64_t q_offset, int cmp_ratio) {
  constexpr int H = kHeadTiles * 16;
  constexpr int kElem = kFp8 ? 1 : 2;            // bytes per element
  constexpr int kRegsPerTile = kFp8 ? 8 : 16;    // A/B dwords per lane per 16-row tile (all 128 columns)
  const int b = blockIdx.z;
  const int q0 = blockIdx.x * kQPerWG;
  const int t0 = blockIdx.y * kKeysPerWG;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, g = lane >> 4;

  // causal frontier of this workgroup's queries: key t is valid for query s iff t < nv(s)
  auto nvalid = [&](int s) -> int {
    const int64_t v = (s + q_offset + 1) / cmp_ratio;
    return (int)max((int64_t)0, min((int64_t)s_k, v));
  };
  const int qa = q0 + wave * kQPerWave;
  int nv[kQPerWave];
#pragma unroll
  for (int j = 0; j < kQPerWave; ++j) nv[j] = qa + j < S ? nvalid(qa + j) : 0;
  const int t_end = min(s_k, t0 + kKeysPerWG);

  // A operands (queries) and folded head weights
  uint32_t qa_reg[kQPerWave][kHeadTiles][kRegsPerTile];
  float wv[kQPerWave][kHeadTiles][4];
#pragma unroll
  for (int j = 0; j < kQPerWave; ++j) {
    const int s = min(qa + j, S - 1);
    const int64_t qrow = ((int64_t)b * S + s) * H;
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
      const int head = ht * 16 + col;
      const uint8_t* src = q + (qrow + head) * kD * kElem;
      if (kFp8) {  // lane holds k = 32g .. 32g+31
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
        wv[j][ht][r] = w[qrow + hr] * sc;
      }
    }
  }

  for (int kt = t0; kt < t_end; kt += 16) {
    const int key = kt + col;
    const int keyc = min(key, s_k - 1);
    const bool any_valid = (kt < nv[0]) || (kt < nv[kQPerWave - 1]);
    float acc[kQPerWave];
#pragma unroll
    for (int j = 0; j < kQPerWave; ++j) acc[j] = 0.f;
    if (any_valid) {  // wave-uniform
      uint32_t kb[kRegsPerTile];
      const uint8_t* ksrc = k + ((int64_t)b * s_k + keyc) * kD * kElem;
      if (kFp8) {
        const u32x4* p = reinterpret_cast<const u32x4*>(ksrc + 32 * g);
        const u32x4 x0 = p[0], x1 = p[1];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kb[r] = x0[r];
          kb[4 + r] = x1[r];
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(ksrc + (32 * c + 8 * g) * 2);
#pragma unroll
          for (int r = 0; r < 4; ++r) kb[4 * c + r] = x[r];
        }
      }
#pragma unroll
      for (int j = 0; j < kQPerWave; ++j) {
        float part = 0.f;
#pragma unroll
        for (int ht = 0; ht < kHeadTiles; ++ht) {
          f32x4 c4 = (f32x4){0.f, 0.f, 0.f, 0.f};
          if (kFp8) {
            i32x8 av, bv;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              av[r] = (int)qa_reg[j][ht][r];
              bv[r] = (int)kb[r];
            }
            c4 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c4, 0, 0, 0, 0, 0, 0);
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              u32x4 av, bv;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                av[r] = qa_reg[j][ht][4 * c + r];
                bv[r] = kb[4 * c + r];
              }
              c4 = mfma16x16x32(as_bf16x8(av), as_bf16x8(bv), c4);
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) part = fmaf(wv[j][ht][r], fmaxf(c4[r], 0.f), part);
        }
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        acc[j] = part;
      }
    }
    if (g == 0 && key < t_end) {
      const float ks = k_scale ? k_scale[(int64_t)b * s_k + keyc] : 1.f;
#pragma unroll
      for (int j = 0; j < kQPerWave; ++j) {
        const int s = qa + j;
        if (s < S) scores[((int64_t)b * S + s) * ld + key] = key < nv[j] ? acc[j] * ks : -INFINITY;
      }
    }
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

}  // namespace
}  // namespace dsa

extern "C" int dsa_indexer_fwd(const void* q, const float* q_scale, const void* k, const float* k_scale,
                               const float* w, float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k,
                               int64_t n_heads, int64_t head_dim, int64_t ld_scores, int64_t q_offset,
                               int64_t cmp_ratio, void* stream) {
  using namespace dsa;
  if (!q || !k || !w || !scores) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: null pointer");
  if (batch <= 0 || s_q <= 0 || s_k <= 0 || n_heads <= 0 || head_dim <= 0 || ld_scores < s_k || cmp_ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: bad sizes");
  if (s_q > 65535LL * 8 || batch > 65535 || s_k > 2147483647LL)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_fwd: sizes out of range");
  hipStream_t st = (hipStream_t)stream;
  const bool mfma_shape = head_dim == kD && n_heads % 16 == 0 && n_heads <= 128 && dtype != DSA_F32;
  if (mfma_shape) {
    dim3 grid(ceil_div(s_q, kQPerWG), ceil_div(s_k, kKeysPerWG), (unsigned)batch);
    const uint8_t* qp = (const uint8_t*)q;
    const uint8_t* kp = (const uint8_t*)k;
#define DSA_IDX_LAUNCH(FP8, HT)                                                                              \
  indexer_mfma_kernel<FP8, HT><<<grid, kThreads, 0, st>>>(qp, q_scale, kp, k_scale, w, scores, (int)s_q, (int)s_k, \
                                                          ld_scores, q_offset, (int)cmp_ratio)
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
