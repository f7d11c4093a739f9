// Per-row fp8-e4m3fn quantisation of the indexer operands (one fp32 scale per row):
//   scale[r] = max(amax_i |x[r,i]| / 448, 1e-12),   q[r,i] = e4m3fn(x[r,i] / scale[r])
// where both divisions are correctly rounded fp32 divisions, the cast rounds to nearest
// even and every magnitude that rounds above 448 (and inf / NaN) becomes NaN (0x7f |
// sign): the same bytes as torch's float -> float8_e4m3fn cast of the same fp32 quotient.
// A NaN in a row makes its scale NaN, as torch's amax does.
//
// HBM-bound: a group of G lanes (G = the next power of two >= D/8, at most 64) owns one row,
// each lane eight consecutive elements per chunk (16-byte bf16 loads, 8-byte fp8 stores),
// the row held in registers between the max and the conversion.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 4;  // chunks of 8 elements per lane: D <= 8 * 64 * 4

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// NaN-propagating max of magnitudes (a NaN element makes the row's amax NaN)
__device__ __forceinline__ float max_mag(float m, float v) {
  const float a = fabsf(v);
  return (a > m || a != a) ? a : m;
}

template <typename T, bool kVec>
__global__ void __launch_bounds__(kThreads)
quantize_fp8_kernel(const T* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scale, int64_t rows, int D,
                    int lg) {
  const int G = 1 << lg;
  const int64_t row = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> lg;
  const int l = threadIdx.x & (G - 1);
  const bool active = row < rows;
  const int64_t r = active ? row : rows - 1;  // idle groups of the last workgroup re-read the last row
  const T* xr = x + r * D;
  float v[kMaxChunks][8];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int i0 = 8 * (l + c * G);
    if (kVec) {
      if (i0 < D) {
        if constexpr (sizeof(T) == 2) {
          const uint4 w = *reinterpret_cast<const uint4*>(xr + i0);
          const uint32_t p[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[c][2 * e] = __uint_as_float(p[e] << 16);
            v[c][2 * e + 1] = __uint_as_float(p[e] & 0xffff0000u);
          }
        } else {
          const float4 a = *reinterpret_cast<const float4*>(xr + i0);
          const float4 b = *reinterpret_cast<const float4*>(xr + i0 + 4);
          v[c][0] = a.x, v[c][1] = a.y, v[c][2] = a.z, v[c][3] = a.w;
          v[c][4] = b.x, v[c][5] = b.y, v[c][6] = b.z, v[c][7] = b.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = 0.f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = i0 + e < D ? to_f32(xr[i0 + e]) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = max_mag(amax, v[c][e]);
  }
  for (int m = G >> 1; m >= 1; m >>= 1) amax = max_mag(amax, __shfl_xor(amax, m, 64));
  float s = amax / 448.0f;
  s = s < 1e-12f ? 1e-12f : s;  // (keeps NaN)
  if (!active) return;
  if (l == 0) scale[row] = s;
  uint8_t* qr = q + row * D;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int i0 = 8 * (l + c * G);
    if (i0 >= D) continue;
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = e4m3fn_rne(v[c][e] / s);
    if (kVec) {
      const uint2 w = {b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
      *reinterpret_cast<uint2*>(qr + i0) = w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (i0 + e < D) qr[i0 + e] = (uint8_t)b[e];
    }
  }
}

// Rows of exactly 8 G elements (one 16-byte chunk per lane, bf16): each lane group takes
// kRows rows a grid apart and issues all their loads before the first use, so a wave keeps
// kRows loads in flight and the launch has a quarter of the waves.  Per row the arithmetic
// is quantize_fp8_kernel's, so the bytes are the same.
constexpr int kRows = 4;
__global__ void __launch_bounds__(kThreads)
quantize_fp8_rows_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scale,
                         int64_t rows, int lg) {
  const int G = 1 << lg, D = 8 << lg;
  const int64_t g0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> lg;
  const int64_t ng = ((int64_t)gridDim.x * kThreads) >> lg;
  const int l = threadIdx.x & (G - 1);
  uint4 w[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t row = g0 + i * ng;
    const int64_t r = row < rows ? row : rows - 1;  // (idle groups re-read the last row)
    w[i] = *reinterpret_cast<const uint4*>(x + r * D + 8 * l);
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t row = g0 + i * ng;
    const uint32_t p[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __uint_as_float(p[e] << 16);
      v[2 * e + 1] = __uint_as_float(p[e] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = max_mag(amax, v[e]);
    for (int m = G >> 1; m >= 1; m >>= 1) amax = max_mag(amax, __shfl_xor(amax, m, 64));
    float s = amax / 448.0f;
    s = s < 1e-12f ? 1e-12f : s;  // (keeps NaN)
    if (row >= rows) continue;  // (uniform over the lane group)
    if (l == 0) scale[row] = s;
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = e4m3fn_rne(v[e] / s);
    const uint2 o = {b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
    *reinterpret_cast<uint2*>(q + row * D + 8 * l) = o;
  }
}

template <typename T>
void launch_quantize(bool vec, const void* x, uint8_t* q, float* scale, int64_t rows, int D, int lg, hipStream_t st) {
  const int64_t threads = rows << lg;
  const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads));
  const TimedLaunch tl("quantize_fp8_kernel", st);
  if constexpr (sizeof(T) == 2) {
    if (vec && D == (8 << lg)) {
      const int64_t groups = (rows + kRows - 1) / kRows;
      const dim3 g4((unsigned)(((groups << lg) + kThreads - 1) / kThreads));
      quantize_fp8_rows_kernel<<<g4, kThreads, 0, st>>>(static_cast<const uint16_t*>(x), q, scale, rows, lg);
      return;
    }
  }
  if (vec)
    quantize_fp8_kernel<T, true><<<grid, kThreads, 0, st>>>(static_cast<const T*>(x), q, scale, rows, D, lg);
  else
    quantize_fp8_kernel<T, false><<<grid, kThreads, 0, st>>>(static_cast<const T*>(x), q, scale, rows, D, lg);
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_quantize_fp8_rows(const void* x, int in_dtype, uint8_t* q, float* scale, int64_t rows, int64_t d,
                                     void* stream) {
  using namespace dsa;
  if (!x || !q || !scale) return set_error(DSA_ERR_INVALID_ARG, "dsa_quantize_fp8_rows: null pointer");
  if (rows < 0 || d <= 0) return set_error(DSA_ERR_INVALID_ARG, "dsa_quantize_fp8_rows: bad sizes");
  if (in_dtype != DSA_BF16 && in_dtype != DSA_F32)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_quantize_fp8_rows: input must be bf16 or fp32");
  int lg = 0;
  while ((8 << lg) < d && lg < 6) ++lg;  // G = 2^lg lanes per row
  if (d > (int64_t)8 * (1 << lg) * kMaxChunks)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_quantize_fp8_rows: rows longer than %d elements", 8 * 64 * kMaxChunks);
  if (rows == 0) return DSA_OK;
  if ((rows << lg) / kThreads >= 2147483647LL) return set_error(DSA_ERR_INVALID_ARG, "dsa_quantize_fp8_rows: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const bool vec = d % 8 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 8) == 0;
  if (in_dtype == DSA_BF16)
    launch_quantize<uint16_t>(vec, x, q, scale, rows, (int)d, lg, st);
  else
    launch_quantize<float>(vec, x, q, scale, rows, (int)d, lg, st);
  return check_launch("dsa_quantize_fp8_rows");
}
