// Per-head attention sink of DeepSeek-V4 SparseAttention (a logit with no value in every
// row's softmax), applied around the gathered-attention kernels:
//
//   fold (after the forward):  with m, l the row's max and sum over its keys,
//     m2 = max(m, sink),  a = l e^(m - m2),  s2 = a + e^(sink - m2),
//     O <- O * a / s2 (in place),  (m, l) <- (m2, s2)
//   so the backward's P = exp(x - m2) / s2 already includes the sink;
//   grad (after the backward):  d sink[h] = - sum_rows e^(sink - m2) / s2 * rowsum(dO o O).
//
// Both are HBM-bound streams over O (and dO): a group of 16 lanes per (row, head), 16-byte
// accesses along the row; the gradient keeps one partial per (workgroup, head) and adds it
// with a single fp32 atomic.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kGradRows = 64;  // rows per gradient workgroup

__device__ __forceinline__ float ld_f(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float ld_f(const uint16_t* p, int64_t i) { return bf16_to_f(p[i]); }

struct SinkStats {
  float m2, s2, factor;
};

__device__ __forceinline__ SinkStats sink_stats(float m, float l, float sink) {
  SinkStats r;
  r.m2 = fmaxf(m, sink);
  const float a = l > 0.f ? l * expf(m - r.m2) : 0.f;
  r.s2 = a + expf(sink - r.m2);
  r.factor = a / r.s2;
  return r;
}

// one 16-lane group per (row, head); dv <= 16 * 8 * kChunks
template <typename T>
__global__ void __launch_bounds__(kThreads)
sink_fold_kernel(T* __restrict__ out, float* __restrict__ smax, float* __restrict__ ssum,
                 const float* __restrict__ sinks, int64_t rows_heads, int H, int dv) {
  const int64_t grp = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 4;
  const int l = threadIdx.x & 15;
  if (grp >= rows_heads) return;  // whole 16-lane groups leave together
  const int h = (int)(grp % H);
  const SinkStats st = sink_stats(smax[grp], ssum[grp], sinks[h]);
  T* orow = out + grp * dv;
  if constexpr (sizeof(T) == 2) {
    if (dv % 8 == 0) {
      u32x4* o4 = reinterpret_cast<u32x4*>(orow);
      for (int c = l; c < dv / 8; c += 16) {
        u32x4 v = o4[c];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = pack_bf16x2(bf16_lo(v[r]) * st.factor, bf16_hi(v[r]) * st.factor);
        o4[c] = v;
      }
    } else {
      for (int d = l; d < dv; d += 16) orow[d] = f_to_bf16(bf16_to_f(orow[d]) * st.factor);
    }
  } else {
    for (int d = l; d < dv; d += 16) orow[d] = orow[d] * st.factor;
  }
  if (l == 0) {
    smax[grp] = st.m2;
    ssum[grp] = st.s2;
  }
}

// workgroup = kGradRows rows x 16 heads (16 groups of 16 lanes, one head each)
template <typename T>
__global__ void __launch_bounds__(kThreads)
sink_grad_kernel(const T* __restrict__ out, const T* __restrict__ dout, const float* __restrict__ m2,
                 const float* __restrict__ s2, const float* __restrict__ sinks, float* __restrict__ dsink,
                 int64_t rows, int H, int dv) {
  const int gi = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int h = blockIdx.y * 16 + gi;
  const int64_t r0 = (int64_t)blockIdx.x * kGradRows;
  const int64_t r1 = r0 + kGradRows < rows ? r0 + kGradRows : rows;
  float acc = 0.f;
  if (h < H) {
    const float sink = sinks[h];
    for (int64_t r = r0; r < r1; ++r) {
      const int64_t hr = r * H + h;
      float part = 0.f;
      if constexpr (sizeof(T) == 2) {
        if (dv % 8 == 0) {
          const u32x4* o4 = reinterpret_cast<const u32x4*>(out + hr * dv);
          const u32x4* d4 = reinterpret_cast<const u32x4*>(dout + hr * dv);
          for (int c = l; c < dv / 8; c += 16) {
            const u32x4 ov = o4[c], gv = d4[c];
#pragma unroll
            for (int q = 0; q < 4; ++q) part += bf16_lo(gv[q]) * bf16_lo(ov[q]) + bf16_hi(gv[q]) * bf16_hi(ov[q]);
          }
        } else {
          for (int d = l; d < dv; d += 16) part += ld_f(dout, hr * dv + d) * ld_f(out, hr * dv + d);
        }
      } else {
        for (int d = l; d < dv; d += 16) part += dout[hr * dv + d] * out[hr * dv + d];
      }
      acc += expf(sink - m2[hr]) / s2[hr] * part;
    }
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (l == 0 && h < H) atomicAdd(&dsink[h], -acc);
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_attn_sink_fold(void* out, float* softmax_max, float* softmax_sum, const float* sinks, int dtype,
                                  int64_t rows, int64_t n_heads, int64_t d_v, void* stream) {
  using namespace dsa;
  if (!out || !softmax_max || !softmax_sum || !sinks) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_fold: null pointer");
  if (rows < 0 || n_heads <= 0 || d_v <= 0 || d_v > (1 << 20))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_fold: bad sizes");
  if (dtype != DSA_BF16 && dtype != DSA_F32) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_fold: dtype %d", dtype);
  const int64_t n = rows * n_heads;
  if (n == 0) return DSA_OK;
  if ((n * 16 + kThreads - 1) / kThreads > 2147483647LL) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_fold: too many rows");
  const unsigned grid = (unsigned)((n * 16 + kThreads - 1) / kThreads);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DSA_BF16)
    sink_fold_kernel<uint16_t><<<grid, kThreads, 0, st>>>((uint16_t*)out, softmax_max, softmax_sum, sinks, n,
                                                          (int)n_heads, (int)d_v);
  else
    sink_fold_kernel<float><<<grid, kThreads, 0, st>>>((float*)out, softmax_max, softmax_sum, sinks, n, (int)n_heads,
                                                       (int)d_v);
  return check_launch("dsa_attn_sink_fold");
}

extern "C" int dsa_attn_sink_grad(const void* out, const void* dout, const float* softmax_max,
                                  const float* softmax_sum, const float* sinks, float* dsink, int dtype, int64_t rows,
                                  int64_t n_heads, int64_t d_v, void* stream) {
  using namespace dsa;
  if (!out || !dout || !softmax_max || !softmax_sum || !sinks || !dsink)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_grad: null pointer");
  if (rows < 0 || n_heads <= 0 || d_v <= 0 || d_v > (1 << 20))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_grad: bad sizes");
  if (dtype != DSA_BF16 && dtype != DSA_F32) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_grad: dtype %d", dtype);
  if (rows == 0) return DSA_OK;
  if ((rows + kGradRows - 1) / kGradRows > 2147483647LL) return set_error(DSA_ERR_INVALID_ARG, "dsa_attn_sink_grad: too many rows");
  const dim3 grid((unsigned)((rows + kGradRows - 1) / kGradRows), (unsigned)((n_heads + 15) / 16));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DSA_BF16)
    sink_grad_kernel<uint16_t><<<grid, kThreads, 0, st>>>((const uint16_t*)out, (const uint16_t*)dout, softmax_max,
                                                          softmax_sum, sinks, dsink, rows, (int)n_heads, (int)d_v);
  else
    sink_grad_kernel<float><<<grid, kThreads, 0, st>>>((const float*)out, (const float*)dout, softmax_max,
                                                       softmax_sum, sinks, dsink, rows, (int)n_heads, (int)d_v);
  return check_launch("dsa_attn_sink_grad");
}
