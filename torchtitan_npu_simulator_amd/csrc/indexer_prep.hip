// Indexer input producer: RoPE, Hadamard rotation and fp8-e4m3 per-row quantisation of the
// lightning indexer's query / key rows in one pass (DeepSeek-V3.2 Indexer.forward and
// DeepSeek-V4 Indexer.forward up to the index-score einsum).
//
// Per row x of D = 128 bf16 values (one query head or one key):
//   1. RoPE on the rope_dim features starting at rope_start, in fp32, rounded to bf16:
//      pairs (a, b) -> (a c - b s, a s + b c) with (c, s) = cs[pos][i] for pair i; the pairs
//      are (rope_start + 2i, rope_start + 2i + 1) when interleaved and
//      (rope_start + i, rope_start + i + rope_dim/2) otherwise (the V3.2 indexer's blocked
//      layout);
//   2. y = bf16(bf16(H x) * D^-0.5) with H the Sylvester Hadamard matrix (natural order,
//      H[i][j] = (-1)^popcount(i & j)), summed in fp32 by a radix-2 butterfly;
//   3. optionally fp8: scale = max(amax |y| / 448, 1e-12), q = e4m3fn(y / scale) rounded to
//      nearest even (the rule of dsa_quantize_fp8_rows).
// The bf16 rounding points are the reference's: RoPE output cast to the model dtype, the
// bf16 linear, then the bf16 scale multiply.
//
// HBM-bound: a 16-lane group per row (four rows per wave), lane l holding features
// 8l .. 8l+7 (16-byte loads and stores coalesced along the row).  Every cross-lane step --
// the butterfly's strides 8 .. 64, the V3.2 rope partner four lanes away and the amax --
// is a DPP lane exchange inside the 16-lane row.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f(f_to_bf16(x)); }

__global__ void __launch_bounds__(kThreads)
indexer_prep_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, uint8_t* __restrict__ q8,
                    float* __restrict__ scale, int64_t vecs, int heads, int64_t seq_len, const float* __restrict__ cs,
                    int64_t n_pos, const int32_t* __restrict__ positions, int64_t pos_offset, int rope_dim,
                    int rope_start, int interleaved, int hadamard) {
  const int64_t v_raw = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 4;
  const int l = threadIdx.x & 15;
  const bool active = v_raw < vecs;
  const int64_t v = active ? v_raw : vecs - 1;  // idle groups of the last wave redo the last row
  const int f0 = 8 * l;
  float e[8];
  {
    const u32x4 w = reinterpret_cast<const u32x4*>(x + v * kD)[l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[2 * i] = bf16_lo(w[i]);
      e[2 * i + 1] = bf16_hi(w[i]);
    }
  }

  // ---- 1. RoPE (fp32, rounded to bf16) ----
  if (rope_dim > 0) {
    const int64_t row = v / heads;
    const int64_t pos = positions ? (int64_t)positions[row] : pos_offset + row % seq_len;
    const bool pos_ok = pos >= 0 && pos < n_pos;  // rows outside the table keep their features
    const float* cp = cs + (pos_ok ? pos : 0) * rope_dim;
    const int lf = f0 - rope_start;  // local feature of e[0]
    const bool in_rope = pos_ok && lf >= 0 && lf < rope_dim;
    if (interleaved) {
      // pairs (lf + 2i, lf + 2i + 1) inside the lane, angles lf/2 + i
      if (in_rope) {
        const float4 c01 = *reinterpret_cast<const float4*>(cp + lf);
        const float4 c23 = *reinterpret_cast<const float4*>(cp + lf + 4);
        const float cc[4] = {c01.x, c01.z, c23.x, c23.z}, ss[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = e[2 * i], b = e[2 * i + 1];
          e[2 * i] = round_bf16(a * cc[i] - b * ss[i]);
          e[2 * i + 1] = round_bf16(a * ss[i] + b * cc[i]);
        }
      }
    } else {
      // pairs (i, i + 32) of a 64-feature block: the partner lane is four lanes away
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = lane_xor<4>(e[i]);
      if (in_rope) {
        const bool lower = lf < 32;
        const int a0 = lower ? lf : lf - 32;  // angle of e[0]
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float2 c = reinterpret_cast<const float2*>(cp)[a0 + i];
          e[i] = lower ? round_bf16(e[i] * c.x - p[i] * c.y) : round_bf16(p[i] * c.y + e[i] * c.x);
        }
      }
    }
  }

  // ---- 2. Hadamard: y = bf16(bf16(H x) * D^-0.5) ----
  if (hadamard) {
    // feature strides 1, 2, 4 inside the lane
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!(i & h)) {
          const float a = e[i], b = e[i + h];
          e[i] = a + b;
          e[i + h] = a - b;
        }
    // strides 8 .. 64 across the lanes of the row: lane bit k <-> feature stride 8 * 2^k
    static_for<4>([&](auto k) {
      constexpr int m = 1 << decltype(k)::value;
      const bool upper = l & m;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o = lane_xor<m>(e[i]);
        e[i] = upper ? o - e[i] : e[i] + o;
      }
    });
    const float sc = 0.08838834764831845f;  // 128^-0.5 rounded to fp32
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = round_bf16(round_bf16(e[i]) * sc);
  }
  if (y && active) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(e[2 * i], e[2 * i + 1]);
    reinterpret_cast<u32x4*>(y + v * kD)[l] = w;
  }

  // ---- 3. fp8-e4m3 with a per-row scale ----
  if (q8) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = fabsf(e[i]);
      amax = (a > amax || a != a) ? a : amax;  // a NaN makes the row's amax NaN
    }
    static_for<4>([&](auto k) {
      constexpr int m = 1 << decltype(k)::value;
      const float o = lane_xor<m>(amax);
      amax = (o > amax || o != o) ? o : amax;
    });
    float s = amax / 448.0f;
    s = s < 1e-12f ? 1e-12f : s;  // (keeps NaN)
    if (active) {
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = e4m3fn_rne(e[i] / s);
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 w = {b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
      reinterpret_cast<u32x2*>(q8 + v * kD)[l] = w;
      if (l == 0 && scale) scale[v] = s;
    }
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_indexer_prep(const void* x, void* y, uint8_t* q8, float* scale, int64_t rows, int64_t heads,
                                int64_t d, int64_t seq_len, const float* rope_cs, int64_t n_pos,
                                const int32_t* positions, int64_t pos_offset, int64_t rope_dim, int64_t rope_start,
                                int interleaved, int hadamard, void* stream) {
  using namespace dsa;
  if (!x) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: null input");
  if (!y && !q8) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: no output requested");
  if (q8 && !scale) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: fp8 output needs the scale output");
  if (rows < 0 || heads <= 0 || seq_len <= 0) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: bad sizes");
  if (d != kD) return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_prep: D=%lld (the producer takes D = 128)",
                                (long long)d);
  if (rope_dim < 0 || rope_start < 0 || rope_start + rope_dim > kD ||
      (rope_dim > 0 && (interleaved ? (rope_dim % 8 || rope_start % 8) : (rope_dim != 64 || rope_start % 64))))
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_prep: rope features [%lld, %lld) (interleaved: multiples of "
                     "8; blocked: 64 features starting at 0 or 64)", (long long)rope_start,
                     (long long)(rope_start + rope_dim));
  if (rope_dim > 0 && (!rope_cs || n_pos <= 0))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: RoPE needs the cos/sin table");
  const int64_t vecs = rows * heads;
  if (vecs == 0) return DSA_OK;
  const int64_t grid = (vecs * 16 + kThreads - 1) / kThreads;
  if (grid > INT32_MAX) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: too many rows");
  const TimedLaunch tl("indexer_prep_kernel", (hipStream_t)stream);
  indexer_prep_kernel<<<(unsigned)grid, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, (uint16_t*)y, q8, scale, vecs, (int)heads, seq_len, rope_cs, n_pos, positions, pos_offset,
      (int)rope_dim, (int)rope_start, interleaved ? 1 : 0, hadamard ? 1 : 0);
  return check_launch("dsa_indexer_prep");
}
