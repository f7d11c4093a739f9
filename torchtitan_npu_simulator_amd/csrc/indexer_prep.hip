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
// HBM-bound: one wave per row, lane l holds features 2l, 2l+1 (4-byte loads and stores
// coalesced along the row); the butterfly's cross-lane stages are lane exchanges.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f(f_to_bf16(x)); }

template <int kMask>
__device__ __forceinline__ float lane_swap(float x) {
  return __shfl_xor(x, kMask, 64);
}

__global__ void __launch_bounds__(kThreads)
indexer_prep_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, uint8_t* __restrict__ q8,
                    float* __restrict__ scale, int64_t vecs, int heads, int64_t seq_len, const float* __restrict__ cs,
                    int64_t n_pos, const int32_t* __restrict__ positions, int64_t pos_offset, int rope_dim,
                    int rope_start, int interleaved, int hadamard) {
  const int64_t v = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (v >= vecs) return;  // whole waves: v is wave-uniform
  const uint32_t w = reinterpret_cast<const uint32_t*>(x + v * kD)[lane];
  float e0 = bf16_lo(w), e1 = bf16_hi(w);
  const int f0 = 2 * lane;  // features f0, f0 + 1

  // ---- 1. RoPE (fp32, rounded to bf16) ----
  if (rope_dim > 0) {
    const int64_t row = v / heads;
    const int64_t pos = positions ? (int64_t)positions[row] : pos_offset + row % seq_len;
    const bool pos_ok = pos >= 0 && pos < n_pos;  // rows outside the table keep their features
    const int half = rope_dim / 2;
    const int lf = f0 - rope_start;  // local feature index of e0
    const bool in_rope = lf >= 0 && lf < rope_dim;
    if (interleaved) {
      // pair (lf, lf + 1) lives in this lane: angle lf / 2
      if (in_rope && pos_ok) {
        const float2 c = reinterpret_cast<const float2*>(cs + pos * rope_dim)[lf / 2];
        const float a = e0, b = e1;
        e0 = round_bf16(a * c.x - b * c.y);
        e1 = round_bf16(a * c.y + b * c.x);
      }
    } else {
      // pair (i, i + half): the partner features sit half / 2 lanes away
      const int dl = half / 2;
      const bool lower = in_rope && lf < half;
      const int partner = in_rope ? (lower ? lane + dl : lane - dl) : lane;
      const float p0 = __shfl(e0, partner, 64), p1 = __shfl(e1, partner, 64);
      if (in_rope && pos_ok) {
        const int i0 = lower ? lf : lf - half;  // angle of e0 (e1: i0 + 1)
        const float2* cp = reinterpret_cast<const float2*>(cs + pos * rope_dim);
        const float2 c0 = cp[i0], c1 = cp[i0 + 1];
        if (lower) {  // real parts: a c - b s with b = partner
          e0 = round_bf16(e0 * c0.x - p0 * c0.y);
          e1 = round_bf16(e1 * c1.x - p1 * c1.y);
        } else {  // imaginary parts: a s + b c with a = partner
          e0 = round_bf16(p0 * c0.y + e0 * c0.x);
          e1 = round_bf16(p1 * c1.y + e1 * c1.x);
        }
      }
    }
  }

  // ---- 2. Hadamard: y = bf16(bf16(H x) * D^-0.5) ----
  if (hadamard) {
    // stage h = 1 inside the lane, then h = 2 .. 64 across lanes (feature bit k <-> lane bit k-1)
    float s0 = e0 + e1, s1 = e0 - e1;
    e0 = s0;
    e1 = s1;
    static_for<6>([&](auto k) {
      constexpr int m = 1 << decltype(k)::value;  // lane mask of feature stride 2m
      const float o0 = lane_swap<m>(e0), o1 = lane_swap<m>(e1);
      const bool upper = lane & m;
      e0 = upper ? o0 - e0 : e0 + o0;
      e1 = upper ? o1 - e1 : e1 + o1;
    });
    const float sc = 0.08838834764831845f;  // 128^-0.5 rounded to fp32
    e0 = round_bf16(round_bf16(e0) * sc);
    e1 = round_bf16(round_bf16(e1) * sc);
  }
  if (y) reinterpret_cast<uint32_t*>(y + v * kD)[lane] = pack_bf16x2(e0, e1);

  // ---- 3. fp8-e4m3 with a per-row scale ----
  if (q8) {
    float amax = fmaxf(fabsf(e0), fabsf(e1));
    if (e0 != e0 || e1 != e1) amax = __int_as_float(0x7fc00000);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float o = __shfl_xor(amax, m, 64);
      amax = (o > amax || o != o) ? o : amax;
    }
    float s = amax / 448.0f;
    s = s < 1e-12f ? 1e-12f : s;  // (keeps NaN)
    const uint32_t b0 = e4m3fn_rne(e0 / s), b1 = e4m3fn_rne(e1 / s);
    reinterpret_cast<uint16_t*>(q8 + v * kD)[lane] = (uint16_t)(b0 | (b1 << 8));
    if (lane == 0 && scale) scale[v] = s;
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
  if (rope_dim < 0 || rope_dim % 4 != 0 || rope_start < 0 || rope_start % 2 != 0 || rope_start + rope_dim > kD)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: rope features [%lld, %lld) (need rope_dim a multiple "
                     "of 4 inside [0, 128) starting at an even feature)", (long long)rope_start,
                     (long long)(rope_start + rope_dim));
  if (rope_dim > 0 && (!rope_cs || n_pos <= 0))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: RoPE needs the cos/sin table");
  const int64_t vecs = rows * heads;
  if (vecs == 0) return DSA_OK;
  const int64_t grid = (vecs * 64 + kThreads - 1) / kThreads;
  if (grid > INT32_MAX) return set_error(DSA_ERR_INVALID_ARG, "dsa_indexer_prep: too many rows");
  indexer_prep_kernel<<<(unsigned)grid, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, (uint16_t*)y, q8, scale, vecs, (int)heads, seq_len, rope_cs, n_pos, positions, pos_offset,
      (int)rope_dim, (int)rope_start, interleaved ? 1 : 0, hadamard ? 1 : 0);
  return check_launch("dsa_indexer_prep");
}
