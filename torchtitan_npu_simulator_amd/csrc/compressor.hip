// Block KV compressor (DeepSeek-V4): softmax-gated pooling of ratio-token blocks.
//
// out[b, c, f] = sum_i softmax_i(g_i) x_i over the block's slots, where slot i of block c
//   without overlap: x = kv[b, c*r + i, f],        g = score[b, c*r + i, f] + ape[i, f]
//   with overlap (coff = 2), 2r slots: i < r  -> previous block's features 0..D
//                   x = kv[b, (c-1)*r + i, f],     g = score[...] + ape[i, f]   (absent for c = 0)
//                                       i >= r -> current block's features D..2D
//                   x = kv[b, c*r + i-r, D + f],   g = score[...] + ape[i-r, D + f]
// then optionally RMSNorm over f of the bf16-rounded pooled row times norm_weight, and
// optionally RoPE on the last rope_dim features (interleaved pairs (2i, 2i+1), angle i at
// the block's position, in fp32 on the row as stored: bf16-rounded when the output is
// bf16), as Compressor._forward_bsnd / _forward_tnd apply it after the norm.  The block's
// position is that of its first token: c * ratio, or positions[first token] when token
// positions are given (rows whose position falls outside the cos/sin table keep their
// features).
//
// Packed varlen ("TND") batches give each block's first token explicitly (block_starts,
// whole r-token blocks inside one request): block c pools tokens block_starts[c] + i, and
// with overlap its first r slots come from the previous listed block, block_starts[c-1],
// when c > 0 and the block's position (positions[block_starts[c]]) is at least r.
//
// HBM-bound streaming: a row group of D/4 lanes owns one compressed block, each lane four
// consecutive features (16-byte loads, coalesced along the row); a 256-lane workgroup
// holds 256 / (D/4) row groups.  Each input row is read once per block that uses it (the
// overlap re-read of the previous block's first half comes from L2).  The softmax is
// computed online per feature in fp32 with expf.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
compressor_kernel(const float* __restrict__ kv, const float* __restrict__ score, const float* __restrict__ ape,
                  const float* __restrict__ norm_w, void* __restrict__ out, int out_bf16, int64_t n_blocks_total,
                  int nb, int D, int r, int overlap, float eps, const int64_t* __restrict__ block_starts,
                  const int32_t* __restrict__ positions, int64_t n_tokens, const float* __restrict__ rope_cs,
                  int64_t n_pos, int rope_dim) {
  extern __shared__ float red[];  // [row groups][lanes_per_group / 64 + 1]
  const int lanes = D / 4;        // lanes per row group
  const int groups = kThreads / lanes;
  const int g = threadIdx.x / lanes, l = threadIdx.x - g * lanes;
  const int64_t blk = (int64_t)blockIdx.x * groups + g;
  const bool active = blk < n_blocks_total;  // D is a power of two: groups tile the workgroup
  const int64_t b = active ? blk / nb : 0;
  const int c = active ? (int)(blk - b * nb) : 0;
  const int coff = overlap ? 2 : 1;
  const int64_t row_elems = (int64_t)coff * D;
  const int f = 4 * l;

  float m[4], s[4], acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    m[u] = -INFINITY;
    s[u] = 0.f;
    acc[u] = 0.f;
  }
  auto consume = [&](const float* xrow, const float* grow, const float* arow) {
    const float4 x = *reinterpret_cast<const float4*>(xrow);
    const float4 gg = *reinterpret_cast<const float4*>(grow);
    const float4 a = *reinterpret_cast<const float4*>(arow);
    const float xv[4] = {x.x, x.y, x.z, x.w};
    const float gv[4] = {gg.x + a.x, gg.y + a.y, gg.z + a.z, gg.w + a.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float mn = fmaxf(m[u], gv[u]);
      const float sc = expf(m[u] - mn);  // 0 on the first slot (m = -inf)
      const float e = expf(gv[u] - mn);
      s[u] = s[u] * sc + e;
      acc[u] = acc[u] * sc + e * xv[u];
      m[u] = mn;
    }
  };
  // first token of the block and of the block whose first half overlaps it
  int64_t cur = 0, prev = 0;
  bool has_prev = false, usable = active;
  if (active) {
    if (block_starts) {
      cur = block_starts[c];
      usable = cur >= 0 && cur <= n_tokens - r;  // out-of-range starts pool nothing
      if (usable && overlap && c > 0 && positions[cur] >= r) {
        prev = block_starts[c - 1];
        has_prev = prev >= 0 && prev <= n_tokens - r;
      }
    } else {
      cur = b * (int64_t)nb * r + (int64_t)c * r;
      prev = cur - r;
      has_prev = overlap && c > 0;
    }
  }
  if (usable) {
    if (has_prev) {
      for (int i = 0; i < r; ++i) {
        const int64_t row = (prev + i) * row_elems;
        consume(kv + row + f, score + row + f, ape + (int64_t)i * row_elems + f);
      }
    }
    const int off = overlap ? D : 0;
    for (int i = 0; i < r; ++i) {
      const int64_t row = (cur + i) * row_elems;
      consume(kv + row + off + f, score + row + off + f, ape + (int64_t)i * row_elems + off + f);
    }
  }
  float pooled[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) pooled[u] = s[u] > 0.f ? acc[u] / s[u] : 0.f;

  if (norm_w) {
    // RMSNorm of the bf16-rounded pooled row (fp32 arithmetic)
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pooled[u] = bf16_to_f(f_to_bf16(pooled[u]));
      ss += pooled[u] * pooled[u];
    }
    // reduce over the row group's lanes: wave-level then across waves of the group
    const int wpg = (lanes + 63) / 64;  // waves per row group (a group of < 64 lanes sits inside one wave)
    if (lanes >= 64) {
      ss = wave_sum(ss);
      const int w_in_g = l / 64;
      if ((l & 63) == 0) red[g * (wpg + 1) + w_in_g] = ss;
      __syncthreads();
      float t = 0.f;
      for (int w = 0; w < wpg; ++w) t += red[g * (wpg + 1) + w];
      ss = t;
    } else {
      for (int mk = lanes >> 1; mk >= 1; mk >>= 1) ss += __shfl_xor(ss, mk, 64);
    }
    const float inv = rsqrtf(ss / (float)D + eps);
    const float4 w4 = *reinterpret_cast<const float4*>(norm_w + f);
    pooled[0] *= inv * w4.x;
    pooled[1] *= inv * w4.y;
    pooled[2] *= inv * w4.z;
    pooled[3] *= inv * w4.w;
  }
  if (rope_cs && usable && f >= D - rope_dim) {
    // RoPE of the stored row: this lane's features are the pairs (f, f+1), (f+2, f+3)
    const int64_t pos = positions ? (int64_t)positions[cur] : (int64_t)c * r;
    if (pos >= 0 && pos < n_pos) {
      if (out_bf16)
#pragma unroll
        for (int u = 0; u < 4; ++u) pooled[u] = bf16_to_f(f_to_bf16(pooled[u]));
      const float4 cs4 = *reinterpret_cast<const float4*>(rope_cs + pos * rope_dim + (f - (D - rope_dim)));
      const float a0 = pooled[0], b0 = pooled[1], a1 = pooled[2], b1 = pooled[3];
      pooled[0] = a0 * cs4.x - b0 * cs4.y;
      pooled[1] = a0 * cs4.y + b0 * cs4.x;
      pooled[2] = a1 * cs4.z - b1 * cs4.w;
      pooled[3] = a1 * cs4.w + b1 * cs4.z;
    }
  }
  if (!active) return;
  const int64_t o = blk * (int64_t)D + f;
  if (out_bf16) {
    uint2 v;
    v.x = pack_bf16x2(pooled[0], pooled[1]);
    v.y = pack_bf16x2(pooled[2], pooled[3]);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = v;
  } else {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + o) =
        make_float4(pooled[0], pooled[1], pooled[2], pooled[3]);
  }
}

}  // namespace
}  // namespace dsa

namespace dsa {
namespace {
int check_rope(const char* what, const float* rope_cs, int64_t n_pos, int64_t rope_dim, int64_t d) {
  if (!rope_cs) return DSA_OK;
  if (rope_dim <= 0 || rope_dim % 4 != 0 || rope_dim > d || n_pos <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "%s: rope_dim=%lld with %lld positions (needs a multiple of 4 <= D)", what,
                     (long long)rope_dim, (long long)n_pos);
  return DSA_OK;
}
}  // namespace
}  // namespace dsa

extern "C" int dsa_compressor_fwd(const float* kv, const float* score, const float* ape, const float* norm_weight,
                                  void* out, int out_dtype, int64_t batch, int64_t s, int64_t d, int64_t ratio,
                                  int overlap, float norm_eps, const float* rope_cs, int64_t n_pos, int64_t rope_dim,
                                  const int32_t* positions, void* stream) {
  using namespace dsa;
  if (!kv || !score || !ape || !out) return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd: null pointer");
  if (int rc = check_rope("dsa_compressor_fwd", rope_cs, n_pos, rope_dim, d)) return rc;
  if (batch <= 0 || s <= 0 || d <= 0 || ratio <= 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd: bad sizes");
  if (s % ratio != 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd: seqlen (%lld) must be divisible by ratio (%lld)",
                     (long long)s, (long long)ratio);
  if (d < 4 || d > 4 * kThreads || (d & (d - 1)) != 0)  // row groups tile the workgroup exactly
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd: D=%lld (needs a power of two in [4, 1024])",
                     (long long)d);
  if (out_dtype != DSA_F32 && out_dtype != DSA_BF16)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd: out dtype %d", out_dtype);
  const int64_t nb = s / ratio;
  if (nb > INT32_MAX || ratio > 65536) return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd: sizes out of range");
  const int lanes = (int)(d / 4);
  const int groups = kThreads / lanes;
  const int64_t total = batch * nb;
  const int64_t grid = (total + groups - 1) / groups;
  if (grid > INT32_MAX) return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd: too many blocks");
  const size_t shm = (size_t)groups * ((lanes + 63) / 64 + 1) * sizeof(float);
  const TimedLaunch tl("compressor_kernel", (hipStream_t)stream);
  compressor_kernel<<<(unsigned)grid, kThreads, shm, (hipStream_t)stream>>>(
      kv, score, ape, norm_weight, out, out_dtype == DSA_BF16, total, (int)nb, (int)d, (int)ratio, overlap ? 1 : 0,
      norm_eps, nullptr, positions, batch * s, rope_cs, n_pos, (int)rope_dim);
  return check_launch("dsa_compressor_fwd");
}

extern "C" int dsa_compressor_fwd_tnd(const float* kv, const float* score, const float* ape,
                                      const float* norm_weight, void* out, int out_dtype, int64_t n_tokens, int64_t d,
                                      int64_t ratio, int overlap, const int64_t* block_starts, int64_t n_blocks,
                                      const int32_t* positions, float norm_eps, const float* rope_cs, int64_t n_pos,
                                      int64_t rope_dim, void* stream) {
  using namespace dsa;
  if (!kv || !score || !ape || !out || (n_blocks > 0 && !block_starts))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd_tnd: null pointer");
  if (int rc = check_rope("dsa_compressor_fwd_tnd", rope_cs, n_pos, rope_dim, d)) return rc;
  if (rope_cs && !positions)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd_tnd: RoPE needs the token positions");
  if (overlap && !positions)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd_tnd: overlap needs the token positions");
  if (n_tokens <= 0 || d <= 0 || ratio <= 0 || n_blocks < 0)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd_tnd: bad sizes");
  if (d < 4 || d > 4 * kThreads || (d & (d - 1)) != 0)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd_tnd: D=%lld (needs a power of two in [4, 1024])",
                     (long long)d);
  if (out_dtype != DSA_F32 && out_dtype != DSA_BF16)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd_tnd: out dtype %d", out_dtype);
  if (n_blocks > INT32_MAX || ratio > 65536)
    return set_error(DSA_ERR_INVALID_ARG, "dsa_compressor_fwd_tnd: sizes out of range");
  if (n_blocks == 0) return DSA_OK;
  const int lanes = (int)(d / 4);
  const int groups = kThreads / lanes;
  const int64_t grid = (n_blocks + groups - 1) / groups;
  const size_t shm = (size_t)groups * ((lanes + 63) / 64 + 1) * sizeof(float);
  const TimedLaunch tl("compressor_kernel", (hipStream_t)stream);
  compressor_kernel<<<(unsigned)grid, kThreads, shm, (hipStream_t)stream>>>(
      kv, score, ape, norm_weight, out, out_dtype == DSA_BF16, n_blocks, (int)n_blocks, (int)d, (int)ratio,
      overlap ? 1 : 0, norm_eps, block_starts, positions, n_tokens, rope_cs, n_pos, (int)rope_dim);
  return check_launch("dsa_compressor_fwd_tnd");
}
