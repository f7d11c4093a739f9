// Shared device/host helpers for the DSA HIP kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "dsa_mi355x.h"

namespace dsa {

// ----- vector types used as MFMA operands -----
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ----- error plumbing (host) -----
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// per-row top-k (topk.hip): dsa_topk with an optional candidate workspace of
// topk_cand_bytes(batch * s_q, k) bytes, which rows longer than 16384 keys use to select
// from one read of their scores
// With ``win`` (device int32 [2 * win_rows]: each row's first valid key, then the end of its
// window, the layout indexer_fwd_tnd writes) row r's valid prefix is win[win_rows + r] -
// win[r] instead of the causal rule.
int topk_rows(const float* scores, int32_t* indices, float* values, int64_t batch, int64_t s_q, int64_t s_k,
              int64_t ld_scores, int64_t k, int64_t q_offset, int64_t cmp_ratio, int64_t index_offset, void* cand_ws,
              void* stream, const int* win = nullptr, int64_t win_rows = 0);
int64_t topk_cand_bytes(int64_t rows, int64_t k);

// ----- lightning-indexer scores shared by the entry points (host) -----
// dsa_indexer_fwd_ws's work; fill_masked = false leaves the key spans that lie past every
// query's causal frontier of a tile unwritten (for consumers that read only each row's
// valid prefix t < (s + q_offset + 1) / cmp_ratio, such as dsa_topk).
int indexer_fwd(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                float* scores, int dtype, int64_t batch, int64_t s_q, int64_t s_k, int64_t n_heads,
                int64_t head_dim, int64_t ld_scores, int64_t q_offset, int64_t cmp_ratio, void* workspace,
                int64_t workspace_bytes, void* stream, bool fill_masked);

// Packed rows with their key windows on the device (indexer_tile_kernel's kTnd mode): the
// tiling of the tile kernel that dsa_indexer_fwd would run for this shape (query rows per
// group, keys per span; false if the shape has no tile kernel), and the scores of ``rows``
// rows from the geometry array ``tnd`` of ``ngroups`` groups (layout in indexer.hip).
bool indexer_tnd_tiling(int dtype, int64_t n_heads, int64_t head_dim, int* group_rows, int* span_keys);
int indexer_fwd_tnd(const void* q, const float* q_scale, const void* k, const float* k_scale, const float* w,
                    float* scores, int dtype, int64_t rows, int64_t s_k, int64_t n_heads, int64_t head_dim,
                    int64_t ld_scores, const int* tnd, int64_t ngroups, void* workspace, int64_t workspace_bytes,
                    void* stream);

// ----- optional per-kernel timing (host) -----
// While dsa_kernel_timing(1) is in force, a TimedLaunch scope around a kernel launch
// records a HIP event before and after it on the launch stream; dsa_kernel_timing_get
// sums the elapsed times per kernel name.  Off (no event calls) by default.
bool kernel_timing_on();
void kernel_timing_begin(hipStream_t st, hipEvent_t* ev);
void kernel_timing_end(const char* name, hipStream_t st, hipEvent_t* ev);
struct TimedLaunch {
  const char* name;
  hipStream_t st;
  hipEvent_t ev[2] = {nullptr, nullptr};
  TimedLaunch(const char* n, hipStream_t s) : name(n), st(s) {
    if (kernel_timing_on()) kernel_timing_begin(st, ev);
  }
  ~TimedLaunch() {
    if (ev[0]) kernel_timing_end(name, st, ev);
  }
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;
};

// Row of a one-workgroup-per-row launch: the rows in descending order.  Workgroups are
// dispatched in id order and a causal row's work grows with its token, so the longest
// rows start first and the short ones fill the CUs that finish early, instead of the last
// long rows running alone at the end.  Rows are independent, so results do not change.
// (The gather kernels keep the ascending order: in this one the forward and the score
// gradient kernel ran 1-1.5 % slower.)
__device__ __forceinline__ int launch_row() { return (int)(gridDim.x - 1u - blockIdx.x); }

// ----- bf16 helpers -----
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// LDS addressing through pointers (not integers): constant offsets added to an
// address-space-3 pointer fold into the ds_read offset field, integer arithmetic does not.
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4_ptr_t;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_ptr_t;
__device__ __forceinline__ lds_char* lds_bytes(void* generic_lds_ptr) {
  return (lds_char*)(uint32_t)(uintptr_t)generic_lds_ptr;
}
__device__ __forceinline__ u32x4 lds_read16(const lds_char* p) { return *(const lds_u32x4_ptr_t*)p; }
// transposed 4 x 16-bit reads of two row groups, packed as the 8 bf16 of an MFMA operand
__device__ __forceinline__ u32x4 lds_read_tr_pair(const lds_char* p1, const lds_char* p2) {
  const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr_t*)p1);
  const i16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr_t*)p2);
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 w1 = __builtin_bit_cast(u32x2, v1);
  const u32x2 w2 = __builtin_bit_cast(u32x2, v2);
  return (u32x4){w1[0], w1[1], w2[0], w2[1]};
}

// exchanges with the lane 16 / 32 apart without the LDS path (gfx950 v_permlane*_swap):
// the swap returns (own, partner) in some order, so a commutative op of the pair is the
// xor-reduction step
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fp32 -> OCP e4m3fn byte, round to nearest even
__device__ __forceinline__ uint32_t e4m3fn_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sgn = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return sgn | 0x7fu;  // inf, NaN
  uint32_t enc;
  if (a < 0x3c800000u) {
    // below 2^-6: multiples of 2^-9 (the scaling is exact); 8 encodes 2^-6 itself
    enc = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t mant = a & 0x7fffffu;
    enc = (((a >> 23) - 120u) << 3) | (mant >> 20);  // exponent rebiased 127 -> 7, 3 mantissa bits
    const uint32_t rest = mant & 0xfffffu;
    enc += (rest > 0x80000u) || (rest == 0x80000u && (enc & 1u));  // carries into the exponent
  }
  return sgn | (enc > 0x7eu ? 0x7fu : enc);
}

// relu as one integer max on the bit pattern (negative floats, -0 included, have the sign
// bit set and compare below 0): a float max would add a canonicalising max per operand in
// IEEE mode.  +NaN passes through like torch.relu.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// value of the lane whose index differs in bit 0..3 (mask 1, 2, 4, 8), through DPP moves
// (VALU, no LDS round trip): quad_perm [1,0,3,2] and [2,3,0,1]; xor 4 = half-row mirror
// (i -> 7 - i) then quad_perm [3,2,1,0]; xor 8 = rotate the 16-lane row by 8
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}
template <int kMask>
__device__ __forceinline__ float lane_xor(float x) {
  static_assert(kMask == 1 || kMask == 2 || kMask == 4 || kMask == 8, "DPP lane exchange within 16-lane rows");
  if constexpr (kMask == 1) return dpp_mov<0xB1>(x);
  else if constexpr (kMask == 2) return dpp_mov<0x4E>(x);
  else if constexpr (kMask == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(x));
  else return dpp_mov<0x128>(x);
}

// wave-level helpers (64-wide)
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// LDS chunk swizzles.  Conflict rules of gfx950's LDS, measured per instruction with the
// bank-conflict counter over full-wave address patterns (a group of lanes is served
// together and must hit distinct slots of the period; equal addresses broadcast):
//   ds_read_b128            4 groups of 16 lanes: each half-wave split by the parity of
//                           lane bits 2..4; 16-byte slots of a 256-byte period
//   ds_read_b64, ..._tr_b16 half-waves; 8-byte slots of a 256-byte period
//   ds_read_b32             half-waves; 4-byte slots of a 128-byte period
//   ds_write_b128           8-lane groups; 16-byte slots of a 128-byte period
//   ds_write_b64            16-lane groups; 8-byte slots of a 128-byte period
// Each swizzle below was chosen by exhaustive search over the linear (XOR) maps of the row
// bits against every access pattern of the kernels that use it.
//
// swz8: 16-byte chunk c of row r lives at chunk c ^ swz8(r); any 8 consecutive rows get
// distinct values.
__device__ __forceinline__ int swz8(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }
// swz_kv: tiles of 1152-byte latent-KV rows (72 chunks; rows alternate between the two
// 128-byte halves of the period): row bits 1, 2, 3 reversed, so the A-operand b128 reads
// of one chunk column by 32 rows and the transposed b64 reads of 4 rows x 4 chunks are
// conflict-free.  Values are < 8, so XOR keeps a chunk inside its aligned group of 8 and
// commutes with the kernels' +8-chunk offsets; it ignores row bit 4.  (On 1024-byte rows
// the b128 reads keep a 2-way conflict: a 16-row read group needs 16 distinct values.)
__device__ __forceinline__ int swz_kv(int r) { return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// swz_a16: the same 1152-byte KV rows read as A operands of v_mfma_f32_16x16x32 (16-lane
// group g reads chunk 4s + g of rows 16x + 0..15): row bits 1, 2 kept in place, which makes
// those b128 reads conflict-free; values < 8 as for swz_kv.
__device__ __forceinline__ int swz_a16(int r) { return r & 6; }
// swz16: for rows whose stride is a multiple of 256 B with >= 16 chunks: 16 consecutive
// rows reading one chunk column hit 16 distinct 16-byte slots.
__device__ __forceinline__ int swz16(int r) { return r & 15; }
// swz_kl: 256-byte rows of 16 chunks read both ways (the indexer KL key tile and q): b128
// reads of one chunk column (4c + lane / 16) by 16 consecutive rows, and transposed b64
// reads of rows 8g + 0..3 (+4) by the two lane quarters of a half-wave.
__device__ __forceinline__ int swz_kl(int r) { return ((r & 7) << 1) ^ (((r >> 3) & 1) * 9); }

// 16-byte-per-lane DMA from global memory straight into LDS (global_load_lds_dwordx4):
// lane i reads gbase + voff and writes LDS byte lds_base + 16 i.  gbase and lds_base must
// be wave-uniform.  Issued from inline assembly on purpose: the compiler then does not
// treat every later LDS read as dependent on the DMA (it would otherwise wait for all DMAs
// in flight before each ds_read), so the caller must wait for completion itself
// (s_waitcnt vmcnt) before reading the destination.  The LDS address travels in M0, bound
// by the "{m0}" operand constraint, so the compiler itself writes M0 and knows its value.
__device__ __forceinline__ void dma16_to_lds(const void* gbase, uint32_t voff, uint32_t lds_base) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(gbase), "{m0}"(m0v) : "memory");
}
// 4-byte-per-lane variant: lane i writes LDS byte lds_base + 4 i.
__device__ __forceinline__ void dma4_to_lds(const void* gbase, uint32_t voff, uint32_t lds_base) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(gbase), "{m0}"(m0v) : "memory");
}

// compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1, expanded by the
// front end (a large "#pragma unroll" body may be left rolled by the optimizer, which turns
// register arrays indexed by the loop variable into scratch memory)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

inline unsigned ceil_div(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// ----- packed ("TND") batches with device cu_seqlens -----
// Row s of a packed batch belongs to sequence i with cu_q[i] <= s < cu_q[i+1]; its keys are
// the sequence's [cu_k[i], cu_k[i+1]) and, under sparse_mode 3, the first
// (s - cu_q[i] + off + 1) / cmp_ratio of them with off = max(0, cmp_ratio * len_k +
// residual - len_q) (the bottom-right causal rule of one sequence, as the host schedule
// applies it per sequence).  Everything is clamped into [0, t_k) so that garbage lengths
// cannot address outside the key tensor.
__device__ __forceinline__ void tnd_row_window(const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                                               const int32_t* __restrict__ res, int n_seq, int64_t s, int cmp_ratio,
                                               bool causal, int t_k, int& first, int& end) {
  int lo = 0, hi = n_seq - 1;  // the last sequence whose start is <= s
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu_q[mid] <= s) lo = mid;
    else hi = mid - 1;
  }
  const int64_t q0 = cu_q[lo], q1 = cu_q[lo + 1];
  const int64_t k0 = min<int64_t>(max<int64_t>(cu_k[lo], 0), t_k);
  const int64_t lk = min<int64_t>(max<int64_t>((int64_t)cu_k[lo + 1] - k0, 0), t_k - k0);
  int64_t nv = 0;
  if (s >= q0 && s < q1) {
    const int64_t r = res ? max<int64_t>(res[lo], 0) : 0;
    const int64_t off = causal ? max<int64_t>(0, cmp_ratio * lk + r - (q1 - q0)) : ((int64_t)1 << 40);
    nv = min<int64_t>(max<int64_t>((s - q0 + off + 1) / cmp_ratio, 0), lk);
  }
  first = (int)k0;
  end = (int)(k0 + nv);
}


}  // namespace dsa
