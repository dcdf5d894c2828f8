// common.h - device helpers shared by the gfx950 kernels.
//
// Wave64 reductions, fp16 conversion, and the Q8_0 activation quantiser used
// in GEMV prologues and epilogues.  All code is written for CDNA4 (gfx950):
// 64-lane wavefronts, v_dot4 integer dot products, 160 KB LDS per CU.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define LLMRS_WAVE 64

namespace llmrs {

__device__ __forceinline__ int lane_id() { return threadIdx.x & (LLMRS_WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / LLMRS_WAVE; }

// Butterfly sums / maxima over `width` lanes (power of two, <= 64).
template <int W = LLMRS_WAVE>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, W);
  return v;
}
template <int W = LLMRS_WAVE>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, W);
  return v;
}
template <int W = LLMRS_WAVE>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, W));
  return v;
}

// Wave64 sum with DPP row operations (quad_perm, half-row mirror, row
// mirror) and the four row totals added in lane order 0, 16, 32, 48.  The
// result is uniform across the wave; the summation order is fixed, so equal
// inputs give bit-equal sums.
template <int CTRL>
__device__ __forceinline__ float dpp_c(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_c<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_c<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_c<0x141>(v);  // row_half_mirror
  v = v + dpp_c<0x140>(v);  // row_mirror: every lane holds its row's sum
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return ((r0 + r1) + r2) + r3;
}
// Maximum over each 16-lane row (quad exchanges, then the half-row and row
// mirrors); every lane of the row holds the result.
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dpp_c<0xB1>(v));
  v = fmaxf(v, dpp_c<0x4E>(v));
  v = fmaxf(v, dpp_c<0x141>(v));
  return fmaxf(v, dpp_c<0x140>(v));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_c<0xB1>(v));
  v = fmaxf(v, dpp_c<0x4E>(v));
  v = fmaxf(v, dpp_c<0x141>(v));
  v = fmaxf(v, dpp_c<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The value held by lane l ^ 32 (l ^ 16): with both operands v, gfx950's
// v_permlane32_swap (v_permlane16_swap) returns the lower and the upper half
// (the even and the odd 16-lane row) of v side by side, in VALU time rather
// than an LDS permute's round trip.
__device__ __forceinline__ float xor32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(lane_id() < 32 ? p[1] : p[0]);
}
__device__ __forceinline__ float xor16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane_id() & 16) ? p[0] : p[1]);
}

__device__ __forceinline__ float h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
// a * (float)h, rounded once as the f32 product, for the f16 h in the low
// (high) half of w: the mixed-precision FMA with an addend of -0, whose sum
// with the exact product is the product itself (sign of zero included).
// One instruction instead of a conversion and a multiply; equal to them bit
// for bit on gfx950 for every f16 pattern in either half against 8192 f32
// values (signed zeros, denormals, infinities, NaNs, random bit patterns).
// An addend of +0 would turn a -0 product into +0.
__device__ __forceinline__ float mul_f16lo(float a, unsigned w) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[0,1,0]" : "=v"(d) : "v"(a), "v"(w));
  return d;
}
__device__ __forceinline__ float mul_f16hi(float a, unsigned w) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(d) : "v"(a), "v"(w));
  return d;
}
// IEEE binary16 round-to-nearest-even.
__device__ __forceinline__ uint16_t f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// One Q8_0 code for x with inverse scale inv (cpu.rs:736-740):
// round-half-away-from-zero, clamp to [-127, 127], NaN -> 0.  The rounding
// is trunc(p + copysign(0.5 - 2^-25, p)): three instructions instead of the
// six of roundf, and equal to roundf for every non-NaN float (checked
// exhaustively over all 2^32 bit patterns; 0.5 - 2^-25 keeps p = 0.5 - 2^-25
// from rounding up, and the sum of a half-integer and it rounds away from
// zero).  The NaN case is a select, not a branch.
__device__ __forceinline__ int q8_code(float x, float inv) {
  const float p = x * inv;
  float r = __builtin_truncf(p + __builtin_copysignf(0.49999997f, p));
  r = fminf(127.0f, fmaxf(-127.0f, r));
  return p != p ? 0 : (int)r;  // Rust's `NaN as i8` is 0
}

// Quantise 32 values held one per lane of a 32-lane group (lanes with the
// same lane_id()/32).  Returns this lane's code, writes the group's scale to
// *d_out (the same value in every lane of the group).  Follows
// quantize_row_q8_0 (cpu.rs:724-743): d = amax/127, inv = 1/d; the amax fold
// starts at 0 and ignores NaN, as fmaxf does.
__device__ __forceinline__ int q8_group32(float x, float* d_out) {
  float amax = fmaxf(0.0f, group_max<32>(fabsf(x)));
  if (amax == 0.0f) {
    *d_out = 0.0f;
    return 0;
  }
  float d = amax / 127.0f;
  float inv = 1.0f / d;
  *d_out = d;
  return q8_code(x, inv);
}

// ---- device-coherent memory operations ---------------------------------
// Data produced and consumed inside one launch by workgroups on different
// XCDs (the fused layer launches, the attention combine) moves with device-scope (sc1) buffer
// loads and stores: they bypass the per-XCD L2 copies, so no L2 write-back
// or invalidate is needed at barriers.  The base must be wave-uniform; the
// descriptor covers 2 GiB from it.
typedef unsigned int dev_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // buffer cache-policy bit for device scope on gfx950
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ float dev_ldf(const void* base, int byte_off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(base), byte_off, 0, kSc1));
}
__device__ __forceinline__ unsigned dev_ldu(const void* base, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(base), byte_off, 0, kSc1);
}
typedef unsigned int dev_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ dev_u32x2 dev_ld8(const void* base, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ dev_u32x4 dev_ld16(const void* base, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ void dev_stf(void* base, int byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ void dev_stu(void* base, int byte_off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ void dev_st16(void* base, int byte_off, dev_u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, dev_rsrc(base), byte_off, 0, kSc1);
}
// XCD-local exchange between workgroups on one XCD: stores land in its L2
// (the vector L1 writes through), loads skip the L1 (sc0) and read the L2.
constexpr int kSc0 = 1;
__device__ __forceinline__ void xcd_st16(void* base, int byte_off, dev_u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, dev_rsrc(base), byte_off, 0, 0);
}
__device__ __forceinline__ void xcd_stu(void* base, int byte_off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, dev_rsrc(base), byte_off, 0, 0);
}
__device__ __forceinline__ dev_u32x4 xcd_ld16(const void* base, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(dev_rsrc(base), byte_off, 0, kSc0);
}
// A descriptor whose record count ends `bytes` past `base` (wave-uniform):
// loads at or beyond it read zero with no memory access (buffer range
// checking), so a loop over a variable number of items needs no per-load
// select.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ dev_u32x2 xcd_ld8(const void* base, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(dev_rsrc(base), byte_off, 0, kSc0);
}
__device__ __forceinline__ float xcd_ldf(const void* base, int byte_off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(base), byte_off, 0, kSc0));
}
__device__ __forceinline__ void dev_st8(void* base, int byte_off, int8_t v) {
  __builtin_amdgcn_raw_buffer_store_b8((unsigned char)v, dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ void dev_st_u16(void* base, int byte_off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, dev_rsrc(base), byte_off, 0, kSc1);
}

// f32 activation element, plain or device-scope.
template <bool DEV>
__device__ __forceinline__ float ld_act(const float* base, size_t idx) {
  if (DEV) return dev_ldf(base, (int)(idx * 4));
  return base[idx];
}
template <bool DEV>
__device__ __forceinline__ void st_act(float* base, size_t idx, float v) {
  if (DEV) dev_stf(base, (int)(idx * 4), v);
  else base[idx] = v;
}

// Packed 4 x int8 dot product with int32 accumulation (v_dot4c_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

}  // namespace llmrs
