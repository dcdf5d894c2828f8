// gemv_core.h - the batch-1 dequant-GEMV machinery of the decode GEMV
// kernels (gemv.hip).
//
// y[row] = sum_b isum_b(row) * (d_w[row,b] * d_a[b]) where isum_b is the exact
// int32 dot product of one 32-element block of weight codes with the Q8_0
// activation codes.  This is the reference CPU GEMV (cpu.rs:49-111,
// kernel_avx2 cpu.rs:888-941) with the block loop spread over the 64 lanes of
// a wavefront and the lane partials summed by a fixed DPP tree; isum_b is
// bit-exact, only the f32 summation order differs.
//
// Device weight layout (written by the host at upload): for an [n, k] matrix
// with nb = k/32 blocks per row, codes [n][nb][B] (B = 16 bytes for Q4_0:
// byte i = e[i] | e[i+16] << 4; B = 32 bytes for Q8_0), then scales [n][nb]
// (fp16, or f32 for the reference's Q4 storage).
//
// Work decomposition.  A "row group" is R consecutive rows; a "unit" is one
// row group times 64*U consecutive blocks: lane l of the wave owns blocks
// b = base + 64*u + l (u < U), so every weight load instruction of a wave
// reads 64 consecutive 16-byte blocks of one row (1 KB, fully coalesced).
// Waves walk their units in order, two units in flight: the weights of unit
// i+2 are requested right after unit i is consumed, and the first units are
// requested with the activation prologue, so HBM latency overlaps the
// prologue.  Row groups are dealt to the waves of `nwg`
// workgroups round-robin (whole 64-row tiles per workgroup for the SwiGLU
// epilogue, which needs matching gate and up rows).
//
// The activation vector is quantised once per workgroup into LDS (prologue):
//   PRO_QUANT  Q8_0 of an f32 row                     (matmul_transposed)
//   PRO_NORM   RMSNorm then Q8_0 of an f32 row
//   PRO_Q8     already-quantised codes from global      (O, down)
//   PRO_NQ     codes of RMSNorm(x) from the producer    (QKV, gate|up, lm_head):
//              Q8_0 codes of x*w with per-block scales d' = amax(x*w)/127 and
//              per-block sums of x^2; the prologue adds the sums, forms
//              s = 1/sqrt(ss/k + eps) and uses d = d' * s
// and each row group is finished in an epilogue:
//   EPI_STORE  y = acc
//   EPI_RESID  y = acc + res
//   EPI_SILU   gate|up rows interleaved in tiles of 32+32; m = silu(g)*u,
//              written as f32 and as Q8_0 codes for the down projection
//   EPI_ARGMAX logits plus a per-workgroup (max, index) partial (lm_head)
//   EPI_NQ     y = acc + res in tiles of 32 rows, then the PRO_NQ operand of
//              the next RMSNorm (weight norm_next): codes, d' and sum of y^2
//              per 32-row block (O + residual, down + residual)
//
// Why PRO_NQ / EPI_NQ: RMSNorm then Q8_0 (cpu.rs:381-389, 724-743) computes
// y = (x*s)*w, d = amax(y)/127, q = round(y/d).  The codes do not depend on
// the positive factor s (it scales y and d alike), so the producer, which
// holds x but not s (a sum over the whole vector), quantises x*w; the
// consumer applies s to the 32x fewer scales.  Only the rounding differs from
// the reference's order (a code moves only where x*w/d' sits within a few ulps
// of a rounding midpoint), and every consumer workgroup loads k + k/8 bytes
// instead of 8k bytes of f32 input and norm weights, with no quantiser
// arithmetic in its prologue.
// DEV = true moves the activations, results and partials with device-scope
// loads and stores (for a producer and consumer in one launch; the decode
// kernels use DEV = false).
#pragma once
#include "common.h"
#include "../kernel_args.h"

namespace llmrs {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { WT_Q4H = 0, WT_Q4F = 1, WT_Q8H = 2 };
enum { PRO_QUANT = 0, PRO_NORM = 1, PRO_Q8 = 2, PRO_NQ = 3 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_ARGMAX = 3, EPI_NQ = 4 };

// Waves per workgroup: 4, or 8 for a code object built with
// LLMRS_GEMV_WAVES=8 (gemv_w8.hip: the 32-row-tile producers, which run one
// workgroup per tile on half the CUs at the 8B width and need twice the
// loads in flight per CU).
#ifndef LLMRS_GEMV_WAVES
#define LLMRS_GEMV_WAVES 4
#endif
constexpr int kThreads = LLMRS_GEMV_WAVES * LLMRS_WAVE;
constexpr int kWaves = LLMRS_GEMV_WAVES;
constexpr int kSiluTile = 64;  // rows per SwiGLU tile: 32 gate + 32 up
constexpr int kNqTile = 32;    // rows per EPI_NQ tile: one Q8_0 block of y
// Rows per tile of the tiled epilogues (0: row groups dealt singly).
__host__ __device__ constexpr int epi_tile(int epi) {
  return epi == EPI_SILU ? kSiluTile : epi == EPI_NQ ? kNqTile : 0;
}

// Raw scale bits: the conversion happens at use, so a load never has to
// complete before the next one is issued.
template <int WT>
__device__ __forceinline__ unsigned load_wscale_raw(const void* ws, size_t i) {
  if (WT == WT_Q4F) return __builtin_nontemporal_load((const unsigned*)ws + i);
  return __builtin_nontemporal_load((const uint16_t*)ws + i);
}
template <int WT>
__device__ __forceinline__ float wscale(unsigned raw) {
  if (WT == WT_Q4F) return __uint_as_float(raw);
  return h2f((uint16_t)raw);
}

// Quantise the 32 values v[] of one block to Q8_0 (cpu.rs:724-743): amax
// from 0, d = amax/127, inv = 1/d, round-half-away, clamp to +-127.  Writes
// 8 packed dwords, the scale and (for Q4 weights) -8 * sum(codes).
template <bool Q4>
__device__ __forceinline__ void quant_block(const float* v, int blk, int8_t* s_q, float* s_d,
                                            int* s_off) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  int packed[8];
  int csum = 0;
  float d = 0.0f;
  if (amax == 0.0f) {
#pragma unroll
    for (int j = 0; j < 8; ++j) packed[j] = 0;
  } else {
    d = amax / 127.0f;
    const float inv = 1.0f / d;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      unsigned w = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = q8_code(v[4 * j + e], inv);
        csum += q;
        w |= ((unsigned)q & 0xFFu) << (8 * e);
      }
      packed[j] = (int)w;
    }
  }
  i32x4* dst = (i32x4*)(s_q + 32 * blk);
  dst[0] = i32x4{packed[0], packed[1], packed[2], packed[3]};
  dst[1] = i32x4{packed[4], packed[5], packed[6], packed[7]};
  s_d[blk] = d;
  if (Q4) s_off[blk] = -8 * csum;
}

// Q8_0 of one 32-element block held by 32/EPT adjacent lanes, EPT values
// each (lane t holds elements [t*EPT, (t+1)*EPT) of the row; block t*EPT/32).
// Same arithmetic as quant_block; the amax is combined across the lanes.
template <bool Q4, int EPT>
__device__ __forceinline__ void quant_part(const float* v, int t, int8_t* s_q, float* s_d, int* s_off) {
  constexpr int LPB = 32 / EPT;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < EPT; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int o = LPB / 2; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, LPB));
  int packed[EPT / 4];
  int csum = 0;
  float d = 0.0f;
  if (amax == 0.0f) {
#pragma unroll
    for (int j = 0; j < EPT / 4; ++j) packed[j] = 0;
  } else {
    d = amax / 127.0f;
    const float inv = 1.0f / d;
#pragma unroll
    for (int j = 0; j < EPT / 4; ++j) {
      unsigned w = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = q8_code(v[4 * j + e], inv);
        csum += q;
        w |= ((unsigned)q & 0xFFu) << (8 * e);
      }
      packed[j] = (int)w;
    }
  }
  int* dst = (int*)(s_q + EPT * t);
#pragma unroll
  for (int j = 0; j < EPT / 4; ++j) dst[j] = packed[j];
  if (Q4) {
#pragma unroll
    for (int o = LPB / 2; o > 0; o >>= 1) csum += __shfl_xor(csum, o, LPB);
  }
  if ((t % LPB) == 0) {
    const int blk = t / LPB;
    s_d[blk] = d;
    if (Q4) s_off[blk] = -8 * csum;
  }
}

template <bool DEV>
__device__ __forceinline__ f32x4 ld_act4(const float* base, size_t idx) {
  if (DEV) {
    const dev_u32x4 u = dev_ld16(base, (int)(idx * 4));
    return f32x4{__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
  }
  return *(const f32x4*)(base + idx);
}

// Prologue: the activation row as Q8_0 in LDS.  s_q holds the codes in
// natural order, s_d the block scales, s_off = -8 * sum(codes) per block (the
// Q4 offset: sum (q-8)*a = sum q*a - 8*sum a, with q in 0..15 read as int8).
// One thread per block; blocks beyond the workgroup size loop.
template <int PRO, bool Q4, bool DEV>
__device__ __forceinline__ void load_activation(const GemvArgs& a, int mrow, int8_t* s_q,
                                                float* s_d, int* s_off, float* s_red) {
  const int k = a.k, nb = k >> 5, tid = threadIdx.x;
  if (PRO == PRO_Q8 || PRO == PRO_NQ) {
    const int rb = mrow * nb;  // the row's first block (row-batched launches)
    float scale = 1.0f;
    if (PRO == PRO_NQ) {  // s from the per-block sums of squares
      float ss = 0.0f;
      for (int b = tid; b < nb; b += kThreads) ss = ss + ld_act<DEV>(a.xss, rb + b);
      ss = wave_sum(ss);
      if (lane_id() == 0) s_red[wave_id()] = ss;
      __syncthreads();
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) tot = tot + s_red[w];
      scale = 1.0f / sqrtf(tot / (float)k + a.eps);
    }
    for (int b = tid; b < nb; b += kThreads) {
      i32x4 c0, c1;
      if (DEV) {
        const dev_u32x4 u0 = dev_ld16(a.xq, 32 * (rb + b)), u1 = dev_ld16(a.xq, 32 * (rb + b) + 16);
        c0 = i32x4{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w};
        c1 = i32x4{(int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
      } else {
        const i32x4* src = (const i32x4*)(a.xq + 32 * ((size_t)rb + b));
        c0 = src[0];
        c1 = src[1];
      }
      i32x4* dst = (i32x4*)(s_q + 32 * b);
      dst[0] = c0;
      dst[1] = c1;
      s_d[b] = PRO == PRO_NQ ? ld_act<DEV>(a.xd, rb + b) * scale : ld_act<DEV>(a.xd, rb + b);
      if (Q4) {
        int s = 0;
        s = dot4(c0.x, 0x01010101, s);
        s = dot4(c0.y, 0x01010101, s);
        s = dot4(c0.z, 0x01010101, s);
        s = dot4(c0.w, 0x01010101, s);
        s = dot4(c1.x, 0x01010101, s);
        s = dot4(c1.y, 0x01010101, s);
        s = dot4(c1.z, 0x01010101, s);
        s = dot4(c1.w, 0x01010101, s);
        s_off[b] = -8 * s;
      }
    }
    return;
  }
  const size_t xrow = (size_t)mrow * k;
  if (nb <= kThreads) {
    // One block per thread: x is read once, kept in registers for both the
    // sum of squares and the quantisation.
    const int b = tid < nb ? tid : nb - 1;
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 t = ld_act4<DEV>(a.x, xrow + 32 * b + 4 * j);
      v[4 * j] = t.x;
      v[4 * j + 1] = t.y;
      v[4 * j + 2] = t.z;
      v[4 * j + 3] = t.w;
    }
    float scale = 1.0f;
    if (PRO == PRO_NORM) {
      // cpu.rs:381-383: ss = sum v*v; rms = sqrt(ss/n + eps); scale = 1/rms.
      float ss = 0.0f;
      if (tid < nb) {
#pragma unroll
        for (int i = 0; i < 32; ++i) ss = ss + v[i] * v[i];
      }
      ss = wave_sum(ss);
      if (lane_id() == 0) s_red[wave_id()] = ss;
      __syncthreads();
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) tot = tot + s_red[w];
      const float rms = sqrtf(tot / (float)k + a.eps);
      scale = 1.0f / rms;
      const f32x4* wsrc = (const f32x4*)(a.norm_w + 32 * b);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4 t = wsrc[j];
        v[4 * j] = v[4 * j] * scale * t.x;  // cpu.rs:389: x * s * w
        v[4 * j + 1] = v[4 * j + 1] * scale * t.y;
        v[4 * j + 2] = v[4 * j + 2] * scale * t.z;
        v[4 * j + 3] = v[4 * j + 3] * scale * t.w;
      }
    }
    if (tid < nb) quant_block<Q4>(v, b, s_q, s_d, s_off);
    return;
  }
  float scale = 1.0f;
  if (PRO == PRO_NORM) {
    // cpu.rs:381-383: ss = sum v*v; rms = sqrt(ss/n + eps); scale = 1/rms.
    float ss = 0.0f;
    for (int b = tid; b < nb; b += kThreads) {
      f32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = ld_act4<DEV>(a.x, xrow + 32 * b + 4 * j);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        ss = ss + v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) s_red[wave_id()] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot = tot + s_red[w];
    const float rms = sqrtf(tot / (float)k + a.eps);
    scale = 1.0f / rms;
  }
  for (int b = tid; b < nb; b += kThreads) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 t = ld_act4<DEV>(a.x, xrow + 32 * b + 4 * j);
      v[4 * j] = t.x;
      v[4 * j + 1] = t.y;
      v[4 * j + 2] = t.z;
      v[4 * j + 3] = t.w;
    }
    if (PRO == PRO_NORM) {
      const f32x4* wsrc = (const f32x4*)(a.norm_w + 32 * b);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4 t = wsrc[j];
        v[4 * j] = v[4 * j] * scale * t.x;  // cpu.rs:389: x * s * w
        v[4 * j + 1] = v[4 * j + 1] * scale * t.y;
        v[4 * j + 2] = v[4 * j + 2] * scale * t.z;
        v[4 * j + 3] = v[4 * j + 3] * scale * t.w;
      }
    }
    quant_block<Q4>(v, b, s_q, s_d, s_off);
  }
}

// The prologue in two halves: issue_activation() requests this thread's
// activation values (and RMSNorm weights) into registers, finish_activation()
// turns them into the LDS operand.  gemv_body issues them BEFORE the weight
// prefetch: a wave's loads complete in issue order, so activation loads
// issued after the prefetch could only be used once every prefetched weight
// had arrived, and no further weight loads would be issued until the
// prologue's second round trip and reductions were done.  Issued first, the
// prologue overlaps the prefetch and the weight stream never pauses.
// Register-resident when k <= 32 * kThreads (RMSNorm / plain quantisation)
// or k <= 32 * kQ8Blocks * kThreads (Q8 codes); larger inputs fall back to
// load_activation after the prefetch.
constexpr int kQ8Blocks = 4;

template <int PRO>
struct ActRegs {
  static constexpr bool CODES = PRO == PRO_Q8 || PRO == PRO_NQ;
  f32x4 x[CODES ? 1 : 8];
  f32x4 w[PRO == PRO_NORM ? 8 : 1];
  i32x4 c0[CODES ? kQ8Blocks : 1];
  i32x4 c1[CODES ? kQ8Blocks : 1];
  float d[CODES ? kQ8Blocks : 1];
  float ss;  // PRO_NQ: this thread's block sum of squares
};

// Elements per thread when the whole input spreads evenly over the
// workgroup in runs of 8, 16 or 32 (k = 2048, 4096, 8192); 0 otherwise.
__device__ __forceinline__ int act_ept(int k) {
  return (k == 8 * kThreads || k == 16 * kThreads || k == 32 * kThreads) ? k / kThreads : 0;
}

template <int PRO>
__device__ __forceinline__ bool act_in_regs(int k) {
  const int nb = k >> 5;
  return PRO == PRO_Q8 ? nb <= kQ8Blocks * kThreads : nb <= kThreads;  // PRO_NQ: one block per thread
}

template <int PRO, bool DEV>
__device__ __forceinline__ void issue_activation(const GemvArgs& a, int mrow, ActRegs<PRO>& r) {
  const int k = a.k, nb = k >> 5, tid = threadIdx.x;
  if (!act_in_regs<PRO>(k)) return;
  if (PRO == PRO_Q8 || PRO == PRO_NQ) {
    const int rb = mrow * nb;  // the row's first block (row-batched launches)
    if (PRO == PRO_NQ) r.ss = ld_act<DEV>(a.xss, rb + min(tid, nb - 1));  // clamped; masked at use
#pragma unroll
    for (int i = 0; i < (PRO == PRO_NQ ? 1 : kQ8Blocks); ++i) {
      const int b = min(tid + kThreads * i, nb - 1);  // clamped; extra ones unused
      if (kThreads * i < nb) {
        if (DEV) {
          const dev_u32x4 u0 = dev_ld16(a.xq, 32 * (rb + b)), u1 = dev_ld16(a.xq, 32 * (rb + b) + 16);
          r.c0[i] = i32x4{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w};
          r.c1[i] = i32x4{(int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
        } else {
          const i32x4* src = (const i32x4*)(a.xq + 32 * ((size_t)rb + b));
          r.c0[i] = src[0];
          r.c1[i] = src[1];
        }
        r.d[i] = ld_act<DEV>(a.xd, rb + b);
      }
    }
    return;
  }
  // k = kThreads * ept: thread t owns elements [t*ept, (t+1)*ept); else one
  // 32-element block per thread.
  const int ept = act_ept(k);
  const size_t xrow = (size_t)mrow * k;
  const int e0 = ept ? tid * ept : 32 * (tid < nb ? tid : nb - 1);
  const int nv = ept ? ept / 4 : 8;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < nv) r.x[j] = ld_act4<DEV>(a.x, xrow + e0 + 4 * j);
  if (PRO == PRO_NORM) {
    const f32x4* wsrc = (const f32x4*)(a.norm_w + e0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < nv) r.w[j] = wsrc[j];
  }
}

// Profiling stamps of one workgroup (100 MHz clock), kept in registers and
// stored once at the end of the kernel: a store issued mid-kernel would make
// the next reuse of its data registers wait for every outstanding load.
// 0 start, 1 operand ready, 2 loop done, 3 end, 4 input arrived, 5 norm
// scale known, 6 operand quantised, 7 where it ran: XCC id << 32 | HW_ID.
struct Stamps {
  bool on;
  unsigned long long t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  __device__ __forceinline__ void rec(int i) {
    if (on) t[i] = __builtin_amdgcn_s_memrealtime();
  }
  __device__ __forceinline__ void write(unsigned long long* dst) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = t[i];
  }
};

// RMSNorm (PRO_NORM) and Q8_0 of the register-resident row: EPT values per
// thread (EPT = 32 also covers one block per thread with nb <= kThreads).
template <int PRO, bool Q4, int EPT>
__device__ __forceinline__ void finish_norm(const GemvArgs& a, ActRegs<PRO>& r, int8_t* s_q, float* s_d,
                                            int* s_off, float* s_red, Stamps& ts) {
  const int k = a.k, nb = k >> 5, tid = threadIdx.x;
  const bool active = EPT < 32 || tid < nb;
  float v[EPT];
#pragma unroll
  for (int j = 0; j < EPT / 4; ++j) {
    v[4 * j] = r.x[j].x;
    v[4 * j + 1] = r.x[j].y;
    v[4 * j + 2] = r.x[j].z;
    v[4 * j + 3] = r.x[j].w;
  }
  if (PRO == PRO_NORM) {
    // cpu.rs:381-383: ss = sum v*v; rms = sqrt(ss/n + eps); scale = 1/rms.
    float ss = 0.0f;
    if (active) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) ss = ss + v[i] * v[i];
    }
    ts.rec(4);
    ss = wave_sum(ss);
    if (lane_id() == 0) s_red[wave_id()] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot = tot + s_red[w];
    const float rms = sqrtf(tot / (float)k + a.eps);
    const float scale = 1.0f / rms;
    ts.rec(5);
#pragma unroll
    for (int j = 0; j < EPT / 4; ++j) {
      v[4 * j] = v[4 * j] * scale * r.w[j].x;  // cpu.rs:389: x * s * w
      v[4 * j + 1] = v[4 * j + 1] * scale * r.w[j].y;
      v[4 * j + 2] = v[4 * j + 2] * scale * r.w[j].z;
      v[4 * j + 3] = v[4 * j + 3] * scale * r.w[j].w;
    }
  }
  if (EPT < 32) quant_part<Q4, EPT>(v, tid, s_q, s_d, s_off);
  else if (active) quant_block<Q4>(v, tid, s_q, s_d, s_off);
  ts.rec(6);
}

template <int PRO, bool Q4, bool DEV>
__device__ __forceinline__ void finish_activation(const GemvArgs& a, int mrow, ActRegs<PRO>& r,
                                                  int8_t* s_q, float* s_d, int* s_off, float* s_red,
                                                  Stamps& ts) {
  const int k = a.k, nb = k >> 5, tid = threadIdx.x;
  if (!act_in_regs<PRO>(k)) {
    load_activation<PRO, Q4, DEV>(a, mrow, s_q, s_d, s_off, s_red);
    return;
  }
  if (PRO == PRO_Q8 || PRO == PRO_NQ) {
    float scale = 1.0f;
    if (PRO == PRO_NQ) {
      // RMSNorm factor (cpu.rs:381-383) from the producer's block sums of
      // squares: rms = sqrt(ss/n + eps), s = 1/rms; the scales become d' * s.
      float ss = tid < nb ? r.ss : 0.0f;
      ts.rec(4);
      ss = wave_sum(ss);
      if (lane_id() == 0) s_red[wave_id()] = ss;
      __syncthreads();
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) tot = tot + s_red[w];
      const float rms = sqrtf(tot / (float)k + a.eps);
      scale = 1.0f / rms;
      ts.rec(5);
    }
#pragma unroll
    for (int i = 0; i < (PRO == PRO_NQ ? 1 : kQ8Blocks); ++i) {
      const int b = tid + kThreads * i;
      if (kThreads * i < nb && b < nb) {
        i32x4* dst = (i32x4*)(s_q + 32 * b);
        dst[0] = r.c0[i];
        dst[1] = r.c1[i];
        s_d[b] = PRO == PRO_NQ ? r.d[i] * scale : r.d[i];
        if (Q4) {
          int s = 0;
          s = dot4(r.c0[i].x, 0x01010101, s);
          s = dot4(r.c0[i].y, 0x01010101, s);
          s = dot4(r.c0[i].z, 0x01010101, s);
          s = dot4(r.c0[i].w, 0x01010101, s);
          s = dot4(r.c1[i].x, 0x01010101, s);
          s = dot4(r.c1[i].y, 0x01010101, s);
          s = dot4(r.c1[i].z, 0x01010101, s);
          s = dot4(r.c1[i].w, 0x01010101, s);
          s_off[b] = -8 * s;
        }
      }
    }
    return;
  }
  switch (act_ept(k)) {
    case 8: finish_norm<PRO, Q4, 8>(a, r, s_q, s_d, s_off, s_red, ts); break;
    case 16: finish_norm<PRO, Q4, 16>(a, r, s_q, s_d, s_off, s_red, ts); break;
    default: finish_norm<PRO, Q4, 32>(a, r, s_q, s_d, s_off, s_red, ts); break;
  }
}

// Pair order for argmax: larger value wins, lower index breaks ties.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Weights of one unit held in registers.
template <int WT, int R, int U>
struct UnitRegs {
  u32x4 c0[R][U];
  u32x4 c1[R][WT == WT_Q8H ? U : 1];
  unsigned sc[R][U];  // raw scale bits
};

template <int WT, int EPI, int R, int U>
struct Gemv {
  static constexpr bool Q4 = (WT != WT_Q8H);
  static constexpr int BS = Q4 ? 16 : 32;       // code bytes per block
  static constexpr int BPU = LLMRS_WAVE * U;    // blocks per unit
  static constexpr int TILE = epi_tile(EPI);             // rows per tile (tiled epilogues)
  static constexpr int TRG = TILE ? TILE / R / kWaves : 1;  // row groups per wave per tile
  static_assert(TILE == 0 || (TILE % (R * kWaves) == 0), "a tile must split evenly over the waves");

  const GemvArgs& a;
  int nb, nchunk, nrg, lane, wave, wg, nwg, nunits;

  __device__ Gemv(const GemvArgs& args, int wg_, int nwg_) : a(args), wg(wg_), nwg(nwg_) {
    nb = a.k >> 5;
    nchunk = (nb + BPU - 1) / BPU;
    nrg = (a.n + R - 1) / R;
    lane = lane_id();
    wave = wave_id();
    // Units of this wave: row groups j = 0, 1, ... each of nchunk units.  For
    // the SwiGLU epilogue every wave of a workgroup walks the same number of
    // tiles, so the per-tile barriers are uniform.
    int ngroups;
    if constexpr (TILE > 0) {
      const int ntiles = (a.n + TILE - 1) / TILE;
      const int my_tiles = wg < ntiles ? (ntiles - 1 - wg) / nwg + 1 : 0;
      ngroups = my_tiles * TRG;
    } else {
      const int first = wg * kWaves + wave;
      const int stride = nwg * kWaves;
      ngroups = first < nrg ? (nrg - 1 - first) / stride + 1 : 0;
    }
    nunits = ngroups * nchunk;
  }

  // Row group of the j-th group this wave processes (-1 past the end).
  __device__ __forceinline__ int row_group(int j) const {
    if constexpr (TILE > 0) {
      const int tile = wg + (j / TRG) * nwg;
      const int rg = tile * (TILE / R) + wave * TRG + (j % TRG);
      return rg < nrg ? rg : -1;
    }
    const int rg = wg * kWaves + wave + j * nwg * kWaves;
    return rg < nrg ? rg : -1;
  }

  // Loads are unconditional: out-of-range rows and blocks read a clamped,
  // valid address and are masked at use (blocks) or never written (rows),
  // so the wave issues every load of the unit back to back.
  __device__ __forceinline__ void load(UnitRegs<WT, R, U>& u, int unit) const {
    const int rg = unit < 0 ? -1 : row_group(unit / nchunk);
    const int b0 = (unit < 0 ? 0 : unit % nchunk) * BPU + lane;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(max(rg * R + r, 0), a.n - 1);
#pragma unroll
      for (int v = 0; v < U; ++v) {
        const int b = min(b0 + LLMRS_WAVE * v, nb - 1);
        const size_t blk = (size_t)row * nb + b;
        u.c0[r][v] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * BS));
        if (!Q4) u.c1[r][v] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * BS + 16));
        u.sc[r][v] = load_wscale_raw<WT>(a.ws, blk);
      }
    }
  }

  // The first two units, before the prologue (or a barrier).
  __device__ __forceinline__ void prefetch(UnitRegs<WT, R, U>& ua, UnitRegs<WT, R, U>& ub) const {
    load(ua, nunits > 0 ? 0 : -1);
    load(ub, nunits > 1 ? 1 : -1);
  }

  // acc[r] += sum over the unit's blocks of isum * (d_w * d_a)  (cpu.rs:913,932)
  __device__ __forceinline__ void compute(const UnitRegs<WT, R, U>& u, int unit, float* acc,
                                          const int8_t* s_q, const float* s_d,
                                          const int* s_off) const {
    const int b0 = (unit % nchunk) * BPU + lane;
#pragma unroll
    for (int v = 0; v < U; ++v) {
      // Branch-free: a block past the row end (partial last chunk) reads a
      // clamped block and contributes 0.  Divergent branches here would make
      // the compiler drain every outstanding load at the join.
      const int bb = b0 + LLMRS_WAVE * v;
      const bool ok = bb < nb;
      const int b = ok ? bb : nb - 1;
      {
        const i32x4* aq = (const i32x4*)(s_q + 32 * b);
        const i32x4 a0 = aq[0], a1 = aq[1];
        const float da = s_d[b];
        const int off = Q4 ? s_off[b] : 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int s = off;
          const u32x4 w = u.c0[r][v];
          if (Q4) {
            const unsigned M = 0x0F0F0F0Fu;
            // low nibbles of dword j = elements 4j..4j+3, high = 16+4j..
            s = dot4((int)(w.x & M), a0.x, s);
            s = dot4((int)(w.y & M), a0.y, s);
            s = dot4((int)(w.z & M), a0.z, s);
            s = dot4((int)(w.w & M), a0.w, s);
            s = dot4((int)((w.x >> 4) & M), a1.x, s);
            s = dot4((int)((w.y >> 4) & M), a1.y, s);
            s = dot4((int)((w.z >> 4) & M), a1.z, s);
            s = dot4((int)((w.w >> 4) & M), a1.w, s);
          } else {
            const u32x4 w1 = u.c1[r][v];
            s = dot4((int)w.x, a0.x, s);
            s = dot4((int)w.y, a0.y, s);
            s = dot4((int)w.z, a0.z, s);
            s = dot4((int)w.w, a0.w, s);
            s = dot4((int)w1.x, a1.x, s);
            s = dot4((int)w1.y, a1.y, s);
            s = dot4((int)w1.z, a1.z, s);
            s = dot4((int)w1.w, a1.w, s);
          }
          const float t = (float)s * (wscale<WT>(u.sc[r][v]) * da);
          acc[r] = acc[r] + (ok ? t : 0.0f);
        }
      }
    }
  }
};

// LDS used by gemv_body beyond the activation area.
struct GemvShared {
  float red[kWaves];
  float bv[kWaves];
  int bi[kWaves];
};

// Bytes of the activation area in LDS for an input of length k.
__host__ __device__ constexpr size_t gemv_act_lds(int k) { return gemv_act_bytes(k); }
static_assert(kWaves == 4 || kWaves == 8, "gemv_lds_bytes takes the wave count");

// One GEMV over the waves of workgroup `wg` of `nwg`: prologue, pipelined
// unit loop, epilogues.  `ua`/`ub` hold the first two units already when
// `preloaded`; otherwise PRE of them (0-2) are requested before the
// activation prologue and the rest right after it.  Requests issued before
// the prologue overlap its latency, but they also queue ahead of the
// activation loads of later workgroups; the best depth depends on the
// launch (measured: 1 for the 64-row-tile SwiGLU GEMV, 2 otherwise).
// Argmax partials go to slot `wg`.
//
// The unit loop issues no global stores and has no divergent branches, and
// the last two units are peeled off so it never requests weights it will not
// use: the memory counter of a wave is in order, so a store, or a branch
// join the compiler cannot count through, inside the loop would make the
// next compute wait for every outstanding load and collapse the two-unit
// pipeline.  Row results go to LDS and are written after the loop.
template <int WT, int PRO, int EPI, int R, int U, bool DEV, int PRE = 2>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, int mrow, int wg, int nwg,
                                          UnitRegs<WT, R, U>& ua, UnitRegs<WT, R, U>& ub,
                                          bool preloaded, uint8_t* act, GemvShared& sh) {
  typedef Gemv<WT, EPI, R, U> G;
  const int k = a.k, nb = k >> 5;
  int8_t* s_q = (int8_t*)act;
  float* s_d = (float*)(act + k);
  int* s_off = (int*)(act + k + 4 * nb);
  float* s_out = (float*)(act + (gemv_act_lds(k) + 15) / 16 * 16);
  G g(a, wg, nwg);
  const int lane = g.lane, wave = g.wave, tid = threadIdx.x;
  const int nunits = g.nunits;
  // Row groups per wave (non-SwiGLU): the wave's slice of s_out.
  const int gmax = (g.nrg + nwg * kWaves - 1) / (nwg * kWaves);
  Stamps ts;
  ts.on = a.ts != nullptr;
  ts.rec(0);
  if (ts.on)
    ts.t[7] = ((unsigned long long)__builtin_amdgcn_s_getreg((15 << 11) | 20) << 32) |
              (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);

  // The residual of this lane's first output row is requested with the
  // activations: loaded in the epilogue it would cost a whole memory round
  // trip after the unit loop.  The row is clamped instead of tested, so the
  // prologue has no branch at which the compiler would wait for the loads.
  float res0 = 0.0f, wn0 = 0.0f;
  {
    ActRegs<PRO> ar;
    issue_activation<PRO, DEV>(a, mrow, ar);
    if (EPI == EPI_RESID) {
      const int nv = (nunits / g.nchunk) * R;
      const int v = min(lane, max(nv - 1, 0));
      const int rg = max(g.row_group(v / R), 0);
      const int row = min(rg * R + v % R, a.n - 1);
      res0 = ld_act<DEV>(a.res, (size_t)mrow * a.n + row);
    }
    if (EPI == EPI_NQ) {  // residual and next-norm weight of the first 8 tiles' rows
      const int row = min((wg + (tid / 32) * nwg) * kNqTile + tid % 32, a.n - 1);
      res0 = ld_act<DEV>(a.res, (size_t)mrow * a.n + row);
      wn0 = a.norm_next[row];
    }
    if (!preloaded && PRE > 0) g.load(ua, nunits > 0 ? 0 : -1);
    if (!preloaded && PRE > 1) g.load(ub, nunits > 1 ? 1 : -1);
    finish_activation<PRO, G::Q4, DEV>(a, mrow, ar, s_q, s_d, s_off, sh.red, ts);
  }
  if (!preloaded && PRE < 1) g.load(ua, nunits > 0 ? 0 : -1);
  if (!preloaded && PRE < 2) g.load(ub, nunits > 1 ? 1 : -1);
  __syncthreads();
  ts.rec(1);

  float best_v = -INFINITY;
  int best_i = 0x7fffffff;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  // Finish unit i: on the last chunk of a row group, reduce the lane
  // partials and park the R results in LDS (lane r writes row r).
  auto finish = [&](int i) {
    if ((i % g.nchunk) != g.nchunk - 1) return;
    const int j = i / g.nchunk;
    float vals[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      vals[r] = wave_sum(acc[r]);
      acc[r] = 0.0f;
    }
    if (EPI == EPI_ARGMAX) {
      const int rg = g.row_group(j);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = rg * R + r;
        if (rg >= 0 && row < a.n && better(vals[r], row, best_v, best_i)) {
          best_v = vals[r];
          best_i = row;
        }
      }
    }
    float out = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane == r) out = vals[r];
    int slot;
    if (G::TILE)
      slot = (j / G::TRG) * G::TILE + wave * (G::TRG * R) + (j % G::TRG) * R;
    else
      slot = (wave * gmax + j) * R;
    if (lane < R) s_out[slot + lane] = out;
  };

  int i = 0;
  for (; i + 3 < nunits; i += 2) {
    g.compute(ua, i, acc, s_q, s_d, s_off);
    g.load(ua, i + 2);
    finish(i);
    g.compute(ub, i + 1, acc, s_q, s_d, s_off);
    g.load(ub, i + 3);
    finish(i + 1);
  }
  // Tail: 0-3 units left, at most one more load.
  if (i + 2 < nunits) {
    g.compute(ua, i, acc, s_q, s_d, s_off);
    g.load(ua, i + 2);
    finish(i);
    g.compute(ub, i + 1, acc, s_q, s_d, s_off);
    finish(i + 1);
    g.compute(ua, i + 2, acc, s_q, s_d, s_off);
    finish(i + 2);
  } else if (i + 1 < nunits) {
    g.compute(ua, i, acc, s_q, s_d, s_off);
    finish(i);
    g.compute(ub, i + 1, acc, s_q, s_d, s_off);
    finish(i + 1);
  } else if (i < nunits) {
    g.compute(ua, i, acc, s_q, s_d, s_off);
    finish(i);
  }
  ts.rec(2);

  // Epilogues from the parked results.
  const size_t ybase = (size_t)mrow * a.n;
  if (EPI == EPI_SILU) {
    __syncthreads();
    const int ntiles = (a.n + kSiluTile - 1) / kSiluTile;
    const int my_tiles = wg < ntiles ? (ntiles - 1 - wg) / nwg + 1 : 0;
    // 32 threads per tile: tile = 32 gate rows then the 32 matching up rows
    // (layer.rs:72-79); m = silu(g) * u and its Q8_0 block.
    for (int q0 = 0; q0 < my_tiles; q0 += kThreads / 32) {
      const int q = q0 + tid / 32, e = tid % 32;
      if (q < my_tiles) {  // uniform per 32-lane half-wave
        const int tile = wg + q * nwg;
        const float gv = s_out[q * kSiluTile + e], uv = s_out[q * kSiluTile + 32 + e];
        const float mv = (gv / (1.0f + expf(-gv))) * uv;
        const int idx = mrow * (a.n / 2) + tile * 32 + e;  // m row mrow (row-batched launches)
        if (a.y) st_act<DEV>(a.y, idx, mv);
        float d;
        const int qc = q8_group32(mv, &d);
        if (DEV) dev_st8(a.yq, idx, (int8_t)qc);
        else a.yq[idx] = (int8_t)qc;
        if (e == 0) st_act<DEV>(a.yd, mrow * (a.n / 64) + tile, d);
      }
    }
  } else if (EPI == EPI_NQ) {
    __syncthreads();
    const int ntiles = (a.n + kNqTile - 1) / kNqTile;
    const int my_tiles = wg < ntiles ? (ntiles - 1 - wg) / nwg + 1 : 0;
    // 32 threads per tile: y = acc + res (layer.rs:386,403), then the next
    // RMSNorm's operand: Q8_0 of y*w (d' = amax/127, cpu.rs:724-743) and the
    // block's sum of y^2.
    for (int q0 = 0; q0 < my_tiles; q0 += kThreads / 32) {
      const int q = q0 + tid / 32, e = tid % 32;
      if (q < my_tiles) {  // uniform per 32-lane half-wave
        const int tile = wg + q * nwg;
        const int row = tile * kNqTile + e;
        const bool ok = row < a.n;
        const float rv = q0 == 0 ? res0 : (ok ? ld_act<DEV>(a.res, ybase + row) : 0.0f);
        const float wv = q0 == 0 ? wn0 : (ok ? a.norm_next[row] : 0.0f);
        const float yv = s_out[q * kNqTile + e] + rv;
        if (ok) st_act<DEV>(a.y, ybase + row, yv);
        const float z = ok ? yv * wv : 0.0f;
        float d;
        const int qc = q8_group32(z, &d);
        const float ss = group_sum<32>(ok ? yv * yv : 0.0f);
        if (ok) a.yq[row] = (int8_t)qc;
        if (e == 0) {
          a.yd[tile] = d;
          a.yss[tile] = ss;
        }
      }
    }
  } else if (EPI == EPI_STORE || EPI == EPI_RESID || (EPI == EPI_ARGMAX && a.y)) {
    // This wave's rows: value v = j * R + r of its slice, one per lane.
    const int nv = (nunits / g.nchunk) * R;
    for (int v0 = 0; v0 < nv; v0 += LLMRS_WAVE) {
      const int v = v0 + lane;
      const int rg = v < nv ? g.row_group(v / R) : -1;
      const int row = rg * R + v % R;
      if (rg >= 0 && row < a.n) {
        float out = s_out[wave * gmax * R + v];
        if (EPI == EPI_RESID) {
          float rv = res0;  // requested in the prologue for v0 == 0
          if (v0 > 0) rv = ld_act<DEV>(a.res, ybase + row);
          out = out + rv;  // layer.rs:386,403
        }
        st_act<DEV>(a.y, ybase + row, out);
      }
    }
  }

  if (EPI == EPI_ARGMAX) {
    if (lane == 0) {
      sh.bv[wave] = best_v;
      sh.bi[wave] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kWaves; ++w)
        if (better(sh.bv[w], sh.bi[w], best_v, best_i)) {
          best_v = sh.bv[w];
          best_i = sh.bi[w];
        }
      st_act<DEV>(a.part_val, wg, best_v);
      if (DEV) dev_stu(a.part_idx, 4 * wg, (unsigned)best_i);
      else a.part_idx[wg] = best_i;
    }
  }
  ts.rec(3);
  if (ts.on && tid == 0) ts.write(a.ts + 8 * ((size_t)mrow * nwg + wg));
  // Test probe: the prologue's operand, copied after every load has been
  // consumed so the unit pipeline is unaffected.
  if (a.probe_xq && wg == 0 && mrow == 0) {
    for (int i = tid; i < k; i += kThreads) a.probe_xq[i] = s_q[i];
    for (int b = tid; b < nb; b += kThreads) a.probe_xd[b] = s_d[b];
  }
}

}  // namespace llmrs
