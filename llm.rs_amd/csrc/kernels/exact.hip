// exact.hip - the decode step in the reference's f32 operation order, for
// gfx950 (a model with llmrs_model_set_exact, or created with LLMRS_EXACT=1).
//
// The fast decode kernels (gemv.hip, attention.hip) compute every integer
// block sum exactly but add the f32 terms in wave-parallel orders, so their
// outputs differ from the reference's in the last bits, and on
// ill-conditioned weights the differences reach the logits.  These kernels
// add in the reference's own order, so that for the same weights and tokens
// every value - norms, codes, projections, attention, logits, the greedy
// stream - equals the reference CPU path's (x86-64 build) bit for bit:
//   exact_norm_q8   RMSNorm with one sequential f32 fold of x*x
//                   (cpu.rs:381-389), then Q8_0 (cpu.rs:724-743)
//   exact_gemv_*    per output row, total = total + isum_b * (d_w * d_a) for
//                   b = 0, 1, ... (kernel_avx2, cpu.rs:903-938); a wave per
//                   row computes the terms of 64 blocks at once, then adds
//                   them in block order
//   exact_attn_*    one workgroup per query head: RoPE (cpu.rs:345-354),
//                   K/V append, sequential q.k dots (matmul_slice,
//                   cpu.rs:230-269) times 1/sqrt(hd) (layer.rs:257-258),
//                   softmax with a sequential sum (cpu.rs:395-423), P.V
//                   sequential over positions (layer.rs:276-299), ctx Q8_0
//   exact_silu_q8   g / (1 + exp(-g)) * u (layer.rs:75-79) with glibc's
//                   expf (exact_math.h), Q8_0 of the product
// The lm_head runs exact_gemv with the argmax partials of argmax_final.
// A batched prompt is the same computation row by row (the reference's
// batched path adds in the same per-row orders), so prompts run as
// consecutive single-row steps.
#include "common.h"
#include "exact_math.h"
#include "gemv_core.h"
#include "../kernel_args.h"

using namespace llmrs;

namespace {

constexpr int kT = 256;

// ---- RMSNorm + Q8_0 ---------------------------------------------------------
// One workgroup; x staged in LDS (n <= 32768 floats), one lane folds x*x in
// index order.  n is a multiple of 32, so a 32-lane group holds one block.
__device__ __forceinline__ void norm_q8(const ExactNormArgs& a) {
  extern __shared__ __align__(16) float sx[];
  __shared__ float s_scale;
  const int tid = threadIdx.x;
  for (int i = tid; i < a.n; i += kT) sx[i] = a.x[i];
  __syncthreads();
  if (tid == 0) {
    float ss = 0.0f;
    for (int i = 0; i < a.n; i += 4) {
      const f32x4 v = *(const f32x4*)(sx + i);
      ss = ss + v[0] * v[0];
      ss = ss + v[1] * v[1];
      ss = ss + v[2] * v[2];
      ss = ss + v[3] * v[3];
    }
    const float rms = __builtin_sqrtf(ss / (float)a.n + a.eps);
    s_scale = 1.0f / rms;
  }
  __syncthreads();
  const float s = s_scale;
  for (int i = tid; i < a.n; i += kT) {
    const float y = sx[i] * s * a.w[i];
    float d;
    const int q = q8_group32(y, &d);
    a.xq[i] = (int8_t)q;
    if ((tid & 31) == 0) a.xd[i >> 5] = d;
    if (a.y) a.y[i] = y;
  }
}

// ---- GEMV -----------------------------------------------------------------
// Exact integer sum of one block of weight codes with activation codes
// (device Q4 layout: byte i = e[i] | e[i+16] << 4, value q - 8).
template <int WT>
__device__ __forceinline__ int block_isum(const uint8_t* wblk, const int8_t* ablk) {
  const i32x4 a0 = *(const i32x4*)ablk, a1 = *(const i32x4*)(ablk + 16);
  int s = 0;
  if (WT == WT_Q8H) {
    const i32x4 w0 = *(const i32x4*)wblk, w1 = *(const i32x4*)(wblk + 16);
    s = dot4(w0.x, a0.x, s);
    s = dot4(w0.y, a0.y, s);
    s = dot4(w0.z, a0.z, s);
    s = dot4(w0.w, a0.w, s);
    s = dot4(w1.x, a1.x, s);
    s = dot4(w1.y, a1.y, s);
    s = dot4(w1.z, a1.z, s);
    s = dot4(w1.w, a1.w, s);
  } else {
    const u32x4 w = *(const u32x4*)wblk;
    const unsigned M = 0x0F0F0F0Fu;
    s = dot4((int)(w.x & M), a0.x, s);
    s = dot4((int)(w.y & M), a0.y, s);
    s = dot4((int)(w.z & M), a0.z, s);
    s = dot4((int)(w.w & M), a0.w, s);
    s = dot4((int)((w.x >> 4) & M), a1.x, s);
    s = dot4((int)((w.y >> 4) & M), a1.y, s);
    s = dot4((int)((w.z >> 4) & M), a1.z, s);
    s = dot4((int)((w.w >> 4) & M), a1.w, s);
    int sa = 0;
    sa = dot4(a0.x, 0x01010101, sa);
    sa = dot4(a0.y, 0x01010101, sa);
    sa = dot4(a0.z, 0x01010101, sa);
    sa = dot4(a0.w, 0x01010101, sa);
    sa = dot4(a1.x, 0x01010101, sa);
    sa = dot4(a1.y, 0x01010101, sa);
    sa = dot4(a1.z, 0x01010101, sa);
    sa = dot4(a1.w, 0x01010101, sa);
    s -= 8 * sa;
  }
  return s;
}

// EPI: EPI_STORE (y = total), EPI_RESID (y = total + res), EPI_ARGMAX
// (logits into y when set, and this workgroup's (max, lowest index) into
// part_val / part_idx[blockIdx.x]).  Waves take rows round-robin.
template <int WT, int EPI>
__device__ __forceinline__ void gemv(const ExactGemvArgs& a) {
  constexpr int BS = WT == WT_Q8H ? 32 : 16;
  __shared__ float s_bv[kT / LLMRS_WAVE];
  __shared__ int s_bi[kT / LLMRS_WAVE];
  const int lane = lane_id(), wave = wave_id();
  const int nb = a.k >> 5;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int row = blockIdx.x * (kT / LLMRS_WAVE) + wave; row < a.n; row += gridDim.x * (kT / LLMRS_WAVE)) {
    float total = 0.0f;
    for (int c = 0; c < nb; c += LLMRS_WAVE) {
      const int b = c + lane;
      float p = 0.0f;
      if (b < nb) {
        const size_t blk = (size_t)row * nb + b;
        const int isum = block_isum<WT>(a.wq + blk * BS, a.xq + 32 * b);
        p = (float)isum * (wscale<WT>(load_wscale_raw<WT>(a.ws, blk)) * a.xd[b]);
      }
      const int cnt = min(LLMRS_WAVE, nb - c);
      for (int l = 0; l < cnt; ++l) total = total + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), l));
    }
    if (lane == 0) {
      if (EPI == EPI_RESID) a.y[row] = total + a.res[row];
      else if (a.y) a.y[row] = total;
    }
    if (EPI == EPI_ARGMAX && better(total, row, bv, bi)) {
      bv = total;
      bi = row;
    }
  }
  if (EPI == EPI_ARGMAX) {
    if (lane == 0) {
      s_bv[wave] = bv;
      s_bi[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kT / LLMRS_WAVE; ++w)
        if (better(s_bv[w], s_bi[w], bv, bi)) {
          bv = s_bv[w];
          bi = s_bi[w];
        }
      a.part_val[blockIdx.x] = bv;
      a.part_idx[blockIdx.x] = bi;
    }
  }
}

// ---- attention -------------------------------------------------------------
// One workgroup per query head h (KV head g = h / n_rep) at the device
// position pos: scores, exponentials and probabilities of the pos + 1
// positions in LDS.  The new K/V row is rotated and rounded to the cache
// type by every workgroup of the group (the values are identical) and
// stored by the group's first; each workgroup uses its own copy for
// position pos, so no workgroup reads a row another is writing.
template <int HD, bool F16>
__device__ __forceinline__ void attn(const ExactAttnArgs& a) {
  constexpr int MID = HD / 2;
  extern __shared__ __align__(16) float s_p[];  // [pos + 1]
  __shared__ __align__(16) float s_q[HD];
  __shared__ __align__(16) float s_k[HD];
  __shared__ float s_v[HD];
  __shared__ float s_red[kT / LLMRS_WAVE];
  __shared__ float s_inv;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int h = blockIdx.x, n_rep = a.nq / a.nkv, g = h / n_rep;
  const int pos = *a.pos_ptr, T = pos + 1;
  const size_t head = (size_t)g * a.max_seq * HD;
  if (tid < MID) {  // rotate-half RoPE of q and the new k (cpu.rs:345-354)
    const float co = a.rope_cos[(size_t)pos * MID + tid], sn = a.rope_sin[(size_t)pos * MID + tid];
    const float* q = a.qkv + (size_t)h * HD;
    float re = q[tid], im = q[tid + MID];
    s_q[tid] = re * co - im * sn;
    s_q[tid + MID] = re * sn + im * co;
    const float* k = a.qkv + (size_t)(a.nq + g) * HD;
    const float* v = a.qkv + (size_t)(a.nq + a.nkv + g) * HD;
    re = k[tid];
    im = k[tid + MID];
    float kv[4] = {re * co - im * sn, re * sn + im * co, v[tid], v[tid + MID]};
    const int dd[4] = {tid, tid + MID, tid, tid + MID};
    const bool owner = h % n_rep == 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool is_k = j < 2;
      if (F16) {
        const uint16_t b = f2h(kv[j]);
        kv[j] = h2f(b);
        if (owner) {
          if (is_k) ((uint16_t*)a.kc)[head + (size_t)pos * HD + dd[j]] = b;
          else ((uint16_t*)a.vc)[head + v_offset(pos, dd[j], HD, true)] = b;
        }
      } else if (owner) {
        if (is_k) ((float*)a.kc)[head + (size_t)pos * HD + dd[j]] = kv[j];
        else ((float*)a.vc)[head + v_offset(pos, dd[j], HD, false)] = kv[j];
      }
      (is_k ? s_k : s_v)[dd[j]] = kv[j];
    }
  }
  __syncthreads();
  // scores: sequential dot over the head dims, then the scale
  float mx = -3.40282347e+38f;  // f32::MIN (cpu.rs:408)
  for (int t = tid; t < T; t += kT) {
    float s = 0.0f;
    if (t == pos) {
      for (int e = 0; e < HD; ++e) s = s + s_q[e] * s_k[e];
    } else if (F16) {
      const uint16_t* kr = (const uint16_t*)a.kc + head + (size_t)t * HD;
      for (int e = 0; e < HD; e += 8) {
        const u32x4 w = *(const u32x4*)(kr + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s = s + s_q[e + 2 * i] * h2f((uint16_t)(w[i] & 0xFFFF));
          s = s + s_q[e + 2 * i + 1] * h2f((uint16_t)(w[i] >> 16));
        }
      }
    } else {
      const float* kr = (const float*)a.kc + head + (size_t)t * HD;
      for (int e = 0; e < HD; e += 4) {
        const f32x4 w = *(const f32x4*)(kr + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) s = s + s_q[e + i] * w[i];
      }
    }
    s = s * a.scale;
    s_p[t] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  mx = s_red[0];
#pragma unroll
  for (int w = 1; w < kT / LLMRS_WAVE; ++w) mx = fmaxf(mx, s_red[w]);
  for (int t = tid; t < T; t += kT) s_p[t] = exact_expf(s_p[t] - mx);
  __syncthreads();
  if (tid == 0) {  // sequential sum of the exponentials
    float sum = 0.0f;
    int t = 0;
    for (; t + 4 <= T; t += 4) {
      const f32x4 e = *(const f32x4*)(s_p + t);
      sum = sum + e[0];
      sum = sum + e[1];
      sum = sum + e[2];
      sum = sum + e[3];
    }
    for (; t < T; ++t) sum = sum + s_p[t];
    s_inv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = s_inv;
  for (int t = tid; t < T; t += kT) s_p[t] = s_p[t] * inv;
  __syncthreads();
  if (tid < HD) {  // ctx[d] = sum over t of p_t * V[t][d], sequential in t
    const int d = tid;
    float s = 0.0f;
    int t = 0;
    if (F16) {  // blocked V: the 8 positions of a block are 16 contiguous bytes per dim
      const uint16_t* vr = (const uint16_t*)a.vc + head;
      for (; t + 8 <= pos; t += 8) {
        const u32x4 w = *(const u32x4*)(vr + v_offset(t, d, HD, true));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s = s + s_p[t + 2 * i] * h2f((uint16_t)(w[i] & 0xFFFF));
          s = s + s_p[t + 2 * i + 1] * h2f((uint16_t)(w[i] >> 16));
        }
      }
      for (; t < pos; ++t) s = s + s_p[t] * h2f(vr[v_offset(t, d, HD, true)]);
    } else {
      const float* vr = (const float*)a.vc + head;
      for (; t < pos; ++t) s = s + s_p[t] * vr[(size_t)t * HD + d];
    }
    s = s + s_p[pos] * s_v[d];
    const size_t e = (size_t)h * HD + d;
    a.ctx[e] = s;
    float dq;
    const int q = q8_group32(s, &dq);
    a.ctx_q[e] = (int8_t)q;
    if ((d & 31) == 0) a.ctx_d[e >> 5] = dq;
  }
}

// ---- SwiGLU ------------------------------------------------------------------
// m[j] = silu(gate[j]) * up[j] from the gate|up GEMV's rows (runs of 32 gate
// rows then the 32 matching up rows), then Q8_0 of m.
__device__ __forceinline__ void silu_q8(const ExactSiluArgs& a) {
  const int j = blockIdx.x * kT + threadIdx.x;
  if (j >= a.n) return;  // n % 32 == 0: whole 32-lane groups leave together
  const size_t r = (size_t)(j >> 5) * 64 + (j & 31);
  const float g = a.gu[r], u = a.gu[r + 32];
  const float silu = g / (1.0f + exact_expf(-g));
  const float m = silu * u;
  float d;
  const int q = q8_group32(m, &d);
  a.mq[j] = (int8_t)q;
  if ((j & 31) == 0) a.md[j >> 5] = d;
  if (a.mf) a.mf[j] = m;
}

}  // namespace

extern "C" __global__ __launch_bounds__(kT) void exact_norm_q8(ExactNormArgs a) { norm_q8(a); }
extern "C" __global__ __launch_bounds__(kT) void exact_silu_q8(ExactSiluArgs a) { silu_q8(a); }

#define LLMRS_EXACT_GEMV(tag, WT)                                                                     \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_store(ExactGemvArgs a) {      \
    gemv<WT, EPI_STORE>(a);                                                                         \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_resid(ExactGemvArgs a) {      \
    gemv<WT, EPI_RESID>(a);                                                                         \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_argmax(ExactGemvArgs a) {     \
    gemv<WT, EPI_ARGMAX>(a);                                                                        \
  }
LLMRS_EXACT_GEMV(q4h, WT_Q4H)
LLMRS_EXACT_GEMV(q4f, WT_Q4F)
LLMRS_EXACT_GEMV(q8h, WT_Q8H)

#define LLMRS_EXACT_ATTN(name, HD, F16) \
  extern "C" __global__ __launch_bounds__(kT) void name(ExactAttnArgs a) { attn<HD, F16>(a); }
LLMRS_EXACT_ATTN(exact_attn_hd64_f16, 64, true)
LLMRS_EXACT_ATTN(exact_attn_hd128_f16, 128, true)
LLMRS_EXACT_ATTN(exact_attn_hd64_f32, 64, false)
LLMRS_EXACT_ATTN(exact_attn_hd128_f32, 128, false)
