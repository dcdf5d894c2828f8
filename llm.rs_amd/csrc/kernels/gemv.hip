// gemv.hip - batch-1 dequant-GEMV for gfx950 (CDNA4).
//
// y[row] = sum_b isum_b(row) * (d_w[row,b] * d_a[b]) where isum_b is the exact
// int32 dot product of one 32-element block of weight codes with the Q8_0
// activation codes.  This is the reference CPU GEMV (cpu.rs:49-111,
// kernel_avx2 cpu.rs:888-941) with the block loop spread over the 64 lanes of
// a wavefront and the partial sums reduced across lanes; isum_b is bit-exact,
// only the f32 summation order differs.
//
// Device weight layout (written by the host at upload): for an [n, k] matrix
// with nb = k/32 blocks per row, codes [n][nb][B] (B = 16 bytes for Q4_0:
// byte i = e[i] | e[i+16] << 4; B = 32 bytes for Q8_0), then scales [n][nb]
// (fp16, or f32 for the reference's Q4 storage).  Lane l of a wave reads
// block l, l+64, ... of a row: 64 lanes x 16 B = one 1 KB coalesced load.
//
// The activation vector is quantised once per workgroup into LDS (prologue):
//   PRO_QUANT  Q8_0 of an f32 row                     (matmul_transposed)
//   PRO_NORM   RMSNorm then Q8_0                        (QKV, gate|up, lm_head)
//   PRO_Q8     already-quantised codes from global      (O, down)
// and the result tile is finished in an epilogue:
//   EPI_STORE  y = acc
//   EPI_RESID  y = acc + res                            (O + residual, down + residual)
//   EPI_SILU   gate|up rows interleaved in tiles of 32+32; m = silu(g)*u,
//              written as f32 and as Q8_0 codes for the down projection
//   EPI_ARGMAX logits plus a per-workgroup (max, index) partial (lm_head)
#include "common.h"
#include "../kernel_args.h"

using namespace llmrs;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

enum { WT_Q4H = 0, WT_Q4F = 1, WT_Q8H = 2 };
enum { PRO_QUANT = 0, PRO_NORM = 1, PRO_Q8 = 2 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_ARGMAX = 3 };


template <int WT>
__device__ __forceinline__ float load_wscale(const void* ws, size_t i) {
  if (WT == WT_Q4F) return __builtin_nontemporal_load((const float*)ws + i);
  return h2f(__builtin_nontemporal_load((const uint16_t*)ws + i));
}

// Prologue: the activation row as Q8_0 in LDS.  s_q holds the codes in
// natural order, s_d the block scales, s_off = -8 * sum(codes) per block (the
// Q4 offset: sum (q-8)*a = sum q*a - 8*sum a, with q in 0..15 read as int8).
template <int PRO, bool Q4>
__device__ __forceinline__ void load_activation(const GemvArgs& a, int mrow, int8_t* s_q,
                                                float* s_d, int* s_off, float* s_red) {
  const int k = a.k, nb = k >> 5, tid = threadIdx.x;
  if (PRO == PRO_Q8) {
    const int* src = (const int*)a.xq;
    int* dst = (int*)s_q;
    for (int i = tid; i < (k >> 2); i += blockDim.x) dst[i] = src[i];
    for (int b = tid; b < nb; b += blockDim.x) s_d[b] = a.xd[b];
    if (Q4) {
      __syncthreads();
      for (int b = tid; b < nb; b += blockDim.x) {
        int s = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) s = dot4(dst[8 * b + j], 0x01010101, s);
        s_off[b] = -8 * s;
      }
    }
    return;
  }
  const float* x = a.x + (size_t)mrow * k;
  float scale = 1.0f;
  if (PRO == PRO_NORM) {
    // cpu.rs:381-383: ss = sum v*v; rms = sqrt(ss/n + eps); scale = 1/rms.
    float ss = 0.0f;
    for (int i = tid; i < k; i += blockDim.x) ss = ss + x[i] * x[i];
    ss = group_sum(ss);
    if (lane_id() == 0) s_red[wave_id()] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < (int)(blockDim.x / LLMRS_WAVE); ++w) tot = tot + s_red[w];
    float rms = sqrtf(tot / (float)k + a.eps);
    scale = 1.0f / rms;
  }
  const int grp = tid >> 5, gl = tid & 31, ngrp = blockDim.x >> 5;
  for (int b = grp; b < nb; b += ngrp) {
    float v = x[32 * b + gl];
    if (PRO == PRO_NORM) v = v * scale * a.norm_w[32 * b + gl];  // cpu.rs:389
    float d;
    int q = q8_group32(v, &d);
    s_q[32 * b + gl] = (int8_t)q;
    if (Q4) {
      int sq = group_sum_i<32>(q);
      if (gl == 0) s_off[b] = -8 * sq;
    }
    if (gl == 0) s_d[b] = d;
  }
}

// Pair order for argmax: larger value wins, lower index breaks ties.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int WT, int PRO, int EPI, int R, int P>
__device__ __forceinline__ void gemv_impl(const GemvArgs& a) {
  constexpr bool Q4 = (WT != WT_Q8H);
  constexpr int ROWS_TILE = 4 * R * P;  // 4 waves per workgroup
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float s_out[ROWS_TILE];
  __shared__ float s_red[8];
  __shared__ float s_bv[8];
  __shared__ int s_bi[8];

  const int k = a.k, nb = k >> 5;
  int8_t* s_q = (int8_t*)smem;
  float* s_d = (float*)(smem + k);
  int* s_off = (int*)(smem + k + 4 * nb);
  const int mrow = blockIdx.y;

  load_activation<PRO, Q4>(a, mrow, s_q, s_d, s_off, s_red);
  __syncthreads();

  const int lane = lane_id(), wave = wave_id(), tid = threadIdx.x;
  const int ntiles = (a.n + ROWS_TILE - 1) / ROWS_TILE;
  const i32x4* s_q4 = (const i32x4*)s_q;
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;

  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int row0 = tile * ROWS_TILE + p * 4 * R + wave * R;
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0f;
      for (int b = lane; b < nb; b += LLMRS_WAVE) {
        const i32x4 a0 = s_q4[2 * b];
        const i32x4 a1 = s_q4[2 * b + 1];
        const float da = s_d[b];
        const int off = Q4 ? s_off[b] : 0;
        u32x4 w0[R], w1[R];
        float dw[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = row0 + r;
          if (row < a.n) {
            const size_t blk = (size_t)row * nb + b;
            if (Q4) {
              w0[r] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * 16));
            } else {
              w0[r] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * 32));
              w1[r] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * 32 + 16));
            }
            dw[r] = load_wscale<WT>(a.ws, blk);
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (row0 + r < a.n) {
            int s = off;
            if (Q4) {
              const unsigned M = 0x0F0F0F0Fu;
              // low nibbles of dword j = elements 4j..4j+3, high = 16+4j..
              s = dot4((int)(w0[r].x & M), a0.x, s);
              s = dot4((int)(w0[r].y & M), a0.y, s);
              s = dot4((int)(w0[r].z & M), a0.z, s);
              s = dot4((int)(w0[r].w & M), a0.w, s);
              s = dot4((int)((w0[r].x >> 4) & M), a1.x, s);
              s = dot4((int)((w0[r].y >> 4) & M), a1.y, s);
              s = dot4((int)((w0[r].z >> 4) & M), a1.z, s);
              s = dot4((int)((w0[r].w >> 4) & M), a1.w, s);
            } else {
              s = dot4((int)w0[r].x, a0.x, s);
              s = dot4((int)w0[r].y, a0.y, s);
              s = dot4((int)w0[r].z, a0.z, s);
              s = dot4((int)w0[r].w, a0.w, s);
              s = dot4((int)w1[r].x, a1.x, s);
              s = dot4((int)w1[r].y, a1.y, s);
              s = dot4((int)w1[r].z, a1.z, s);
              s = dot4((int)w1[r].w, a1.w, s);
            }
            // cpu.rs:913,932: total += block_sum * (d_w * d_a)
            acc[r] = acc[r] + (float)s * (dw[r] * da);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v = group_sum(acc[r]);
        if (lane == 0) s_out[p * 4 * R + wave * R + r] = v;
      }
    }
    __syncthreads();

    const size_t ybase = (size_t)mrow * a.n;
    if (EPI == EPI_STORE || EPI == EPI_RESID) {
      if (tid < ROWS_TILE) {
        const int row = tile * ROWS_TILE + tid;
        if (row < a.n) {
          float v = s_out[tid];
          if (EPI == EPI_RESID) v = v + a.res[ybase + row];  // layer.rs:386,403
          a.y[ybase + row] = v;
        }
      }
    } else if (EPI == EPI_SILU) {
      // Tile = 32 gate rows then the 32 matching up rows (layer.rs:72-79).
      if (tid < 32) {
        const float g = s_out[tid], u = s_out[32 + tid];
        const float mv = (g / (1.0f + expf(-g))) * u;
        const int i = tile * 32 + tid;
        if (a.y) a.y[i] = mv;
        float d;
        const int q = q8_group32(mv, &d);
        a.yq[i] = (int8_t)q;
        if (tid == 0) a.yd[tile] = d;
      }
    } else if (EPI == EPI_ARGMAX) {
      if (tid < ROWS_TILE) {
        const int row = tile * ROWS_TILE + tid;
        if (row < a.n) {
          const float v = s_out[tid];
          if (a.y) a.y[row] = v;
          if (better(v, row, best_v, best_i)) {
            best_v = v;
            best_i = row;
          }
        }
      }
    }
    __syncthreads();
  }

  if (EPI == EPI_ARGMAX) {
    // Workgroup reduction of (value, index) pairs.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(best_v, o);
      int oi = __shfl_xor(best_i, o);
      if (better(ov, oi, best_v, best_i)) {
        best_v = ov;
        best_i = oi;
      }
    }
    if (lane == 0) {
      s_bv[wave] = best_v;
      s_bi[wave] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < (int)(blockDim.x / LLMRS_WAVE); ++w)
        if (better(s_bv[w], s_bi[w], best_v, best_i)) {
          best_v = s_bv[w];
          best_i = s_bi[w];
        }
      a.part_val[blockIdx.x] = best_v;
      a.part_idx[blockIdx.x] = best_i;
    }
  }
}

#define LLMRS_GEMV(name, WT, PRO, EPI, R, P)                                       \
  extern "C" __global__ __launch_bounds__(256) void name(GemvArgs a) {             \
    gemv_impl<WT, PRO, EPI, R, P>(a);                                              \
  }

#define LLMRS_GEMV_FAMILY(tag, WT)                                          \
  LLMRS_GEMV(gemv_##tag##_quant_store, WT, PRO_QUANT, EPI_STORE, 4, 1)      \
  LLMRS_GEMV(gemv_##tag##_norm_store, WT, PRO_NORM, EPI_STORE, 4, 1)        \
  LLMRS_GEMV(gemv_##tag##_q8_resid, WT, PRO_Q8, EPI_RESID, 4, 1)            \
  LLMRS_GEMV(gemv_##tag##_norm_silu, WT, PRO_NORM, EPI_SILU, 4, 4)          \
  LLMRS_GEMV(gemv_##tag##_norm_argmax, WT, PRO_NORM, EPI_ARGMAX, 4, 1)

LLMRS_GEMV_FAMILY(q4h, WT_Q4H)
LLMRS_GEMV_FAMILY(q4f, WT_Q4F)
LLMRS_GEMV_FAMILY(q8h, WT_Q8H)

// Final reduction of the lm_head partials and the greedy step bookkeeping:
// next = argmax (lowest index on ties); gen[pos+1] = next; tokens[pos+1] =
// next once the prompt is consumed; pos += 1.
extern "C" __global__ __launch_bounds__(256) void argmax_final(ArgmaxFinalArgs a) {
  __shared__ float s_bv[8];
  __shared__ int s_bi[8];
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < a.nparts; i += blockDim.x)
    if (better(a.part_val[i], a.part_idx[i], bv, bi)) {
      bv = a.part_val[i];
      bi = a.part_idx[i];
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bv, o);
    int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_bv[wave] = bv;
    s_bi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < (int)(blockDim.x / LLMRS_WAVE); ++w)
      if (better(s_bv[w], s_bi[w], bv, bi)) {
        bv = s_bv[w];
        bi = s_bi[w];
      }
    if (bi == 0x7fffffff) bi = 0;  // every logit NaN
    const int pos = *a.pos;
    if (pos + 1 < a.cap) {
      a.gen[pos + 1] = bi;
      if (pos + 1 >= *a.n_prompt) a.tokens[pos + 1] = bi;
    }
    *a.pos = pos + 1;
  }
}
