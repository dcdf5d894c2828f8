// prefill.hip - batched prompt processing (prefill) for gfx950.
//
// Reference: LlamaModel::forward over a chunk of M tokens (model.rs:17-49,
// layer.rs:373-406; the prompt step of main.rs:134-190).  The reference's
// M > 1 GEMM quantises every activation row to Q8_0 and runs the Q4 x Q8
// block loop per output element (cpu.rs:90-110, kernel_avx2 cpu.rs:888-941):
//   y[t][r] = (...((0 + isum_0 * s_0) + isum_1 * s_1) + ...),  s_b = d_w[r,b] * d_a[t,b]
// with isum_b the exact int32 dot product of one 32-element block.
//
// gemm_*: one v_mfma_i32_32x32x32_i8 per 32-block gives isum_b for a 32 x 32
// (token x row) tile exactly; the epilogue applies the reference's scale and
// f32 accumulation in the same block order, so every GEMM output is
// bit-identical to the reference for identical activation codes.  The f32
// epilogue (convert, two multiplies, add per element and block) is the
// kernel's bottleneck, not the MFMA: four VALU operations per 32 MACs.
//
// Workgroup tile 128 tokens x 128 rows, four waves of 64 x 64 (2 x 2 MFMA
// tiles).  Operands come straight from global memory (the token rows and
// weight rows are L2-resident across the grid): lane l reads the 16 codes
// k = 16*(l/32) .. +15 of token / weight row l % 32 for each block; Q4 codes
// become (q - 8) bytes with ((q | 0x80) - 8) ^ 0x80.  Activation scales are
// staged in LDS 16 blocks at a time.
#include "attn_core.h"
#include "gemv_core.h"

using namespace llmrs;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

constexpr int kBM = 128, kBN = 128;  // workgroup tile (tokens x rows)
constexpr int kKCH = 16;             // blocks of activation scales per LDS chunk

// 16 Q4 codes (low or high nibbles of a 16-byte block) as int8 (q - 8).
__device__ __forceinline__ v4i q4_bytes(u32x4 w, int high) {
  const unsigned M = 0x0F0F0F0Fu;
  u32x4 q;
  if (high) q = u32x4{(w.x >> 4) & M, (w.y >> 4) & M, (w.z >> 4) & M, (w.w >> 4) & M};
  else q = u32x4{w.x & M, w.y & M, w.z & M, w.w & M};
  // per byte: ((q + 128) - 8) - 128 without borrows between bytes
  const u32x4 r = ((q | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  return v4i{(int)r.x, (int)r.y, (int)r.z, (int)r.w};
}

template <int WT>
__device__ __forceinline__ void load_b(const PrefillGemmArgs& a, const uint8_t* row, size_t srow,
                                       int b, int high, v4i& bv, float& dw) {
  if (WT == WT_Q8H) {
    const i32x4 v = *(const i32x4*)(row + (size_t)b * 32 + 16 * high);
    bv = v4i{v.x, v.y, v.z, v.w};
  } else {
    bv = q4_bytes(*(const u32x4*)(row + (size_t)b * 16), high);
  }
  dw = wscale<WT>(load_wscale_raw<WT>(a.ws, srow + b));
}

}  // namespace

template <int WT, int EPI>
__device__ __forceinline__ void gemm_impl(const PrefillGemmArgs& a) {
  constexpr int BS = WT == WT_Q8H ? 32 : 16;
  __shared__ float s_da[kKCH][kBM];
  const int lane = lane_id(), wave = wave_id(), tid = threadIdx.x;
  const int half = lane >> 5, col = lane & 31;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int nb = a.K >> 5;

  const int8_t* arow[2];
  const uint8_t* brow[2];
  size_t srow[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int tok = min(m0 + wm + 32 * t + col, a.M - 1);
    arow[t] = a.xq + (size_t)tok * a.K + 16 * half;
    const int r = min(n0 + wn + 32 * t + col, a.N - 1);
    brow[t] = a.wq + (size_t)r * nb * BS;
    srow[t] = (size_t)r * nb;
  }

  float acc[2][2][16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][r][i] = 0.0f;

  // operands of the next block, loaded one block ahead
  v4i An[2], Bn[2];
  float dwn[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    An[t] = *(const v4i*)(arow[t]);
    load_b<WT>(a, brow[t], srow[t], 0, half, Bn[t], dwn[t]);
  }

  for (int b0 = 0; b0 < nb; b0 += kKCH) {
    __syncthreads();  // the previous chunk of scales is consumed
    for (int i = tid; i < kKCH * kBM; i += kThreads) {
      const int kb = i / kBM, t = i % kBM;
      const int tok = min(m0 + t, a.M - 1);
      s_da[kb][t] = (b0 + kb < nb) ? a.xd[(size_t)tok * nb + b0 + kb] : 0.0f;
    }
    __syncthreads();
    const int kend = min(kKCH, nb - b0);
    for (int kb = 0; kb < kend; ++kb) {
      const int b = b0 + kb;
      v4i A[2] = {An[0], An[1]}, B[2] = {Bn[0], Bn[1]};
      const float dw[2] = {dwn[0], dwn[1]};
      if (b + 1 < nb) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          An[t] = *(const v4i*)(arow[t] + (size_t)(b + 1) * 32);
          load_b<WT>(a, brow[t], srow[t], b + 1, half, Bn[t], dwn[t]);
        }
      }
      v16i p[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 2; ++r) p[t][r] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[t], B[r], v16i{}, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // token of register i: 8*(i/4) + 4*half + i%4 within the 32-token tile
        float da[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = *(const f32x4*)&s_da[kb][wm + 32 * t + 8 * g + 4 * half];
          da[4 * g] = v.x;
          da[4 * g + 1] = v.y;
          da[4 * g + 2] = v.z;
          da[4 * g + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int i = 0; i < 16; ++i)  // cpu.rs:913,932: total += isum * (d_w * d_a)
            acc[t][r][i] = acc[t][r][i] + (float)p[t][r][i] * (dw[r] * da[i]);
      }
    }
  }

  // Epilogues.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = m0 + wm + 32 * t + 8 * (i / 4) + 4 * half + (i % 4);
      if (EPI == EPI_SILU) {
        // rows n0+wn .. +31 are gate, +32 .. +63 the matching up rows
        // (layer.rs:72-79); m index j = (n0+wn)/2 + col.
        const float g = acc[t][0][i], u = acc[t][1][i];
        const float mv = (g / (1.0f + expf(-g))) * u;
        const int run = (n0 + wn) / 64;
        const int j = run * 32 + col;
        float amax = fabsf(mv);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
        const float d = amax / 127.0f;
        const float inv = amax == 0.0f ? 0.0f : 1.0f / d;
        if (tok < a.M && n0 + wn < a.N) {
          if (a.y) a.y[(size_t)tok * a.ldy + j] = mv;
          a.yq[(size_t)tok * (a.N / 2) + j] = amax == 0.0f ? (int8_t)0 : (int8_t)q8_code(mv, inv);
          if (col == 0) a.yd[(size_t)tok * (a.N / 64) + run] = amax == 0.0f ? 0.0f : d;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int row = n0 + wn + 32 * r + col;
          if (tok < a.M && row < a.N) {
            float v = acc[t][r][i];
            if (EPI == EPI_RESID) v = v + a.res[(size_t)tok * a.N + row];  // layer.rs:386,403
            a.y[(size_t)tok * a.ldy + row] = v;
          }
        }
      }
    }
  }
}

#define LLMRS_GEMM(name, WT, EPI)                                                 \
  extern "C" __global__ __launch_bounds__(kThreads) void name(PrefillGemmArgs a) { \
    gemm_impl<WT, EPI>(a);                                                        \
  }
LLMRS_GEMM(gemm_q4h_store, WT_Q4H, EPI_STORE)
LLMRS_GEMM(gemm_q4h_resid, WT_Q4H, EPI_RESID)
LLMRS_GEMM(gemm_q4h_silu, WT_Q4H, EPI_SILU)
LLMRS_GEMM(gemm_q4f_store, WT_Q4F, EPI_STORE)
LLMRS_GEMM(gemm_q4f_resid, WT_Q4F, EPI_RESID)
LLMRS_GEMM(gemm_q4f_silu, WT_Q4F, EPI_SILU)
LLMRS_GEMM(gemm_q8h_store, WT_Q8H, EPI_STORE)
LLMRS_GEMM(gemm_q8h_resid, WT_Q8H, EPI_RESID)
LLMRS_GEMM(gemm_q8h_silu, WT_Q8H, EPI_SILU)

// Per-row RMSNorm + Q8_0 (w != null) or plain Q8_0 (w == null): the GEMV
// prologue's arithmetic (same summation order), one workgroup per row, so a
// row gets the same codes here as in the decode path.
extern "C" __global__ __launch_bounds__(kThreads) void prefill_rows_q8(PrefillRowArgs r) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float s_red[kWaves];
  GemvArgs g{};
  g.k = r.dim;
  g.x = r.x;
  g.norm_w = r.w;
  g.eps = r.eps;
  const int nb = r.dim >> 5;
  int8_t* s_q = (int8_t*)smem;
  float* s_d = (float*)(smem + r.dim);
  int* s_off = (int*)(smem + r.dim + 4 * nb);
  const int row = blockIdx.x;
  if (r.w) load_activation<PRO_NORM, false, false>(g, row, s_q, s_d, s_off, s_red);
  else load_activation<PRO_QUANT, false, false>(g, row, s_q, s_d, s_off, s_red);
  __syncthreads();
  const i32x4* src = (const i32x4*)s_q;
  i32x4* dst = (i32x4*)(r.xq + (size_t)row * r.dim);
  for (int i = threadIdx.x; i < r.dim / 16; i += kThreads) dst[i] = src[i];
  for (int b = threadIdx.x; b < nb; b += kThreads) r.xd[(size_t)row * nb + b] = s_d[b];
}

// RoPE of q and k (cpu.rs:326-357, per head, position start_pos + t) and the
// K/V append (layer.rs:219-246): one thread per (token, head, pair).
extern "C" __global__ __launch_bounds__(256) void prefill_rope_kv(PrefillRopeArgs r) {
  const int mid = r.hd / 2;
  const int heads = r.nq + 2 * r.nkv;
  const long total = (long)r.M * heads * mid;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int j = (int)(i % mid);
    const int h = (int)((i / mid) % heads);
    const int t = (int)(i / ((long)mid * heads));
    const int pos = r.start_pos + t;
    const float* src = r.qkv + (size_t)t * r.qkv_rows + (size_t)h * r.hd;
    const float c = r.rope_cos[(size_t)pos * mid + j], s = r.rope_sin[(size_t)pos * mid + j];
    if (h < r.nq) {
      const float re = src[j], im = src[j + mid];
      float* q = r.q + (size_t)t * r.nq * r.hd + (size_t)h * r.hd;
      q[j] = re * c - im * s;
      q[j + mid] = re * s + im * c;
    } else if (h < r.nq + r.nkv) {
      const int g = h - r.nq;
      const float re = src[j], im = src[j + mid];
      const float k0 = re * c - im * s, k1 = re * s + im * c;
      const size_t o = ((size_t)g * r.max_seq + pos) * r.hd;
      if (r.kv16) {
        ((uint16_t*)r.kc)[o + j] = f2h(k0);
        ((uint16_t*)r.kc)[o + j + mid] = f2h(k1);
      } else {
        ((float*)r.kc)[o + j] = k0;
        ((float*)r.kc)[o + j + mid] = k1;
      }
    } else {
      const int g = h - r.nq - r.nkv;
      const size_t o = ((size_t)g * r.max_seq + pos) * r.hd;
      if (r.kv16) {
        ((uint16_t*)r.vc)[o + j] = f2h(src[j]);
        ((uint16_t*)r.vc)[o + j + mid] = f2h(src[j + mid]);
      } else {
        ((float*)r.vc)[o + j] = src[j];
        ((float*)r.vc)[o + j + mid] = src[j + mid];
      }
    }
  }
}

// Causal prefill attention (layer.rs:248-326): one workgroup per (32-query
// tile, query head).  Per key tile (64 positions for an f16 cache, 32 for
// f32): scores in 2 x 4 register blocks (f32 q times the stored K, staged in
// LDS in the cache's type), online softmax per query row (16-lane
// reductions), P.V in 2 x (HD/16) blocks; the causal mask keeps key
// j <= start_pos + t (layer.rs:264-266).  ctx is written as f32 and as Q8_0.
template <int HD, bool KV16>
__device__ __forceinline__ void attn_prefill_impl(const PrefillAttnArgs& a) {
  typedef typename KvType<KV16>::T kv_t;
  constexpr int QT = 32, KT = KV16 ? 64 : 32;
  constexpr int KPT = KT / 16;       // keys per thread in the score block
  constexpr int DPT = HD / 16;       // head dims per thread in P.V
  constexpr int KS = HD + (KV16 ? 8 : 4);  // padded LDS row (elements)
  __shared__ __align__(16) float s_q[QT][HD + 4];
  __shared__ __align__(16) kv_t s_k[KT][KS];
  __shared__ __align__(16) kv_t s_v[KT][KS];
  __shared__ float s_p[QT][KT + 4];

  const int tid = threadIdx.x;
  const int q0 = blockIdx.x * QT, h = blockIdx.y;
  const int g = h / (a.nq / a.nkv);
  const int qi = tid / 16, ki = tid % 16;  // rows 2qi, 2qi+1; keys KPT*ki..; dims DPT*ki..
  const int qdim = a.nq * HD;
  const kv_t* kc = (const kv_t*)a.kc + (size_t)g * a.max_seq * HD;
  const kv_t* vc = (const kv_t*)a.vc + (size_t)g * a.max_seq * HD;

  for (int i = tid; i < QT * HD; i += 256) {
    const int r = i / HD, d = i % HD;
    const int t = min(q0 + r, a.M - 1);
    s_q[r][d] = a.q[(size_t)t * qdim + (size_t)h * HD + d];
  }
  float m[2], l[2], o[2][DPT];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) o[r][e] = 0.0f;
  }
  // keys up to the last query's position
  const int kend = a.start_pos + min(q0 + QT, a.M);
  for (int k0 = 0; k0 < kend; k0 += KT) {
    __syncthreads();
#pragma unroll 2
    for (int i = tid; i < KT * HD; i += 256) {
      const int r = i / HD, d = i % HD;
      const int t = min(k0 + r, kend - 1);
      s_k[r][d] = kc[(size_t)t * HD + d];
      s_v[r][d] = vc[(size_t)t * HD + d];
    }
    __syncthreads();
    float sc[2][KPT];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < KPT; ++c) sc[r][c] = 0.0f;
#pragma unroll 2
    for (int d = 0; d < HD; d += 4) {
      f32x4 qv[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) qv[r] = *(const f32x4*)&s_q[2 * qi + r][d];
#pragma unroll
      for (int c = 0; c < KPT; ++c) {
        const kv_t* kr = &s_k[KPT * ki + c][d];
        const float k0f = kv_to_f<KV16>(kr[0]), k1f = kv_to_f<KV16>(kr[1]);
        const float k2f = kv_to_f<KV16>(kr[2]), k3f = kv_to_f<KV16>(kr[3]);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          float s2 = sc[r][c];
          s2 = __builtin_fmaf(qv[r].x, k0f, s2);
          s2 = __builtin_fmaf(qv[r].y, k1f, s2);
          s2 = __builtin_fmaf(qv[r].z, k2f, s2);
          s2 = __builtin_fmaf(qv[r].w, k3f, s2);
          sc[r][c] = s2;
        }
      }
    }
    // mask, online softmax per query row (16 lanes share a row pair)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int qpos = a.start_pos + q0 + 2 * qi + r;
      float rmax = -INFINITY;
#pragma unroll
      for (int c = 0; c < KPT; ++c) {
        const int kpos = k0 + KPT * ki + c;
        sc[r][c] = (kpos <= qpos && kpos < kend) ? sc[r][c] * a.scale : -INFINITY;
        rmax = fmaxf(rmax, sc[r][c]);
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) rmax = fmaxf(rmax, __shfl_xor(rmax, off, 16));
      const float mnew = fmaxf(m[r], rmax);
      const float corr = (m[r] == -INFINITY) ? 0.0f : expf(m[r] - mnew);
      float psum = 0.0f;
#pragma unroll
      for (int c = 0; c < KPT; ++c) {
        const float p = (sc[r][c] == -INFINITY) ? 0.0f : expf(sc[r][c] - mnew);
        s_p[2 * qi + r][KPT * ki + c] = p;
        psum += p;
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) psum += __shfl_xor(psum, off, 16);
      l[r] = l[r] * corr + psum;
      m[r] = mnew;
#pragma unroll
      for (int e = 0; e < DPT; ++e) o[r][e] = o[r][e] * corr;
    }
    __syncthreads();
    // P.V: rows 2qi.., dims DPT*ki..
    const int kvalid = min(KT, kend - k0);
#pragma unroll 4
    for (int kk = 0; kk < kvalid; ++kk) {
      const float p0 = s_p[2 * qi][kk], p1 = s_p[2 * qi + 1][kk];
      const kv_t* vr = &s_v[kk][DPT * ki];
#pragma unroll
      for (int e = 0; e < DPT; ++e) {
        const float vv = kv_to_f<KV16>(vr[e]);
        o[0][e] = __builtin_fmaf(p0, vv, o[0][e]);
        o[1][e] = __builtin_fmaf(p1, vv, o[1][e]);
      }
    }
  }
  // ctx rows (f32 and Q8_0): a 32-dim block spans 32/DPT threads of a row.
  constexpr int TPB = 32 / DPT;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int t = q0 + 2 * qi + r;
    float v[DPT];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      v[e] = o[r][e] / l[r];
      amax = fmaxf(amax, fabsf(v[e]));
    }
#pragma unroll
    for (int off = TPB / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, TPB));
    const float d = amax / 127.0f;
    const float inv = amax == 0.0f ? 0.0f : 1.0f / d;
    if (t < a.M) {
      const size_t base = (size_t)t * qdim + (size_t)h * HD + DPT * ki;
#pragma unroll
      for (int e = 0; e < DPT; ++e) {
        if (a.ctx) a.ctx[base + e] = v[e];
        a.ctx_q[base + e] = amax == 0.0f ? (int8_t)0 : (int8_t)q8_code(v[e], inv);
      }
      if ((ki % TPB) == 0) a.ctx_d[base / 32] = amax == 0.0f ? 0.0f : d;
    }
  }
}

#define LLMRS_ATTN_PREFILL(name, HD, KV16)                                        \
  extern "C" __global__ __launch_bounds__(256) void name(PrefillAttnArgs a) {   \
    attn_prefill_impl<HD, KV16>(a);                                             \
  }
LLMRS_ATTN_PREFILL(attn_prefill_hd64_f32, 64, false)
LLMRS_ATTN_PREFILL(attn_prefill_hd64_f16, 64, true)
LLMRS_ATTN_PREFILL(attn_prefill_hd128_f32, 128, false)
LLMRS_ATTN_PREFILL(attn_prefill_hd128_f16, 128, true)
