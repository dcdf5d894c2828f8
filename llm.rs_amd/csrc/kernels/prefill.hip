// prefill.hip - batched prompt processing (prefill) for gfx950.
//
// Reference: LlamaModel::forward over a chunk of M tokens (model.rs:17-49,
// layer.rs:373-406; the prompt step of main.rs:134-190).  The reference's
// M > 1 GEMM quantises every activation row to Q8_0 and runs the Q4 x Q8
// block loop per output element (cpu.rs:90-110, kernel_avx2 cpu.rs:888-941):
//   y[t][r] = (...((0 + isum_0 * s_0) + isum_1 * s_1) + ...),  s_b = d_w[r,b] * d_a[t,b]
// with isum_b the exact int32 dot product of one 32-element block.
//
// gemm_*: per 32-element block and 32 x 32 (token x row) tile, one
// v_mfma_i32_32x32x32_i8 gives every isum_b exactly, and one two-block
// v_mfma_f32_32x32x1_2b_f32 per token tile gives the scales
// s_b = d_w * d_a of both row tiles, each as a single IEEE product (round to
// nearest even, the same value as the reference's f32 multiply).  Lane
// 32 blk + i supplies row / column i of block blk, and block blk's results
// sit in registers 16 blk .. 16 blk + 15 in the layout of a one-block
// 32 x 32 MFMA (checked on the device), so no operand is wasted.  The epilogue per element and
// block is then the reference's own two roundings, total = total + isum * s,
// in block order, so every output is bit-identical to the reference for
// identical activation codes.  Three VALU operations per element and block
// (convert, multiply, add) bound the kernel, not the MFMA.
//
// Workgroup tile 128 tokens x 128 rows, four waves of 64 x 64 (2 x 2 MFMA
// tiles).  Operands are staged in LDS four blocks at a time, double-buffered:
// the global loads of stage s+1 are issued before stage s is computed and
// written to LDS after it, so their latency hides behind a whole stage.
// LDS layouts make each MFMA operand read conflict-free: 16-byte chunk
// (c, token) lives at c * 128 + (token ^ c), so the 32 lanes of a half-wave
// read 32 distinct consecutive chunks.  Q4 codes become (q - 8) bytes with
// ((q | 0x80) - 8) ^ 0x80.
#include "attn_core.h"
#include "exact_math.h"
#include "gemv_core.h"

using namespace llmrs;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

namespace {

#ifndef LLMRS_GEMM_WAVES
#define LLMRS_GEMM_WAVES 2    // workgroups per CU the register budget allows
#endif
constexpr int kBM = 128, kBN = 128;  // workgroup tile (tokens x rows)
constexpr int kKB = 4;               // 32-element blocks per pipeline stage

// 16 Q4 codes (low or high nibbles of a 16-byte block) as int8 (q - 8).
// Branch-free: the half-wave selects its nibble with a per-lane shift.
__device__ __forceinline__ v4i q4_bytes(u32x4 w, int high) {
  const unsigned M = 0x0F0F0F0Fu, sh = 4u * (unsigned)high;
  const u32x4 q = u32x4{(w.x >> sh) & M, (w.y >> sh) & M, (w.z >> sh) & M, (w.w >> sh) & M};
  // per byte: ((q + 128) - 8) - 128 without borrows between bytes
  const u32x4 r = ((q | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  return v4i{(int)r.x, (int)r.y, (int)r.z, (int)r.w};
}

// LDS of one pipeline stage (bytes): activation codes and weight codes as
// int8 in 16-byte chunks, chunk (c, i) at c * 128 + (i ^ c) for c = 2 b + h
// (codes 16 h .. 16 h + 15 of block b) and token / row i, then f32 scales
// d_w [kKB][SW] and d_a [kKB][SW] (rows padded by 4).  A half-wave's MFMA
// operand read is a permutation of 32 consecutive chunks, and the XOR and
// the padding spread the staging writes (8 chunks of one token, 4 scales of
// one row) over distinct banks.
struct GemmStage {
  static constexpr int A = 0;
  static constexpr int B = A + 2 * kKB * kBM * 16;
  static constexpr int DW = B + 2 * kKB * kBN * 16;
  static constexpr int SW = kBN + 4;            // padded scale row (floats)
  static constexpr int DA = DW + kKB * SW * 4;
  static constexpr int BYTES = DA + kKB * SW * 4;
};

template <int WT>
struct GemmLoads {
  static constexpr int BCH = WT == WT_Q8H ? 2 : 1;             // 16-byte chunks per weight block
  static constexpr int A_PER_T = 2 * kKB * kBM / 256;          // activation chunks per thread
  static constexpr int B_PER_T = kKB * BCH * kBN / 256;        // weight chunks per thread
  static constexpr int S_PER_T = kKB * kBN / 256;              // scales per thread (d_w and d_a)
};

// MFMA operands of one block for a wave's 2 x 2 tiles: codes, d_a of the
// lane's token in each token tile, d_w of the lane's row in row tile
// `half` (the two-block scale MFMA takes row tile blk from lanes 32 blk..).
struct GemmOps {
  v4i A[2], B[2];
  float da[2], dw;
};

}  // namespace

// First token and row of this workgroup's tile (PrefillGemmArgs::group_m).
// Both steps are bijections on [0, tiles): the XCD deal when the tile count
// is a multiple of 8, the grouped walk for any grid.
__device__ __forceinline__ void gemm_tile(const PrefillGemmArgs& a, int& m0, int& n0) {
  const int gx = gridDim.x, gy = gridDim.y, T = gx * gy;
  if (a.group_m <= 0) {
    m0 = blockIdx.y * kBM;
    n0 = blockIdx.x * kBN;
    return;
  }
  int t = blockIdx.x + blockIdx.y * gx;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int gsz = a.group_m * gx, g = t / gsz, fm = g * a.group_m;
  const int gm = min(gy - fm, a.group_m), r = t - g * gsz;
  m0 = (fm + r % gm) * kBM;
  n0 = (r / gm) * kBN;
}

template <int WT, int EPI>
__device__ __forceinline__ void gemm_impl(const PrefillGemmArgs& a, uint8_t* lds) {
  typedef GemmStage S;
  typedef GemmLoads<WT> G;
  constexpr int BCH = G::BCH;
  const int lane = lane_id(), wave = wave_id(), tid = threadIdx.x;
  const int half = lane >> 5, col = lane & 31;
  int m0, n0;
  gemm_tile(a, m0, n0);
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int nb = a.K >> 5;
  const int nstage = (nb + kKB - 1) / kKB;

  // ---- staging: global -> registers -> LDS -------------------------------
  // activation chunk q: token q / (2 kKB), c = q % (2 kKB); weight chunk q:
  // row q / (kKB BCH), chunk q % (kKB BCH) of that row's stage bytes;
  // scales: (token | row) q / kKB, block q % kKB.  Scales stay raw until the
  // LDS write, so nothing waits on the loads before the stage's compute.
  i32x4 ra[G::A_PER_T], rb[G::B_PER_T];
  unsigned rdw[G::S_PER_T];
  float rda[G::S_PER_T];
  auto load_stage = [&](int st) {
    const int b0 = st * kKB;
#pragma unroll
    for (int j = 0; j < G::A_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int tok = min(m0 + q / (2 * kKB), a.M - 1);
      const int c = q % (2 * kKB);
      const int blk = min(b0 + c / 2, nb - 1);
      ra[j] = *(const i32x4*)(a.xq + (size_t)tok * a.K + (size_t)blk * 32 + 16 * (c & 1));
    }
#pragma unroll
    for (int j = 0; j < G::B_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int row = min(n0 + q / (kKB * BCH), a.N - 1);
      const int c = q % (kKB * BCH);
      const int blk = min(b0 + c / BCH, nb - 1);
      rb[j] = *(const i32x4*)(a.wq + ((size_t)row * nb + blk) * (16 * BCH) + 16 * (c % BCH));
    }
#pragma unroll
    for (int j = 0; j < G::S_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int blk = min(b0 + q % kKB, nb - 1);
      const int row = min(n0 + q / kKB, a.N - 1);
      const size_t si = (size_t)row * nb + blk;
      rdw[j] = WT == WT_Q4F ? ((const unsigned*)a.ws)[si] : ((const uint16_t*)a.ws)[si];
      const int tok = min(m0 + q / kKB, a.M - 1);
      rda[j] = a.xd[(size_t)tok * nb + blk];
    }
  };
  auto store_stage = [&](int buf) {
    uint8_t* base = lds + buf * S::BYTES;
#pragma unroll
    for (int j = 0; j < G::A_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int tok = q / (2 * kKB), c = q % (2 * kKB);
      *(i32x4*)(base + S::A + (c * kBM + (tok ^ c)) * 16) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < G::B_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int row = q / (kKB * BCH), c = q % (kKB * BCH);
      if (WT == WT_Q8H) {
        *(i32x4*)(base + S::B + (c * kBN + (row ^ c)) * 16) = rb[j];
      } else {  // one Q4 block: low nibbles are codes 0..15, high 16..31
        const u32x4 w = u32x4{(unsigned)rb[j].x, (unsigned)rb[j].y, (unsigned)rb[j].z, (unsigned)rb[j].w};
        const v4i lo = q4_bytes(w, 0), hi = q4_bytes(w, 1);
        *(v4i*)(base + S::B + ((2 * c) * kBN + (row ^ (2 * c))) * 16) = lo;
        *(v4i*)(base + S::B + ((2 * c + 1) * kBN + (row ^ (2 * c + 1))) * 16) = hi;
      }
    }
#pragma unroll
    for (int j = 0; j < G::S_PER_T; ++j) {
      const int q = tid + 256 * j;
      const int b = q % kKB, r = q / kKB;
      ((float*)(base + S::DW))[b * S::SW + r] = wscale<WT>(rdw[j]);
      ((float*)(base + S::DA))[b * S::SW + r] = rda[j];
    }
  };

  // ---- compute -------------------------------------------------------------
  // Per-lane LDS offsets of the operands (the block adds a constant).
  int offA[2], offB[2], offDA[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    offA[t] = S::A + (half * kBM + wm + 32 * t) * 16;  // + (col ^ c) per block
    offB[t] = S::B + (half * kBN + wn + 32 * t) * 16;
    offDA[t] = S::DA + (wm + 32 * t + col) * 4;
  }
  const int offDW = S::DW + (wn + 32 * half + col) * 4;  // row tile `half` (two-block MFMA)
  auto load_ops = [&](const uint8_t* base, int b, GemmOps& o) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int cx = (col ^ half) ^ (2 * b);  // token / row swizzle of chunk c = 2 b + half
      const i32x4 va = *(const i32x4*)(base + offA[t] + (b * (2 * kBM) + cx) * 16);
      o.A[t] = v4i{va.x, va.y, va.z, va.w};
      const i32x4 vb = *(const i32x4*)(base + offB[t] + (b * (2 * kBN) + cx) * 16);
      o.B[t] = v4i{vb.x, vb.y, vb.z, vb.w};
      o.da[t] = *(const float*)(base + offDA[t] + b * (S::SW * 4));
    }
    o.dw = *(const float*)(base + offDW + b * (S::SW * 4));
  };

  float acc[2][2][16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][r][i] = 0.0f;
  // sc: both row tiles' scales of token tile t (registers 16 r ..).
  auto epi = [&](int t, int r, const v16i& p, const v32f& sc) {
#pragma unroll
    for (int i = 0; i < 16; ++i)  // cpu.rs:913,932: total += isum * (d_w * d_a)
      acc[t][r][i] = acc[t][r][i] + (float)p[i] * sc[16 * r + i];
  };

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int st = 0; st < nstage; ++st) {
    if (st + 1 < nstage) load_stage(st + 1);
    const uint8_t* base = lds + (st & 1) * S::BYTES;
    const int kvalid = min(kKB, nb - st * kKB);
    if (kvalid == kKB) {
      // Software pipeline over the stage's 4 kKB tiles k = 4 b + 2 t + r:
      // the MFMAs of tile k+1 are issued before the VALU work of tile k, and
      // the operands of block b+1 are read while block b is in flight.
      GemmOps o[2];
      v16i P[2];
      v32f SC;  // scales of the current (block, token tile) pair, both row tiles
      load_ops(base, 0, o[0]);
      P[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o[0].A[0], o[0].B[0], v16i{}, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < 4 * kKB; ++k) {
        const int b = k / 4, t = (k / 2) % 2, r = k % 2;
        // The pair's scale MFMA at its r = 0 tile, then the next tile's
        // integer MFMA, whose issue covers the scale MFMA's latency.
        if (r == 0) SC = __builtin_amdgcn_mfma_f32_32x32x1f32(o[b % 2].da[t], o[b % 2].dw, v32f{}, 0, 0, 0);
        if (k % 4 == 0 && b + 1 < kKB) load_ops(base, b + 1, o[(b + 1) % 2]);
        if (k + 1 < 4 * kKB) {
          const int kn = k + 1;
          const GemmOps& on = o[(kn / 4) % 2];
          P[kn % 2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(on.A[(kn / 2) % 2], on.B[kn % 2], v16i{}, 0, 0, 0);
        }
        epi(t, r, P[k % 2], SC);
      }
    } else {
      for (int b = 0; b < kvalid; ++b) {
        GemmOps o;
        load_ops(base, b, o);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(o.da[t], o.dw, v32f{}, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.A[t], o.B[r], v16i{}, 0, 0, 0);
            epi(t, r, p, sc);
          }
        }
      }
    }
    if (st + 1 < nstage) store_stage((st + 1) & 1);
    __syncthreads();
  }

  // Epilogues.  Register i of a tile holds token 8 (i / 4) + 4 half + i % 4
  // and row col.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = m0 + wm + 32 * t + 8 * (i / 4) + 4 * half + (i % 4);
      if (EPI == EPI_SILU) {
        // rows n0+wn .. +31 are gate, +32 .. +63 the matching up rows
        // (layer.rs:72-79); m index j = (n0+wn)/2 + col.
        const float g = acc[t][0][i], u = acc[t][1][i];
        const float mv = (g / (1.0f + exact_expf(-g))) * u;  // glibc expf (exact_math.h)
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

// Dynamic LDS: two pipeline stages, gemm_lds_bytes(weights) at launch.
static_assert(2 * GemmStage::BYTES == gemm_lds_bytes(), "GEMM LDS size");
#define LLMRS_GEMM(name, WT, EPI)                                                 \
  extern "C" __global__ __launch_bounds__(kThreads, LLMRS_GEMM_WAVES) void name(PrefillGemmArgs a) { \
    extern __shared__ __align__(16) uint8_t gemm_lds[];                            \
    gemm_impl<WT, EPI>(a, gemm_lds);                                              \
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
  if (r.layout == kActNatural) {
    const i32x4* src = (const i32x4*)s_q;
    i32x4* dst = (i32x4*)(r.xq + (size_t)row * r.dim);
    for (int i = threadIdx.x; i < r.dim / 16; i += kThreads) dst[i] = src[i];
  } else {
    int8_t* dst = r.xq + (size_t)row * r.dim;
    for (int i = threadIdx.x; i < r.dim; i += kThreads) dst[act_offset(i, r.layout)] = s_q[i];
  }
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
      if (r.kv16) {  // blocked V layout (v_offset)
        const size_t hb = (size_t)g * r.max_seq * r.hd;
        ((uint16_t*)r.vc)[hb + v_offset(pos, j, r.hd, true)] = f2h(src[j]);
        ((uint16_t*)r.vc)[hb + v_offset(pos, j + mid, r.hd, true)] = f2h(src[j + mid]);
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
      s_v[r][d] = vc[v_offset(t, d, HD, KV16)];
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
        a.ctx_q[(size_t)t * qdim + act_offset(h * HD + DPT * ki + e, a.ctx_layout)] =
            amax == 0.0f ? (int8_t)0 : (int8_t)q8_code(v[e], inv);
      }
      if ((ki % TPB) == 0) a.ctx_d[base / 32] = amax == 0.0f ? 0.0f : d;
    }
  }
}

// Causal prefill attention on the matrix cores, f16 K/V cache.  One
// workgroup of 8 waves per (32-query tile, KV group): wave w takes query head
// g * n_rep + w % 4 (+4, +8, ... for larger groups) and key stream w / 4,
// which covers the even or odd key tiles, so the four heads share each
// staged K/V tile and the two streams halve the serial path of long tiles.
// Per key tile of 32:
//   S^T = K Q^T        (v_mfma_f32_32x32x16_f16; q split into f16 hi + lo,
//                       so the products carry ~22 bits of q, as in f32)
//   online softmax      one query per lane column: row max / sum over the
//                       lane's 16 keys and its partner lane's 16; exp as
//                       exp2 of log2(e)-scaled scores
//   O^T += V^T P^T      (P split into f16 hi + lo; keys taken in the order
//                       the S^T registers hold them, V^T staged to match)
// The two streams' (max, sum, O) are merged through LDS at the end.  The
// causal mask keeps key j <= start_pos + t (layer.rs:264-266).  Query tiles
// run longest-first.  ctx is written as Q8_0 (and f32 when asked).
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

template <int HD>
struct AttnMfmaLds {
  static constexpr int KT = 32;                 // keys per tile
  static constexpr int KROW = HD * 2 + 16;      // padded K row (bytes)
  static constexpr int VROW = KT * 2 + 8;       // padded V^T row (bytes)
  static constexpr int K = 0;
  static constexpr int V = K + KT * KROW;
  static constexpr int TILE = V + HD * VROW;    // one staged tile
  static constexpr int BYTES = 2 * TILE;        // the even and odd tiles
  // merge area (reuses the tiles): per head, lane: 16 O values of one pass + m, l
  static constexpr int MERGE = 4 * 64 * 18 * 4;
  static_assert(MERGE <= BYTES, "merge area fits in the tile buffers");
};

template <int HD>
__device__ __forceinline__ void attn_prefill_mfma_impl(const PrefillAttnArgs& a) {
  typedef AttnMfmaLds<HD> LY;
  constexpr int NS = HD / 16, ND = HD / 32, KT = LY::KT;
  constexpr float kLog2e = 1.4426950408889634f;
  __shared__ __align__(16) uint8_t lds[LY::BYTES];
  const int lane = lane_id(), wave = wave_id(), tid = threadIdx.x;
  const int h2 = lane >> 5, col = lane & 31;
  const int hw = wave & 3, stream = wave >> 2;
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 32, g = blockIdx.y;  // longest tiles first
  const int n_rep = a.nq / a.nkv;
  const int qdim = a.nq * HD;
  const uint16_t* kc = (const uint16_t*)a.kc + (size_t)g * a.max_seq * HD;
  const uint16_t* vc = (const uint16_t*)a.vc + (size_t)g * a.max_seq * HD;
  const int kend = a.start_pos + min(q0 + 32, a.M);  // keys [0, kend)
  const int ntile = (kend + KT - 1) / KT;
  const int npair = (ntile + 1) / 2;
  const int myq = q0 + col;
  const int qpos = a.start_pos + myq;
  const float sl2 = a.scale * kLog2e;

  for (int rp = 0; rp < n_rep; rp += 4) {
    const int r = rp + hw;
    const bool active = r < n_rep;  // wave-uniform
    const int h = g * n_rep + min(r, n_rep - 1);
    v8h qh[NS], ql[NS];
    {
      const float* qrow = a.q + (size_t)min(myq, a.M - 1) * qdim + (size_t)h * HD;
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        const f32x4 x0 = *(const f32x4*)(qrow + 16 * sl + 8 * h2);
        const f32x4 x1 = *(const f32x4*)(qrow + 16 * sl + 8 * h2 + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const _Float16 hi = (_Float16)xv[j];
          qh[sl][j] = hi;
          ql[sl][j] = (_Float16)(xv[j] - (float)hi);
        }
      }
    }
    v16f o[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = v16f{};
    float m = -INFINITY, l = 0.0f;  // m in the log2 domain

    // K rows [key][HD] and V^T [HD][key] of tile pair (2i, 2i+1): thread
    // chunk c < 2 * 32 * HD / 8 = (tile c / (32 HD / 8), then key and 8-dim
    // part of K, or dim and 8-key block of the blocked V); keys clamped
    // (those past kend are masked below).  Loaded a pair ahead.
    constexpr int CPT = 2 * KT * HD / 8 / 512;
    u32x4 rk[CPT], rv[CPT];
    auto fetch = [&](int pr) {
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int c = tid + 512 * j;
        const int t = c / (KT * HD / 8), cc = c % (KT * HD / 8);
        const int key = cc / (HD / 8), part = cc % (HD / 8);
        rk[j] = *(const u32x4*)(kc + (size_t)min((2 * pr + t) * KT + key, kend - 1) * HD + part * 8);
        const int vb = cc / HD, vd = cc % HD;
        rv[j] = *(const u32x4*)(vc + v_offset(min((2 * pr + t) * KT + 8 * vb, kend - 1) & ~7, vd, HD, true));
      }
    };
    fetch(0);
    for (int pr = 0; pr < npair; ++pr) {
      __syncthreads();  // the previous pair is consumed
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int c = tid + 512 * j;
        const int t = c / (KT * HD / 8), cc = c % (KT * HD / 8);
        const int key = cc / (HD / 8), part = cc % (HD / 8);
        uint8_t* tb = lds + t * LY::TILE;
        *(u32x4*)(tb + LY::K + key * LY::KROW + part * 16) = rk[j];
        const int vb = cc / HD, vd = cc % HD;  // keys 8 vb .. 8 vb + 7 of dim vd
        uint2* vdst = (uint2*)(tb + LY::V + vd * LY::VROW + vb * 16);
        vdst[0] = make_uint2(rv[j].x, rv[j].y);
        vdst[1] = make_uint2(rv[j].z, rv[j].w);
      }
      __syncthreads();
      if (pr + 1 < npair) fetch(pr + 1);
      const int kt = 2 * pr + stream;
      if (!active || kt >= ntile) continue;
      const uint8_t* tb = lds + stream * LY::TILE;
      // S^T: lane holds keys kt*32 + 8(i/4) + 4 h2 + i%4 for query col
      v16f st = v16f{};
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        const v8h kop = *(const v8h*)(tb + LY::K + col * LY::KROW + (16 * sl + 8 * h2) * 2);
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qh[sl], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, ql[sl], st, 0, 0, 0);
      }
      float p[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kt * KT + 8 * (i / 4) + 4 * h2 + (i % 4);
        p[i] = key <= qpos ? st[i] * sl2 : -INFINITY;
        mloc = fmaxf(mloc, p[i]);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      // The stream's first tile holds a key <= qpos for every query (key 0
      // or, for stream 1, key 32 <= qpos whenever that tile is reached with
      // an unmasked key); a fully masked tile keeps mn = m.
      const float mn = fmaxf(m, mloc);
      const float corr = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
      float lsum = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(p[i] - mn);
        lsum += p[i];
      }
      lsum += __shfl_xor(lsum, 32);
      l = l * corr + lsum;
      m = mn;
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[d][i] *= corr;
      // O^T += V^T P^T over the two 16-key slices
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        v8h ph, pl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = p[8 * s2 + j];
          const _Float16 hi = (_Float16)x;
          ph[j] = hi;
          pl[j] = (_Float16)(x - (float)hi);
        }
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          const uint8_t* vrow = tb + LY::V + (32 * d + col) * LY::VROW;
          const v4h v0 = *(const v4h*)(vrow + (16 * s2 + 4 * h2) * 2);
          const v4h v1 = *(const v4h*)(vrow + (16 * s2 + 8 + 4 * h2) * 2);
          const v8h vop = v8h{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, ph, o[d], 0, 0, 0);
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pl, o[d], 0, 0, 0);
        }
      }
    }
    // Merge stream 1 into stream 0 through LDS, one 32-dim block at a time.
    float* mg = (float*)lds + (hw * 64 + lane) * 18;
    float m1 = -INFINITY, l1 = 0.0f, c0 = 1.0f, c1 = 0.0f;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      __syncthreads();  // tiles (or the previous block) consumed
      if (stream == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) mg[i] = o[d][i];
        mg[16] = m;
        mg[17] = l;
      }
      __syncthreads();
      if (stream == 0) {
        if (d == 0) {
          m1 = mg[16];
          l1 = mg[17];
          const float mm = fmaxf(m, m1);  // finite: stream 0 saw key 0
          c0 = __builtin_amdgcn_exp2f(m - mm);
          c1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
          l = l * c0 + l1 * c1;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) o[d][i] = o[d][i] * c0 + mg[i] * c1;
      }
    }
    __syncthreads();  // merge reads done before the next pass stages tiles
    if (!active || stream != 0) continue;
    // o[d][i] = O[query col][dim 32 d + 8 (i/4) + 4 h2 + i%4] * l
    const float inv_l = 1.0f / l;
    const bool write = myq < a.M;
    const size_t base = (size_t)min(myq, a.M - 1) * qdim + (size_t)h * HD;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      float v[16];
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        v[i] = o[d][i] * inv_l;
        amax = fmaxf(amax, fabsf(v[i]));
      }
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const float dq = amax / 127.0f;
      const float inv = amax == 0.0f ? 0.0f : 1.0f / dq;
      if (write) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const size_t e = base + 32 * d + 8 * gq + 4 * h2;
          unsigned w = 0;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int q8 = amax == 0.0f ? 0 : q8_code(v[4 * gq + c], inv);
            w |= ((unsigned)q8 & 0xFFu) << (8 * c);
          }
          *(unsigned*)(a.ctx_q + (base - (size_t)h * HD) +
                       act_offset(h * HD + 32 * d + 8 * gq + 4 * h2, a.ctx_layout)) = w;
          if (a.ctx) *(f32x4*)(a.ctx + e) = f32x4{v[4 * gq], v[4 * gq + 1], v[4 * gq + 2], v[4 * gq + 3]};
        }
        if (h2 == 0) a.ctx_d[base / 32 + d] = amax == 0.0f ? 0.0f : dq;
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(512) void attn_prefill_mfma_hd64(PrefillAttnArgs a) {
  attn_prefill_mfma_impl<64>(a);
}
extern "C" __global__ __launch_bounds__(512) void attn_prefill_mfma_hd128(PrefillAttnArgs a) {
  attn_prefill_mfma_impl<128>(a);
}

#define LLMRS_ATTN_PREFILL(name, HD, KV16)                                        \
  extern "C" __global__ __launch_bounds__(256) void name(PrefillAttnArgs a) {   \
    attn_prefill_impl<HD, KV16>(a);                                             \
  }
LLMRS_ATTN_PREFILL(attn_prefill_hd64_f32, 64, false)
LLMRS_ATTN_PREFILL(attn_prefill_hd64_f16, 64, true)
LLMRS_ATTN_PREFILL(attn_prefill_hd128_f32, 128, false)
LLMRS_ATTN_PREFILL(attn_prefill_hd128_f16, 128, true)
