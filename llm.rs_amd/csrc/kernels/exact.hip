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
//                   b = 0, 1, ... (kernel_avx2, cpu.rs:903-938); the block
//                   terms are computed lane-parallel and parked in LDS, and
//                   one lane per row adds them in block order
//   exact_attn_*    one workgroup per query head: RoPE (cpu.rs:345-354),
//                   K/V append, sequential q.k dots (matmul_slice,
//                   cpu.rs:230-269) times 1/sqrt(hd) (layer.rs:257-258),
//                   softmax with a sequential sum (cpu.rs:395-423), P.V
//                   sequential over positions (layer.rs:276-299), ctx Q8_0
//   exact_gemv_*_silu  the gate|up GEMV (same block order) finished with
//                   g / (1 + exp(-g)) * u (layer.rs:75-79) with glibc's expf
//                   (exact_math.h) and the Q8_0 of the product
// The lm_head runs exact_gemv with the argmax partials of argmax_final.
// A prompt of M rows runs as the reference's batched forward does, row by
// row in its per-row orders: exact_norm_q8 over the M rows (one workgroup
// each), the prefill GEMMs (prefill.hip, sgemm.hip: the same block loop,
// bit-identical, glibc's expf in their SwiGLU epilogue), the prefill RoPE /
// append, and exact_attn_prefill_* (one workgroup per query head and row).
#include "common.h"
#include "exact_math.h"
#include "gemv_core.h"
#include "../kernel_args.h"

using namespace llmrs;

namespace {

constexpr int kT = 256;

// ---- sequential sums by chunks ---------------------------------------------
// The reference folds sums in index order, one rounding per term:
//   sum = (...((0 + v[0]) + v[1]) + ...) + v[n-1]
// (the RMSNorm sum of squares, cpu.rs:381; the softmax denominator,
// cpu.rs:413-415).  seq_sum evaluates that fold with the NW waves of a
// workgroup: wave c owns chunk c (NW chunks of equal length in index order)
// and folds it from kWin consecutive f32 start values at once, one per lane,
// centred on the exact sum of the terms before the chunk (added in f64):
// lane l starts at the float whose bit pattern is the centre's plus
// l - kWin/2.  A fold from a given start is a fixed sequence of IEEE
// additions, so when the sequential total at the chunk's start is one of
// those floats, the lane that started there ends with exactly the sequential
// total at the chunk's end.  Wave 0 then walks the chunks in order, with
// every chunk's ends in registers (lane l: the end from start l), and takes
// each chunk's end by the bit distance of the running total from the chunk's
// centre; when the total lies outside the window (the rounding drift of a
// long run of equal terms, for instance) it folds that chunk itself from the
// total.  Either way the result is the sequential fold, bit for bit.  On
// real rows of non-negative terms the fold drifts from the exact sum by well
// under kWin/2 ulps at every chunk start, so the walk rarely folds.
constexpr int kWin = LLMRS_WAVE;  // start values per chunk, one per lane

template <int NW>
struct FoldShared {
  double part[NW];      // sum of each chunk's terms (f64)
  unsigned centre[NW];  // bit pattern of each chunk's centre start value
  float end[NW][kWin];  // chunk c folded from the start value of lane l
  float total;
};

// One lane's fold of v[i0..i1) from acc in index order (i1 - i0 a multiple
// of 32, i0 a multiple of 4, v 16-byte aligned), reading the terms 32 at a
// time with the next 32 requested before the current ones are added.  With
// constant bounds the compiler unrolls it completely.
__device__ __forceinline__ float fold_range(const float* v, int i0, int i1, float acc) {
  if (i0 >= i1) return acc;
  f32x4 A[8], B[8];
  auto load = [&](f32x4 (&r)[8], int i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = *(const f32x4*)(v + i + 4 * j);
  };
  auto add = [&](const f32x4 (&r)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc = acc + r[j][0];
      acc = acc + r[j][1];
      acc = acc + r[j][2];
      acc = acc + r[j][3];
    }
  };
  load(A, i0);
  for (int i = i0;; i += 64) {
    const bool more = i + 32 < i1;
    if (more) load(B, i + 32);
    add(A);
    if (!more) break;
    const bool more2 = i + 64 < i1;
    if (more2) load(A, i + 64);
    add(B);
    if (!more2) break;
  }
  return acc;
}
// The same for any i1 >= i0: whole groups of 32, then the rest one by one.
__device__ __forceinline__ float fold_any(const float* v, int i0, int i1, float acc) {
  const int i32 = i0 + (i1 - i0) / 32 * 32;
  acc = fold_range(v, i0, i32, acc);
  for (int i = i32; i < i1; ++i) acc = acc + v[i];
  return acc;
}

// Wave64 sum of doubles with DPP row operations (as wave_sum); uniform.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v = v + dpp_d<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_d<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_d<0x141>(v);  // row_half_mirror
  v = v + dpp_d<0x140>(v);  // row_mirror
  return ((readlane_d(v, 0) + readlane_d(v, 16)) + readlane_d(v, 32)) + readlane_d(v, 48);
}

// The sequential sum of v[0..n) (v in LDS, 16-byte aligned, written before
// the call and visible to every thread), by all NW waves of the workgroup;
// every thread returns it.  WHOLE32: n is a multiple of 32 (so is every
// chunk).
template <int NW, bool WHOLE32>
__device__ __forceinline__ float seq_sum(const float* v, int n, FoldShared<NW>& sh) {
  const int lane = lane_id(), wave = wave_id();
  const int len = (n + NW * 32 - 1) / (NW * 32) * 32;
  const int c0 = min(wave * len, n), c1 = min(c0 + len, n);
  double p = 0.0;
  for (int i = c0 + lane; i < c1; i += LLMRS_WAVE) p += (double)v[i];
  p = wave_sum_d(p);
  if (lane == 0) sh.part[wave] = p;
  __syncthreads();
  double before = 0.0;
  for (int c = 0; c < wave; ++c) before += sh.part[c];
  const unsigned centre = __float_as_uint((float)before);
  // chunk 0 starts from the fold's own 0
  const float start = wave == 0 ? 0.0f : __uint_as_float(centre + (unsigned)lane - (unsigned)(kWin / 2));
  sh.end[wave][lane] = WHOLE32 ? fold_range(v, c0, c1, start) : fold_any(v, c0, c1, start);
  if (lane == 0) sh.centre[wave] = centre;
  __syncthreads();
  if (wave == 0) {  // the walk, uniform over wave 0
    float e[NW];
#pragma unroll
    for (int c = 0; c < NW; ++c) e[c] = sh.end[c][lane];
    float ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[0]), 0));
#pragma unroll
    for (int c = 1; c < NW; ++c) {
      if (c * len < n) {
        const unsigned cen = (unsigned)__builtin_amdgcn_readfirstlane((int)sh.centre[c]);
        const unsigned j = __float_as_uint(ss) - cen + (unsigned)(kWin / 2);
        const float f = j < (unsigned)kWin ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[c]), (int)j))
                                           : WHOLE32 ? fold_range(v, c * len, min(c * len + len, n), ss)
                                                     : fold_any(v, c * len, min(c * len + len, n), ss);
        ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f)));
      }
    }
    if (lane == 0) sh.total = ss;
  }
  __syncthreads();
  return sh.total;
}

// ---- RMSNorm + Q8_0 ---------------------------------------------------------
// One workgroup of kNT threads per row.  All threads square the row into LDS
// (each product is the reference's own rounding of x*x), seq_sum folds the
// squares (cpu.rs:381), then y = (x*s)*w and its Q8_0 blocks.  n <= 32768 and
// a multiple of 32, so a 32-lane group holds one block.
constexpr int kNT = 1024;              // threads of the norm workgroup
constexpr int kNW = kNT / LLMRS_WAVE;  // fold chunks, one per wave

// 1/rms of the squares sq[0..n) (cpu.rs:381-383), all threads.
__device__ __forceinline__ float fold_scale(const float* sq, int n, float eps, FoldShared<kNW>& sh) {
  const float ss = seq_sum<kNW, true>(sq, n, sh);
  const float rms = __builtin_sqrtf(ss / (float)n + eps);
  return 1.0f / rms;
}

// The row this workgroup normalises.
struct NormRow {
  const float* x;
  const float* w;
  int8_t* xq;
  float* xd;
  float* y;
  int n, layout;
  float eps;
};

// y = (x*s)*w (cpu.rs:389) and its Q8_0 block; element i is held by lane
// i % 32 of a 32-lane group.
__device__ __forceinline__ void norm_out(const NormRow& a, int i, float x, float s, float w) {
  const float y = x * s * w;
  float d;
  const int q = q8_group32(y, &d);
  a.xq[act_offset(i, a.layout)] = (int8_t)q;
  if ((i & 31) == 0) a.xd[i >> 5] = d;
  if (a.y) a.y[i] = y;
}

// n == kNT * EPT: thread t holds elements t + kNT*j of x and w in registers
// from the start, so nothing is loaded after the fold.
template <int EPT>
__device__ __forceinline__ void norm_q8_regs(const NormRow& a, float* sq, FoldShared<kNW>& sh) {
  const int tid = threadIdx.x;
  float xv[EPT], wv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) xv[j] = a.x[tid + kNT * j];
#pragma unroll
  for (int j = 0; j < EPT; ++j) wv[j] = a.w[tid + kNT * j];
#pragma unroll
  for (int j = 0; j < EPT; ++j) sq[tid + kNT * j] = xv[j] * xv[j];
  __syncthreads();
  const float s = fold_scale(sq, a.n, a.eps, sh);
#pragma unroll
  for (int j = 0; j < EPT; ++j) norm_out(a, tid + kNT * j, xv[j], s, wv[j]);
}

__device__ __forceinline__ void norm_q8(const ExactNormArgs& args) {
  extern __shared__ __align__(16) float sq[];
  __shared__ FoldShared<kNW> sh;
  const size_t ro = (size_t)blockIdx.x * args.n;  // this workgroup's row
  const NormRow a{args.x + ro, args.w, args.xq + ro, args.xd + ro / 32, args.y ? args.y + ro : nullptr,
                  args.n, args.layout, args.eps};
  switch (a.n) {
    case 2 * kNT: norm_q8_regs<2>(a, sq, sh); return;
    case 4 * kNT: norm_q8_regs<4>(a, sq, sh); return;
    case 8 * kNT: norm_q8_regs<8>(a, sq, sh); return;
    default: break;
  }
  const int tid = threadIdx.x;
  for (int i = tid; i < a.n; i += kNT) {
    const float v = a.x[i];
    sq[i] = v * v;
  }
  __syncthreads();
  const float s = fold_scale(sq, a.n, a.eps, sh);
  for (int i = tid; i < a.n; i += kNT) norm_out(a, i, a.x[i], s, a.w[i]);
}

// ---- GEMV -----------------------------------------------------------------
// A workgroup tile is 4 * RW rows: wave w computes the block terms of rows
// w, w + 4, ... (lanes over 64 blocks, coalesced loads), parks them in LDS,
// and lane r of wave 0 adds row r's terms to its total in block order.  RW
// is 2 (8-row tiles), or 16 for the SwiGLU launch, whose tile is one 64-row
// group of 32 gate and the 32 matching up rows.
template <int EPI>
constexpr int ex_rows_per_wave() { return EPI == EPI_SILU ? kSiluTile / 4 : 2; }

// The loads of one 64-block chunk for a wave's rows.
template <int WT, int RW>
struct ExChunk {
  i32x4 a0, a1;                                // activation codes of block b
  float da;                                    // activation scale of block b
  u32x4 w0[RW], w1[WT == WT_Q8H ? RW : 1];     // weight codes (Q8: two halves)
  unsigned sc[RW];                             // raw weight scales
};

template <int WT, int RW>
__device__ __forceinline__ void ex_load(const ExactGemvArgs& a, int row0, int c, int nb, ExChunk<WT, RW>& r) {
  constexpr int BS = WT == WT_Q8H ? 32 : 16;
  const int b = min(c + lane_id(), nb - 1);  // clamped: terms past the row end are not folded
  r.a0 = *(const i32x4*)(a.xq + 32 * b);
  r.a1 = *(const i32x4*)(a.xq + 32 * b + 16);
  r.da = a.xd[b];
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    const int row = min(row0 + wave_id() + 4 * j, a.n - 1);
    const size_t blk = (size_t)row * nb + b;
    r.w0[j] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * BS));
    if (WT == WT_Q8H) r.w1[j] = __builtin_nontemporal_load((const u32x4*)(a.wq + blk * BS + 16));
    r.sc[j] = load_wscale_raw<WT>(a.ws, blk);
  }
}

// Exact integer sum of one block: device Q4 layout (byte i = e[i] | e[i+16]
// << 4, value q - 8) or Q8 codes, against the activation codes.
template <int WT, int RW>
__device__ __forceinline__ int ex_isum(const ExChunk<WT, RW>& r, int j) {
  int s = 0;
  if (WT == WT_Q8H) {
    const u32x4 w0 = r.w0[j], w1 = r.w1[j];
    s = dot4((int)w0.x, r.a0.x, s);
    s = dot4((int)w0.y, r.a0.y, s);
    s = dot4((int)w0.z, r.a0.z, s);
    s = dot4((int)w0.w, r.a0.w, s);
    s = dot4((int)w1.x, r.a1.x, s);
    s = dot4((int)w1.y, r.a1.y, s);
    s = dot4((int)w1.z, r.a1.z, s);
    s = dot4((int)w1.w, r.a1.w, s);
  } else {
    const u32x4 w = r.w0[j];
    const unsigned M = 0x0F0F0F0Fu;
    s = dot4((int)(w.x & M), r.a0.x, s);
    s = dot4((int)(w.y & M), r.a0.y, s);
    s = dot4((int)(w.z & M), r.a0.z, s);
    s = dot4((int)(w.w & M), r.a0.w, s);
    s = dot4((int)((w.x >> 4) & M), r.a1.x, s);
    s = dot4((int)((w.y >> 4) & M), r.a1.y, s);
    s = dot4((int)((w.z >> 4) & M), r.a1.z, s);
    s = dot4((int)((w.w >> 4) & M), r.a1.w, s);
  }
  return s;
}

// The Q4 offset -8 * sum(a) of block b (0 for Q8 weights).
template <int WT, int RW>
__device__ __forceinline__ int ex_offset(const ExChunk<WT, RW>& r) {
  if (WT == WT_Q8H) return 0;
  int sa = 0;
  sa = dot4(r.a0.x, 0x01010101, sa);
  sa = dot4(r.a0.y, 0x01010101, sa);
  sa = dot4(r.a0.z, 0x01010101, sa);
  sa = dot4(r.a0.w, 0x01010101, sa);
  sa = dot4(r.a1.x, 0x01010101, sa);
  sa = dot4(r.a1.y, 0x01010101, sa);
  sa = dot4(r.a1.z, 0x01010101, sa);
  sa = dot4(r.a1.w, 0x01010101, sa);
  return -8 * sa;
}

// Chunk loads in flight per wave: the loads of item i + PF are issued right
// after item i is computed, so PF - 1 items' loads are outstanding while an
// item is computed.  Q8 chunks carry twice the weight bytes; three of them
// keep the 8-row kernels at four workgroups per CU.  A SwiGLU chunk holds 16
// rows per wave: two Q4 chunks fit the registers of two workgroups per CU,
// one Q8 chunk (at the 1B width K = 2048 is a single chunk anyway).
template <int WT, int EPI>
constexpr int ex_prefetch() {
  if (EPI == EPI_SILU) return WT == WT_Q8H ? 1 : 2;
  return WT == WT_Q8H ? 3 : 4;
}

// EPI: EPI_STORE (y = total), EPI_RESID (y = total + res), EPI_ARGMAX
// (logits into y when set, and this workgroup's (max, lowest index) into
// part_val / part_idx[blockIdx.x]), EPI_SILU (gate|up rows, one 64-row group
// per tile: m = g / (1 + expf(-g)) * u (layer.rs:75-79, glibc's expf) into y
// when set, and its Q8_0 codes and scale into mq / md).  Workgroups take
// tiles round-robin and walk their (tile, 64-block chunk) items in order
// through a ring of loads, across tile boundaries.
template <int WT, int EPI>
__device__ __forceinline__ void gemv(const ExactGemvArgs& a) {
  constexpr bool SILU = EPI == EPI_SILU;
  constexpr int RW = ex_rows_per_wave<EPI>();
  constexpr int R = 4 * RW;  // rows per tile
  // Block terms of two items (a row padded to 68 floats: the 16-byte reads
  // of the folding lanes cover distinct banks in groups of 8).  Item i writes
  // buffer i % 2 while wave 0 may still fold item i - 1 from the other; it
  // cannot be two items ahead, since the barrier of item i - 1 waits for
  // wave 0's fold of item i - 2.
  constexpr int kPad = LLMRS_WAVE + 4;
  __shared__ __align__(16) float s_p[2][R][kPad];
  __shared__ uint64_t s_exptab[SILU ? 32 : 1];  // exact_expf's table (visible after the first barrier)
  if (SILU && threadIdx.x < 32) s_exptab[threadIdx.x] = expf_detail::kT[threadIdx.x];
  const int lane = lane_id(), wave = wave_id();
  const int nb = a.k >> 5, nch = (nb + LLMRS_WAVE - 1) / LLMRS_WAVE;
  const int ntiles = (a.n + R - 1) / R;
  const int my_tiles = (int)blockIdx.x < ntiles ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int nitems = my_tiles * nch;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  float total = 0.0f;  // lane r < R of wave 0: row row0 + r of the current tile
  auto row0_of = [&](int item) { return ((int)blockIdx.x + (item / nch) * (int)gridDim.x) * R; };
  auto load = [&](int item, ExChunk<WT, RW>& r) {
    ex_load<WT, RW>(a, row0_of(item), (item % nch) * LLMRS_WAVE, nb, r);
  };
  // one item: the wave's block terms into LDS, then wave 0 folds them; the
  // tile's last chunk writes its rows
  auto step = [&](int item, const ExChunk<WT, RW>& r) {
    const int c = (item % nch) * LLMRS_WAVE;
    const int off = ex_offset<WT, RW>(r);
    float(*buf)[kPad] = s_p[item & 1];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      const int isum = ex_isum<WT, RW>(r, j) + off;
      buf[wave + 4 * j][lane] = (float)isum * (wscale<WT>(r.sc[j]) * r.da);
    }
    __syncthreads();
    if (wave == 0 && lane < R) {
      const int cnt = min(LLMRS_WAVE, nb - c);
      if (cnt == LLMRS_WAVE) {  // 16 terms at a time, the next 16 read before these are added
        f32x4 t[2][4];
        const f32x4* src = (const f32x4*)buf[lane];
#pragma unroll
        for (int q = 0; q < 4; ++q) t[0][q] = src[q];
#pragma unroll
        for (int g = 0; g < LLMRS_WAVE / 16; ++g) {
          if (g + 1 < LLMRS_WAVE / 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) t[(g + 1) & 1][q] = src[4 * (g + 1) + q];
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            total = total + t[g & 1][q][0];
            total = total + t[g & 1][q][1];
            total = total + t[g & 1][q][2];
            total = total + t[g & 1][q][3];
          }
        }
      } else {
        for (int l = 0; l < cnt; ++l) total = total + buf[lane][l];
      }
      const int row = row0_of(item) + lane;
      if (item % nch == nch - 1) {
        if (SILU) {  // lanes 0-31 hold the gate rows, 32-63 the up rows
          const float u = __shfl(total, lane + 32);
          if (lane < 32) {
            const float silu = total / (1.0f + exact_expf(-total, s_exptab));
            const float m = silu * u;
            float d;
            const int q = q8_group32(m, &d);
            const int j = row0_of(item) / 2 + lane;
            a.mq[j] = (int8_t)q;
            if (lane == 0) a.md[j >> 5] = d;
            if (a.y) a.y[j] = m;
          }
        } else if (row < a.n) {
          if (EPI == EPI_RESID) a.y[row] = total + a.res[row];
          else if (a.y) a.y[row] = total;
          if (EPI == EPI_ARGMAX && better(total, row, bv, bi)) {
            bv = total;
            bi = row;
          }
        }
        total = 0.0f;
      }
    }
  };
  constexpr int PF = ex_prefetch<WT, EPI>();
  ExChunk<WT, RW> ring[PF];
#pragma unroll
  for (int s = 0; s < PF; ++s)
    if (s < nitems) load(s, ring[s]);
  for (int i = 0; i < nitems; i += PF) {
#pragma unroll
    for (int s = 0; s < PF; ++s) {
      if (i + s < nitems) {
        step(i + s, ring[s]);
        if (i + s + PF < nitems) load(i + s + PF, ring[s]);
      }
    }
  }
  if (EPI == EPI_ARGMAX && wave == 0) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      a.part_val[blockIdx.x] = bv;
      a.part_idx[blockIdx.x] = bi;
    }
  }
}

// ---- attention -------------------------------------------------------------
constexpr int kVTile = 16384;  // bytes of V per LDS tile
constexpr int kChunkedSum = 384;  // softmax rows from this length sum by chunks

// LDS of one query row's attention (the scores are the dynamic LDS); V tiles
// for f32 caches only.
template <int HD, bool F16>
struct AttnShared {
  float q[HD], k[HD], v[HD];
  uint64_t exptab[32];  // exact_expf's table
  float red[kT / LLMRS_WAVE];
  FoldShared<kT / LLMRS_WAVE> fold;
  u32x4 vt[F16 ? 1 : 2][F16 ? 1 : kVTile / 16];  // V tiles
};

// One query row's attention over the KV head at kbase / vbase: cache rows
// 0 .. ncache-1, then (OWN) the row at position ncache from sh.k / sh.v.
// Scores: the sequential dot over the head dims of q and each row, then
// times the scale (matmul_slice cpu.rs:230-269, layer.rs:257-258); softmax
// with the maximum from f32::MIN, glibc's expf, the sequential sum (seq_sum
// for long rows) and e * (1/sum) (cpu.rs:395-423); ctx[d] = sum over the
// rows of p * V[d], sequential (layer.rs:276-299).  f16 caches: in decode
// each thread requests its next K row before it folds the current one; thread d < HD
// reads dim d of the blocked V rows (8 positions per 16-byte load) straight
// from memory, kVRing blocks ahead in decode (the first ones before the
// softmax).  f32 caches:
// V rows pass through LDS in 16 KB tiles that every thread loads
// (coalesced), each tile requested while the previous one is added; `first`
// holds the first tile's loads, issued by the caller.  Returns ctx[d] for
// thread d < HD.
constexpr int kVRing = 16;
// Start of a query row's attention: exact_expf's table into LDS (visible
// after the caller's barrier).
template <int HD, bool F16>
__device__ __forceinline__ void attn_start(AttnShared<HD, F16>& sh) {
  if (threadIdx.x < 32) sh.exptab[threadIdx.x] = expf_detail::kT[threadIdx.x];
}


template <int HD, bool F16, bool OWN>
__device__ __forceinline__ float attn_row(const char* kbase, const char* vbase, size_t head_bytes, int ncache,
                                          float scale, float* s_p, AttnShared<HD, F16>& sh,
                                          const u32x4 (&first)[kVTile / 16 / kT]) {
  constexpr int VB = F16 ? 2 : 4;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int T = ncache + (OWN ? 1 : 0);
  const int d = tid;
  const u32x4* vb = (const u32x4*)vbase + d;  // block b of dim d at vb[b * HD] (f16)
  const int nblk = (ncache + 7) / 8;
  // scores: sequential dot over the head dims, then the scale
  float mx = -3.40282347e+38f;  // f32::MIN (cpu.rs:408)
  auto own_dot = [&]() {
    float s = 0.0f;
    for (int e = 0; e < HD; ++e) s = s + sh.q[e] * sh.k[e];
    return s;
  };
  if constexpr (F16) {
    constexpr int KW = HD * 2 / 16;  // 16-byte words per K row
    auto kload = [&](int t, u32x4 (&w)[KW]) {
      const u32x4* kr = (const u32x4*)(kbase + (size_t)t * HD * 2);
#pragma unroll
      for (int j = 0; j < KW; ++j) w[j] = kr[j];
    };
    auto score = [&](int t, const u32x4 (&w)[KW]) {
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < KW; ++j) {
        const f32x4 qa = *(const f32x4*)&sh.q[8 * j], qb = *(const f32x4*)&sh.q[8 * j + 4];
        const float qv[8] = {qa[0], qa[1], qa[2], qa[3], qb[0], qb[1], qb[2], qb[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s = s + mul_f16lo(qv[2 * i], w[j][i]);
          s = s + mul_f16hi(qv[2 * i + 1], w[j][i]);
        }
      }
      s = s * scale;
      s_p[t] = s;
      mx = fmaxf(mx, s);
    };
    // loads are unconditional (rows clamped into the cache; a clamped row is
    // never scored), so the next row's load never waits on the current one
    const int last = max(ncache - 1, 0);
    u32x4 ka[KW];
    int t = tid;
    if constexpr (OWN) {  // decode: 32 workgroups, registers to spare
      u32x4 kb[KW];
      kload(min(t, last), ka);
      while (t < ncache) {
        const int t2 = t + kT;
        kload(min(t2, last), kb);
        score(t, ka);
        if (t2 >= ncache) break;
        const int t3 = t2 + kT;
        kload(min(t3, last), ka);
        score(t2, kb);
        t = t3;
      }
    } else {  // prompt rows: many workgroups per CU, one K row per thread at a time
      for (; t < ncache; t += kT) {
        kload(t, ka);
        score(t, ka);
      }
    }
    if (OWN && tid == ncache % kT) {  // the new row, from LDS
      const float s = own_dot() * scale;
      s_p[ncache] = s;
      mx = fmaxf(mx, s);
    }
  } else {
    for (int t = tid; t < T; t += kT) {
      float s = 0.0f;
      if (OWN && t == ncache) {
        s = own_dot();
      } else {
        const float* kr = (const float*)kbase + (size_t)t * HD;
        for (int e = 0; e < HD; e += 4) {
          const f32x4 w = *(const f32x4*)(kr + e);
#pragma unroll
          for (int i = 0; i < 4; ++i) s = s + sh.q[e + i] * w[i];
        }
      }
      s = s * scale;
      s_p[t] = s;
      mx = fmaxf(mx, s);
    }
  }
  // f16: the first V blocks of dim d, requested before the softmax (blocks
  // clamped into the cache, unconditionally, as the K rows); prompt rows keep
  // half the ring (their workgroups share a CU)
  constexpr int RS = F16 ? (OWN ? kVRing : kVRing / 2) : 1;
  const int lastb = max(nblk - 1, 0);
  u32x4 ring[RS];
  if (F16 && d < HD) {
#pragma unroll
    for (int j = 0; j < RS; ++j) ring[j] = vb[(size_t)min(j, lastb) * HD];
  }
  mx = wave_max(mx);
  if (lane == 0) sh.red[wave] = mx;
  __syncthreads();
  mx = sh.red[0];
#pragma unroll
  for (int w = 1; w < kT / LLMRS_WAVE; ++w) mx = fmaxf(mx, sh.red[w]);
  for (int t = tid; t < T; t += kT) s_p[t] = exact_expf(s_p[t] - mx, sh.exptab);
  __syncthreads();
  // the sequential sum of the exponentials: by chunks for long rows, by one
  // lane below kChunkedSum terms (where the chunks' fixed cost exceeds the
  // fold); both give the same sum
  float sum;
  if (T >= kChunkedSum) {
    sum = seq_sum<kT / LLMRS_WAVE, false>(s_p, T, sh.fold);
  } else {
    if (tid == 0) {
      float acc = 0.0f;
      int t = 0;
      for (; t + 4 <= T; t += 4) {
        const f32x4 e = *(const f32x4*)(s_p + t);
        acc = acc + e[0];
        acc = acc + e[1];
        acc = acc + e[2];
        acc = acc + e[3];
      }
      for (; t < T; ++t) acc = acc + s_p[t];
      sh.fold.total = acc;
    }
    __syncthreads();
    sum = sh.fold.total;
  }
  const float inv = 1.0f / sum;
  for (int t = tid; t < T; t += kT) s_p[t] = s_p[t] * inv;
  // ctx[d] = sum over t of p_t * V[t][d], sequential in t; the own row last.
  float acc = 0.0f;
  if constexpr (F16) {
    __syncthreads();
    if (d < HD) {
      // 8 positions of one block: p from LDS, V from the block's 16 bytes
      auto block8 = [&](const u32x4& w, int t0, int cnt) {
        if (cnt == 8) {
          const f32x4 p0 = *(const f32x4*)(s_p + t0), p1 = *(const f32x4*)(s_p + t0 + 4);
          acc = acc + mul_f16lo(p0[0], w[0]);
          acc = acc + mul_f16hi(p0[1], w[0]);
          acc = acc + mul_f16lo(p0[2], w[1]);
          acc = acc + mul_f16hi(p0[3], w[1]);
          acc = acc + mul_f16lo(p1[0], w[2]);
          acc = acc + mul_f16hi(p1[1], w[2]);
          acc = acc + mul_f16lo(p1[2], w[3]);
          acc = acc + mul_f16hi(p1[3], w[3]);
        } else {  // the last, partial block: rows past ncache are not added
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (e < cnt) acc = acc + s_p[t0 + e] * h2f((uint16_t)(w[e / 2] >> (16 * (e & 1))));
        }
      };
      const int nfull = ncache / 8;
      // the last whole blocks from slot 0 of a round, then the partial one
      auto tail = [&](const u32x4 (&r)[RS], int b0) {
#pragma unroll
        for (int j = 0; j < RS; ++j) {
          const int b = b0 + j;
          if (b < nfull) block8(r[j], 8 * b, 8);
          else if (b == nfull && 8 * b < ncache) block8(r[j], 8 * b, ncache - 8 * b);
        }
      };
      // whole rounds of the ring without a branch, the next round's loads
      // (clamped, unconditional) issued as each block is consumed
      int b0 = 0;
      for (; b0 + RS <= nfull; b0 += RS) {
#pragma unroll
        for (int j = 0; j < RS; ++j) {
          const u32x4 w = ring[j];
          ring[j] = vb[(size_t)min(b0 + j + RS, lastb) * HD];
          block8(w, 8 * (b0 + j), 8);
        }
      }
      tail(ring, b0);
    }
  } else {
    constexpr int TP = kVTile / (HD * VB);  // positions per tile, a multiple of 8
    constexpr int LPT = kVTile / 16 / kT;   // 16-byte loads per thread per tile
    const int ntile = (ncache + TP - 1) / TP;
    u32x4 st[LPT];
#pragma unroll
    for (int l = 0; l < LPT; ++l) st[l] = first[l];
    auto vload = [&](int tile) {  // rows past ncache read stale (in-bounds) bytes, never added
#pragma unroll
      for (int l = 0; l < LPT; ++l) {
        const size_t off = min((size_t)tile * kVTile + 16 * (size_t)(tid + kT * l), head_bytes - 16);
        st[l] = *(const u32x4*)(vbase + off);
      }
    };
    auto vstore = [&](int buf) {
#pragma unroll
      for (int l = 0; l < LPT; ++l) sh.vt[buf][tid + kT * l] = st[l];
    };
    if (ntile > 0) vstore(0);
    __syncthreads();
    for (int i = 0; i < ntile; ++i) {
      if (i + 1 < ntile) vload(i + 1);
      if (d < HD) {
        const int t0 = i * TP, t1 = min(t0 + TP, ncache);
        const float* vt = (const float*)sh.vt[i & 1];
        for (int t = t0; t < t1; ++t) acc = acc + s_p[t] * vt[(t - t0) * HD + d];
      }
      if (i + 1 < ntile) vstore((i + 1) & 1);
      __syncthreads();
    }
  }
  if (OWN && d < HD) acc = acc + s_p[ncache] * sh.v[d];
  return acc;
}

// The first V tile's loads (tile 0 of the KV head; f32 caches), issued at
// kernel start.
template <int HD, bool F16>
__device__ __forceinline__ void attn_first_tile(const char* vbase, size_t head_bytes, u32x4 (&st)[kVTile / 16 / kT]) {
  if (F16) return;
#pragma unroll
  for (int l = 0; l < kVTile / 16 / kT; ++l)
    st[l] = *(const u32x4*)(vbase + min(16 * (size_t)(threadIdx.x + kT * l), head_bytes - 16));
}

// Decode: one workgroup per query head h (KV head g = h / n_rep) at the
// device position pos.  The new K/V row is rotated and rounded to the
// cache type by every workgroup of the group (the values are identical) and
// stored by the group's first; each workgroup uses its own copy for
// position pos, so no workgroup adds a value another is writing (a V tile
// may hold the bytes of row pos mid-write; only rows below pos are added).
template <int HD, bool F16>
__device__ __forceinline__ void attn(const ExactAttnArgs& a) {
  constexpr int MID = HD / 2, VB = F16 ? 2 : 4;
  extern __shared__ __align__(16) float s_p[];  // [pos + 1]
  __shared__ __align__(16) AttnShared<HD, F16> sh;
  const int tid = threadIdx.x;
  const int h = blockIdx.x, n_rep = a.nq / a.nkv, g = h / n_rep;
  const int pos = *a.pos_ptr;
  const size_t head = (size_t)g * a.max_seq * HD;
  const size_t head_bytes = (size_t)a.max_seq * HD * VB;
  const char* kbase = (const char*)a.kc + head * VB;
  const char* vbase = (const char*)a.vc + head * VB;
  u32x4 first[kVTile / 16 / kT];
  attn_first_tile<HD, F16>(vbase, head_bytes, first);
  attn_start<HD, F16>(sh);
  if (tid < MID) {  // rotate-half RoPE of q and the new k (cpu.rs:345-354)
    const float co = a.rope_cos[(size_t)pos * MID + tid], sn = a.rope_sin[(size_t)pos * MID + tid];
    const float* q = a.qkv + (size_t)h * HD;
    float re = q[tid], im = q[tid + MID];
    sh.q[tid] = re * co - im * sn;
    sh.q[tid + MID] = re * sn + im * co;
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
      (is_k ? sh.k : sh.v)[dd[j]] = kv[j];
    }
  }
  __syncthreads();
  const float acc = attn_row<HD, F16, true>(kbase, vbase, head_bytes, pos, a.scale, s_p, sh, first);
  if (tid < HD) {
    const size_t e = (size_t)h * HD + tid;
    a.ctx[e] = acc;
    float dq;
    const int q = q8_group32(acc, &dq);
    a.ctx_q[e] = (int8_t)q;
    if ((tid & 31) == 0) a.ctx_d[e >> 5] = dq;
  }
}

// Prompt rows: one workgroup per (query head h, row t) at position
// start_pos + t over the cache rows 0 .. start_pos + t, which the RoPE /
// append launch has written (layer.rs:248-270: the causal mask keeps
// j <= start_pos + t); q rotated, ctx as f32 (optional) and Q8_0 in the
// operand order ctx_layout.
template <int HD, bool F16>
__device__ __forceinline__ void attn_prefill(const PrefillAttnArgs& a) {
  constexpr int VB = F16 ? 2 : 4;
  extern __shared__ __align__(16) float s_p[];  // [start_pos + t + 1]
  __shared__ __align__(16) AttnShared<HD, F16> sh;
  const int tid = threadIdx.x;
  const int h = blockIdx.x, t = blockIdx.y, g = h / (a.nq / a.nkv);
  const int pos = a.start_pos + t;
  const size_t head_bytes = (size_t)a.max_seq * HD * VB;
  const char* kbase = (const char*)a.kc + (size_t)g * head_bytes;
  const char* vbase = (const char*)a.vc + (size_t)g * head_bytes;
  u32x4 first[kVTile / 16 / kT];
  attn_first_tile<HD, F16>(vbase, head_bytes, first);
  attn_start<HD, F16>(sh);
  const int qd = a.nq * HD;
  if (tid < HD) sh.q[tid] = a.q[(size_t)t * qd + (size_t)h * HD + tid];
  __syncthreads();
  const float acc = attn_row<HD, F16, false>(kbase, vbase, head_bytes, pos + 1, a.scale, s_p, sh, first);
  if (tid < HD) {
    const int e = h * HD + tid;
    if (a.ctx) a.ctx[(size_t)t * qd + e] = acc;
    float dq;
    const int q = q8_group32(acc, &dq);
    a.ctx_q[(size_t)t * qd + act_offset(e, a.ctx_layout)] = (int8_t)q;
    if ((tid & 31) == 0) a.ctx_d[(size_t)t * (qd / 32) + (e >> 5)] = dq;
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(kNT) void exact_norm_q8(ExactNormArgs a) { norm_q8(a); }

#define LLMRS_EXACT_GEMV(tag, WT)                                                                     \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_store(ExactGemvArgs a) {      \
    gemv<WT, EPI_STORE>(a);                                                                         \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_resid(ExactGemvArgs a) {      \
    gemv<WT, EPI_RESID>(a);                                                                         \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_argmax(ExactGemvArgs a) {     \
    gemv<WT, EPI_ARGMAX>(a);                                                                        \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(kT) void exact_gemv_##tag##_silu(ExactGemvArgs a) {       \
    gemv<WT, EPI_SILU>(a);                                                                          \
  }
LLMRS_EXACT_GEMV(q4h, WT_Q4H)
LLMRS_EXACT_GEMV(q4f, WT_Q4F)
LLMRS_EXACT_GEMV(q8h, WT_Q8H)

#define LLMRS_EXACT_ATTN(tag, HD, F16)                                                                    \
  extern "C" __global__ __launch_bounds__(kT) void exact_attn_##tag(ExactAttnArgs a) { attn<HD, F16>(a); } \
  extern "C" __global__ __launch_bounds__(kT) void exact_attn_prefill_##tag(PrefillAttnArgs a) {        \
    attn_prefill<HD, F16>(a);                                                                        \
  }
LLMRS_EXACT_ATTN(hd64_f16, 64, true)
LLMRS_EXACT_ATTN(hd128_f16, 128, true)
LLMRS_EXACT_ATTN(hd64_f32, 64, false)
LLMRS_EXACT_ATTN(hd128_f32, 128, false)
