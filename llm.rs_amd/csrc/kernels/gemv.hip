// gemv.hip - standalone batch-1 dequant-GEMV kernels for gfx950 (CDNA4).
//
// Entry points over the shared machinery of gemv_core.h (which documents the
// arithmetic, the weight layout and the work decomposition): one launch per
// GEMV, row groups dealt to the waves of the whole grid.  Used by the trait
// operator Backend::matmul_transposed (src/backend.rs:24) and by the
// per-kernel decode step; argmax_final closes the lm_head GEMV.
#include "gemv_core.h"

using namespace llmrs;

// Weight units requested before the activation prologue: one for the
// SwiGLU GEMV with the RMSNorm prologue (earlier weight requests delay its
// 32 KB of activation loads), two otherwise.
template <int PRO, int EPI>
constexpr int pre_units() { return EPI == EPI_SILU && PRO == PRO_NORM ? 1 : 2; }

template <int WT, int PRO, int EPI, int R, int U>
__device__ __forceinline__ void gemv_impl(const GemvArgs& a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  UnitRegs<WT, R, U> ua, ub;
  gemv_body<WT, PRO, EPI, R, U, false, pre_units<PRO, EPI>()>(a, blockIdx.y, blockIdx.x, gridDim.x, ua, ub,
                                                               false, smem, sh);
}

// Row-batched launch (batched decode): batch_rows rows of Q8_0 activation
// codes over batch_nwg workgroups per row.  Workgroups are dealt to the 8 XCDs
// by linear index mod 8, so the linear index is split as xcd + 8 * (row + rows
// * (wg / 8)) with xcd = wg % 8: the rows' workgroups for one slice of the
// weights run on one XCD, close together in dispatch order, and the weights
// stream from HBM about once, the other rows reading them from that L2.
template <int WT, int EPI, int R, int U>
__device__ __forceinline__ void gemv_batch_impl(const GemvArgs& a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  const int L = blockIdx.x, xcd = L & 7, rest = L >> 3;
  const int mrow = rest % a.batch_rows, wg = xcd + 8 * (rest / a.batch_rows);
  if (wg >= a.batch_nwg) return;  // padding to whole groups of 8
  UnitRegs<WT, R, U> ua, ub;
  gemv_body<WT, PRO_Q8, EPI, R, U, false, 2>(a, mrow, wg, a.batch_nwg, ua, ub, false, smem, sh);
}

#define LLMRS_GEMV_B(name, WT, EPI, R, U)                                          \
  extern "C" __global__ __launch_bounds__(kThreads) void name(GemvArgs a) {        \
    gemv_batch_impl<WT, EPI, R, U>(a);                                             \
  }

#define LLMRS_GEMV(name, WT, PRO, EPI, R, U)                                       \
  extern "C" __global__ __launch_bounds__(kThreads) void name(GemvArgs a) {        \
    gemv_impl<WT, PRO, EPI, R, U>(a);                                              \
  }

// Variant names: gemv_<weights>_<prologue>_<epilogue>_r<R>u<U>; row-batched
// gemv_<weights>_q8b_<epilogue>_r<R>u<U>.
#define LLMRS_GEMV_FAMILY(tag, WT, U)                                                     \
  LLMRS_GEMV(gemv_##tag##_quant_store_r4u##U, WT, PRO_QUANT, EPI_STORE, 4, U)             \
  LLMRS_GEMV(gemv_##tag##_norm_store_r2u##U, WT, PRO_NORM, EPI_STORE, 2, U)               \
  LLMRS_GEMV(gemv_##tag##_norm_store_r4u##U, WT, PRO_NORM, EPI_STORE, 4, U)               \
  LLMRS_GEMV(gemv_##tag##_q8_resid_r2u##U, WT, PRO_Q8, EPI_RESID, 2, U)                   \
  LLMRS_GEMV(gemv_##tag##_q8_resid_r4u##U, WT, PRO_Q8, EPI_RESID, 4, U)                   \
  LLMRS_GEMV(gemv_##tag##_norm_silu_r4u##U, WT, PRO_NORM, EPI_SILU, 4, U)                 \
  LLMRS_GEMV(gemv_##tag##_norm_argmax_r4u##U, WT, PRO_NORM, EPI_ARGMAX, 4, U)               \
  LLMRS_GEMV(gemv_##tag##_nq_store_r2u##U, WT, PRO_NQ, EPI_STORE, 2, U)                   \
  LLMRS_GEMV(gemv_##tag##_nq_silu_r4u##U, WT, PRO_NQ, EPI_SILU, 4, U)                     \
  LLMRS_GEMV(gemv_##tag##_nq_argmax_r4u##U, WT, PRO_NQ, EPI_ARGMAX, 4, U)                 \
  LLMRS_GEMV_B(gemv_##tag##_q8b_store_r2u##U, WT, EPI_STORE, 2, U)                        \
  LLMRS_GEMV_B(gemv_##tag##_q8b_resid_r2u##U, WT, EPI_RESID, 2, U)                        \
  LLMRS_GEMV_B(gemv_##tag##_q8b_silu_r4u##U, WT, EPI_SILU, 4, U)

LLMRS_GEMV_FAMILY(q4h, WT_Q4H, 1)
LLMRS_GEMV_FAMILY(q4h, WT_Q4H, 2)
LLMRS_GEMV_FAMILY(q4f, WT_Q4F, 1)
LLMRS_GEMV_FAMILY(q4f, WT_Q4F, 2)
LLMRS_GEMV_FAMILY(q8h, WT_Q8H, 1)
LLMRS_GEMV_FAMILY(q8h, WT_Q8H, 2)

// Final reduction of the lm_head partials and the greedy step bookkeeping:
// next = argmax (lowest index on ties); gen[pos+1] = next; tokens[pos+1] =
// next once the prompt is consumed; pos += 1.
// Block sizes of the launches below (their launch bounds): the block size
// read at run time would be a vector load from the dispatch arguments and a
// wait on every outstanding memory operation.
constexpr int kArgmaxFinalThreads = 256, kArgmaxBatchThreads = 1024;

extern "C" __global__ __launch_bounds__(kArgmaxFinalThreads) void argmax_final(ArgmaxFinalArgs a) {
  __shared__ float s_bv[8];
  __shared__ int s_bi[8];
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < a.nparts; i += kArgmaxFinalThreads)
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
    for (int w = 1; w < kArgmaxFinalThreads / LLMRS_WAVE; ++w)
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

// Greedy step of a batch: workgroup b takes the argmax of logits row b
// (lowest index on ties; every logit NaN gives 0) and advances sequence b
// as argmax_final advances one sequence (its prompt is consumed: the id is
// both produced and the next input).  16-byte loads, four per thread in
// flight.
extern "C" __global__ __launch_bounds__(kArgmaxBatchThreads) void argmax_batch(ArgmaxBatchArgs a) {
  __shared__ float s_bv[16];
  __shared__ int s_bi[16];
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id(), b = blockIdx.x;
  const float* row = a.logits + (size_t)b * a.vocab;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  auto take = [&](float v, int i) {
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  };
  // rows start 16-byte aligned when vocab % 4 == 0; else scalar loads
  const int nv = a.vocab % 4 == 0 ? a.vocab / 4 : 0;
  const f32x4* row4 = (const f32x4*)row;
  for (int v0 = tid; v0 < nv; v0 += 4 * kArgmaxBatchThreads) {
    f32x4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int v = v0 + u * kArgmaxBatchThreads;
      x[u] = v < nv ? row4[v] : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int v = v0 + u * kArgmaxBatchThreads;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (v < nv) take(x[u][e], 4 * v + e);
    }
  }
  for (int i = 4 * nv + tid; i < a.vocab; i += kArgmaxBatchThreads) take(row[i], i);
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
    s_bv[wave] = bv;
    s_bi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxBatchThreads / LLMRS_WAVE; ++w)
      if (better(s_bv[w], s_bi[w], bv, bi)) {
        bv = s_bv[w];
        bi = s_bi[w];
      }
    if (bi == 0x7fffffff) bi = 0;
    const int pos = a.pos[b];
    if (pos + 1 < a.cap) {
      a.gen[(size_t)b * a.cap + pos + 1] = bi;
      a.tokens[(size_t)b * a.cap + pos + 1] = bi;
    }
    a.pos[b] = pos + 1;
  }
}
