// gemv_w8.hip - decode GEMV kernels with 8 waves (512 threads) per
// workgroup: the residual GEMVs that also produce the next RMSNorm's operand
// in 32-row tiles (EPI_NQ of gemv_core.h, which documents the arithmetic),
// one workgroup per tile.  Used when the tiles fill the GPU (hidden 8192 on
// 256 CUs: measured 110.2 vs 103.9 tok/s on the 70B-shaped decode, the
// gate|up GEMV at 5.9 TB/s); at hidden 4096 the 128 tiles leave half the
// CUs idle and the producers lose more than the consumers gain.
#define LLMRS_GEMV_WAVES 8
#include "gemv_core.h"

using namespace llmrs;

template <int WT, int R, int U>
__device__ __forceinline__ void gemv_w8_impl(const GemvArgs& a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  UnitRegs<WT, R, U> ua, ub;
  gemv_body<WT, PRO_Q8, EPI_NQ, R, U, false, 2>(a, blockIdx.y, blockIdx.x, gridDim.x, ua, ub, false, smem, sh);
}

// The SwiGLU GEMV with its RMSNorm prologue (gate|up) when its 64-row tiles
// outnumber the CUs: one workgroup per CU looping over the tiles, so the
// prologue runs once per CU, not once per co-resident workgroup (8B shape,
// 448 tiles: 15.0 vs 15.3 us per launch, decode 723.9 vs 719.5 tok/s; at
// 256 tiles or fewer the 4-wave kernel is faster).
// One unit requested before the prologue (8B shape: 15.0 us per launch;
// 16.0 with two, 16.0 with none).
template <int WT, int R, int U>
__device__ __forceinline__ void gemv_w8_silu_impl(const GemvArgs& a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  UnitRegs<WT, R, U> ua, ub;
  gemv_body<WT, PRO_NORM, EPI_SILU, R, U, false, 1>(a, blockIdx.y, blockIdx.x, gridDim.x, ua, ub, false, smem, sh);
}

// Variant names: gemv_<weights>_q8_nq_r<R>u<U>_w8, gemv_<weights>_norm_silu_r4u<U>_w8.
#define LLMRS_GEMV_W8(tag, WT, R, U)                                                          \
  extern "C" __global__ __launch_bounds__(kThreads) void gemv_##tag##_q8_nq_r##R##u##U##_w8(GemvArgs a) { \
    gemv_w8_impl<WT, R, U>(a);                                                                \
  }

LLMRS_GEMV_W8(q4h, WT_Q4H, 2, 1)
LLMRS_GEMV_W8(q4h, WT_Q4H, 2, 2)
LLMRS_GEMV_W8(q4f, WT_Q4F, 2, 1)
LLMRS_GEMV_W8(q4f, WT_Q4F, 2, 2)
LLMRS_GEMV_W8(q8h, WT_Q8H, 2, 1)
LLMRS_GEMV_W8(q8h, WT_Q8H, 2, 2)

#define LLMRS_GEMV_W8_SILU(tag, WT, U)                                                          \
  extern "C" __global__ __launch_bounds__(kThreads) void gemv_##tag##_norm_silu_r4u##U##_w8(GemvArgs a) { \
    gemv_w8_silu_impl<WT, 4, U>(a);                                                             \
  }
LLMRS_GEMV_W8_SILU(q4h, WT_Q4H, 1)
LLMRS_GEMV_W8_SILU(q4h, WT_Q4H, 2)
LLMRS_GEMV_W8_SILU(q4f, WT_Q4F, 1)
LLMRS_GEMV_W8_SILU(q4f, WT_Q4F, 2)
LLMRS_GEMV_W8_SILU(q8h, WT_Q8H, 1)
LLMRS_GEMV_W8_SILU(q8h, WT_Q8H, 2)
