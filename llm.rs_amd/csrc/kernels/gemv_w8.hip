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

// Variant names: gemv_<weights>_q8_nq_r<R>u<U>_w8.
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
