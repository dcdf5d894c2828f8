// attention.hip - standalone batch-1 decode attention kernels for gfx950.
//
// One launch per layer: grid (nsplit, nkv), one work item of attn_core.h
// (which documents the algorithm) per workgroup.  Reference:
// LlamaAttention::forward with seq == 1 (layer.rs:175-299).
#include "attn_core.h"

using namespace llmrs;

template <int HD, bool KV16, int S>
__device__ __forceinline__ void attn_decode_impl(const AttnArgs& a) {
  __shared__ __align__(16) uint8_t lds[AttnLds<HD, KV16, S>::BYTES];
  attn_item<HD, KV16, false, S>(a, blockIdx.y, blockIdx.x, *a.pos_ptr, lds);
}

// Variant names: attn_decode_hd<HD>_<cache>[_s<streams>].
#define LLMRS_ATTN(name, HD, KV16, S)                                              \
  extern "C" __global__ __launch_bounds__(256 * S) void name(AttnArgs a) {        \
    attn_decode_impl<HD, KV16, S>(a);                                             \
  }

LLMRS_ATTN(attn_decode_hd64_f32, 64, false, 1)
LLMRS_ATTN(attn_decode_hd64_f16, 64, true, 1)
LLMRS_ATTN(attn_decode_hd128_f32, 128, false, 1)
LLMRS_ATTN(attn_decode_hd128_f16, 128, true, 1)
LLMRS_ATTN(attn_decode_hd64_f32_s4, 64, false, 4)
LLMRS_ATTN(attn_decode_hd64_f16_s4, 64, true, 4)
LLMRS_ATTN(attn_decode_hd128_f32_s4, 128, false, 4)
LLMRS_ATTN(attn_decode_hd128_f16_s4, 128, true, 4)
