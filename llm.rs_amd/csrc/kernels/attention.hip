// attention.hip - standalone batch-1 decode attention kernels for gfx950.
//
// One launch per layer, one work item per workgroup, grid (nsplit, nkv).
// f16 caches run on the matrix cores (attn_mfma.h, which documents the
// algorithm and the blocked V layout); f32 caches on the vector ALUs
// (attn_core.h).  Reference: LlamaAttention::forward with seq == 1
// (layer.rs:175-299).
#include "attn_core.h"
#include "attn_mfma.h"

using namespace llmrs;

// Sequence blockIdx.z of a batched decode launch (grid.z > 1): its buffers.
template <int HD>
__device__ __forceinline__ AttnArgs sequence_args(const AttnArgs& a0) {
  AttnArgs a = a0;
  const int z = blockIdx.z;
  if (z) {
    const size_t qd = (size_t)a.nq * HD;
    a.qkv += (size_t)z * (a.nq + 2 * a.nkv) * HD;
    a.pos_ptr += z;
    a.kc = (uint8_t*)a.kc + z * a.kv_batch_bytes;
    a.vc = (uint8_t*)a.vc + z * a.kv_batch_bytes;
    a.part_o += (size_t)z * qd * a.nsplit;
    a.part_ml += (size_t)z * a.nq * ml_stride(a.nsplit) * 2;
    a.counters += (size_t)z * a.nkv * kTicketStride;
    a.ctx += z * qd;
    a.ctx_q += z * qd;
    a.ctx_d += z * qd / 32;
    if (a.rope_now) a.rope_now += (size_t)z * HD;
    a.ts = nullptr;
  }
  return a;
}

template <int HD, int S, bool LOCAL>
__device__ __forceinline__ void attn_decode_impl(const AttnArgs& a0) {
  __shared__ __align__(16) uint8_t lds[AttnLds<HD, false, S>::BYTES];
  const AttnArgs a = sequence_args<HD>(a0);
  // LOCAL: KV head = linear workgroup index % nkv (one XCD per head)
  const int lin = blockIdx.x + blockIdx.y * gridDim.x;
  const int g = LOCAL ? lin % a.nkv : blockIdx.y, split = LOCAL ? lin / a.nkv : blockIdx.x;
  attn_item<HD, false, false, S, LOCAL>(a, g, split, *a.pos_ptr, lds);
}

template <int HD, int TW, bool LOCAL>
__device__ __forceinline__ void attn_decode_mfma_impl(const AttnArgs& a0) {
  __shared__ __align__(16) uint8_t lds[MfmaAttnLds<HD, TW>::BYTES];
  const AttnArgs a = sequence_args<HD>(a0);
  attn_mfma_item<HD, TW, LOCAL>(a, *a.pos_ptr, lds);
}

// Variant names: attn_decode_hd<HD>_f32[_s<streams>][_l], where _l is the
// XCD-local split exchange (a KV head's workgroups on one XCD).
#define LLMRS_ATTN(name, HD, S, LOCAL)                                             \
  extern "C" __global__ __launch_bounds__(256 * S) void name(AttnArgs a) {        \
    attn_decode_impl<HD, S, LOCAL>(a);                                            \
  }
LLMRS_ATTN(attn_decode_hd64_f32, 64, 1, false)
LLMRS_ATTN(attn_decode_hd128_f32, 128, 1, false)
LLMRS_ATTN(attn_decode_hd64_f32_s4, 64, 4, false)
LLMRS_ATTN(attn_decode_hd128_f32_s4, 128, 4, false)
LLMRS_ATTN(attn_decode_hd64_f32_l, 64, 1, true)
LLMRS_ATTN(attn_decode_hd128_f32_l, 128, 1, true)
LLMRS_ATTN(attn_decode_hd64_f32_s4_l, 64, 4, true)
LLMRS_ATTN(attn_decode_hd128_f32_s4_l, 128, 4, true)

// attn_decode_mfma_hd<HD>_w<tile waves>[_l]: max(4, tile waves) waves
#define LLMRS_ATTN_MFMA(name, HD, TW, LOCAL)                                            \
  extern "C" __global__ __launch_bounds__(64 * (TW > 4 ? TW : 4)) void name(AttnArgs a) { \
    attn_decode_mfma_impl<HD, TW, LOCAL>(a);                                           \
  }
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w1, 64, 1, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w4, 64, 4, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w8, 64, 8, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w1, 128, 1, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w4, 128, 4, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w8, 128, 8, false)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w1_l, 64, 1, true)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w4_l, 64, 4, true)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd64_w8_l, 64, 8, true)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w1_l, 128, 1, true)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w4_l, 128, 4, true)
LLMRS_ATTN_MFMA(attn_decode_mfma_hd128_w8_l, 128, 8, true)
