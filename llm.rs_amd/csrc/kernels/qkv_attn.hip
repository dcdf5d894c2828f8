// qkv_attn.hip - the Q|K|V projection and the decode attention of one layer
// in one launch (batch 1, f16 KV cache, 8 KV heads).
//
// Reference: LlamaAttention::forward at seq == 1 (layer.rs:175-333): q, k
// and v from the RMSNorm'd input (layer.rs:177-179, 377), RoPE, the K/V
// append and attention over the cache (layer.rs:216-299).
//
// Why one launch: with grouped-query attention a KV head's attention reads
// only that head's rows of the projection - its n_rep query heads, its key
// and its value row - so the hand-off from the projection to the attention
// stays inside one KV head.  Workgroups are dealt to the 8 XCDs by linear
// index mod 8; with KV head g = linear index % 8 every workgroup of head g
// runs on one XCD, computes a share of head g's (n_rep + 2) * hd projection
// rows (the decode GEMV of gemv_core.h over mapped rows, stored through the
// vector L1 into that XCD's L2), counts itself in with an atomic in that L2,
// and waits until all nsplit workgroups of the head have; then it runs its
// attention split (attn_mfma.h) reading q, k and v from the L2.  The first
// K/V tile of the split is requested before the projection, so the cache
// reads overlap the weight stream, and the kernel boundary between the two
// (a launch and the attention's first memory round trips) is gone.
//
// Progress: the grid is nkv * nsplit workgroups of 256 threads with nsplit =
// CUs / nkv, one per CU; the host launches it only where every workgroup
// fits on the device at once (so a waiting workgroup never holds a slot
// that one it waits for needs) and where a probe launch showed the XCD
// dealing.  The wait is bounded: past spin_limit polls a workgroup sets the
// error word and carries on, so the grid always drains; the host reports it.
#include "attn_mfma.h"
#include "gemv_core.h"

using namespace llmrs;

namespace {

// Read-modify-writes in the XCD's L2 (atomics execute there).  The poll adds
// 0 with sequentially consistent ordering: LLVM rewrites an idempotent
// relaxed or acquire RMW into a plain load, which the vector L1 could serve
// from a stale line; a seq_cst one stays an atomic.
__device__ __forceinline__ int l2_fetch_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int l2_poll(int* p) {
  return __hip_atomic_fetch_add(p, 0, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_WORKGROUP);
}

}  // namespace

template <int WT, int PRO, int HD, int U>
__device__ __forceinline__ void qkv_attn_impl(const QkvAttnArgs& f) {
  extern __shared__ __align__(16) uint8_t smem[];  // the GEMV's operand and parked rows
  __shared__ GemvShared sh;
  __shared__ __align__(16) uint8_t alds[MfmaAttnLds<HD, 1>::BYTES];
  const AttnArgs& a = f.attn;
  const int lin = blockIdx.x + blockIdx.y * gridDim.x;
  const int g = lin % a.nkv, split = lin / a.nkv;
  const int n_rep = a.nq / a.nkv;
  GemvArgs ga = f.gemv;  // n = (n_rep + 2) * HD logical rows: head g's q, k, v
  ga.map_n1 = n_rep * HD;
  ga.map_n2 = HD;
  ga.map_b0 = g * n_rep * HD;
  ga.map_b1 = (a.nq + g) * HD;
  ga.map_b2 = (a.nq + a.nkv + g) * HD;
  if (g != 0) {  // the operand probe: one copy
    ga.probe_xq = nullptr;
    ga.probe_xd = nullptr;
  }
  const int pos = *a.pos_ptr;
  attn_mfma_item<HD, 1, true>(a, pos, alds, [&] {
    UnitRegs<WT, 2, U> ua, ub;
    gemv_body<WT, PRO, EPI_STORE, 2, U, false, 2, true>(ga, 0, split, a.nsplit, ua, ub, false, smem, sh);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's rows have reached the L2
    __syncthreads();
    unsigned long long t_rows = 0;
    if (f.ts_mid) t_rows = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      int* cnt = a.counters + g * kTicketStride + kArrivalWord;
      int seen = l2_fetch_add(cnt, 1) + 1;
      int spins = 0;
      while (seen < a.nsplit && spins < f.spin_limit) {
        seen = l2_poll(cnt);
        ++spins;
      }
      if (seen < a.nsplit) *f.err = 2;
      if (f.ts_mid) {
        unsigned long long* d = f.ts_mid + 2 * ((size_t)g * a.nsplit + split);
        d[0] = t_rows;
        d[1] = __builtin_amdgcn_s_memrealtime();
      }
    }
    __syncthreads();
  });
}

// qkv_attn_<weights>_<prologue>_hd<HD>_u<U>: the decode GEMV's prologue
// (norm: RMSNorm + Q8_0 of x; nq: the producer's codes of x*w) and units of
// 64*U blocks.
#define LLMRS_QKV_ATTN(name, WT, PRO, HD, U)                                       \
  extern "C" __global__ __launch_bounds__(256) void name(QkvAttnArgs f) {         \
    qkv_attn_impl<WT, PRO, HD, U>(f);                                             \
  }
#define LLMRS_QKV_ATTN_HD(tag, WT, PRO, ptag)                                      \
  LLMRS_QKV_ATTN(qkv_attn_##tag##_##ptag##_hd64_u1, WT, PRO, 64, 1)                \
  LLMRS_QKV_ATTN(qkv_attn_##tag##_##ptag##_hd64_u2, WT, PRO, 64, 2)                \
  LLMRS_QKV_ATTN(qkv_attn_##tag##_##ptag##_hd128_u1, WT, PRO, 128, 1)              \
  LLMRS_QKV_ATTN(qkv_attn_##tag##_##ptag##_hd128_u2, WT, PRO, 128, 2)
LLMRS_QKV_ATTN_HD(q4h, WT_Q4H, PRO_NORM, norm)
LLMRS_QKV_ATTN_HD(q4h, WT_Q4H, PRO_NQ, nq)
LLMRS_QKV_ATTN_HD(q4f, WT_Q4F, PRO_NORM, norm)
LLMRS_QKV_ATTN_HD(q4f, WT_Q4F, PRO_NQ, nq)
LLMRS_QKV_ATTN_HD(q8h, WT_Q8H, PRO_NORM, norm)
LLMRS_QKV_ATTN_HD(q8h, WT_Q8H, PRO_NQ, nq)
