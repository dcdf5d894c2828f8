// layer.hip - the batch-1 decode layer in three launches instead of five.
//
// Reference: LlamaBlock::forward (layer.rs:373-406) at seq == 1:
//   qkv = W_qkv . Q8(RMSNorm(x))                       (layer.rs:177-179, 377)
//   ctx = attention(rope(q), cache + rope(k), v)        (layer.rs:175-333)
//   h   = x + W_o . ctx                                 (layer.rs:329-332, 386)
//   m   = silu(W_gate h') * (W_up h'), h' = Q8(RMSNorm(h))  (layer.rs:37-89, 393)
//   x   = h + W_down . m                                (layer.rs:93-96, 403)
// The Q|K|V GEMV stays a launch of its own (gemv.hip); attention + O and
// gate|up + down are one launch each.
//
// Why: on MI355X every kernel boundary costs a launch (~1.6 us in a graph)
// plus a ramp in which the new kernel's first weight loads are still in
// flight.  Inside one launch the grid is split into two roles, producer
// workgroups first.  A consumer workgroup first requests its first weight
// units (weights never depend on activations), then waits for its
// producers' completion flags, so its weight stream overlaps the producer's
// latency-bound tail (the attention chain, the gate|up tail) instead of
// following it.  Data produced and consumed inside a launch moves with
// device-scope (sc1) loads and stores, which bypass the per-XCD L2 copies; a
// producer workgroup waits for its stores to complete before it sets its
// flag.
//
// Progress: workgroups are dispatched in increasing index order, producers
// before consumers, so a waiting consumer never holds a slot its producer
// still needs to start.  Every wait is nevertheless bounded: a workgroup
// whose wait exceeds the spin limit sets the error word and leaves, the
// waits of its own consumers then time out as well and the grid drains; the
// host checks the error word.
#include "attn_core.h"
#include "gemv_core.h"

using namespace llmrs;

namespace {

constexpr long kSpinLimit = 1L << 21;

// Completion flags instead of shared counters: every producer workgroup
// stores the step's epoch into its own word (no read-modify-write, so no
// serialisation of hundreds of atomics on one address, measured at ~40 ns
// each), and a consumer's first wave loads all of its producer's words at
// once.  Epochs increase every decode step, so flags never need clearing.
__device__ __forceinline__ void set_flag(unsigned* flag, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete (device-visible)
  __syncthreads();                // ... and every other wave's
  if (threadIdx.x == 0) dev_stu(flag, 0, epoch);
}

// Wave 0 polls flags[0..n) until every word equals epoch; false when the
// spin limit was hit (the error word is set) or another workgroup failed.
__device__ __forceinline__ bool wait_flags(const unsigned* flags, int n, unsigned epoch, int* err,
                                           unsigned* s_word) {
  if (threadIdx.x < LLMRS_WAVE) {
    const int lane = threadIdx.x;
    long spins = 0;
    unsigned bad = 0;
    for (;;) {
      bool ok = true;
      for (int i = lane; i < n; i += LLMRS_WAVE) ok &= dev_ldu(flags, 4 * i) == epoch;
      if (__all(ok)) break;
      if (++spins > kSpinLimit || dev_ldu(err, 0) != 0) {
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) {
      if (bad) dev_stu(err, 0, 1u);
      *s_word = bad;
    }
  }
  __syncthreads();
  return *s_word == 0;
}

}  // namespace

// Profiling stamps of one workgroup, kept in registers and stored on exit:
// 0 start, 1 producer wait released, 2 own work done, 3 end.
struct LayerStamps {
  unsigned long long* dst;
  unsigned long long t[4] = {0, 0, 0, 0};
  __device__ __forceinline__ void rec(int i) {
    if (dst) t[i] = __builtin_amdgcn_s_memrealtime();
  }
  __device__ __forceinline__ ~LayerStamps() {
    if (dst && threadIdx.x == 0) {
      t[3] = __builtin_amdgcn_s_memrealtime();
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = t[i];
    }
  }
};

// Attention + O projection in one launch: the attention items first, then
// the O workgroups, which request their weights, wait for every KV head's
// combined ctx, and finish h = x + W_o . ctx.
template <int WT, int HD, bool KV16, int UH>
__device__ __forceinline__ void attn_o_impl(const LayerArgs& L) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  __shared__ unsigned s_word;
  const int H = L.hidden;
  int wg = blockIdx.x;
  const unsigned epoch = *L.epoch;
  unsigned* f_attn = L.flags;
  LayerStamps st;
  st.dst = L.ts ? L.ts + 4 * (size_t)blockIdx.x : nullptr;
  st.rec(0);

  if (wg < L.n_attn) {
    AttnArgs a{};
    a.qkv = L.qkv;
    a.pos_ptr = L.pos_ptr;
    a.kc = L.w.kc;
    a.vc = L.w.vc;
    a.rope_cos = L.rope_cos;
    a.rope_sin = L.rope_sin;
    a.part_o = L.part_o;
    a.part_ml = L.part_ml;
    a.counters = L.counters;
    a.ctx = L.ctx;
    a.ctx_q = L.ctx_q;
    a.ctx_d = L.ctx_d;
    a.max_seq = L.max_seq;
    a.nq = L.nq;
    a.nkv = L.nkv;
    a.nsplit = L.nsplit;
    a.scale = L.attn_scale;
    // q/k/v and the cache come from earlier launches: plain loads
    const bool combined = attn_item<HD, KV16, false>(a, wg / L.nsplit, wg % L.nsplit, *L.pos_ptr, smem);
    st.rec(2);
    if (combined) set_flag(f_attn + wg / L.nsplit, epoch);
    return;
  }
  wg -= L.n_attn;
  GemvArgs g{};
  g.wq = L.w.o_w;
  g.ws = L.w.o_s;
  g.n = H;
  g.k = L.nq * HD;
  g.xq = L.ctx_q;
  g.xd = L.ctx_d;
  g.y = L.h;
  g.res = L.x;
  UnitRegs<WT, 2, UH> ua, ub;
  Gemv<WT, EPI_RESID, 2, UH>(g, wg, L.n_o).prefetch(ua, ub);
  if (!wait_flags(f_attn, L.nkv, epoch, L.err, &s_word)) return;
  st.rec(1);
  gemv_body<WT, PRO_Q8, EPI_RESID, 2, UH, true>(g, 0, wg, L.n_o, ua, ub, true, smem, sh);
  st.rec(2);
}

// gate|up + SwiGLU and down + residual in one launch: the gate|up
// workgroups first, then the down workgroups, which request their weights,
// wait for every gate|up workgroup and finish x = h + W_down . m.
template <int WT, int UH, int UF>
__device__ __forceinline__ void mlp_impl(const LayerArgs& L) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  __shared__ unsigned s_word;
  const int H = L.hidden, F = L.ffn;
  int wg = blockIdx.x;
  const unsigned epoch = *L.epoch;
  unsigned* f_gu = L.flags + L.nkv + L.n_o;
  LayerStamps st;
  st.dst = L.ts ? L.ts + 4 * (size_t)blockIdx.x : nullptr;
  st.rec(0);

  if (wg < L.n_gu) {
    GemvArgs g{};
    g.wq = L.w.gu_w;
    g.ws = L.w.gu_s;
    g.n = 2 * F;
    g.k = H;
    g.x = L.h;
    g.norm_w = L.w.norm_post;
    g.eps = L.eps;
    g.y = L.mf;
    g.yq = L.m_q;
    g.yd = L.m_d;
    UnitRegs<WT, 4, UH> ua, ub;
    gemv_body<WT, PRO_NORM, EPI_SILU, 4, UH, true, 1>(g, 0, wg, L.n_gu, ua, ub, false, smem, sh);
    st.rec(2);
    set_flag(f_gu + wg, epoch);
    return;
  }
  wg -= L.n_gu;
  GemvArgs g{};
  g.wq = L.w.down_w;
  g.ws = L.w.down_s;
  g.n = H;
  g.k = F;
  g.xq = L.m_q;
  g.xd = L.m_d;
  g.y = L.x;
  g.res = L.h;
  UnitRegs<WT, 2, UF> ua, ub;
  Gemv<WT, EPI_RESID, 2, UF>(g, wg, L.n_down).prefetch(ua, ub);
  if (!wait_flags(f_gu, L.n_gu, epoch, L.err, &s_word)) return;
  st.rec(1);
  gemv_body<WT, PRO_Q8, EPI_RESID, 2, UF, true>(g, 0, wg, L.n_down, ua, ub, true, smem, sh);
  st.rec(2);
}

#define LLMRS_ATTN_O(name, WT, HD, KV16, UH)                                    \
  extern "C" __global__ __launch_bounds__(kThreads) void name(LayerArgs L) {   \
    attn_o_impl<WT, HD, KV16, UH>(L);                                         \
  }
#define LLMRS_MLP(name, WT, UH, UF)                                             \
  extern "C" __global__ __launch_bounds__(kThreads) void name(LayerArgs L) {   \
    mlp_impl<WT, UH, UF>(L);                                                  \
  }

#define LLMRS_LAYER_FAMILY(tag, WT)                                  \
  LLMRS_ATTN_O(attn_o_##tag##_hd64_f32_u1, WT, 64, false, 1)         \
  LLMRS_ATTN_O(attn_o_##tag##_hd64_f16_u1, WT, 64, true, 1)          \
  LLMRS_ATTN_O(attn_o_##tag##_hd128_f32_u1, WT, 128, false, 1)       \
  LLMRS_ATTN_O(attn_o_##tag##_hd128_f16_u1, WT, 128, true, 1)        \
  LLMRS_ATTN_O(attn_o_##tag##_hd64_f32_u2, WT, 64, false, 2)         \
  LLMRS_ATTN_O(attn_o_##tag##_hd64_f16_u2, WT, 64, true, 2)          \
  LLMRS_ATTN_O(attn_o_##tag##_hd128_f32_u2, WT, 128, false, 2)       \
  LLMRS_ATTN_O(attn_o_##tag##_hd128_f16_u2, WT, 128, true, 2)        \
  LLMRS_MLP(mlp_##tag##_h1f1, WT, 1, 1)                              \
  LLMRS_MLP(mlp_##tag##_h1f2, WT, 1, 2)                              \
  LLMRS_MLP(mlp_##tag##_h2f1, WT, 2, 1)                              \
  LLMRS_MLP(mlp_##tag##_h2f2, WT, 2, 2)

LLMRS_LAYER_FAMILY(q4h, WT_Q4H)
LLMRS_LAYER_FAMILY(q4f, WT_Q4F)
LLMRS_LAYER_FAMILY(q8h, WT_Q8H)
