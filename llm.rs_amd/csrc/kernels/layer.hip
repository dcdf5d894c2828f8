// layer.hip - one decoder layer of the batch-1 decode step in one launch.
//
// Reference: LlamaBlock::forward (layer.rs:373-406) at seq == 1:
//   qkv = W_qkv . Q8(RMSNorm(x))                       (layer.rs:177-179, 377)
//   ctx = attention(rope(q), cache + rope(k), v)        (layer.rs:175-333)
//   h   = x + W_o . ctx                                 (layer.rs:329-332, 386)
//   m   = silu(W_gate h') * (W_up h'), h' = Q8(RMSNorm(h))  (layer.rs:37-89, 393)
//   x   = h + W_down . m                                (layer.rs:93-96, 403)
//
// Why one launch per layer: on MI355X every kernel boundary costs a launch
// (~1.6 us in a graph) plus a ramp in which the new kernel's first weight
// loads are still in flight, and a batch-1 layer has five dependent steps.
// Here the grid is split into five roles, each a contiguous run of
// workgroups in dependency order.  A consumer role first requests its first
// weight units (weights never depend on activations), then waits on its
// producer's completion flags, so weight streaming overlaps the producer's latency
// (attention, prologues, tails) instead of following it.  Data produced and
// consumed inside the launch moves with device-scope (sc1) loads and stores,
// which bypass the per-XCD L2 copies; a producer workgroup waits for its
// stores to complete before it sets its flag.
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

template <int WT, int HD, bool KV16, int UH, int UF>
__device__ __forceinline__ void layer_impl(const LayerArgs& L) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  __shared__ unsigned s_word;
  const int H = L.hidden, F = L.ffn;
  int wg = blockIdx.x;
  const unsigned epoch = *L.epoch;
  unsigned* f_qkv = L.flags;
  unsigned* f_attn = f_qkv + L.n_qkv;
  unsigned* f_o = f_attn + L.nkv;
  unsigned* f_gu = f_o + L.n_o;
  LayerStamps st;
  st.dst = L.ts ? L.ts + 4 * (size_t)blockIdx.x : nullptr;
  st.rec(0);

  // ---- Q|K|V: qkv = W_qkv . Q8(RMSNorm(x)) --------------------------------
  if (wg < L.n_qkv) {
    GemvArgs g{};
    g.wq = L.w.qkv_w;
    g.ws = L.w.qkv_s;
    g.n = L.qkv_rows;
    g.k = H;
    g.x = L.x;
    g.norm_w = L.w.norm_in;
    g.eps = L.eps;
    g.y = L.qkv;
    UnitRegs<WT, 2, UH> ua, ub;
    gemv_body<WT, PRO_NORM, EPI_STORE, 2, UH, true>(g, 0, wg, L.n_qkv, ua, ub, false, smem, sh);
    st.rec(2);
    set_flag(f_qkv + wg, epoch);
    return;
  }
  wg -= L.n_qkv;

  // ---- attention: one (KV head, split) item per workgroup ----------------
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
    const int pos = *L.pos_ptr;
    auto wait_qkv = [&]() {
      const bool ok = wait_flags(f_qkv, L.n_qkv, epoch, L.err, &s_word);
      st.rec(1);
      return ok;
    };
    const bool combined = attn_item<HD, KV16, true>(a, wg / L.nsplit, wg % L.nsplit, pos, smem, wait_qkv);
    st.rec(2);
    if (combined) set_flag(f_attn + wg / L.nsplit, epoch);
    return;
  }
  wg -= L.n_attn;

  // ---- O + residual: h = x + W_o . ctx ------------------------------------
  if (wg < L.n_o) {
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
    set_flag(f_o + wg, epoch);
    return;
  }
  wg -= L.n_o;

  // ---- gate|up + SwiGLU: m = silu(g) * u (+ Q8) --------------------------
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
    UnitRegs<WT, 2, UH> ua, ub;
    Gemv<WT, EPI_SILU, 2, UH>(g, wg, L.n_gu).prefetch(ua, ub);
    if (!wait_flags(f_o, L.n_o, epoch, L.err, &s_word)) return;
    st.rec(1);
    gemv_body<WT, PRO_NORM, EPI_SILU, 2, UH, true>(g, 0, wg, L.n_gu, ua, ub, true, smem, sh);
    st.rec(2);
    set_flag(f_gu + wg, epoch);
    return;
  }
  wg -= L.n_gu;

  // ---- down + residual: x = h + W_down . m --------------------------------
  {
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
}

#define LLMRS_LAYER(name, WT, HD, KV16, UH, UF)                                  \
  extern "C" __global__ __launch_bounds__(kThreads) void name(LayerArgs L) {      \
    layer_impl<WT, HD, KV16, UH, UF>(L);                                      \
  }

#define LLMRS_LAYER_FAMILY(tag, WT)                                          \
  LLMRS_LAYER(layer_##tag##_hd64_f32_h1f2, WT, 64, false, 1, 2)              \
  LLMRS_LAYER(layer_##tag##_hd64_f16_h1f2, WT, 64, true, 1, 2)               \
  LLMRS_LAYER(layer_##tag##_hd128_f32_h1f2, WT, 128, false, 1, 2)            \
  LLMRS_LAYER(layer_##tag##_hd128_f16_h1f2, WT, 128, true, 1, 2)             \
  LLMRS_LAYER(layer_##tag##_hd64_f32_h2f1, WT, 64, false, 2, 1)              \
  LLMRS_LAYER(layer_##tag##_hd64_f16_h2f1, WT, 64, true, 2, 1)               \
  LLMRS_LAYER(layer_##tag##_hd128_f32_h2f1, WT, 128, false, 2, 1)            \
  LLMRS_LAYER(layer_##tag##_hd128_f16_h2f1, WT, 128, true, 2, 1)

LLMRS_LAYER_FAMILY(q4h, WT_Q4H)
LLMRS_LAYER_FAMILY(q4f, WT_Q4F)
LLMRS_LAYER_FAMILY(q8h, WT_Q8H)
