// decode.hip - persistent batch-1 decode for gfx950: every layer of every
// decode step in one cooperative launch.
//
// Reference: LlamaModel::forward (model.rs:17-49) over LlamaBlock::forward
// (layer.rs:373-406), driven like src/main.rs:128-327 with argmax in place
// of sampling.  Per step and layer the grid runs five phases separated by
// grid barriers:
//   QKV   qkv = W_qkv . Q8(RMSNorm(x))                  (layer.rs:177-179)
//   ATTN  rope, KV append, split attention, ctx (+Q8)    (layer.rs:175-333)
//   O     h = x + W_o . ctx                               (layer.rs:329-332,386)
//   GU    m = silu(W_gate h') * (W_up h'), h' = Q8(RMSNorm(h))  (layer.rs:37-89)
//   DOWN  x = h + W_down . m                              (layer.rs:93-96,403)
// then, when the step's token is needed, LM (logits and per-workgroup argmax
// partials, model.rs:39-47) and a barrier, after which every workgroup
// reduces the partials itself (no further barrier) and knows the next token.
//
// Why one launch: on MI355X every kernel boundary writes back all eight XCD
// L2s, a fixed 3-5 us per kernel that, at five kernels per layer, is as long
// as streaming the layer's weights.  Inside this kernel the phases hand data
// over with device-scope (sc1) loads and stores, which bypass the per-XCD L2
// copies, so a barrier needs no cache maintenance: it is two relaxed
// atomics (per-XCD-group counter, then a top counter) and a spin on the top
// counter.  Before every barrier each wave requests the first two units of
// weights of the next GEMV phase (weights never depend on activations), so
// HBM streams while the grid synchronises.
//
// Every spin is bounded: a workgroup whose wait exceeds the limit sets the
// error word and leaves, so the others' waits time out as well and the grid
// drains.  The host reports the error; nothing spins forever.
#include "attn_core.h"
#include "gemv_core.h"

using namespace llmrs;

namespace {

constexpr long kSpinLimit = 1L << 22;
constexpr int kGroups = 8;  // one barrier counter per XCD (workgroups are dealt round-robin)

__device__ __forceinline__ unsigned ld_dev_u(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_dev_u(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Hierarchical grid barrier.  Word 0 is the top counter, word 64*(1+i) the
// counter of group i (workgroups wg with wg % ng == i); 256-byte spacing
// keeps the counters in separate cache lines.
struct GridBarrier {
  unsigned* top;
  unsigned* grp;
  int ng;
  unsigned gsize;
  unsigned round;
  int* abort_flag;  // LDS
  int* err;

  __device__ GridBarrier(unsigned* words, int wg, int nwg, int* lds_abort, int* err_)
      : top(words), abort_flag(lds_abort), err(err_) {
    ng = nwg < kGroups ? nwg : kGroups;
    const int gi = wg % ng;
    grp = words + 64 * (1 + gi);
    gsize = (unsigned)((nwg - 1 - gi) / ng + 1);
    round = 0;
  }

  // Arrival, in two halves so the next phase's weight loads can be issued
  // in between.  publish() waits until this workgroup's stores have
  // completed, then arrives: the counter atomics are issued while nothing
  // else is outstanding (on gfx9 loads, stores and atomics share one
  // in-order counter, so an arrival issued after the prefetch would wait for
  // the prefetch's HBM latency before the last arriver could advance the top
  // counter).  wait() spins on the top counter; it returns false when this
  // workgroup must leave (a wait timed out).
  __device__ __forceinline__ void publish() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ++round;
    if (threadIdx.x == 0) {
      const unsigned t = add_dev_u(grp, 1u);
      if (t == gsize * round - 1) add_dev_u(top, 1u);
    }
  }
  __device__ __forceinline__ bool wait() {
    if (threadIdx.x == 0) {
      const unsigned target = (unsigned)ng * round;
      long spins = 0;
      int bad = 0;
      while (ld_dev_u(top) < target) {
        if (++spins > kSpinLimit) {
          bad = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (bad) atomicExch(err, 1);
      *abort_flag = bad;
    }
    __syncthreads();
    return *abort_flag == 0;
  }
};

// Greedy choice from the per-workgroup partials (argmax_final's rule).
__device__ __forceinline__ int reduce_argmax(const float* pv, const int* pi, int n, float* s_v, int* s_i) {
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float v = dev_ldf(pv, 4 * i);
    const int ix = (int)dev_ldu(pi, 4 * i);
    if (better(v, ix, bv, bi)) {
      bv = v;
      bi = ix;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  if (lane_id() == 0) {
    s_v[wave_id()] = bv;
    s_i[wave_id()] = bi;
  }
  __syncthreads();
  bv = s_v[0];
  bi = s_i[0];
  for (int w = 1; w < kWaves; ++w)
    if (better(s_v[w], s_i[w], bv, bi)) {
      bv = s_v[w];
      bi = s_i[w];
    }
  return bi == 0x7fffffff ? 0 : bi;  // every logit NaN
}

}  // namespace

// Phase timestamps: workgroup 0 records the 100 MHz real-time counter when a
// phase's own work ends and when the following barrier releases it, layer by
// layer, for the first step of the launch (profiling only; null = off).
// Layer 1 of the first step is also recorded for every workgroup, after the
// per-layer block: ts[10 L + 10 wg + slot].
#define LLMRS_TS(slot)                                                              \
  do {                                                                              \
    if (d.ts && s == 0 && tid == 0) {                                               \
      if (wg == 0) d.ts[(size_t)l * 10 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
      if (l == 1) d.ts[(size_t)L * 10 + (size_t)wg * 10 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
    }                                                                               \
  } while (0)

template <int WT, int HD, bool KV16, int U>
__device__ __forceinline__ void decode_impl(const DecodeArgs& d) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ GemvShared sh;
  __shared__ int s_abort;
  const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x;
  GridBarrier bar(d.bar, wg, nwg, &s_abort, d.err);

  const int H = d.hidden, F = d.ffn, L = d.n_layers;
  const int items = d.nkv * d.nsplit;

  // One pair of unit registers for every GEMV phase (R = 2 rows per unit):
  // the next phase's first units are loaded into them before each barrier.
  UnitRegs<WT, 2, U> ra, rb;

  auto args_qkv = [&](int l, const float* xin) {
    const LayerDesc& Ld = d.layers[l];
    GemvArgs g{};
    g.wq = Ld.qkv_w;
    g.ws = Ld.qkv_s;
    g.n = d.qkv_rows;
    g.k = H;
    g.x = xin;
    g.norm_w = Ld.norm_in;
    g.eps = d.eps;
    g.y = d.qkv;
    return g;
  };
  auto args_o = [&](int l, const float* xin) {
    const LayerDesc& Ld = d.layers[l];
    GemvArgs g{};
    g.wq = Ld.o_w;
    g.ws = Ld.o_s;
    g.n = H;
    g.k = d.nq * HD;
    g.xq = d.ctx_q;
    g.xd = d.ctx_d;
    g.y = d.h;
    g.res = xin;
    return g;
  };
  auto args_gu = [&](int l) {
    const LayerDesc& Ld = d.layers[l];
    GemvArgs g{};
    g.wq = Ld.gu_w;
    g.ws = Ld.gu_s;
    g.n = 2 * F;
    g.k = H;
    g.x = d.h;
    g.norm_w = Ld.norm_post;
    g.eps = d.eps;
    g.y = d.mf;
    g.yq = d.m_q;
    g.yd = d.m_d;
    return g;
  };
  auto args_down = [&](int l) {
    const LayerDesc& Ld = d.layers[l];
    GemvArgs g{};
    g.wq = Ld.down_w;
    g.ws = Ld.down_s;
    g.n = H;
    g.k = F;
    g.xq = d.m_q;
    g.xd = d.m_d;
    g.y = d.x;
    g.res = d.h;
    return g;
  };
  auto args_lm = [&](float* logits) {
    GemvArgs g{};
    g.wq = d.lm_w;
    g.ws = d.lm_s;
    g.n = d.vocab;
    g.k = H;
    g.x = d.x;
    g.norm_w = d.final_norm;
    g.eps = d.eps;
    g.y = logits;
    g.part_val = d.part_val;
    g.part_idx = d.part_idx;
    return g;
  };

  int next_tok = 0;
  bool qkv_pre = false;  // ra/rb hold the first units of the coming QKV phase
  for (int s = 0; s < d.n_steps; ++s) {
    const int pos = d.pos0 + s;
    // Prompt ids, and the id the previous launch produced, come from memory.
    const int tok = (s == 0 || pos < d.n_prompt) ? d.tokens[pos] : next_tok;
    const float* xin = d.embed + (size_t)tok * H;  // main.rs:159-167
    const bool need_lm = pos + 1 >= d.n_prompt;
    for (int l = 0; l < L; ++l) {
      // QKV
      {
        const GemvArgs g = args_qkv(l, xin);
        gemv_body<WT, PRO_NORM, EPI_STORE, 2, U, true>(g, 0, wg, nwg, ra, rb, qkv_pre, smem, sh);
      }
      LLMRS_TS(0);
      bar.publish();
      // the O weights do not depend on the attention: request them now
      Gemv<WT, EPI_RESID, 2, U>(args_o(l, xin), wg, nwg).prefetch(ra, rb);
      if (!bar.wait()) return;
      LLMRS_TS(1);
      // ATTN
      {
        AttnArgs a{};
        const LayerDesc& Ld = d.layers[l];
        a.qkv = d.qkv;
        a.kc = Ld.kc;
        a.vc = Ld.vc;
        a.rope_cos = d.rope_cos;
        a.rope_sin = d.rope_sin;
        a.part_o = d.part_o;
        a.part_ml = d.part_ml;
        a.counters = d.counters + (size_t)l * d.nkv;
        a.ctx = d.ctx;
        a.ctx_q = d.ctx_q;
        a.ctx_d = d.ctx_d;
        a.max_seq = d.max_seq;
        a.nq = d.nq;
        a.nkv = d.nkv;
        a.nsplit = d.nsplit;
        a.scale = d.attn_scale;
        a.ts = (d.ts && s == 0 && l == 1) ? d.ts + (size_t)L * 10 + (size_t)nwg * 10 : nullptr;
        for (int it = wg; it < items; it += nwg)
          attn_item<HD, KV16, true>(a, it / d.nsplit, it % d.nsplit, pos, smem);
      }
      LLMRS_TS(2);
      bar.publish();
      if (!bar.wait()) return;
      LLMRS_TS(3);
      // O + residual
      {
        const GemvArgs g = args_o(l, xin);
        gemv_body<WT, PRO_Q8, EPI_RESID, 2, U, true>(g, 0, wg, nwg, ra, rb, true, smem, sh);
      }
      LLMRS_TS(4);
      bar.publish();
      Gemv<WT, EPI_SILU, 2, U>(args_gu(l), wg, nwg).prefetch(ra, rb);
      if (!bar.wait()) return;
      LLMRS_TS(5);
      // gate|up + SwiGLU
      {
        const GemvArgs g = args_gu(l);
        gemv_body<WT, PRO_NORM, EPI_SILU, 2, U, true>(g, 0, wg, nwg, ra, rb, true, smem, sh);
      }
      LLMRS_TS(6);
      bar.publish();
      Gemv<WT, EPI_RESID, 2, U>(args_down(l), wg, nwg).prefetch(ra, rb);
      if (!bar.wait()) return;
      LLMRS_TS(7);
      // down + residual
      {
        const GemvArgs g = args_down(l);
        gemv_body<WT, PRO_Q8, EPI_RESID, 2, U, true>(g, 0, wg, nwg, ra, rb, true, smem, sh);
      }
      LLMRS_TS(8);
      bar.publish();
      {
        if (l + 1 < L) {
          Gemv<WT, EPI_STORE, 2, U>(args_qkv(l + 1, d.x), wg, nwg).prefetch(ra, rb);
          qkv_pre = true;
        } else if (need_lm) {
          Gemv<WT, EPI_ARGMAX, 2, U>(args_lm(nullptr), wg, nwg).prefetch(ra, rb);
          qkv_pre = false;
        } else {
          // next step, layer 0 (its input row is not needed to fetch weights)
          Gemv<WT, EPI_STORE, 2, U>(args_qkv(0, d.embed), wg, nwg).prefetch(ra, rb);
          qkv_pre = true;
        }
      }
      if (!bar.wait()) return;
      LLMRS_TS(9);
      xin = d.x;
    }
    if (need_lm) {
      float* logits = (s == d.n_steps - 1) ? d.logits : nullptr;
      const GemvArgs g = args_lm(logits);
      gemv_body<WT, PRO_NORM, EPI_ARGMAX, 2, U, true>(g, 0, wg, nwg, ra, rb, true, smem, sh);
      bar.publish();
      if (s + 1 < d.n_steps) {
        Gemv<WT, EPI_STORE, 2, U>(args_qkv(0, d.embed), wg, nwg).prefetch(ra, rb);
        qkv_pre = true;
      }
      if (!bar.wait()) return;
      next_tok = reduce_argmax(d.part_val, d.part_idx, nwg, sh.bv, sh.bi);
      if (wg == 0 && tid == 0 && pos + 1 < d.cap) {
        d.gen[pos + 1] = next_tok;
        if (pos + 1 >= d.n_prompt) d.tokens_out[pos + 1] = next_tok;
      }
    }
  }
  if (wg == 0 && tid == 0) *d.pos_out = d.pos0 + d.n_steps;
}

#define LLMRS_DECODE(name, WT, HD, KV16, U)                                          \
  extern "C" __global__ __launch_bounds__(kThreads, 2) void name(DecodeArgs d) {     \
    decode_impl<WT, HD, KV16, U>(d);                                                 \
  }

#define LLMRS_DECODE_FAMILY(tag, WT)                                  \
  LLMRS_DECODE(decode_##tag##_hd64_f32_u1, WT, 64, false, 1)          \
  LLMRS_DECODE(decode_##tag##_hd64_f16_u1, WT, 64, true, 1)           \
  LLMRS_DECODE(decode_##tag##_hd64_f32_u2, WT, 64, false, 2)          \
  LLMRS_DECODE(decode_##tag##_hd64_f16_u2, WT, 64, true, 2)           \
  LLMRS_DECODE(decode_##tag##_hd128_f32_u1, WT, 128, false, 1)        \
  LLMRS_DECODE(decode_##tag##_hd128_f16_u1, WT, 128, true, 1)         \
  LLMRS_DECODE(decode_##tag##_hd128_f32_u2, WT, 128, false, 2)        \
  LLMRS_DECODE(decode_##tag##_hd128_f16_u2, WT, 128, true, 2)

LLMRS_DECODE_FAMILY(q4h, WT_Q4H)
LLMRS_DECODE_FAMILY(q4f, WT_Q4F)
LLMRS_DECODE_FAMILY(q8h, WT_Q8H)
