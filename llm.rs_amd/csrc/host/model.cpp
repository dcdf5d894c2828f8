// model.cpp - the HBM-resident decode model and its per-token kernel sequence.
//
// One decode position = 5 kernels per layer + 3 (LlamaModel::forward,
// model.rs:17-49, over LlamaBlock::forward, layer.rs:373-406):
//   embed_gather                      x = E[token[pos]]          (main.rs:159-167)
//   per layer:
//     gemv *_norm_store   (Q|K|V)     qkv = W_qkv . Q8(RMSNorm(x))  (layer.rs:177-179)
//     attn_decode                     rope, KV append, attention, ctx (+Q8)
//     gemv *_q8_resid     (O)         h = x + W_o . ctx             (layer.rs:329-332,386)
//     gemv *_norm_silu    (gate|up)   m = silu(g)*u (+Q8)           (layer.rs:40-89)
//     gemv *_q8_resid     (down)      x = h + W_down . m            (layer.rs:93-96,403)
//   gemv *_norm_argmax    (lm_head)   logits, partial argmax        (model.rs:39-47)
//   argmax_final                      next token, pos += 1
// Every kernel reads the position from device memory, so one captured HIP
// graph replays every step with no host round trip.
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <tuple>

#include "../kernel_args.h"
#include "internal.h"

using namespace llmrs;

namespace {

struct DevLinear {
  uint8_t* codes = nullptr;
  void* scales = nullptr;
  int n = 0, k = 0;
  size_t bytes = 0;
};

struct LayerBufs {
  DevLinear qkv, o, gu, down;
  float* norm[2] = {nullptr, nullptr};
  void* kc = nullptr;
  void* vc = nullptr;
  unsigned set_mask = 0;  // bit s = linear slot s uploaded; bits 8,9 = norms
};

int env_int(const char* name, int def) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : def;
}
std::string env_str(const char* name) {
  const char* v = std::getenv(name);
  return v ? std::string(v) : std::string();
}

// Batched decode runs its linear layers on the row-batched decode GEMV up to
// this many sequences (8B shape, ms per step GEMV / skinny GEMM: B = 1 1.63 /
// 2.73, 2 1.94 / 2.84, 4 2.66 / 3.04, 8 4.00 / 3.26); LLMRS_BATCH_GEMM=gemv,
// skinny or prefill forces one path.
constexpr int kBatchGemvMax = 4;

}  // namespace

struct llmrs_model {
  llmrs_model_config c{};
  int wt = WT_Q4H;
  int qkv_rows = 0;
  std::vector<LayerBufs> layers;
  float* embed = nullptr;
  float* final_norm = nullptr;
  DevLinear lm_head;
  bool embed_set = false, final_set = false, lm_set = false;
  // activations and state
  float *x = nullptr, *h = nullptr, *qkv = nullptr, *ctxv = nullptr, *mf = nullptr;
  float *logits = nullptr, *ctx_d = nullptr, *m_d = nullptr, *part_o = nullptr, *part_ml = nullptr;
  float *part_val = nullptr, *rope_cos = nullptr, *rope_sin = nullptr, *trace = nullptr;
  float* rope_now = nullptr;  // [hd]: the step position's RoPE row (embed_gather -> attention)
  int8_t *ctx_q = nullptr, *m_q = nullptr;
  // RMSNorm operands from the producers (gemv_core.h PRO_NQ): codes of x*w,
  // d' and sums of squares per block, of x (Q|K|V and lm_head input) and of
  // h (gate|up input)
  int8_t *x_q = nullptr, *h_q = nullptr;
  float *x_d = nullptr, *x_ss = nullptr, *h_d = nullptr, *h_ss = nullptr;
  // producer-side norm operands: x's (down -> next Q|K|V and lm_head,
  // embedding -> layer 0) and h's (O -> gate|up); false: RMSNorm + Q8_0
  // inside the consumers
  bool nq_x = true, nq_h = true;
  int *part_idx = nullptr, *counters = nullptr, *tokens = nullptr, *gen = nullptr;
  int *pos = nullptr, *n_prompt = nullptr, *err = nullptr;
  int nsplit = 1, lm_grid = 1, cap = 0;
  // decode attention layout: tile streams per workgroup of the vector kernel
  // (f32 caches, 256 threads each), tile waves per 256-thread workgroup of
  // the matrix-core kernel (f16 caches)
  int attn_streams = 1, attn_waves = 1;
  // decode attention: the splits of a KV head on one XCD, exchanging
  // partials through its L2 (the attention kernels' _l variants)
  bool attn_local = false;
  // batches created on this model and not yet freed: the model outlives them
  int live_batches = 0;
  // single-sequence steps on the reference-order kernels (exact.hip)
  bool exact = false;
  float* ex_part_val = nullptr;  // [exact_gemv_cap()] argmax partials of the exact lm_head
  int* ex_part_idx = nullptr;
  size_t host_pos = 0;
  bool begun = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool graph_failed = false;
  int host_n_prompt = 0;
  // sampling in place of the greedy argmax (llmrs_model_set_sampling)
  bool sampling = false;
  llmrs_sampling samp{};
  float* probs = nullptr;      // [vocab] sampler scratch, allocated on first use
  llmrs::SampleState* samp_state = nullptr;
  int* eos = nullptr;          // [LLMRS_MAX_EOS]
  int* stopped = nullptr;      // an end-of-sequence id was drawn
  // batched prompt (prefill) buffers for chunks of up to pf_cap rows,
  // allocated on first use
  int pf_cap = 0;
  float *pf_x = nullptr, *pf_h = nullptr, *pf_qkv = nullptr, *pf_q = nullptr;
  float *pf_ad = nullptr, *pf_ctx_d = nullptr, *pf_m_d = nullptr;
  int8_t *pf_aq = nullptr, *pf_ctx_q = nullptr, *pf_m_q = nullptr;
  int* pf_start = nullptr;   // first position of the chunk (device copy)
  std::vector<void*> allocs;

  template <class T>
  T* dalloc(size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    if (hipMalloc(&p, bytes) != hipSuccess) {
      (void)hipGetLastError();
      fail(LLMRS_E_OOM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    allocs.push_back(p);
    LLMRS_HIP(hipMemsetAsync(p, 0, bytes, ctx().stream));
    return (T*)p;
  }
  void alloc_linear(DevLinear& L, int n, int k) {
    L.n = n;
    L.k = k;
    const size_t nb = (size_t)k / 32;
    const size_t code_bytes = (size_t)n * nb * block_code_bytes(wt);
    const size_t off = align_up(code_bytes, 256);
    L.bytes = off + (size_t)n * nb * block_scale_bytes(wt);
    L.codes = dalloc<uint8_t>(L.bytes);
    L.scales = L.codes + off;
  }
  ~llmrs_model() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (void* p : allocs) (void)hipFree(p);
  }
};

namespace {

size_t kv_elem_bytes(const llmrs_model* m) { return m->c.kv_dtype == LLMRS_F16 ? 2 : 4; }
// Cache rows per KV head: max_seq rounded up to whole attention tiles.
int kv_rows(const llmrs_model* m) { return llmrs::kv_rows(m->c.max_seq); }
size_t kv_layer_elems(const llmrs_model* m) {
  return (size_t)m->c.n_kv_heads * kv_rows(m) * m->c.head_dim;
}

// Records a (name, algorithmic bytes, start, end) tuple per launch when
// profiling - the events take the dispatch's own start and end timestamps -
// otherwise a plain launch.
struct Launcher {
  hipStream_t s;
  std::vector<std::tuple<std::string, double, hipEvent_t, hipEvent_t>>* rec = nullptr;
  template <class A>
  void operator()(const std::string& name, double bytes, dim3 g, dim3 b, size_t lds, const A& args) {
    if (!rec) {
      launch(name, g, b, lds, s, args);
      return;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    LLMRS_HIP(hipEventCreate(&e0));
    LLMRS_HIP(hipEventCreate(&e1));
    rec->emplace_back(name, bytes, e0, e1);
    launch_timed(name, g, b, lds, s, args, e0, e1);
  }
};

double linear_weight_bytes(const llmrs_model* m, const DevLinear& L) {
  const double nb = L.k / 32.0;
  return (double)L.n * nb * (block_code_bytes(m->wt) + block_scale_bytes(m->wt));
}

void enqueue_head(llmrs_model* m, Launcher& L, bool write_logits, int8_t* probe_xq = nullptr,
                  float* probe_xd = nullptr);

// The decode-attention kernel of this model (attention.hip).
std::string attn_kernel(const llmrs_model* m) {
  const char* local = m->attn_local ? "_l" : "";
  if (m->c.kv_dtype == LLMRS_F16)
    return "attn_decode_mfma_hd" + std::to_string(m->c.head_dim) + "_w" + std::to_string(m->attn_waves) + local;
  return "attn_decode_hd" + std::to_string(m->c.head_dim) + "_f32" + (m->attn_streams > 1 ? "_s4" : "") + local;
}
// Its threads per workgroup.
unsigned attn_threads(const llmrs_model* m) {
  return m->c.kv_dtype == LLMRS_F16 ? 64u * (unsigned)std::max(4, m->attn_waves) : 256u * (unsigned)m->attn_streams;
}

// x = the embedding of the token at the device position, or (x_in set) the
// row x_in; with the consumers' RMSNorm folded into the producers, also the
// first RMSNorm's operand of x with weight norm_w (PRO_NQ of gemv_core.h).
// Kernel arguments of the sampling parameters; the caller fills the buffers.
SampleArgs sample_args(const llmrs_sampling& s, int vocab) {
  SampleArgs a{};
  a.vocab = vocab;
  a.groups = llmrs::sample_groups(vocab);
  a.penalty = s.repeat_penalty;
  a.temperature = s.temperature;
  a.top_p = s.top_p;
  a.window = s.penalty_window;
  a.seed = s.seed;
  a.n_eos = s.n_eos;
  a.step_override = -1;
  return a;
}

void check_sampling(const llmrs_sampling& s, int vocab) {
  LLMRS_REQUIRE(std::isfinite(s.temperature) && s.temperature > 0.0f, LLMRS_E_INVALID,
                "temperature must be finite and > 0");
  LLMRS_REQUIRE(std::isfinite(s.top_p), LLMRS_E_INVALID, "top_p must be finite");
  LLMRS_REQUIRE(std::isfinite(s.repeat_penalty) && s.repeat_penalty > 0.0f, LLMRS_E_INVALID,
                "repeat_penalty must be finite and > 0");
  LLMRS_REQUIRE(s.n_eos >= 0 && s.n_eos <= LLMRS_MAX_EOS, LLMRS_E_INVALID, "n_eos must be in [0, 8]");
  LLMRS_REQUIRE(vocab > 0 && vocab <= llmrs::kSampleMaxVocab, LLMRS_E_INVALID,
                "sampling supports vocabularies up to 262144 ids");
}

// The sampler's launch chain (sample.hip): prep, probs, the refine levels
// (top-p only), pick.  Work figures: bytes of the launch's vocabulary passes.
void enqueue_sample(Launcher& L, const SampleArgs& a) {
  const dim3 grid((unsigned)a.groups), block((unsigned)llmrs::kSampleThreads);
  const double V = a.vocab;
  L("sample_prep", 8.0 * V, grid, block, 0, a);
  L("sample_probs", 8.0 * V, grid, block, 0, a);
  if (a.top_p < 1.0f)
    for (int i = 0; i < llmrs::kSampleRefines; ++i) L("sample_refine", 4.0 * V, grid, block, 0, a);
  L("sample_pick", 4.0 * V, grid, block, 0, a);
}

void enqueue_embed(llmrs_model* m, Launcher& L, const float* x_in, const float* norm_w) {
  const int H = m->c.hidden;
  EmbedArgs e{};
  e.table = m->embed;
  e.tokens = m->tokens;
  e.pos_ptr = m->pos;
  e.x = m->x;
  e.err = m->err;
  e.hidden = H;
  e.vocab = m->c.vocab;
  if (m->nq_x) {
    e.norm_w = norm_w;
    e.xq = m->x_q;
    e.xd = m->x_d;
    e.xss = m->x_ss;
  }
  e.x_in = x_in;
  e.rope_cos = m->rope_cos;
  e.rope_sin = m->rope_sin;
  e.rope_now = m->rope_now;
  e.rope_mid = m->c.head_dim / 2;
  e.rope_rows = m->c.max_seq;  // rows of the RoPE tables
  L("embed_gather", (m->nq_x ? 9.25 : 8.0) * H, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, e);
}

// The decode GEMV of one linear slot of layer li (LLMRS_W_Q = the stacked
// Q|K|V rows, LLMRS_W_O, LLMRS_W_GATE = gate|up, LLMRS_W_DOWN) with its fused
// prologue and epilogue, on the decode activation buffers.
// `probe_xq` / `probe_xd` (test probes, may be null) receive the Q8_0
// operand the GEMV's prologue built.
void enqueue_linear(llmrs_model* m, Launcher& L, int li, int slot, int8_t* probe_xq = nullptr,
                    float* probe_xd = nullptr, unsigned long long* stamps = nullptr) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_heads, F = c.ffn;
  const int cus = ctx().num_cus;
  LayerBufs& Lb = m->layers[li];
  GemvArgs g{};
  const char* kind = nullptr;
  double bytes = 0.0;
  switch (slot) {
    case LLMRS_W_Q:  // Q|K|V, RMSNorm prologue (layer.rs:378)
      g.wq = Lb.qkv.codes;
      g.ws = Lb.qkv.scales;
      g.n = Lb.qkv.n;
      g.k = H;
      g.eps = c.rms_eps;
      g.y = m->qkv;
      if (m->nq_x) {
        g.xq = m->x_q;
        g.xd = m->x_d;
        g.xss = m->x_ss;
        kind = "nq_store";
        bytes = linear_weight_bytes(m, Lb.qkv) + 1.125 * H + 4.0 * g.n;
      } else {
        g.x = m->x;
        g.norm_w = Lb.norm[0];
        kind = "norm_store";
        bytes = linear_weight_bytes(m, Lb.qkv) + 8.0 * H + 4.0 * g.n;
      }
      break;
    case LLMRS_W_O:  // O projection + residual (layer.rs:386)
      g.wq = Lb.o.codes;
      g.ws = Lb.o.scales;
      g.n = H;
      g.k = nq * hd;
      g.xq = m->ctx_q;
      g.xd = m->ctx_d;
      g.y = m->h;
      g.res = m->x;
      kind = "q8_resid";
      bytes = linear_weight_bytes(m, Lb.o) + 1.125 * g.k + 8.0 * H;
      if (m->nq_h) {  // and the post-attention RMSNorm's operand (layer.rs:393)
        g.norm_next = Lb.norm[1];
        g.yq = m->h_q;
        g.yd = m->h_d;
        g.yss = m->h_ss;
        kind = "q8_nq";
        bytes += 5.25 * H;
      }
      break;
    case LLMRS_W_GATE:  // gate|up + SiLU (layer.rs:40-89, 400)
      g.wq = Lb.gu.codes;
      g.ws = Lb.gu.scales;
      g.n = 2 * F;
      g.k = H;
      g.eps = c.rms_eps;
      g.y = m->mf;
      g.yq = m->m_q;
      g.yd = m->m_d;
      if (m->nq_h) {
        g.xq = m->h_q;
        g.xd = m->h_d;
        g.xss = m->h_ss;
        kind = "nq_silu";
        bytes = linear_weight_bytes(m, Lb.gu) + 1.125 * H + 5.125 * F;
      } else {
        g.x = m->h;
        g.norm_w = Lb.norm[1];
        kind = "norm_silu";
        bytes = linear_weight_bytes(m, Lb.gu) + 8.0 * H + 5.125 * F;
      }
      break;
    case LLMRS_W_DOWN:  // down projection + residual (layer.rs:403)
      g.wq = Lb.down.codes;
      g.ws = Lb.down.scales;
      g.n = H;
      g.k = F;
      g.xq = m->m_q;
      g.xd = m->m_d;
      g.y = m->x;
      g.res = m->h;
      kind = "q8_resid";
      bytes = linear_weight_bytes(m, Lb.down) + 1.125 * F + 8.0 * H;
      if (m->nq_x) {  // and the next RMSNorm's operand: next layer's input norm or the final norm
        g.norm_next = li + 1 < c.n_layers ? m->layers[li + 1].norm[0] : m->final_norm;
        g.yq = m->x_q;
        g.yd = m->x_d;
        g.yss = m->x_ss;
        kind = "q8_nq";
        bytes += 5.25 * H;
      }
      break;
    default:
      fail(LLMRS_E_INVALID, "enqueue_linear: slot must be Q, O, GATE or DOWN");
  }
  g.probe_xq = probe_xq;
  g.probe_xd = probe_xd;
  g.ts = stamps;
  const GemvPlan p = gemv_plan(m->wt, kind, g.n, g.k, cus);
  L(p.name, bytes, dim3(p.grid), dim3(p.threads), p.lds, g);
}

// Workgroups of the decode GEMV of a linear slot (for stamp buffers).
unsigned linear_grid(llmrs_model* m, int slot) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden, F = c.ffn, qd = c.n_heads * c.head_dim, cus = ctx().num_cus;
  switch (slot) {
    case LLMRS_W_Q: return gemv_plan(m->wt, m->nq_x ? "nq_store" : "norm_store", m->qkv_rows, H, cus).grid;
    case LLMRS_W_O: return gemv_plan(m->wt, m->nq_h ? "q8_nq" : "q8_resid", H, qd, cus).grid;
    case LLMRS_W_GATE: return gemv_plan(m->wt, m->nq_h ? "nq_silu" : "norm_silu", 2 * F, H, cus).grid;
    case LLMRS_W_DOWN: return gemv_plan(m->wt, m->nq_x ? "q8_nq" : "q8_resid", H, F, cus).grid;
  }
  fail(LLMRS_E_INVALID, "slot must be Q, O, GATE or DOWN");
}

// Decode attention of layer li at the device position: RoPE of q and the new
// k, K/V append, attention over the cache, ctx as f32 and Q8_0.
void enqueue_attention(llmrs_model* m, Launcher& L, int li, unsigned long long* stamps = nullptr) {
  const llmrs_model_config& c = m->c;
  const int hd = c.head_dim, nkv = c.n_kv_heads;
  LayerBufs& Lb = m->layers[li];
  AttnArgs a{};
  a.qkv = m->qkv;
  a.pos_ptr = m->pos;
  a.kc = (uint8_t*)Lb.kc;
  a.vc = (uint8_t*)Lb.vc;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.rope_now = m->rope_now;
  a.part_o = m->part_o;
  a.part_ml = m->part_ml;
  a.counters = m->counters + (size_t)li * nkv * llmrs::kTicketStride;
  a.ctx = m->ctxv;
  a.ctx_q = m->ctx_q;
  a.ctx_d = m->ctx_d;
  a.max_seq = kv_rows(m);
  a.nq = c.n_heads;
  a.nkv = nkv;
  a.nsplit = m->nsplit;
  a.scale = 1.0f / std::sqrt((float)hd);  // layer.rs:258
  a.ts = stamps;
  const double kvb = 2.0 * nkv * (double)(m->host_pos + 1) * hd * kv_elem_bytes(m);
  L(attn_kernel(m), kvb, dim3((unsigned)m->nsplit, (unsigned)nkv), dim3(attn_threads(m)), 0, a);
}

void enqueue_exact_step(llmrs_model* m, Launcher& L, bool write_logits, float* trace_dev);

void enqueue_step(llmrs_model* m, Launcher& L, bool write_logits, float* trace_dev) {
  if (m->exact) {
    enqueue_exact_step(m, L, write_logits, trace_dev);
    return;
  }
  const llmrs_model_config& c = m->c;
  const int H = c.hidden;

  enqueue_embed(m, L, nullptr, m->layers[0].norm[0]);

  for (int li = 0; li < c.n_layers; ++li) {
    if (trace_dev)
      LLMRS_HIP(hipMemcpyAsync(trace_dev + (size_t)li * H, m->x, H * sizeof(float),
                               hipMemcpyDeviceToDevice, L.s));
    enqueue_linear(m, L, li, LLMRS_W_Q);
    enqueue_attention(m, L, li);
    enqueue_linear(m, L, li, LLMRS_W_O);
    enqueue_linear(m, L, li, LLMRS_W_GATE);
    enqueue_linear(m, L, li, LLMRS_W_DOWN);
  }
  if (trace_dev)
    LLMRS_HIP(hipMemcpyAsync(trace_dev + (size_t)c.n_layers * H, m->x, H * sizeof(float),
                             hipMemcpyDeviceToDevice, L.s));
  enqueue_head(m, L, write_logits);
}

// Final RMSNorm + lm_head GEMV of the row in m->x, then the greedy step
// bookkeeping at the device position (model.rs:39-47, main.rs:185-190).
void enqueue_head(llmrs_model* m, Launcher& L, bool write_logits, int8_t* probe_xq, float* probe_xd) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden;
  const int cus = ctx().num_cus;
  {  // lm_head + argmax
    GemvArgs g{};
    g.wq = m->lm_head.codes;
    g.ws = m->lm_head.scales;
    g.n = c.vocab;
    g.k = H;
    g.eps = c.rms_eps;
    if (m->nq_x) {
      g.xq = m->x_q;
      g.xd = m->x_d;
      g.xss = m->x_ss;
    } else {
      g.x = m->x;
      g.norm_w = m->final_norm;
    }
    g.y = write_logits || m->sampling ? m->logits : nullptr;
    g.part_val = m->part_val;
    g.part_idx = m->part_idx;
    g.probe_xq = probe_xq;
    g.probe_xd = probe_xd;
    const GemvPlan p = gemv_plan(m->wt, m->nq_x ? "nq_argmax" : "norm_argmax", g.n, g.k, cus);
    LLMRS_REQUIRE((int)p.grid == m->lm_grid, LLMRS_E_INVALID, "lm_head grid changed since model creation");
    L(p.name, linear_weight_bytes(m, m->lm_head) + (m->nq_x ? 1.125 : 8.0) * H, dim3(p.grid), dim3(256), p.lds, g);
  }
  if (m->sampling) {
    SampleArgs a = sample_args(m->samp, c.vocab);
    a.logits = m->logits;
    a.probs = m->probs;
    a.st = m->samp_state;
    a.pos = m->pos;
    a.n_prompt = m->n_prompt;
    a.tokens = m->tokens;
    a.gen = m->gen;
    a.cap = m->cap;
    a.eos = m->eos;
    a.stopped = m->stopped;
    enqueue_sample(L, a);
    return;
  }
  ArgmaxFinalArgs f{m->part_val, m->part_idx, m->lm_grid, m->pos, m->n_prompt, m->tokens, m->gen, m->cap};
  L("argmax_final", 8.0 * m->lm_grid, dim3(1), dim3(256), 0, f);
}

// ---- the decode step in the reference's operation order (exact.hip) --------
// Eight launches per layer: RMSNorm + Q8_0, Q|K|V GEMV, attention, O GEMV +
// residual, RMSNorm + Q8_0, gate|up GEMV, SwiGLU + Q8_0, down GEMV +
// residual; then the final RMSNorm, the lm_head GEMV with argmax partials and
// argmax_final (or the sampler).  Every sum runs in the reference's order,
// so each value equals the reference CPU path's (x86-64 build) bit for bit.

// Cache positions the exact attention keeps in LDS (scores, then
// probabilities): 64 KB.
constexpr int kExactMaxRows = 16384;

// Workgroups of an exact GEMV: one per 8-row tile, at most four per CU (as
// many as are resident at once; they loop over the tiles beyond).
int exact_gemv_cap() { return 4 * ctx().num_cus; }
unsigned exact_gemv_grid(int n) { return (unsigned)std::max(1, std::min((n + 7) / 8, exact_gemv_cap())); }

// RMSNorm + Q8_0 of `rows` rows of hidden floats (one workgroup each; the
// codes in the operand order `layout`).
void exact_norm(llmrs_model* m, Launcher& L, const float* x, const float* w, int8_t* xq, float* xd,
                float* y = nullptr, int rows = 1, int layout = llmrs::kActNatural) {
  const int H = m->c.hidden;
  ExactNormArgs a{x, w, xq, xd, y, H, m->c.rms_eps, layout};
  L("exact_norm_q8", 9.125 * H * rows, dim3((unsigned)rows), dim3(1024), (size_t)H * 4, a);
}

void exact_linear(llmrs_model* m, Launcher& L, const DevLinear& W, const char* epi, const int8_t* xq,
                  const float* xd, float* y, const float* res) {
  ExactGemvArgs a{W.codes, W.scales, xq, xd, y, res, nullptr, nullptr, W.n, W.k, nullptr, nullptr};
  const unsigned grid = exact_gemv_grid(W.n);
  L(std::string("exact_gemv_") + wt_tag(m->wt) + "_" + epi,
    linear_weight_bytes(m, W) + 1.125 * W.k + (res ? 8.0 : 4.0) * W.n, dim3(grid), dim3(256), 0, a);
}

// The gate|up GEMV with the SwiGLU product and its Q8_0 (layer.rs:40,
// 75-79): one workgroup per 64-row group (32 gate + 32 up rows), at most two
// per CU (as many as are resident at once; they loop over the groups beyond).
void exact_gate_up(llmrs_model* m, Launcher& L, const DevLinear& W) {
  const int F = m->c.ffn;
  ExactGemvArgs a{W.codes, W.scales, m->h_q, m->h_d, m->mf, nullptr, nullptr, nullptr, W.n, W.k, m->m_q, m->m_d};
  const unsigned grid = (unsigned)std::max(1, std::min(W.n / 64, 2 * ctx().num_cus));
  L(std::string("exact_gemv_") + wt_tag(m->wt) + "_silu", linear_weight_bytes(m, W) + 1.125 * W.k + 5.125 * F,
    dim3(grid), dim3(256), 0, a);
}

void exact_attention(llmrs_model* m, Launcher& L, int li) {
  const llmrs_model_config& c = m->c;
  const int hd = c.head_dim;
  LayerBufs& Lb = m->layers[li];
  ExactAttnArgs a{m->qkv, m->pos, Lb.kc, Lb.vc, m->rope_cos, m->rope_sin, m->ctxv, m->ctx_q, m->ctx_d,
                  kv_rows(m), c.n_heads, c.n_kv_heads, 1.0f / std::sqrt((float)hd)};  // layer.rs:258
  const std::string name = "exact_attn_hd" + std::to_string(hd) + (c.kv_dtype == LLMRS_F16 ? "_f16" : "_f32");
  const double kvb = 2.0 * c.n_kv_heads * (double)(m->host_pos + 1) * hd * kv_elem_bytes(m);
  L(name, kvb, dim3((unsigned)c.n_heads), dim3(256), (size_t)kv_rows(m) * 4, a);
}

// `after(stage)` (may be empty) runs after stage s of the layer has been
// enqueued: 0 norm, 1 Q|K|V, 2 attention, 3 O, 4 norm, 5 gate|up, 6 SwiGLU,
// 7 down.
void enqueue_exact_layer(llmrs_model* m, Launcher& L, int li, const std::function<void(int)>& after = {}) {
  LayerBufs& Lb = m->layers[li];
  auto done = [&](int s) {
    if (after) after(s);
  };
  exact_norm(m, L, m->x, Lb.norm[0], m->x_q, m->x_d);                      // layer.rs:378
  done(0);
  exact_linear(m, L, Lb.qkv, "store", m->x_q, m->x_d, m->qkv, nullptr);    // layer.rs:177-179
  done(1);
  exact_attention(m, L, li);                                               // layer.rs:216-326
  done(2);
  exact_linear(m, L, Lb.o, "resid", m->ctx_q, m->ctx_d, m->h, m->x);      // layer.rs:332,386
  done(3);
  exact_norm(m, L, m->h, Lb.norm[1], m->h_q, m->h_d);                      // layer.rs:393
  done(4);
  exact_gate_up(m, L, Lb.gu);                                              // layer.rs:40,75-79
  done(5);
  done(6);
  exact_linear(m, L, Lb.down, "resid", m->m_q, m->m_d, m->x, m->h);       // layer.rs:93-96,403
  done(7);
}

// Final RMSNorm, lm_head with argmax partials, then argmax_final or the
// sampler (model.rs:39-47, main.rs:185-190).
void enqueue_exact_head(llmrs_model* m, Launcher& L, bool write_logits) {
  const llmrs_model_config& c = m->c;
  exact_norm(m, L, m->x, m->final_norm, m->x_q, m->x_d);
  const unsigned grid = exact_gemv_grid(c.vocab);
  ExactGemvArgs a{m->lm_head.codes, m->lm_head.scales, m->x_q, m->x_d,
                  write_logits || m->sampling ? m->logits : nullptr, nullptr, m->ex_part_val, m->ex_part_idx,
                  c.vocab, c.hidden, nullptr, nullptr};
  L(std::string("exact_gemv_") + wt_tag(m->wt) + "_argmax", linear_weight_bytes(m, m->lm_head) + 1.125 * c.hidden,
    dim3(grid), dim3(256), 0, a);
  if (m->sampling) {
    SampleArgs s = sample_args(m->samp, c.vocab);
    s.logits = m->logits;
    s.probs = m->probs;
    s.st = m->samp_state;
    s.pos = m->pos;
    s.n_prompt = m->n_prompt;
    s.tokens = m->tokens;
    s.gen = m->gen;
    s.cap = m->cap;
    s.eos = m->eos;
    s.stopped = m->stopped;
    enqueue_sample(L, s);
    return;
  }
  ArgmaxFinalArgs f{m->ex_part_val, m->ex_part_idx, (int)grid, m->pos, m->n_prompt, m->tokens, m->gen, m->cap};
  L("argmax_final", 8.0 * grid, dim3(1), dim3(256), 0, f);
}

void enqueue_exact_step(llmrs_model* m, Launcher& L, bool write_logits, float* trace_dev) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden;
  EmbedArgs e{};  // x = E[token at the device position] (main.rs:159-167)
  e.table = m->embed;
  e.tokens = m->tokens;
  e.pos_ptr = m->pos;
  e.x = m->x;
  e.err = m->err;
  e.hidden = H;
  e.vocab = c.vocab;
  L("embed_gather", 8.0 * H, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, e);
  for (int li = 0; li < c.n_layers; ++li) {
    if (trace_dev)
      LLMRS_HIP(hipMemcpyAsync(trace_dev + (size_t)li * H, m->x, H * sizeof(float), hipMemcpyDeviceToDevice, L.s));
    enqueue_exact_layer(m, L, li);
  }
  if (trace_dev)
    LLMRS_HIP(hipMemcpyAsync(trace_dev + (size_t)c.n_layers * H, m->x, H * sizeof(float),
                             hipMemcpyDeviceToDevice, L.s));
  enqueue_exact_head(m, L, write_logits);
}

// Switches a model between the fast and the reference-order step; the first
// switch to the latter allocates its lm_head partials and resolves its kernels.
void set_exact(llmrs_model* m, bool on) {
  if (on) {
    const llmrs_model_config& c = m->c;
    LLMRS_REQUIRE(kv_rows(m) <= kExactMaxRows, LLMRS_E_INVALID,
                  "the reference-order step supports max_seq up to " + std::to_string(kExactMaxRows));
    if (!m->ex_part_val) {
      m->ex_part_val = m->dalloc<float>((size_t)exact_gemv_cap());
      m->ex_part_idx = m->dalloc<int>((size_t)exact_gemv_cap());
    }
    for (const char* epi : {"store", "resid", "argmax", "silu"})
      (void)kernel(std::string("exact_gemv_") + wt_tag(m->wt) + "_" + epi);
    (void)kernel("exact_norm_q8");
    (void)kernel("exact_attn_hd" + std::to_string(c.head_dim) + (c.kv_dtype == LLMRS_F16 ? "_f16" : "_f32"));
    (void)kernel("exact_attn_prefill_hd" + std::to_string(c.head_dim) + (c.kv_dtype == LLMRS_F16 ? "_f16" : "_f32"));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  }
  if (m->exact != on) {  // the captured step changes
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->graph_failed = false;
  }
  m->exact = on;
}

// Batched prompt processing (prefill).  The reference runs the whole prompt
// as one forward of M rows (main.rs:134-138,179; model.rs:17-49): every
// linear layer quantises each activation row to Q8_0 and runs the block loop
// per output (cpu.rs:90-110), which the exact int8 MFMA GEMM reproduces bit
// for bit; attention is causal over the cache (layer.rs:248-326).  Prompts
// longer than pf_cap rows run as consecutive chunks at increasing start
// positions, which gives the same values: each row's projections depend only
// on that row, and its attention reads the K/V already in the cache.
void ensure_prefill(llmrs_model* m) {
  if (m->pf_cap) return;
  const llmrs_model_config& c = m->c;
  const int cap = std::max(1, std::min(c.max_seq, env_int("LLMRS_PREFILL_CHUNK", 2048)));
  const size_t M = (size_t)cap, H = c.hidden, F = c.ffn, qd = (size_t)c.n_heads * c.head_dim;
  const size_t kmax = std::max(H, std::max(F, qd));
  m->pf_x = m->dalloc<float>(M * H);
  m->pf_h = m->dalloc<float>(M * H);
  m->pf_qkv = m->dalloc<float>(M * m->qkv_rows);
  m->pf_q = m->dalloc<float>(M * qd);
  m->pf_aq = m->dalloc<int8_t>(M * kmax);
  m->pf_ad = m->dalloc<float>(M * kmax / 32);
  m->pf_ctx_q = m->dalloc<int8_t>(M * qd);
  m->pf_ctx_d = m->dalloc<float>(M * qd / 32);
  m->pf_m_q = m->dalloc<int8_t>(M * F);
  m->pf_m_d = m->dalloc<float>(M * F / 32);
  m->pf_start = m->dalloc<int>(1);
  LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  m->pf_cap = cap;
}

std::string gemm_kernel(const llmrs_model* m, const char* epi) {
  return std::string("gemm_") + wt_tag(m->wt) + "_" + epi;
}

// Whether M prefill rows run their linear layers on the skinny GEMM's exact
// launches (sgemm.hip, up to 64 rows; the activation codes then in its
// operand order) rather than the 128 x 128-tile GEMM, which a short prompt
// leaves mostly idle; both are bit-identical to the reference's block loop.
// LLMRS_PREFILL_SKINNY=0 keeps every prefill on the tile GEMM.
bool prefill_skinny(const llmrs_model* m, int M) {
  const llmrs_model_config& c = m->c;
  return M <= 64 && c.hidden % 128 == 0 && c.ffn % 128 == 0 && (c.n_heads * c.head_dim) % 128 == 0 &&
         env_int("LLMRS_PREFILL_SKINNY", 1) != 0;
}

// The skinny GEMM kernel of an epilogue for M rows (store, resid, silu);
// exact: each output's blocks in one wave, in order (prompt prefill).
std::string sgemm_kernel(const llmrs_model* m, const char* epi, int M, bool exact) {
  return std::string("sgemm_") + wt_tag(m->wt) + "_" + epi + "_t" + (M <= 16 ? "1" : M <= 32 ? "2" : "4") +
         (exact ? "_exact" : "");
}

// Launch shape of a skinny GEMM (sgemm.hip): SwiGLU 64 rows per 256-thread
// workgroup; exact store / residual 16 rows per one-wave workgroup; else
// residual 16 and store 32 rows per 256-thread workgroup.
std::pair<dim3, dim3> sgemm_shape(const char* epi, int N, bool exact) {
  const std::string e(epi);
  const int rows = e == "silu" ? 64 : exact || e == "resid" ? 16 : 32;
  const unsigned threads = exact && e != "silu" ? 64 : 256;
  return {dim3((unsigned)((N + rows - 1) / rows)), dim3(threads)};
}

dim3 gemm_grid(int M, int N) { return dim3((unsigned)((N + 127) / 128), (unsigned)((M + 127) / 128)); }

// Device buffers a test probe adds to one prefill layer: ctx and the SwiGLU
// product m as f32 (the production path keeps only their Q8_0 codes).
struct PrefillProbe {
  float* ctx = nullptr;  // [M][nq*hd]
  float* mf = nullptr;   // [M][ffn]
  std::function<void(int)> after;  // called after stage s (0..6) has been enqueued
};

// Layer li of one chunk of M rows at positions [start, start+M), in place on
// pf_x (the residual stream).  Stages: 0 RMSNorm+Q8, 1 Q|K|V GEMM, 2 RoPE +
// K/V append, 3 causal attention, 4 O GEMM + residual, 5 RMSNorm+Q8,
// 6 gate|up GEMM + SwiGLU + Q8, 7 down GEMM + residual.  The recorded figure
// per launch is its FLOPs for the GEMMs and attention, bytes for the rest.
// exact: the RMSNorms and the attention on the reference-order kernels
// (exact.hip; the GEMMs, the RoPE / append and the SwiGLU epilogue already
// compute the reference's values), so every row equals the reference's.
void enqueue_prefill_layer(llmrs_model* m, Launcher& L, int li, size_t start, int M,
                           const PrefillProbe* probe = nullptr, void* kc = nullptr, void* vc = nullptr,
                           bool exact = false) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, F = c.ffn;
  const int QR = m->qkv_rows;
  const bool kv16 = c.kv_dtype == LLMRS_F16;
  const dim3 blk(256);
  auto flops = [](double a, double b, double k) { return 2.0 * a * b * k; };
  auto after = [&](int stage) {
    if (probe && probe->after) probe->after(stage);
  };
  const size_t glds = gemm_lds_bytes();
  const float scale = 1.0f / std::sqrt((float)hd);  // layer.rs:258
  // f16 caches use the matrix-core kernel (LLMRS_PREFILL_ATTN=valu selects the
  // vector kernel, which also serves f32 caches)
  const char* pa = std::getenv("LLMRS_PREFILL_ATTN");
  const bool mfma_attn = kv16 && !(pa && std::string(pa) == "valu");
  const std::string attn = mfma_attn ? "attn_prefill_mfma_hd" + std::to_string(hd)
                                     : "attn_prefill_hd" + std::to_string(hd) + (kv16 ? "_f16" : "_f32");
  // causal score and P.V products over the chunk
  const double attn_flops = 4.0 * nq * hd * ((double)M * start + (double)M * (M + 1) / 2.0);
  LayerBufs& Lb = m->layers[li];
  if (!kc) {  // the model's own cache (a batch slot's otherwise)
    kc = Lb.kc;
    vc = Lb.vc;
  }
  const bool skinny = prefill_skinny(m, M);
  const int layout = skinny ? llmrs::kActMfma : llmrs::kActNatural;
  // One linear layer over the M rows on the tile GEMM or the skinny GEMM.
  auto linear = [&](const char* epi, const DevLinear& W, const int8_t* xq, const float* xd, float* y,
                    const float* res, int8_t* yq, float* yd, int ldy) {
    const double work = flops(M, W.n, W.k);
    if (skinny) {
      SgemmArgs g{xq, xd, W.codes, W.scales, y, res, yq, yd, M, W.n, W.k, ldy, layout};
      const auto sh = sgemm_shape(epi, W.n, true);
      L(sgemm_kernel(m, epi, M, true), work, sh.first, sh.second, 0, g);
    } else {
      PrefillGemmArgs g{xq, xd, W.codes, W.scales, y, res, yq, yd, M, W.n, W.k, ldy, gemm_group_m()};
      L(gemm_kernel(m, epi), work, gemm_grid(M, W.n), blk, glds, g);
    }
  };
  if (exact) {  // RMSNorm + Q8_0 of each row (layer.rs:378; cpu.rs:90-93)
    exact_norm(m, L, m->pf_x, Lb.norm[0], m->pf_aq, m->pf_ad, nullptr, M, layout);
  } else {
    PrefillRowArgs r{m->pf_x, Lb.norm[0], m->pf_aq, m->pf_ad, M, H, c.rms_eps, layout};
    L("prefill_rows_q8", 5.0 * H * M, dim3((unsigned)M), blk, gemv_act_lds_host(H), r);
  }
  after(0);
  linear("store", Lb.qkv, m->pf_aq, m->pf_ad, m->pf_qkv, nullptr, nullptr, nullptr, QR);  // Q|K|V
  after(1);
  {  // RoPE + K/V append
    PrefillRopeArgs r{m->pf_qkv, m->pf_q, kc, vc, m->rope_cos, m->rope_sin, M, nq, nkv, hd,
                      kv_rows(m), (int)start, QR, kv16 ? 1 : 0};
    const long total = (long)M * (nq + 2 * nkv) * (hd / 2);
    const unsigned grid = (unsigned)std::min<long>((total + 255) / 256, 8192);
    L("prefill_rope_kv", 4.0 * QR * M * 2, dim3(grid), blk, 0, r);
  }
  after(2);
  {  // causal attention
    PrefillAttnArgs a{m->pf_q, kc, vc, probe ? probe->ctx : nullptr, m->pf_ctx_q, m->pf_ctx_d, M, nq,
                      nkv, kv_rows(m), (int)start, scale, layout};
    if (exact)  // one workgroup per (query head, row); the scores of up to start + M positions in LDS
      L("exact_attn_prefill_hd" + std::to_string(hd) + (kv16 ? "_f16" : "_f32"), attn_flops,
        dim3((unsigned)nq, (unsigned)M), blk, (start + M) * 4, a);
    else if (mfma_attn)
      L(attn, attn_flops, dim3((unsigned)((M + 31) / 32), (unsigned)nkv), dim3(512), 0, a);
    else
      L(attn, attn_flops, dim3((unsigned)((M + 31) / 32), (unsigned)nq), blk, 0, a);
  }
  after(3);
  linear("resid", Lb.o, m->pf_ctx_q, m->pf_ctx_d, m->pf_h, m->pf_x, nullptr, nullptr, H);  // O + residual
  after(4);
  if (exact) {  // post-attention RMSNorm + Q8_0
    exact_norm(m, L, m->pf_h, Lb.norm[1], m->pf_aq, m->pf_ad, nullptr, M, layout);
  } else {
    PrefillRowArgs r{m->pf_h, Lb.norm[1], m->pf_aq, m->pf_ad, M, H, c.rms_eps, layout};
    L("prefill_rows_q8", 5.0 * H * M, dim3((unsigned)M), blk, gemv_act_lds_host(H), r);
  }
  after(5);
  // gate|up + SiLU + Q8_0 of m (layer.rs:40-89)
  linear("silu", Lb.gu, m->pf_aq, m->pf_ad, probe ? probe->mf : nullptr, nullptr, m->pf_m_q, m->pf_m_d, F);
  after(6);
  linear("resid", Lb.down, m->pf_m_q, m->pf_m_d, m->pf_x, m->pf_h, nullptr, nullptr, H);  // down + residual
  after(7);
}

// One chunk of M <= pf_cap rows at positions [start, start+M): embeddings,
// every layer, and (head) the lm_head of the last row with the greedy step
// at the device position.  trace_dev, when set, is
// [M][n_layers+1][hidden].
void enqueue_prefill(llmrs_model* m, Launcher& L, size_t start, int M, bool head, bool write_logits,
                     float* trace_dev, void* const* kcs = nullptr, void* const* vcs = nullptr, bool exact = false) {
  const llmrs_model_config& c = m->c;
  const int H = c.hidden;
  auto trace = [&](int li) {
    if (trace_dev)
      LLMRS_HIP(hipMemcpy2DAsync(trace_dev + (size_t)li * H, (size_t)(c.n_layers + 1) * H * sizeof(float),
                                 m->pf_x, H * sizeof(float), H * sizeof(float), M,
                                 hipMemcpyDeviceToDevice, L.s));
  };
  EmbedArgs e{};  // no norm operand, no RoPE row: a chunk of rows from *pf_start
  e.table = m->embed;
  e.tokens = m->tokens;
  e.pos_ptr = m->pf_start;
  e.x = m->pf_x;
  e.err = m->err;
  e.hidden = H;
  e.vocab = c.vocab;
  L("embed_gather", 8.0 * H * M, dim3((unsigned)((H + 255) / 256), (unsigned)M), dim3(256), 0, e);
  for (int li = 0; li < c.n_layers; ++li) {
    trace(li);
    enqueue_prefill_layer(m, L, li, start, M, nullptr, kcs ? kcs[li] : nullptr, vcs ? vcs[li] : nullptr, exact);
  }
  trace(c.n_layers);
  if (head && exact) {  // the last row on the reference-order head
    LLMRS_HIP(hipMemcpyAsync(m->x, m->pf_x + (size_t)(M - 1) * H, H * sizeof(float), hipMemcpyDeviceToDevice,
                             L.s));
    enqueue_exact_head(m, L, write_logits);
  } else if (head) {
    if (m->nq_x) {
      enqueue_embed(m, L, m->pf_x + (size_t)(M - 1) * H, m->final_norm);
    } else {
      LLMRS_HIP(hipMemcpyAsync(m->x, m->pf_x + (size_t)(M - 1) * H, H * sizeof(float),
                               hipMemcpyDeviceToDevice, L.s));
    }
    enqueue_head(m, L, write_logits);
  }
}

bool prefill_enabled() { return env_int("LLMRS_PREFILL", 1) != 0; }

void set_state(llmrs_model* m, size_t pos, int n_prompt);

// Runs rows [start, start+n) through the prefill kernels in chunks; the last
// chunk ends with the lm_head and greedy step, leaving the device position
// at start+n.  trace (host, may be null) is [n][n_layers+1][hidden].
void run_prefill(llmrs_model* m, size_t start, size_t n, int n_prompt, bool write_logits, float* trace,
                 void* const* kcs = nullptr, void* const* vcs = nullptr) {
  ensure_prefill(m);
  const llmrs_model_config& c = m->c;
  const size_t rowf = (size_t)(c.n_layers + 1) * c.hidden;
  const bool exact = m->exact && !kcs;  // a batch slot's prompt stays on the fast kernels
  float* tdev = nullptr;
  if (trace) {
    LLMRS_HIP(hipMalloc(&tdev, std::min<size_t>(n, m->pf_cap) * rowf * sizeof(float)));
  }
  try {
    for (size_t done = 0; done < n;) {
      const int M = (int)std::min<size_t>(m->pf_cap, n - done);
      const bool last = done + M == n;
      const int s0 = (int)(start + done);
      LLMRS_HIP(hipMemcpyAsync(m->pf_start, &s0, sizeof(int), hipMemcpyHostToDevice, ctx().stream));
      set_state(m, start + done + M - 1, n_prompt);  // synchronises the stream
      Launcher L{ctx().stream};
      enqueue_prefill(m, L, start + done, M, last, write_logits && last, tdev, kcs, vcs, exact);
      if (trace) {
        LLMRS_HIP(hipMemcpyAsync(trace + done * rowf, tdev, (size_t)M * rowf * sizeof(float),
                                 hipMemcpyDeviceToHost, ctx().stream));
        LLMRS_HIP(hipStreamSynchronize(ctx().stream));
      }
      done += M;
    }
  } catch (...) {
    if (tdev) (void)hipFree(tdev);
    throw;
  }
  if (tdev) {
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    (void)hipFree(tdev);
  }
}

void check_ready(const llmrs_model* m) {
  LLMRS_REQUIRE(m, LLMRS_E_INVALID, "null model");
  LLMRS_REQUIRE(m->embed_set && m->final_set && m->lm_set, LLMRS_E_INVALID,
                "model weights incomplete (embedding / final norm / lm_head)");
  for (size_t i = 0; i < m->layers.size(); ++i)
    LLMRS_REQUIRE(m->layers[i].set_mask == 0x37f, LLMRS_E_INVALID,
                  "layer " + std::to_string(i) + " weights incomplete");
}

void check_err(llmrs_model* m) {
  int e = 0;
  LLMRS_HIP(hipMemcpyAsync(&e, m->err, sizeof(int), hipMemcpyDeviceToHost, ctx().stream));
  LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  if (e) {
    int zero = 0;
    LLMRS_HIP(hipMemcpyAsync(m->err, &zero, sizeof(int), hipMemcpyHostToDevice, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    fail(LLMRS_E_RANGE, "token id out of range [0, vocab)");
  }
}

void set_state(llmrs_model* m, size_t pos, int n_prompt) {
  int v[3] = {(int)pos, n_prompt, 0};
  LLMRS_HIP(hipMemcpyAsync(m->pos, &v[0], sizeof(int), hipMemcpyHostToDevice, ctx().stream));
  LLMRS_HIP(hipMemcpyAsync(m->n_prompt, &v[1], sizeof(int), hipMemcpyHostToDevice, ctx().stream));
  LLMRS_HIP(hipMemcpyAsync(m->stopped, &v[2], sizeof(int), hipMemcpyHostToDevice, ctx().stream));
  LLMRS_HIP(hipStreamSynchronize(ctx().stream));
}

void upload_tokens(llmrs_model* m, size_t pos0, const int32_t* ids, size_t n) {
  for (size_t i = 0; i < n; ++i)
    LLMRS_REQUIRE(ids[i] >= 0 && ids[i] < m->c.vocab, LLMRS_E_RANGE,
                  "token id out of range at index " + std::to_string(i));
  LLMRS_HIP(hipMemcpyAsync(m->tokens + pos0, ids, n * sizeof(int32_t), hipMemcpyHostToDevice,
                           ctx().stream));
  LLMRS_HIP(hipStreamSynchronize(ctx().stream));
}

// One decode position through the captured graph (captured on first use).
void replay_step(llmrs_model* m) {
  hipStream_t s = ctx().stream;
  if (!m->exec && !m->graph_failed && env_int("LLMRS_GRAPH", 1)) {
    Launcher L{s};
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    bool ok = e == hipSuccess;
    if (ok) {
      try {
        enqueue_step(m, L, false, nullptr);
      } catch (const Error&) {
        ok = false;
      }
      hipGraph_t g = nullptr;
      e = hipStreamEndCapture(s, &g);
      ok = ok && e == hipSuccess && g;
      if (ok) {
        m->graph = g;
        ok = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0) == hipSuccess;
      } else if (g) {
        (void)hipGraphDestroy(g);
      }
    }
    if (!ok) {
      (void)hipGetLastError();
      m->graph_failed = true;
      m->exec = nullptr;
      std::fprintf(stderr, "llmrs_hip: HIP graph capture failed; using per-kernel launches\n");
    }
  }
  if (m->exec) {
    LLMRS_HIP(hipGraphLaunch(m->exec, s));
  } else {
    Launcher L{s};
    enqueue_step(m, L, false, nullptr);
  }
}

}  // namespace

extern "C" {

int llmrs_model_create(const llmrs_model_config* cfg, llmrs_model** out) {
  return guard([&] {
    LLMRS_REQUIRE(cfg && out, LLMRS_E_INVALID, "null argument");
    const llmrs_model_config& c = *cfg;
    LLMRS_REQUIRE(c.n_layers > 0 && c.hidden > 0 && c.n_heads > 0 && c.n_kv_heads > 0 &&
                      c.ffn > 0 && c.vocab > 0 && c.max_seq > 0,
                  LLMRS_E_INVALID, "model dimensions must be positive");
    LLMRS_REQUIRE(c.head_dim == 64 || c.head_dim == 128, LLMRS_E_INVALID, "head_dim must be 64 or 128");
    LLMRS_REQUIRE(c.n_heads % c.n_kv_heads == 0 && c.n_heads / c.n_kv_heads <= 8, LLMRS_E_INVALID,
                  "n_heads must be a multiple of n_kv_heads with at most 8 query heads per KV head");
    LLMRS_REQUIRE(c.hidden % 32 == 0 && c.ffn % 32 == 0 && (c.n_heads * c.head_dim) % 32 == 0,
                  LLMRS_E_INVALID, "hidden, ffn and n_heads*head_dim must be multiples of 32");
    LLMRS_REQUIRE(c.hidden <= 32768 && c.ffn <= 32768 && c.n_heads * c.head_dim <= 32768,
                  LLMRS_E_INVALID, "GEMV input length is limited to 32768");
    LLMRS_REQUIRE(c.kv_dtype == LLMRS_F32 || c.kv_dtype == LLMRS_F16, LLMRS_E_INVALID, "kv_dtype");
    // the attention kernels address one layer's K (or V) cache with 32-bit byte offsets
    LLMRS_REQUIRE((double)c.n_kv_heads * llmrs::kv_rows(c.max_seq) * c.head_dim *
                          (c.kv_dtype == LLMRS_F16 ? 2 : 4) <
                      2147483648.0,
                  LLMRS_E_INVALID, "one layer's K cache must stay below 2 GiB (n_kv_heads*max_seq*head_dim)");
    std::unique_ptr<llmrs_model> m(new llmrs_model());
    m->c = c;
    switch (c.weight_dtype) {
      case LLMRS_Q4: m->wt = WT_Q4F; break;
      case LLMRS_Q4_0: m->wt = WT_Q4H; break;
      case LLMRS_Q8_0: m->wt = WT_Q8H; break;
      default: fail(LLMRS_E_DTYPE, "weight_dtype must be LLMRS_Q4, LLMRS_Q4_0 or LLMRS_Q8_0");
    }
    Context& cx = ctx();
    const int H = c.hidden, hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, F = c.ffn;
    m->qkv_rows = (nq + 2 * nkv) * hd;
    m->cap = c.max_seq + 1;
    // Attention splits over the tiles of max_seq.  f16 caches (matrix-core
    // kernel; attn_waves = its tile waves per workgroup): one tile per
    // workgroup up to two workgroups per CU (and the combine's 64 splits),
    // beyond that eight tile waves per workgroup and up to one workgroup per
    // CU.  f32 caches (vector kernel): one tile per split up to two
    // workgroups per CU; longer contexts run 4 tile streams per workgroup
    // (one workgroup per CU) so the split combine stays short.
    const int tiles = llmrs::kv_rows(c.max_seq) / llmrs::kAttnTile;
    int splits;
    m->attn_streams = 1;
    if (c.kv_dtype == LLMRS_F16) {
      int ew = env_int("LLMRS_ATTN_WAVES", 0);  // 0 = by context length; 1, 4 or 8 = forced
      if (ew != 1 && ew != 4 && ew != 8)
        ew = tiles <= std::min(llmrs::kMfmaAttnMaxSplits, 2 * cx.num_cus / nkv) ? 1 : 8;
      m->attn_waves = ew;
      splits = ew == 1 ? tiles : std::min((tiles + ew - 1) / ew, std::max(1, cx.num_cus / nkv));
      splits = std::min(env_int("LLMRS_ATTN_SPLITS", splits), llmrs::kMfmaAttnMaxSplits);
    } else {
      splits = std::min(tiles, std::max(1, 2 * cx.num_cus / nkv));
      const int es = env_int("LLMRS_ATTN_STREAMS", 0);  // 0 = by context length, 1 or 4 = forced
      if (es == 4 || (es == 0 && tiles > splits)) {
        m->attn_streams = 4;
        splits = std::min((tiles + 3) / 4, std::max(1, cx.num_cus / nkv));
      }
      splits = env_int("LLMRS_ATTN_SPLITS", splits);
    }
    m->nsplit = std::max(1, splits);
    // the XCD-local split exchange needs a head's workgroups on one XCD
    m->attn_local = nkv % 8 == 0 && env_int("LLMRS_ATTN_LOCAL", 1) == 1 &&
                    xcd_dealt_mod8((unsigned)m->nsplit, (unsigned)nkv);
    const int psplit = m->nsplit;  // attention partials per query head
    m->lm_grid = (int)gemv_plan(m->wt, "nq_argmax", c.vocab, H, cx.num_cus).grid;
    m->layers.resize(c.n_layers);
    for (auto& L : m->layers) {
      m->alloc_linear(L.qkv, m->qkv_rows, H);
      m->alloc_linear(L.o, H, nq * hd);
      m->alloc_linear(L.gu, 2 * F, H);
      m->alloc_linear(L.down, H, F);
      L.norm[0] = m->dalloc<float>(H);
      L.norm[1] = m->dalloc<float>(H);
      L.kc = m->dalloc<uint8_t>(kv_layer_elems(m.get()) * kv_elem_bytes(m.get()));
      L.vc = m->dalloc<uint8_t>(kv_layer_elems(m.get()) * kv_elem_bytes(m.get()));
    }
    m->alloc_linear(m->lm_head, c.vocab, H);
    m->embed = m->dalloc<float>((size_t)c.vocab * H);
    m->final_norm = m->dalloc<float>(H);
    m->x = m->dalloc<float>(H);
    m->h = m->dalloc<float>(H);
    m->qkv = m->dalloc<float>(m->qkv_rows);
    m->ctxv = m->dalloc<float>((size_t)nq * hd);
    m->ctx_q = m->dalloc<int8_t>((size_t)nq * hd);
    m->ctx_d = m->dalloc<float>((size_t)nq * hd / 32);
    m->mf = m->dalloc<float>(F);
    // Producer-side RMSNorm operands when the producers' 32-row tiles fill
    // the GPU (measured on 256 CUs: hidden 8192, 70B shape, 103.9 -> 110.2
    // tok/s; hidden 4096, 8B shape, the 128-tile O and down GEMVs lose more
    // than the consumers' prologues gain, 724 -> 707).  LLMRS_NQ forces:
    // 0 neither, 1 both, 2 x's only (down's epilogue), 3 h's only (O's).
    const int nqe = env_int("LLMRS_NQ", -1);
    const bool nq_fit = H / 32 <= 256, nq_auto = H / 32 >= cx.num_cus;
    m->nq_x = nq_fit && (nqe >= 0 ? (nqe == 1 || nqe == 2) : nq_auto);
    m->nq_h = nq_fit && (nqe >= 0 ? (nqe == 1 || nqe == 3) : nq_auto);
    m->x_q = m->dalloc<int8_t>(H);
    m->h_q = m->dalloc<int8_t>(H);
    m->x_d = m->dalloc<float>(H / 32);
    m->h_d = m->dalloc<float>(H / 32);
    m->x_ss = m->dalloc<float>(H / 32);
    m->h_ss = m->dalloc<float>(H / 32);
    m->m_q = m->dalloc<int8_t>(F);
    m->m_d = m->dalloc<float>(F / 32);
    m->logits = m->dalloc<float>(c.vocab);
    m->part_o = m->dalloc<float>((size_t)nq * psplit * hd);
    m->part_ml = m->dalloc<float>((size_t)nq * llmrs::ml_stride(psplit) * 2);
    const size_t nparts = (size_t)m->lm_grid;
    m->part_val = m->dalloc<float>(nparts);
    m->part_idx = m->dalloc<int>(nparts);
    m->counters = m->dalloc<int>((size_t)c.n_layers * nkv * llmrs::kTicketStride);
    m->tokens = m->dalloc<int>(m->cap);
    m->gen = m->dalloc<int>(m->cap);
    m->pos = m->dalloc<int>(1);
    m->n_prompt = m->dalloc<int>(1);
    m->err = m->dalloc<int>(1);
    m->stopped = m->dalloc<int>(1);
    m->eos = m->dalloc<int>(LLMRS_MAX_EOS);
    m->trace = m->dalloc<float>((size_t)(c.n_layers + 1) * H);
    {  // RoPE tables for every position (cpu.rs:345-349)
      const size_t mid = hd / 2;
      std::vector<float> cs((size_t)c.max_seq * mid), sn((size_t)c.max_seq * mid);
      rope_table(0, c.max_seq, hd, c.rope_theta, cs.data(), sn.data());
      m->rope_cos = m->dalloc<float>(cs.size());
      m->rope_sin = m->dalloc<float>(sn.size());
      m->rope_now = m->dalloc<float>(hd);
      LLMRS_HIP(hipMemcpyAsync(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, cx.stream));
      LLMRS_HIP(hipMemcpyAsync(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, cx.stream));
    }
    LLMRS_HIP(hipStreamSynchronize(cx.stream));
    // Resolve every kernel of the step now, so graph capture never has to.
    const bool nx = m->nq_x, nh = m->nq_h;
    (void)kernel(gemv_plan(m->wt, nx ? "nq_store" : "norm_store", m->qkv_rows, H, cx.num_cus).name);
    (void)kernel(gemv_plan(m->wt, nh ? "q8_nq" : "q8_resid", H, nq * hd, cx.num_cus).name);
    (void)kernel(gemv_plan(m->wt, nh ? "nq_silu" : "norm_silu", 2 * F, H, cx.num_cus).name);
    (void)kernel(gemv_plan(m->wt, nx ? "q8_nq" : "q8_resid", H, F, cx.num_cus).name);
    (void)kernel(gemv_plan(m->wt, nx ? "nq_argmax" : "norm_argmax", c.vocab, H, cx.num_cus).name);
    (void)kernel("embed_gather");
    (void)kernel("argmax_final");
    for (const char* k : {"sample_prep", "sample_probs", "sample_refine", "sample_pick"})
      (void)kernel(k, dim3(llmrs::kSampleThreads));
    (void)kernel(attn_kernel(m.get()), dim3(attn_threads(m.get())));
    if (env_int("LLMRS_EXACT", 0) == 1) set_exact(m.get(), true);
    *out = m.release();
  });
}

int llmrs_model_free(llmrs_model* m) {
  return guard([&] {
    if (!m) return;
    LLMRS_REQUIRE(m->live_batches == 0, LLMRS_E_INVALID,
                  std::to_string(m->live_batches) + " batch(es) of this model are still alive: free them first");
    (void)hipStreamSynchronize(ctx().stream);
    delete m;
  });
}

int llmrs_model_set_embedding(llmrs_model* m, const float* table) {
  return guard([&] {
    LLMRS_REQUIRE(m && table, LLMRS_E_INVALID, "null argument");
    const size_t bytes = (size_t)m->c.vocab * m->c.hidden * sizeof(float);
    LLMRS_HIP(hipMemcpyAsync(m->embed, table, bytes, hipMemcpyHostToDevice, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    m->embed_set = true;
  });
}

int llmrs_model_set_norm(llmrs_model* m, int layer, int slot, const float* w) {
  return guard([&] {
    LLMRS_REQUIRE(m && w, LLMRS_E_INVALID, "null argument");
    float* dst;
    if (layer < 0 || slot == LLMRS_N_FINAL) {
      dst = m->final_norm;
      m->final_set = true;
    } else {
      LLMRS_REQUIRE(layer < m->c.n_layers && (slot == LLMRS_N_INPUT || slot == LLMRS_N_POST),
                    LLMRS_E_INVALID, "bad norm slot");
      dst = m->layers[layer].norm[slot];
      m->layers[layer].set_mask |= 1u << (8 + slot);
    }
    LLMRS_HIP(hipMemcpyAsync(dst, w, m->c.hidden * sizeof(float), hipMemcpyHostToDevice, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  });
}

}  // extern "C"

namespace {

// Target matrix, source shape and device-row placement of a linear slot
// (loader.rs:113-150,186-190; gate|up interleaved in tiles of 32 rows so one
// GEMV tile owns matching gate and up rows).
struct Placement {
  DevLinear* L;
  size_t rows, k;
  size_t row0;        // first device row
  bool interleave;    // gate/up: runs of 32 rows, device pitch 64 rows
};

Placement place(llmrs_model* m, int layer, int slot) {
  const llmrs_model_config& c = m->c;
  const size_t H = c.hidden, hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, F = c.ffn;
  if (slot == LLMRS_W_LM_HEAD || layer < 0) {
    LLMRS_REQUIRE(slot == LLMRS_W_LM_HEAD, LLMRS_E_INVALID, "layer -1 takes only LLMRS_W_LM_HEAD");
    return {&m->lm_head, (size_t)c.vocab, H, 0, false};
  }
  LLMRS_REQUIRE(layer < c.n_layers, LLMRS_E_INVALID, "layer out of range");
  LayerBufs& Lb = m->layers[layer];
  switch (slot) {
    case LLMRS_W_Q: return {&Lb.qkv, nq * hd, H, 0, false};
    case LLMRS_W_K: return {&Lb.qkv, nkv * hd, H, nq * hd, false};
    case LLMRS_W_V: return {&Lb.qkv, nkv * hd, H, nq * hd + nkv * hd, false};
    case LLMRS_W_O: return {&Lb.o, H, nq * hd, 0, false};
    case LLMRS_W_GATE: return {&Lb.gu, F, H, 0, true};
    case LLMRS_W_UP: return {&Lb.gu, F, H, 32, true};
    case LLMRS_W_DOWN: return {&Lb.down, H, F, 0, false};
  }
  fail(LLMRS_E_INVALID, "bad linear slot");
}

void put_rows(llmrs_model* m, const Placement& p, const std::vector<uint8_t>& codes,
              const std::vector<uint8_t>& scales) {
  const size_t nb = p.k / 32;
  const size_t cb = nb * block_code_bytes(m->wt), sb = nb * block_scale_bytes(m->wt);
  hipStream_t s = ctx().stream;
  uint8_t* dc = p.L->codes;
  uint8_t* ds = (uint8_t*)p.L->scales;
  if (!p.interleave) {
    LLMRS_HIP(hipMemcpyAsync(dc + p.row0 * cb, codes.data(), p.rows * cb, hipMemcpyHostToDevice, s));
    LLMRS_HIP(hipMemcpyAsync(ds + p.row0 * sb, scales.data(), p.rows * sb, hipMemcpyHostToDevice, s));
  } else {
    const size_t runs = p.rows / 32;
    LLMRS_HIP(hipMemcpy2DAsync(dc + p.row0 * cb, 64 * cb, codes.data(), 32 * cb, 32 * cb, runs,
                               hipMemcpyHostToDevice, s));
    LLMRS_HIP(hipMemcpy2DAsync(ds + p.row0 * sb, 64 * sb, scales.data(), 32 * sb, 32 * sb, runs,
                               hipMemcpyHostToDevice, s));
  }
  LLMRS_HIP(hipStreamSynchronize(s));
}

void mark_set(llmrs_model* m, int layer, int slot) {
  if (slot == LLMRS_W_LM_HEAD || layer < 0) m->lm_set = true;
  else m->layers[layer].set_mask |= 1u << slot;
}

}  // namespace

extern "C" {

int llmrs_model_set_linear_q4(llmrs_model* m, int layer, int slot, const uint8_t* qs,
                              const float* scales) {
  return guard([&] {
    LLMRS_REQUIRE(m && qs && scales, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(m->wt == WT_Q4H || m->wt == WT_Q4F, LLMRS_E_DTYPE, "model is not a Q4 model");
    Placement p = place(m, layer, slot);
    const size_t nb = p.k / 32;
    if (m->wt == WT_Q4H)
      LLMRS_REQUIRE(scales_fit_f16(scales, p.rows * nb), LLMRS_E_INVALID,
                    "Q4_0 scales must be exactly representable in fp16 (use LLMRS_Q4)");
    std::vector<uint8_t> codes(p.rows * nb * 16), sc(p.rows * nb * block_scale_bytes(m->wt));
    repack_q4_rows(qs, scales, p.rows, p.k, m->wt, {}, codes.data(), sc.data());
    put_rows(m, p, codes, sc);
    mark_set(m, layer, slot);
  });
}

int llmrs_model_set_linear_q8_0(llmrs_model* m, int layer, int slot, const int8_t* qs,
                                const float* scales) {
  return guard([&] {
    LLMRS_REQUIRE(m && qs && scales, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(m->wt == WT_Q8H, LLMRS_E_DTYPE, "model is not a Q8_0 model");
    Placement p = place(m, layer, slot);
    const size_t nb = p.k / 32;
    LLMRS_REQUIRE(scales_fit_f16(scales, p.rows * nb), LLMRS_E_INVALID,
                  "Q8_0 scales must be exactly representable in fp16");
    std::vector<uint8_t> codes(p.rows * p.k), sc(p.rows * nb * 2);
    repack_q8_rows(qs, scales, p.rows, p.k, {}, codes.data(), sc.data());
    put_rows(m, p, codes, sc);
    mark_set(m, layer, slot);
  });
}

int llmrs_model_kv_write(llmrs_model* m, int layer, int kv_head, size_t pos0, size_t n,
                         const float* k, const float* v) {
  return guard([&] {
    LLMRS_REQUIRE(m && k && v, LLMRS_E_INVALID, "null argument");
    const llmrs_model_config& c = m->c;
    LLMRS_REQUIRE(layer >= 0 && layer < c.n_layers && kv_head >= 0 && kv_head < c.n_kv_heads,
                  LLMRS_E_INVALID, "layer / kv_head out of range");
    LLMRS_REQUIRE(pos0 + n <= (size_t)c.max_seq, LLMRS_E_RANGE, "positions beyond max_seq");
    const int hd = c.head_dim;
    const size_t cnt = n * hd, eb = kv_elem_bytes(m), head = (size_t)kv_head * kv_rows(m) * hd;
    LayerBufs& Lb = m->layers[layer];
    std::vector<uint8_t> kb(cnt * eb);
    std::vector<uint16_t> vb;  // alive until the copies below have completed
    if (eb == 2) {
      // K rows as they are; the f16 V cache is blocked (v_offset): read the
      // 8-position blocks that [pos0, pos0 + n) touches, merge, write back.
      const size_t b0 = pos0 / 8, b1 = (pos0 + n + 7) / 8;
      vb.resize((b1 - b0) * 8 * hd);
      uint16_t* vdev = (uint16_t*)Lb.vc + head + b0 * 8 * hd;
      LLMRS_HIP(hipMemcpyAsync(vb.data(), vdev, vb.size() * 2, hipMemcpyDeviceToHost, ctx().stream));
      LLMRS_HIP(hipStreamSynchronize(ctx().stream));
      for (size_t t = 0; t < n; ++t)
        for (int d = 0; d < hd; ++d) {
          const uint16_t hk = host_f2h(k[t * hd + d]);
          std::memcpy(&kb[2 * (t * hd + d)], &hk, 2);
          vb[llmrs::v_offset(pos0 + t, d, hd, true) - b0 * 8 * hd] = host_f2h(v[t * hd + d]);
        }
      LLMRS_HIP(hipMemcpyAsync(vdev, vb.data(), vb.size() * 2, hipMemcpyHostToDevice, ctx().stream));
    } else {
      std::memcpy(kb.data(), k, cnt * 4);
      LLMRS_HIP(hipMemcpyAsync((float*)Lb.vc + head + pos0 * hd, v, cnt * 4, hipMemcpyHostToDevice, ctx().stream));
    }
    LLMRS_HIP(hipMemcpyAsync((uint8_t*)Lb.kc + (head + pos0 * hd) * eb, kb.data(), kb.size(),
                             hipMemcpyHostToDevice, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  });
}

int llmrs_model_kv_read(llmrs_model* m, int layer, int kv_head, size_t pos0, size_t n, float* k,
                        float* v) {
  return guard([&] {
    LLMRS_REQUIRE(m && k && v, LLMRS_E_INVALID, "null argument");
    const llmrs_model_config& c = m->c;
    LLMRS_REQUIRE(layer >= 0 && layer < c.n_layers && kv_head >= 0 && kv_head < c.n_kv_heads,
                  LLMRS_E_INVALID, "layer / kv_head out of range");
    LLMRS_REQUIRE(pos0 + n <= (size_t)c.max_seq, LLMRS_E_RANGE, "positions beyond max_seq");
    const int hd = c.head_dim;
    const size_t cnt = n * hd, eb = kv_elem_bytes(m), head = (size_t)kv_head * kv_rows(m) * hd;
    LayerBufs& Lb = m->layers[layer];
    std::vector<uint8_t> kb(cnt * eb);
    LLMRS_HIP(hipMemcpyAsync(kb.data(), (uint8_t*)Lb.kc + (head + pos0 * hd) * eb, kb.size(),
                             hipMemcpyDeviceToHost, ctx().stream));
    if (eb == 2) {  // blocked f16 V (v_offset): the 8-position blocks of the range
      const size_t b0 = pos0 / 8, b1 = (pos0 + n + 7) / 8;
      std::vector<uint16_t> vb((b1 - b0) * 8 * hd);
      LLMRS_HIP(hipMemcpyAsync(vb.data(), (uint16_t*)Lb.vc + head + b0 * 8 * hd, vb.size() * 2,
                               hipMemcpyDeviceToHost, ctx().stream));
      LLMRS_HIP(hipStreamSynchronize(ctx().stream));
      for (size_t t = 0; t < n; ++t)
        for (int d = 0; d < hd; ++d) {
          uint16_t hk;
          std::memcpy(&hk, &kb[2 * (t * hd + d)], 2);
          k[t * hd + d] = host_h2f(hk);
          v[t * hd + d] = host_h2f(vb[llmrs::v_offset(pos0 + t, d, hd, true) - b0 * 8 * hd]);
        }
    } else {
      LLMRS_HIP(hipMemcpyAsync(v, (float*)Lb.vc + head + pos0 * hd, cnt * 4, hipMemcpyDeviceToHost, ctx().stream));
      LLMRS_HIP(hipStreamSynchronize(ctx().stream));
      std::memcpy(k, kb.data(), cnt * 4);
    }
  });
}

int llmrs_model_forward(llmrs_model* m, const int32_t* tokens, size_t n, size_t start_pos,
                        float* logits, int32_t* next, float* trace) {
  return guard([&] {
    check_ready(m);
    LLMRS_REQUIRE(tokens && n > 0, LLMRS_E_INVALID, "empty token list");
    LLMRS_REQUIRE(start_pos + n <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "positions beyond max_seq");
    const size_t H = m->c.hidden, L = m->c.n_layers;
    upload_tokens(m, start_pos, tokens, n);
    hipStream_t s = ctx().stream;
    const bool batched = n > 1 && prefill_enabled();
    if (batched)
      run_prefill(m, start_pos, n, INT_MAX, logits != nullptr, trace);
    else
      set_state(m, start_pos, INT_MAX);
    for (size_t i = 0; i < n && !batched; ++i) {
      m->host_pos = start_pos + i;
      Launcher Ln{s};
      enqueue_step(m, Ln, logits && i + 1 == n, trace ? m->trace : nullptr);
      if (trace) {
        LLMRS_HIP(hipMemcpyAsync(trace + i * (L + 1) * H, m->trace, (L + 1) * H * sizeof(float),
                                 hipMemcpyDeviceToHost, s));
        LLMRS_HIP(hipStreamSynchronize(s));
      }
    }
    if (logits)
      LLMRS_HIP(hipMemcpyAsync(logits, m->logits, m->c.vocab * sizeof(float), hipMemcpyDeviceToHost, s));
    if (next) LLMRS_HIP(hipMemcpyAsync(next, m->gen + start_pos + n, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    LLMRS_HIP(hipStreamSynchronize(s));
    check_err(m);
    m->host_pos = start_pos + n;
    m->begun = false;
  });
}

int llmrs_model_begin_at(llmrs_model* m, const int32_t* prompt, size_t n_prompt, size_t start_pos) {
  return guard([&] {
    check_ready(m);
    LLMRS_REQUIRE(prompt && n_prompt > 0, LLMRS_E_INVALID, "empty prompt");
    LLMRS_REQUIRE(start_pos + n_prompt <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "prompt beyond max_seq");
    const size_t end = start_pos + n_prompt;
    upload_tokens(m, start_pos, prompt, n_prompt);
    set_state(m, start_pos, (int)end);
    m->host_n_prompt = (int)end;
    if (n_prompt > 1 && prefill_enabled()) {
      run_prefill(m, start_pos, n_prompt, (int)end, false, nullptr);
    } else {
      for (size_t p = start_pos; p < end; ++p) {
        m->host_pos = p;
        replay_step(m);
      }
    }
    m->host_pos = end;
    m->begun = true;
  });
}

int llmrs_model_begin(llmrs_model* m, const int32_t* prompt, size_t n_prompt) {
  return llmrs_model_begin_at(m, prompt, n_prompt, 0);
}

int llmrs_model_decode_steps(llmrs_model* m, size_t n) {
  return guard([&] {
    LLMRS_REQUIRE(m && m->begun, LLMRS_E_INVALID, "llmrs_model_begin has not been called");
    LLMRS_REQUIRE(m->host_pos + n <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "decode beyond max_seq");
    for (size_t i = 0; i < n; ++i) {
      replay_step(m);
      m->host_pos += 1;
    }
  });
}

int llmrs_model_tokens(llmrs_model* m, int32_t* out, size_t count) {
  return guard([&] {
    LLMRS_REQUIRE(m && out, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(count <= m->host_pos + 1, LLMRS_E_RANGE, "more tokens requested than produced");
    LLMRS_HIP(hipMemcpyAsync(out, m->tokens, count * sizeof(int32_t), hipMemcpyDeviceToHost, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    check_err(m);
  });
}

int llmrs_model_generate(llmrs_model* m, const int32_t* prompt, size_t n_prompt, size_t n_steps,
                         int32_t* out_tokens) {
  int rc = llmrs_model_begin(m, prompt, n_prompt);
  if (rc) return rc;
  if (n_steps == 0) return LLMRS_OK;
  rc = llmrs_model_decode_steps(m, n_steps - 1);
  if (rc) return rc;
  size_t produced = n_steps;
  int32_t stopped = 0;
  rc = llmrs_model_produced(m, &produced, &stopped);
  if (rc) return rc;
  produced = std::min(produced, n_steps);
  std::vector<int32_t> all(n_prompt + n_steps);
  rc = llmrs_model_tokens(m, all.data(), n_prompt + produced);
  if (rc) return rc;
  std::memcpy(out_tokens, all.data() + n_prompt, produced * sizeof(int32_t));
  for (size_t i = produced; i < n_steps; ++i) out_tokens[i] = -1;
  return LLMRS_OK;
}

int llmrs_model_produced(llmrs_model* m, size_t* n, int32_t* stopped) {
  return guard([&] {
    LLMRS_REQUIRE(m && m->begun, LLMRS_E_INVALID, "llmrs_model_begin has not been called");
    int v[2] = {0, 0};
    LLMRS_HIP(hipMemcpyAsync(&v[0], m->pos, sizeof(int), hipMemcpyDeviceToHost, ctx().stream));
    LLMRS_HIP(hipMemcpyAsync(&v[1], m->stopped, sizeof(int), hipMemcpyDeviceToHost, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    // the device position is that of the last token produced (the prompt's
    // last before any)
    if (n) *n = (size_t)std::max(0, v[0] + 1 - m->host_n_prompt);
    if (stopped) *stopped = v[1];
  });
}

int llmrs_model_set_sampling(llmrs_model* m, const llmrs_sampling* s) {
  return guard([&] {
    LLMRS_REQUIRE(m, LLMRS_E_INVALID, "null model");
    if (s) {
      check_sampling(*s, m->c.vocab);
      if (!m->probs) {
        m->probs = m->dalloc<float>(m->c.vocab);
        m->samp_state = (llmrs::SampleState*)m->dalloc<uint8_t>(sizeof(llmrs::SampleState));
      }
      int ids[LLMRS_MAX_EOS] = {};
      std::memcpy(ids, s->eos, sizeof(ids));
      LLMRS_HIP(hipMemcpyAsync(m->eos, ids, sizeof(ids), hipMemcpyHostToDevice, ctx().stream));
      LLMRS_HIP(hipStreamSynchronize(ctx().stream));
      m->samp = *s;
    }
    m->sampling = s != nullptr;
    // the captured step ends with the argmax or the sampler: capture anew
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->graph_failed = false;
  });
}

int llmrs_model_set_exact(llmrs_model* m, int on) {
  return guard([&] {
    LLMRS_REQUIRE(m, LLMRS_E_INVALID, "null model");
    set_exact(m, on != 0);
  });
}

int llmrs_sample_logits(const float* logits, int32_t vocab, const int32_t* history, size_t n_history,
                        const llmrs_sampling* s, uint64_t position, int32_t* token, float* u) {
  return guard([&] {
    LLMRS_REQUIRE(logits && s && (history || n_history == 0), LLMRS_E_INVALID, "null argument");
    check_sampling(*s, vocab);
    LLMRS_REQUIRE(n_history < (size_t)INT_MAX && position < (uint64_t)LLONG_MAX, LLMRS_E_RANGE,
                  "history or position too large");
    hipStream_t st = ctx().stream;
    const size_t V = (size_t)vocab;
    // one allocation: sampler state, logits, probs, history, eos, token, u
    const size_t off_l = align_up(sizeof(llmrs::SampleState), 256);
    const size_t off_p = off_l + V * 4, off_h = off_p + V * 4, off_e = off_h + std::max<size_t>(n_history, 1) * 4;
    const size_t off_t = off_e + LLMRS_MAX_EOS * 4, bytes = off_t + 8;
    uint8_t* d = nullptr;
    LLMRS_HIP(hipMalloc(&d, bytes));
    try {
      LLMRS_HIP(hipMemsetAsync(d, 0, off_l, st));
      LLMRS_HIP(hipMemcpyAsync(d + off_l, logits, V * 4, hipMemcpyHostToDevice, st));
      if (n_history)
        LLMRS_HIP(hipMemcpyAsync(d + off_h, history, n_history * 4, hipMemcpyHostToDevice, st));
      LLMRS_HIP(hipMemcpyAsync(d + off_e, s->eos, LLMRS_MAX_EOS * 4, hipMemcpyHostToDevice, st));
      SampleArgs a = sample_args(*s, vocab);
      a.st = (llmrs::SampleState*)d;
      a.logits = (const float*)(d + off_l);
      a.probs = (float*)(d + off_p);
      a.hist = (const int*)(d + off_h);
      a.n_hist = (int)n_history;
      a.eos = (const int*)(d + off_e);
      a.step_override = (long long)position;
      a.out_token = (int*)(d + off_t);
      a.out_u = (float*)(d + off_t + 4);
      Launcher L{st};
      enqueue_sample(L, a);
      int32_t t = 0;
      float uu = 0.0f;
      LLMRS_HIP(hipMemcpyAsync(&t, d + off_t, 4, hipMemcpyDeviceToHost, st));
      LLMRS_HIP(hipMemcpyAsync(&uu, d + off_t + 4, 4, hipMemcpyDeviceToHost, st));
      LLMRS_HIP(hipStreamSynchronize(st));
      if (token) *token = t;
      if (u) *u = uu;
    } catch (...) {
      (void)hipStreamSynchronize(st);
      (void)hipFree(d);
      throw;
    }
    LLMRS_HIP(hipFree(d));
  });
}

}  // extern "C"

namespace {

// Runs `body` with an event-recording launcher, then reports each launch's
// name, duration and recorded work figure.  Returns the number reported.
template <class F>
int profile_launches(F&& body, char* names, float* ms, double* work, int cap) {
  std::vector<std::tuple<std::string, double, hipEvent_t, hipEvent_t>> rec;
  Launcher L{ctx().stream, &rec};
  try {
    body(L);
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  } catch (...) {
    for (auto& r : rec) {
      (void)hipEventDestroy(std::get<2>(r));
      (void)hipEventDestroy(std::get<3>(r));
    }
    throw;
  }
  int count = 0;
  for (auto& r : rec) {
    float t = 0.0f;
    (void)hipEventElapsedTime(&t, std::get<2>(r), std::get<3>(r));
    if (count < cap) {
      if (names) {
        std::strncpy(names + 32 * count, std::get<0>(r).c_str(), 31);
        names[32 * count + 31] = 0;
      }
      if (ms) ms[count] = t;
      if (work) work[count] = std::get<1>(r);
      ++count;
    }
    (void)hipEventDestroy(std::get<2>(r));
    (void)hipEventDestroy(std::get<3>(r));
  }
  return count;
}

}  // namespace

extern "C" {

int llmrs_model_profile_step(llmrs_model* m, char* names, float* ms, double* bytes, int cap) {
  int count = 0;
  int rc = guard([&] {
    LLMRS_REQUIRE(m && m->begun, LLMRS_E_INVALID, "llmrs_model_begin has not been called");
    LLMRS_REQUIRE(m->host_pos + 1 <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "decode beyond max_seq");
    count = profile_launches([&](Launcher& L) { enqueue_step(m, L, false, nullptr); }, names, ms, bytes,
                             cap);
    m->host_pos += 1;
  });
  return rc ? rc : count;
}

int llmrs_model_time_linear(llmrs_model* m, int slot, int reps, double* us_per_launch,
                            double* bytes_per_launch) {
  return guard([&] {
    LLMRS_REQUIRE(m && m->begun, LLMRS_E_INVALID, "llmrs_model_begin has not been called");
    LLMRS_REQUIRE(us_per_launch && reps > 0, LLMRS_E_INVALID, "null argument or reps < 1");
    hipStream_t s = ctx().stream;
    std::vector<std::tuple<std::string, double, hipEvent_t, hipEvent_t>> rec;
    Launcher probe{s, &rec};
    enqueue_linear(m, probe, 0, slot);  // validates the slot; records the bytes
    LLMRS_HIP(hipStreamSynchronize(s));
    const double bytes = std::get<1>(rec[0]);
    for (auto& r : rec) {
      (void)hipEventDestroy(std::get<2>(r));
      (void)hipEventDestroy(std::get<3>(r));
    }
    hipEvent_t e0, e1;
    LLMRS_HIP(hipEventCreate(&e0));
    LLMRS_HIP(hipEventCreate(&e1));
    Launcher L{s};
    LLMRS_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; ++r)
      for (int li = 0; li < m->c.n_layers; ++li) enqueue_linear(m, L, li, slot);
    LLMRS_HIP(hipEventRecord(e1, s));
    LLMRS_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *us_per_launch = ms * 1e3 / ((double)reps * m->c.n_layers);
    if (bytes_per_launch) *bytes_per_launch = bytes;
  });
}

int llmrs_model_profile_prefill(llmrs_model* m, const int32_t* tokens, size_t n, size_t start_pos,
                                char* names, float* ms, double* work, int cap) {
  int count = 0;
  int rc = guard([&] {
    check_ready(m);
    LLMRS_REQUIRE(tokens && n > 0, LLMRS_E_INVALID, "empty token list");
    LLMRS_REQUIRE(start_pos + n <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "positions beyond max_seq");
    ensure_prefill(m);
    LLMRS_REQUIRE(n <= (size_t)m->pf_cap, LLMRS_E_RANGE, "more rows than one prefill chunk");
    upload_tokens(m, start_pos, tokens, n);
    const int s0 = (int)start_pos;
    LLMRS_HIP(hipMemcpyAsync(m->pf_start, &s0, sizeof(int), hipMemcpyHostToDevice, ctx().stream));
    set_state(m, start_pos + n - 1, INT_MAX);
    count = profile_launches(
        [&](Launcher& L) { enqueue_prefill(m, L, start_pos, (int)n, true, false, nullptr, nullptr, nullptr, m->exact); },
        names, ms,
        work, cap);
    check_err(m);
    m->host_pos = start_pos + n;
    m->begun = false;
  });
  return rc ? rc : count;
}

int llmrs_model_profile_stamps(llmrs_model* m, int layer, int slot, double* out, int cap) {
  int count = 0;
  int rc = guard([&] {
    LLMRS_REQUIRE(m && m->begun && out, LLMRS_E_INVALID, "llmrs_model_begin has not been called");
    LLMRS_REQUIRE(layer >= 0 && layer < m->c.n_layers, LLMRS_E_RANGE, "layer out of range");
    LLMRS_REQUIRE(m->host_pos + 1 <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "decode beyond max_seq");
    const unsigned nwg = slot == -2 ? (unsigned)(m->nsplit * m->c.n_kv_heads) : linear_grid(m, slot);
    const int per = 8;  // stamps per workgroup
    unsigned long long* ts = nullptr;
    LLMRS_HIP(hipMalloc(&ts, (size_t)nwg * per * sizeof(unsigned long long)));
    hipStream_t s = ctx().stream;
    std::vector<unsigned long long> h((size_t)nwg * per);
    try {
      LLMRS_HIP(hipMemsetAsync(ts, 0, h.size() * sizeof(unsigned long long), s));
      const llmrs_model_config& c = m->c;
      Launcher L{s};
      enqueue_embed(m, L, nullptr, m->layers[0].norm[0]);
      for (int li = 0; li < c.n_layers; ++li) {
        enqueue_linear(m, L, li, LLMRS_W_Q, nullptr, nullptr, li == layer && slot == LLMRS_W_Q ? ts : nullptr);
        enqueue_attention(m, L, li, li == layer && slot == -2 ? ts : nullptr);
        enqueue_linear(m, L, li, LLMRS_W_O, nullptr, nullptr, li == layer && slot == LLMRS_W_O ? ts : nullptr);
        enqueue_linear(m, L, li, LLMRS_W_GATE, nullptr, nullptr,
                       li == layer && slot == LLMRS_W_GATE ? ts : nullptr);
        enqueue_linear(m, L, li, LLMRS_W_DOWN, nullptr, nullptr,
                       li == layer && slot == LLMRS_W_DOWN ? ts : nullptr);
      }
      enqueue_head(m, L, false);
      LLMRS_HIP(hipMemcpyAsync(h.data(), ts, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost, s));
      LLMRS_HIP(hipStreamSynchronize(s));
    } catch (...) {
      (void)hipStreamSynchronize(s);
      (void)hipFree(ts);
      throw;
    }
    (void)hipFree(ts);
    m->host_pos += 1;
    // per workgroup: stamps 0-6 in us from the launch's earliest start (-1 =
    // not recorded), then the XCC id and the HW_ID word
    unsigned long long t0 = ~0ull;
    for (unsigned w = 0; w < nwg; ++w)
      if (h[8 * w]) t0 = std::min(t0, h[8 * w]);
    auto us = [&](unsigned long long v) { return v ? (double)(v - t0) / 100.0 : -1.0; };
    for (unsigned w = 0; w < nwg && count + 9 <= cap; ++w) {
      for (int i = 0; i < 7; ++i) out[count++] = us(h[8 * w + i]);
      out[count++] = (double)(h[8 * w + 7] >> 32);
      out[count++] = (double)(h[8 * w + 7] & 0xFFFFFFFFull);
    }
  });
  return rc ? rc : count;
}

int llmrs_model_get_config(const llmrs_model* m, llmrs_model_config* out) {
  return guard([&] {
    LLMRS_REQUIRE(m && out, LLMRS_E_INVALID, "null argument");
    *out = m->c;
  });
}

int llmrs_model_decode_plan(const llmrs_model* m, int32_t out[4]) {
  return guard([&] {
    LLMRS_REQUIRE(m && out, LLMRS_E_INVALID, "null argument");
    out[0] = m->nsplit;
    out[1] = m->c.kv_dtype == LLMRS_F16 ? m->attn_waves : m->attn_streams;
    out[2] = m->attn_local ? 1 : 0;
    out[3] = m->exact ? 1 : 0;
  });
}

double llmrs_model_weight_bytes(const llmrs_model* m) {
  if (!m) return 0.0;
  double b = linear_weight_bytes(m, m->lm_head);
  for (const auto& L : m->layers)
    b += linear_weight_bytes(m, L.qkv) + linear_weight_bytes(m, L.o) + linear_weight_bytes(m, L.gu) +
         linear_weight_bytes(m, L.down);
  return b;
}

}  // extern "C"

// ---- test probes: one layer's kernels on given inputs ----------------------

namespace {

void check_layer_ready(const llmrs_model* m, int layer) {
  LLMRS_REQUIRE(m, LLMRS_E_INVALID, "null model");
  LLMRS_REQUIRE(layer >= 0 && layer < m->c.n_layers, LLMRS_E_RANGE, "layer out of range");
  LLMRS_REQUIRE(m->layers[layer].set_mask == 0x37f, LLMRS_E_INVALID,
                "layer " + std::to_string(layer) + " weights incomplete");
}

// Copies `bytes` from device `src` to host `dst` when dst is set (the stream
// is synchronised by the caller).
void probe_copy(void* dst, const void* src, size_t bytes) {
  if (dst) LLMRS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream));
}

// Device scratch of a probe call, freed on every exit path.
struct ProbeBuf {
  std::vector<void*> ptrs;
  template <class T>
  T* get(size_t count) {
    void* p = nullptr;
    LLMRS_HIP(hipMalloc(&p, std::max<size_t>(count * sizeof(T), 256)));
    ptrs.push_back(p);
    return (T*)p;
  }
  ~ProbeBuf() {
    (void)hipStreamSynchronize(ctx().stream);
    for (void* p : ptrs) (void)hipFree(p);
  }
};

}  // namespace

extern "C" {

int llmrs_model_probe_decode_layer(llmrs_model* m, int layer, size_t pos, const float* x,
                                   llmrs_layer_probe* out) {
  return guard([&] {
    check_layer_ready(m, layer);
    LLMRS_REQUIRE(x && out, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(pos < (size_t)m->c.max_seq, LLMRS_E_RANGE, "position beyond max_seq");
    const llmrs_model_config& c = m->c;
    const size_t H = c.hidden, F = c.ffn, qd = (size_t)c.n_heads * c.head_dim;
    hipStream_t s = ctx().stream;
    ProbeBuf pb;
    int8_t* xq = pb.get<int8_t>(H);
    float* xd = pb.get<float>(H / 32);
    float* xin = pb.get<float>(H);
    set_state(m, pos, INT_MAX);
    m->host_pos = pos;
    LLMRS_HIP(hipMemcpyAsync(xin, x, H * sizeof(float), hipMemcpyHostToDevice, s));
    Launcher L{s};
    auto sync = [&] { LLMRS_HIP(hipStreamSynchronize(s)); };
    if (m->exact) {  // the reference-order kernels, every stage copied out
      LLMRS_HIP(hipMemcpyAsync(m->x, xin, H * sizeof(float), hipMemcpyDeviceToDevice, s));
      enqueue_exact_layer(m, L, layer, [&](int stage) {
        switch (stage) {
          case 0:
            probe_copy(out->xq, m->x_q, H);
            probe_copy(out->xd, m->x_d, H / 32 * sizeof(float));
            break;
          case 1: probe_copy(out->qkv, m->qkv, m->qkv_rows * sizeof(float)); break;
          case 2:
            probe_copy(out->ctx, m->ctxv, qd * sizeof(float));
            probe_copy(out->ctx_q, m->ctx_q, qd);
            probe_copy(out->ctx_d, m->ctx_d, qd / 32 * sizeof(float));
            break;
          case 3: probe_copy(out->h, m->h, H * sizeof(float)); break;
          case 4:
            probe_copy(out->hq, m->h_q, H);
            probe_copy(out->hd, m->h_d, H / 32 * sizeof(float));
            break;
          case 6:
            probe_copy(out->m, m->mf, F * sizeof(float));
            probe_copy(out->m_q, m->m_q, F);
            probe_copy(out->m_d, m->m_d, F / 32 * sizeof(float));
            break;
          case 7: probe_copy(out->out, m->x, H * sizeof(float)); break;
        }
        sync();
      });
      check_err(m);
      m->begun = false;
      return;
    }
    enqueue_embed(m, L, xin, m->layers[layer].norm[0]);
    enqueue_linear(m, L, layer, LLMRS_W_Q, xq, xd);
    probe_copy(out->qkv, m->qkv, m->qkv_rows * sizeof(float));
    probe_copy(out->xq, xq, H);
    probe_copy(out->xd, xd, H / 32 * sizeof(float));
    sync();
    enqueue_attention(m, L, layer);
    probe_copy(out->ctx, m->ctxv, qd * sizeof(float));
    probe_copy(out->ctx_q, m->ctx_q, qd);
    probe_copy(out->ctx_d, m->ctx_d, qd / 32 * sizeof(float));
    sync();
    enqueue_linear(m, L, layer, LLMRS_W_O);
    probe_copy(out->h, m->h, H * sizeof(float));
    sync();
    enqueue_linear(m, L, layer, LLMRS_W_GATE, xq, xd);
    probe_copy(out->hq, xq, H);
    probe_copy(out->hd, xd, H / 32 * sizeof(float));
    probe_copy(out->m, m->mf, F * sizeof(float));
    probe_copy(out->m_q, m->m_q, F);
    probe_copy(out->m_d, m->m_d, F / 32 * sizeof(float));
    sync();
    enqueue_linear(m, L, layer, LLMRS_W_DOWN);
    probe_copy(out->out, m->x, H * sizeof(float));
    sync();
    check_err(m);
    m->begun = false;
  });
}

int llmrs_model_probe_head(llmrs_model* m, const float* x, int8_t* xq, float* xd, float* logits,
                           int32_t* next) {
  return guard([&] {
    LLMRS_REQUIRE(m && x, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(m->final_set && m->lm_set, LLMRS_E_INVALID, "final norm / lm_head not set");
    const size_t H = m->c.hidden;
    hipStream_t s = ctx().stream;
    ProbeBuf pb;
    int8_t* dq = pb.get<int8_t>(H);
    float* dd = pb.get<float>(H / 32);
    float* xin = pb.get<float>(H);
    set_state(m, 0, INT_MAX);
    LLMRS_HIP(hipMemcpyAsync(xin, x, H * sizeof(float), hipMemcpyHostToDevice, s));
    Launcher L{s};
    if (m->exact) {
      LLMRS_HIP(hipMemcpyAsync(m->x, xin, H * sizeof(float), hipMemcpyDeviceToDevice, s));
      enqueue_exact_head(m, L, logits != nullptr);
      dq = m->x_q;
      dd = m->x_d;
    } else {
      enqueue_embed(m, L, xin, m->final_norm);
      enqueue_head(m, L, logits != nullptr, dq, dd);
    }
    probe_copy(xq, dq, H);
    probe_copy(xd, dd, H / 32 * sizeof(float));
    probe_copy(logits, m->logits, (size_t)m->c.vocab * sizeof(float));
    probe_copy(next, m->gen + 1, sizeof(int32_t));
    LLMRS_HIP(hipStreamSynchronize(s));
    m->begun = false;
  });
}

int llmrs_model_probe_prefill_layer(llmrs_model* m, int layer, size_t start_pos, size_t n,
                                    const float* x, llmrs_layer_probe* out) {
  return guard([&] {
    check_layer_ready(m, layer);
    LLMRS_REQUIRE(x && out && n > 0, LLMRS_E_INVALID, "null argument or no rows");
    LLMRS_REQUIRE(start_pos + n <= (size_t)m->c.max_seq, LLMRS_E_RANGE, "positions beyond max_seq");
    ensure_prefill(m);
    LLMRS_REQUIRE(n <= (size_t)m->pf_cap, LLMRS_E_RANGE, "more rows than one prefill chunk");
    const llmrs_model_config& c = m->c;
    const size_t H = c.hidden, F = c.ffn, qd = (size_t)c.n_heads * c.head_dim, M = n;
    hipStream_t s = ctx().stream;
    ProbeBuf pb;
    PrefillProbe p;
    p.ctx = pb.get<float>(M * qd);
    p.mf = pb.get<float>(M * F);
    LLMRS_HIP(hipMemcpyAsync(m->pf_x, x, M * H * sizeof(float), hipMemcpyHostToDevice, s));
    p.after = [&](int stage) {
      switch (stage) {
        case 0:
          probe_copy(out->xq, m->pf_aq, M * H);
          probe_copy(out->xd, m->pf_ad, M * H / 32 * sizeof(float));
          break;
        case 1: probe_copy(out->qkv, m->pf_qkv, M * m->qkv_rows * sizeof(float)); break;
        case 3:
          probe_copy(out->ctx, p.ctx, M * qd * sizeof(float));
          probe_copy(out->ctx_q, m->pf_ctx_q, M * qd);
          probe_copy(out->ctx_d, m->pf_ctx_d, M * qd / 32 * sizeof(float));
          break;
        case 4: probe_copy(out->h, m->pf_h, M * H * sizeof(float)); break;
        case 5:
          probe_copy(out->hq, m->pf_aq, M * H);
          probe_copy(out->hd, m->pf_ad, M * H / 32 * sizeof(float));
          break;
        case 6:
          probe_copy(out->m, p.mf, M * F * sizeof(float));
          probe_copy(out->m_q, m->pf_m_q, M * F);
          probe_copy(out->m_d, m->pf_m_d, M * F / 32 * sizeof(float));
          break;
        case 7: probe_copy(out->out, m->pf_x, M * H * sizeof(float)); break;
      }
      LLMRS_HIP(hipStreamSynchronize(s));
    };
    Launcher L{s};
    enqueue_prefill_layer(m, L, layer, start_pos, (int)M, &p, nullptr, nullptr, m->exact);
    if (prefill_skinny(m, (int)M)) {  // codes back into element order
      auto natural = [&](int8_t* rows, size_t K) {
        if (!rows) return;
        std::vector<int8_t> tmp(K);
        for (size_t t = 0; t < M; ++t) {
          int8_t* r = rows + t * K;
          for (size_t k = 0; k < K; ++k) tmp[k] = r[llmrs::act_offset((int)k, llmrs::kActMfma)];
          std::memcpy(r, tmp.data(), K);
        }
      };
      natural(out->xq, H);
      natural(out->ctx_q, qd);
      natural(out->hq, H);
      natural(out->m_q, F);
    }
    m->begun = false;
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Batched decode: B sequences of one model stepping together, each with its
// own K/V cache, position and token history.  The reference runs one
// sequence; its layer code would take any number of rows (layer.rs:175-333,
// the mask at :264), and a row's values depend only on that row and its own
// cache.  Here the B rows go through every linear layer at once - the exact
// int8 GEMM of the prefill path with M = B, which gives each row the
// reference's per-output block loop (cpu.rs:90-110) - and the decode
// attention runs one grid slice per sequence (grid.z), over that sequence's
// cache at its position.  The head is the lm_head GEMM over the B rows and a
// per-row greedy step.
// ---------------------------------------------------------------------------
struct llmrs_batch {
  llmrs_model* m = nullptr;
  int B = 0, cap = 0;
  size_t kv_bytes = 0;  // one sequence's K (or V) cache of one layer
  std::vector<void*> kc, vc;  // per layer: B caches back to back
  float *x = nullptr, *h = nullptr, *qkv = nullptr, *ctxv = nullptr, *logits = nullptr;
  float *ad = nullptr, *ctx_d = nullptr, *m_d = nullptr, *part_o = nullptr, *part_ml = nullptr;
  float* rope_now = nullptr;  // [B][hd]: each sequence's RoPE row of the step
  int8_t *aq = nullptr, *ctx_q = nullptr, *m_q = nullptr;
  int *pos = nullptr, *tokens = nullptr, *gen = nullptr, *counters = nullptr;
  // linear layers on the decode GEMV over all rows (gemv_*_q8b_*: one
  // workgroup per row and weight slice, the rows' workgroups of a slice on
  // one XCD so that the weights stream from HBM about once and the other rows
  // read them from its L2; up to kBatchGemvMax sequences), on the skinny GEMM
  // (sgemm.hip; token tiles of 16, the activation codes in its operand order)
  // or, beyond 64 sequences or for widths not a multiple of 128, on the
  // prefill GEMM
  bool gemv = false;
  bool skinny = false;
  int layout = llmrs::kActNatural;
  // attention splits per sequence: the model's (planned for one sequence)
  // cut so that the B sequences' workgroups fill the GPU about twice
  int nsplit = 1;
  std::vector<size_t> host_pos;
  std::vector<char> begun;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool graph_failed = false;
  std::vector<void*> allocs;

  template <class T>
  T* dalloc(size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    if (hipMalloc(&p, bytes) != hipSuccess) {
      (void)hipGetLastError();
      fail(LLMRS_E_OOM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    allocs.push_back(p);
    LLMRS_HIP(hipMemsetAsync(p, 0, bytes, ctx().stream));
    return (T*)p;
  }
  ~llmrs_batch() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (void* p : allocs) (void)hipFree(p);
  }
};

namespace {

// Kernel name of a batched linear layer (epi: store, resid, silu).
GemvPlan batch_gemv_plan(const llmrs_batch* b, const char* epi, const DevLinear& W) {
  return gemv_plan(b->m->wt, std::string("q8b_") + epi, W.n, W.k, ctx().num_cus);
}

std::string batch_linear_kernel(const llmrs_batch* b, const char* epi, const DevLinear& W) {
  if (b->gemv) return batch_gemv_plan(b, epi, W).name;
  return b->skinny ? sgemm_kernel(b->m, epi, b->B, false) : gemm_kernel(b->m, epi);
}

// One greedy step of every sequence of the batch.
void enqueue_batch_step(llmrs_batch* b, Launcher& L) {
  llmrs_model* m = b->m;
  const llmrs_model_config& c = m->c;
  const int B = b->B, H = c.hidden, hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads;
  const dim3 blk(256);
  const size_t glds = gemm_lds_bytes();
  // One linear layer over the B rows: Y = X W^T (+ res), or the SwiGLU
  // product's Q8_0 codes; work figure = the weight bytes.
  auto linear = [&](const char* epi, const DevLinear& W, const int8_t* xq, const float* xd, float* y,
                    const float* res, int8_t* yq, float* yd) {
    const std::string name = batch_linear_kernel(b, epi, W);
    const bool silu = std::string(epi) == "silu";
    const double wb = linear_weight_bytes(m, W);
    if (b->gemv) {
      const GemvPlan p = batch_gemv_plan(b, epi, W);
      GemvArgs g{};
      g.wq = W.codes;
      g.ws = W.scales;
      g.n = W.n;
      g.k = W.k;
      g.xq = xq;
      g.xd = xd;
      g.y = y;
      g.res = res;
      g.yq = yq;
      g.yd = yd;
      g.batch_rows = B;
      g.batch_nwg = (int)p.grid;
      L(name, wb, dim3(8u * (unsigned)B * ((p.grid + 7) / 8)), dim3(p.threads), p.lds, g);
    } else if (b->skinny) {
      SgemmArgs g{xq, xd, W.codes, W.scales, y, res, yq, yd, B, W.n, W.k, W.n, b->layout};
      const auto sh = sgemm_shape(epi, W.n, false);
      L(name, wb, sh.first, sh.second, 0, g);
    } else {
      PrefillGemmArgs g{xq, xd, W.codes, W.scales, y, res, yq, yd, B, W.n, W.k, silu ? W.n / 2 : W.n, gemm_group_m()};
      L(name, wb, gemm_grid(B, W.n), blk, glds, g);
    }
  };
  EmbedArgs e{m->embed, b->tokens, b->pos, b->x, m->err, H, c.vocab, nullptr, nullptr, nullptr, nullptr, nullptr,
              b->cap, m->rope_cos, m->rope_sin, b->rope_now, hd / 2, c.max_seq};
  L("embed_gather", 8.0 * H * B, dim3((unsigned)((H + 255) / 256), (unsigned)B), blk, 0, e);
  for (int li = 0; li < c.n_layers; ++li) {
    LayerBufs& Lb = m->layers[li];
    {  // RMSNorm + Q8_0 of each sequence's row (layer.rs:377)
      PrefillRowArgs r{b->x, Lb.norm[0], b->aq, b->ad, B, H, c.rms_eps, b->layout};
      L("prefill_rows_q8", 5.0 * H * B, dim3((unsigned)B), blk, gemv_act_lds_host(H), r);
    }
    linear("store", Lb.qkv, b->aq, b->ad, b->qkv, nullptr, nullptr, nullptr);  // Q|K|V
    {  // decode attention, one grid slice per sequence (RoPE and the K/V append inside)
      AttnArgs a{};
      a.qkv = b->qkv;
      a.pos_ptr = b->pos;
      a.kc = b->kc[li];
      a.vc = b->vc[li];
      a.rope_cos = m->rope_cos;
      a.rope_sin = m->rope_sin;
      a.rope_now = b->rope_now;
      a.part_o = b->part_o;
      a.part_ml = b->part_ml;
      a.counters = b->counters + (size_t)li * B * nkv * llmrs::kTicketStride;
      a.ctx = b->ctxv;
      a.ctx_q = b->ctx_q;
      a.ctx_d = b->ctx_d;
      a.max_seq = kv_rows(m);
      a.nq = nq;
      a.nkv = nkv;
      a.nsplit = b->nsplit;
      a.scale = 1.0f / std::sqrt((float)hd);  // layer.rs:258
      a.kv_batch_bytes = b->kv_bytes;
      a.ctx_layout = b->layout;
      L(attn_kernel(m), 0.0, dim3((unsigned)b->nsplit, (unsigned)nkv, (unsigned)B), dim3(attn_threads(m)), 0, a);
    }
    linear("resid", Lb.o, b->ctx_q, b->ctx_d, b->h, b->x, nullptr, nullptr);  // O + residual (layer.rs:386)
    {  // post-attention RMSNorm + Q8_0
      PrefillRowArgs r{b->h, Lb.norm[1], b->aq, b->ad, B, H, c.rms_eps, b->layout};
      L("prefill_rows_q8", 5.0 * H * B, dim3((unsigned)B), blk, gemv_act_lds_host(H), r);
    }
    linear("silu", Lb.gu, b->aq, b->ad, nullptr, nullptr, b->m_q, b->m_d);  // gate|up + SwiGLU + Q8_0 of m
    linear("resid", Lb.down, b->m_q, b->m_d, b->x, b->h, nullptr, nullptr);  // down + residual (layer.rs:403)
  }
  {  // final RMSNorm (model.rs:39) + lm_head over the B rows, then each row's greedy step
    PrefillRowArgs r{b->x, m->final_norm, b->aq, b->ad, B, H, c.rms_eps, b->layout};
    L("prefill_rows_q8", 5.0 * H * B, dim3((unsigned)B), blk, gemv_act_lds_host(H), r);
    linear("store", m->lm_head, b->aq, b->ad, b->logits, nullptr, nullptr, nullptr);
    ArgmaxBatchArgs am{b->logits, c.vocab, b->pos, b->tokens, b->gen, b->cap};
    L("argmax_batch", 4.0 * c.vocab * B, dim3((unsigned)B), dim3(1024), 0, am);
  }
}

void replay_batch_step(llmrs_batch* b) {
  hipStream_t s = ctx().stream;
  if (!b->exec && !b->graph_failed && env_int("LLMRS_GRAPH", 1)) {
    Launcher L{s};
    bool ok = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess;
    if (ok) {
      try {
        enqueue_batch_step(b, L);
      } catch (const Error&) {
        ok = false;
      }
      hipGraph_t g = nullptr;
      const hipError_t e = hipStreamEndCapture(s, &g);
      ok = ok && e == hipSuccess && g;
      if (ok) {
        b->graph = g;
        ok = hipGraphInstantiate(&b->exec, g, nullptr, nullptr, 0) == hipSuccess;
      } else if (g) {
        (void)hipGraphDestroy(g);
      }
    }
    if (!ok) {
      (void)hipGetLastError();
      b->graph_failed = true;
      b->exec = nullptr;
      std::fprintf(stderr, "llmrs_hip: HIP graph capture failed; using per-kernel launches\n");
    }
  }
  if (b->exec) {
    LLMRS_HIP(hipGraphLaunch(b->exec, s));
  } else {
    Launcher L{s};
    enqueue_batch_step(b, L);
  }
}

}  // namespace

extern "C" {

int llmrs_batch_create(llmrs_model* m, int32_t batch, llmrs_batch** out) {
  return guard([&] {
    check_ready(m);
    LLMRS_REQUIRE(out && batch >= 1 && batch <= 256, LLMRS_E_INVALID, "batch must be in [1, 256]");
    const llmrs_model_config& c = m->c;
    std::unique_ptr<llmrs_batch> b(new llmrs_batch());
    b->m = m;
    b->B = batch;
    b->cap = m->cap;
    b->kv_bytes = align_up(kv_layer_elems(m) * kv_elem_bytes(m), 256);
    const size_t B = (size_t)batch, H = c.hidden, F = c.ffn, qd = (size_t)c.n_heads * c.head_dim;
    for (int li = 0; li < c.n_layers; ++li) {
      b->kc.push_back(b->dalloc<uint8_t>(B * b->kv_bytes));
      b->vc.push_back(b->dalloc<uint8_t>(B * b->kv_bytes));
    }
    b->x = b->dalloc<float>(B * H);
    b->h = b->dalloc<float>(B * H);
    b->qkv = b->dalloc<float>(B * m->qkv_rows);
    b->ctxv = b->dalloc<float>(B * qd);
    b->logits = b->dalloc<float>(B * c.vocab);
    b->aq = b->dalloc<int8_t>(B * H);
    b->ad = b->dalloc<float>(B * H / 32);
    b->ctx_q = b->dalloc<int8_t>(B * qd);
    b->ctx_d = b->dalloc<float>(B * qd / 32);
    b->m_q = b->dalloc<int8_t>(B * F);
    b->m_d = b->dalloc<float>(B * F / 32);
    b->part_o = b->dalloc<float>(B * qd * m->nsplit);
    b->part_ml = b->dalloc<float>(B * c.n_heads * llmrs::ml_stride(m->nsplit) * 2);
    b->counters = b->dalloc<int>((size_t)c.n_layers * B * c.n_kv_heads * llmrs::kTicketStride);
    b->pos = b->dalloc<int>(B);
    b->rope_now = b->dalloc<float>((size_t)B * c.head_dim);
    b->tokens = b->dalloc<int>(B * b->cap);
    b->gen = b->dalloc<int>(B * b->cap);
    b->host_pos.assign(B, 0);
    b->begun.assign(B, 0);
    const int qdim = c.n_heads * c.head_dim;
    const std::string bg = env_str("LLMRS_BATCH_GEMM");  // gemv, skinny or prefill forces one
    b->gemv = bg == "gemv" || (bg.empty() && batch <= kBatchGemvMax);
    b->skinny = !b->gemv && batch <= 64 && c.hidden % 128 == 0 && c.ffn % 128 == 0 && qdim % 128 == 0 &&
                bg != "prefill";
    b->layout = b->skinny ? llmrs::kActMfma : llmrs::kActNatural;
    b->nsplit = std::max(1, std::min(m->nsplit, (2 * ctx().num_cus + batch * c.n_kv_heads - 1) /
                                                     (batch * c.n_kv_heads)));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    (void)kernel("argmax_batch", dim3(1024));
    for (const char* epi : {"store", "resid", "silu"}) {
      const DevLinear& W = std::string(epi) == "store" ? m->lm_head : std::string(epi) == "resid" ? m->layers[0].down
                                                                                             : m->layers[0].gu;
      (void)kernel(batch_linear_kernel(b.get(), epi, W), dim3(256));
    }
    *out = b.release();
    ++m->live_batches;
  });
}

int llmrs_batch_free(llmrs_batch* b) {
  return guard([&] {
    if (!b) return;
    (void)hipStreamSynchronize(ctx().stream);
    --b->m->live_batches;
    delete b;
  });
}

int llmrs_batch_begin(llmrs_batch* b, int32_t slot, const int32_t* prompt, size_t n_prompt) {
  return guard([&] {
    LLMRS_REQUIRE(b && prompt && n_prompt > 0, LLMRS_E_INVALID, "empty prompt");
    LLMRS_REQUIRE(slot >= 0 && slot < b->B, LLMRS_E_RANGE, "slot out of range");
    llmrs_model* m = b->m;
    LLMRS_REQUIRE(!m->sampling, LLMRS_E_INVALID, "batched decoding is greedy: clear the model's sampling first");
    LLMRS_REQUIRE(n_prompt < (size_t)m->c.max_seq, LLMRS_E_RANGE, "prompt beyond max_seq");
    // the prompt through the prefill kernels into the slot's cache, then the
    // lm_head and greedy step of its last row, on the model's own buffers
    upload_tokens(m, 0, prompt, n_prompt);
    set_state(m, 0, (int)n_prompt);
    std::vector<void*> kcs(b->kc.size()), vcs(b->vc.size());
    for (size_t li = 0; li < kcs.size(); ++li) {
      kcs[li] = (uint8_t*)b->kc[li] + (size_t)slot * b->kv_bytes;
      vcs[li] = (uint8_t*)b->vc[li] + (size_t)slot * b->kv_bytes;
    }
    run_prefill(m, 0, n_prompt, (int)n_prompt, false, nullptr, kcs.data(), vcs.data());
    m->begun = false;  // the model's own sequence state was used as scratch
    m->host_pos = n_prompt;
    hipStream_t s = ctx().stream;
    const int p = (int)n_prompt;
    LLMRS_HIP(hipMemcpyAsync(b->tokens + (size_t)slot * b->cap, m->tokens, (n_prompt + 1) * sizeof(int32_t),
                             hipMemcpyDeviceToDevice, s));
    LLMRS_HIP(hipMemcpyAsync(b->gen + (size_t)slot * b->cap, m->gen, (n_prompt + 1) * sizeof(int32_t),
                             hipMemcpyDeviceToDevice, s));
    LLMRS_HIP(hipMemcpyAsync(b->pos + slot, &p, sizeof(int), hipMemcpyHostToDevice, s));
    LLMRS_HIP(hipStreamSynchronize(s));
    check_err(m);
    b->host_pos[slot] = n_prompt;
    b->begun[slot] = 1;
  });
}

int llmrs_batch_decode_steps(llmrs_batch* b, size_t n) {
  return guard([&] {
    LLMRS_REQUIRE(b, LLMRS_E_INVALID, "null batch");
    for (int s = 0; s < b->B; ++s) {
      LLMRS_REQUIRE(b->begun[s], LLMRS_E_INVALID, "slot " + std::to_string(s) + " has not been begun");
      LLMRS_REQUIRE(b->host_pos[s] + n < (size_t)b->m->c.max_seq, LLMRS_E_RANGE,
                    "slot " + std::to_string(s) + " would decode beyond max_seq");
    }
    for (size_t i = 0; i < n; ++i) replay_batch_step(b);
    for (auto& p : b->host_pos) p += n;
  });
}

int llmrs_batch_tokens(llmrs_batch* b, int32_t slot, int32_t* out, size_t count) {
  return guard([&] {
    LLMRS_REQUIRE(b && out, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(slot >= 0 && slot < b->B, LLMRS_E_RANGE, "slot out of range");
    LLMRS_REQUIRE(count <= b->host_pos[slot] + 1, LLMRS_E_RANGE, "more tokens requested than produced");
    LLMRS_HIP(hipMemcpyAsync(out, b->tokens + (size_t)slot * b->cap, count * sizeof(int32_t),
                             hipMemcpyDeviceToHost, ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    check_err(b->m);
  });
}

int llmrs_batch_logits(llmrs_batch* b, float* out) {
  return guard([&] {
    LLMRS_REQUIRE(b && out, LLMRS_E_INVALID, "null argument");
    LLMRS_HIP(hipMemcpyAsync(out, b->logits, (size_t)b->B * b->m->c.vocab * sizeof(float), hipMemcpyDeviceToHost,
                             ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  });
}

int llmrs_batch_profile_step(llmrs_batch* b, char* names, float* ms, double* work, int cap) {
  int count = 0;
  const int rc = guard([&] {
    LLMRS_REQUIRE(b, LLMRS_E_INVALID, "null batch");
    for (int s = 0; s < b->B; ++s)
      LLMRS_REQUIRE(b->begun[s] && b->host_pos[s] + 1 < (size_t)b->m->c.max_seq, LLMRS_E_INVALID,
                    "every slot must be begun, with room for one more step");
    count = profile_launches([&](Launcher& L) { enqueue_batch_step(b, L); }, names, ms, work, cap);
    for (auto& p : b->host_pos) p += 1;
  });
  return rc ? rc : count;
}

}  // extern "C"
