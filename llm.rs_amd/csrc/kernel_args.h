// kernel_args.h - argument blocks of every gfx950 kernel.
//
// Included by the device code (csrc/kernels/*.hip) and by the host library
// (csrc/host/*.cpp), so the by-value kernel argument layout is defined once.
// Plain C structs: pointers, int32, float - identical layout on x86-64 and
// amdgcn.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace llmrs {

// Decode GEMV (gemv.hip).  Which fields are read depends on the prologue /
// epilogue variant encoded in the kernel name.
struct GemvArgs {
  const uint8_t* wq;     // weight codes [n][nb][B]
  const void* ws;        // weight scales [n][nb] (fp16 or f32)
  int n, k;              // rows, columns
  const float* x;        // [m][k] input rows (PRO_QUANT, PRO_NORM)
  const float* norm_w;   // [k] RMSNorm weight (PRO_NORM)
  float eps;
  const int8_t* xq;      // [k] activation codes (PRO_Q8, PRO_NQ: codes of x*w)
  const float* xd;       // [k/32] activation scales (PRO_Q8; PRO_NQ: d' before the RMSNorm factor)
  const float* xss;      // [k/32] per-block sums of x^2 (PRO_NQ)
  float* y;              // [m][n]; EPI_SILU: [n/2] (may be null); EPI_ARGMAX: logits (may be null)
  const float* res;      // [m][n] residual (EPI_RESID, EPI_NQ; may alias y)
  const float* norm_next;  // [n] weight of the RMSNorm the output feeds (EPI_NQ)
  int8_t* yq;            // EPI_SILU: [n/2] codes of silu(g)*u; EPI_NQ: [n] codes of y*norm_next
  float* yd;             // EPI_SILU: [n/64] scales; EPI_NQ: [n/32] d' = amax(y*norm_next)/127
  float* yss;            // [n/32] per-block sums of y^2 (EPI_NQ)
  float* part_val;       // [gridDim.x] (EPI_ARGMAX)
  int* part_idx;         // [gridDim.x] (EPI_ARGMAX)
  unsigned long long* ts;  // profiling: 4 stamps per workgroup (null = off)
  int8_t* probe_xq;      // [k] when set: workgroup 0 copies the Q8_0 activation codes of
  float* probe_xd;       // its prologue and [k/32] their scales here (test probes)
  // Row-batched launches (gemv_*_b): batch_rows activation rows (PRO_Q8 codes
  // [rows][k], scales [rows][k/32]; outputs at the row's stride) over
  // batch_nwg workgroups per row.
  int batch_rows, batch_nwg;
};

// Dynamic LDS of a decode GEMV (gemv_core.h): the quantised activation row
// (k codes, k/32 scales, k/32 Q4 offsets; 16-byte aligned), then the row
// results parked until the unit loop ends: per wave (4 per workgroup) R
// values of each of its row groups, or for a tiled epilogue (`tile` rows:
// 64 for SwiGLU, 32 for the residual + next-norm codes) `tile` values per
// tile of the workgroup.  nwg = workgroups of the launch.
constexpr size_t gemv_act_bytes(int k) { return (size_t)k + 8 * (size_t)(k / 32); }
constexpr size_t gemv_out_floats(int tile, int n, int r, int nwg, int waves = 4) {
  return tile ? (size_t)(((n + tile - 1) / tile + nwg - 1) / nwg) * tile
              : (size_t)((((size_t)n + r - 1) / r + (size_t)nwg * waves - 1) / ((size_t)nwg * waves)) * r * waves;
}
constexpr size_t gemv_lds_bytes(int tile, int n, int k, int r, int nwg, int waves = 4) {
  return (gemv_act_bytes(k) + 15) / 16 * 16 + 4 * gemv_out_floats(tile, n, r, nwg, waves);
}

// lm_head partial reduction + greedy bookkeeping (gemv.hip: argmax_final).
struct ArgmaxFinalArgs {
  const float* part_val;
  const int* part_idx;
  int nparts;
  int* pos;              // device position counter
  const int* n_prompt;
  int* tokens;           // [cap] input id per position
  int* gen;              // [cap] argmax produced at position p, stored at p+1
  int cap;
};

// Activation codes in the skinny GEMM's operand order (sgemm.hip).  Every
// run of 4 blocks (128 elements) is stored as [4 lane groups][4 blocks][8
// bytes]: lane group g's 8 bytes of a block are the elements its weight
// dword multiplies - dword g of a device Q4 block holds elements 4g..4g+3 in
// its low nibbles and 16+4g..16+4g+3 in its high ones (dwords g and g+4 of
// a Q8 block the same elements) - so elements 4g..4g+3, then 16+4g..16+4g+3.
// Aligned runs of 4 elements stay together.  Needs the row length a
// multiple of 128.
enum { kActNatural = 0, kActMfma = 1 };
constexpr int act_offset(int k, int layout) {
  return layout == kActNatural ? k
                               : ((k >> 5) >> 2) * 128 + ((k >> 5) & 3) * 8 + ((k & 31) >> 2 & 3) * 32 +
                                     ((k & 31) >> 4) * 4 + (k & 3);
}

// Skinny GEMM of batched decode (sgemm.hip): Y[t][n] = sum_b isum_b(t, n) *
// (d_w[n,b] * d_a[t,b]) over M <= 64 rows of Q8_0 activation codes (in the
// operand order of the weight type) and an [N, K] quantised weight.
struct SgemmArgs {
  const int8_t* xq;      // [M][K] activation codes, act_offset order
  const float* xd;       // [M][K/32] activation scales
  const uint8_t* wq;     // weight codes [N][nb][B]
  const void* ws;        // weight scales [N][nb]
  float* y;              // [M][ldy] (STORE, RESID)
  const float* res;      // [M][N] residual (RESID; may alias y)
  int8_t* yq;            // SILU: [M][N/2] codes of m, in the order `layout`
  float* yd;             // SILU: [M][N/64] scales of m
  int M, N, K, ldy, layout;
};

// Greedy step of a batch of sequences (gemv.hip: argmax_batch): row b of
// the logits, next = argmax (lowest index on ties), then sequence b's
// bookkeeping as argmax_final does for one sequence.
struct ArgmaxBatchArgs {
  const float* logits;   // [B][vocab]
  int vocab;
  int* pos;              // [B] device positions
  int* tokens;           // [B][cap]
  int* gen;              // [B][cap]
  int cap;
};

// Sampling of the next token (sample.hip): a chain of launches over
// workgroups of kSampleThreads threads, each owning kSampleSlice consecutive
// ids.  Vocabularies up to kSampleMaxVocab ids.
constexpr int kSampleMaxVocab = 262144;
constexpr int kSampleThreads = 256;
constexpr int kSamplePerThread = 2;
constexpr int kSampleSlice = kSampleThreads * kSamplePerThread;
constexpr int kSampleMaxGroups = kSampleMaxVocab / kSampleSlice;
// First-level bins: bits 30..20 of a probability's pattern, plus one bin for
// the part of 1e-5's bin below the candidate threshold; refine levels: bits
// 19..10, then 9..0 inside the selected bin.
constexpr int kSampleL1Bins = 2049;
constexpr int kSampleRBins = 1024;
constexpr int kSampleRefines = 4;  // two levels for the top-p cut, two for the draw
constexpr int sample_groups(int vocab) { return (vocab + kSampleSlice - 1) / kSampleSlice; }

// Device state of one sampler, zero before its first use; every launch
// leaves the counters and histograms it consumed at zero again.
struct SampleState {
  unsigned ticket[4];            // last-workgroup tickets: prep, probs, refine, pick
  float M, S;                    // softmax max and sum
  int mode;                      // selection in progress: 0 none, 1 the top-p cut, 2 the draw
  int level;                     // next refine level (1 or 2)
  int bin1;                      // first-level bin of the selection
  unsigned digit2;               // its second-level digit, once known
  int cut_rank;                  // first-level rank of the cut bin (-1: no cut)
  int pick;                      // workgroup holding the drawn id (-1: none, id 0)
  unsigned vcut, ktie, vsel, ksel;
  unsigned long long target, above, cut_base, cut_above, total, r, pick_base;
  float wg_max[kSampleMaxGroups], wg_sum[kSampleMaxGroups];
  unsigned long long wg_fix[kSampleMaxGroups];
  unsigned l1_n[kSampleL1Bins + 3];
  unsigned long long l1_s[kSampleL1Bins + 3];
  unsigned r_n[kSampleRBins];
  unsigned long long r_s[kSampleRBins];
};

struct SampleArgs {
  const float* logits;   // [vocab] of the step
  float* probs;          // [vocab] scratch
  SampleState* st;
  int vocab, groups;     // groups = sample_groups(vocab)
  int* pos;              // device position (null: probe, no bookkeeping)
  const int* n_prompt;
  int* tokens;           // [cap] ids per position (the penalty history)
  int* gen;              // [cap] drawn id at position p, stored at p+1
  int cap;
  const int* eos;        // end-of-sequence ids
  int n_eos;
  int* stopped;          // set once one is drawn (null: probe)
  float penalty, temperature, top_p;
  int window;            // penalty window (<= 0: the whole history)
  unsigned long long seed;
  long long step_override;  // >= 0: the draw's position (probe), else *pos
  const int* hist;       // probe: explicit history [n_hist] (null: tokens[0..pos])
  int n_hist;
  int* out_token;        // probe outputs (may be null)
  float* out_u;
};

// Decode attention (attention.hip).
struct AttnArgs {
  const float* qkv;        // [nq*hd | nkv*hd | nkv*hd] projections of this token
  const int* pos_ptr;      // device position (the new token's index)
  void* kc;                // this layer's K cache [nkv][max_seq][hd]
  void* vc;                // this layer's V cache [nkv][max_seq rows] (v_offset)
  const float* rope_cos;   // [max_seq][hd/2]
  const float* rope_sin;
  float* part_o;           // [nq][nsplit][hd]
  float* part_ml;          // [nq][ml_stride(nsplit)][2]
  int* counters;           // [nkv][kTicketStride] tickets, zero between launches
  float* ctx;              // [nq*hd]
  int8_t* ctx_q;           // [nq*hd]
  float* ctx_d;            // [nq*hd/32]
  int max_seq, nq, nkv, nsplit;  // max_seq: cache rows per KV head (kv_rows)
  float scale;             // fl(1 / fl(sqrt(hd))), layer.rs:258
  // [hd/2] cos then [hd/2] sin at the step's position, copied from the tables
  // by embed_gather (matrix-core kernel; per sequence: + z * hd)
  const float* rope_now;
  unsigned long long* ts;  // profiling: 8 stage timestamps per item (null = off)
  // Batched decode (grid.z = sequences): sequence z's qkv, position, partials,
  // tickets and ctx rows follow sequence 0's at their natural strides, its
  // K and V caches kv_batch_bytes after sequence 0's; ctx_q in the skinny
  // GEMM's operand order ctx_layout (act_offset within the row).
  size_t kv_batch_bytes;
  int ctx_layout;
};

// Elementwise trait operators (ops.hip).
struct EwArgs {
  float* a;          // in/out
  const float* b;    // second operand
  float* out;        // output (scale)
  float value;       // scale factor
  long n;
};

struct RopeArgs {
  float* x;              // [rows][hd]
  const float* cos_t;    // [rows][hd/2] for positions start_pos + row
  const float* sin_t;
  int rows, hd;
};

struct RowArgs {
  const float* x;
  const float* w;
  float* out;
  int rows, dim;
  float eps;
};

struct MatArgs {
  const float* a;   // [m][k]
  const float* b;   // matmul: [k][n]; matmul_t: [n][k]
  float* out;       // [m][n]
  int m, k, n;
};

struct EmbedArgs {
  const float* table;   // [vocab][hidden]
  const int* tokens;    // [cap]
  const int* pos_ptr;
  float* x;             // [hidden]
  int* err;             // set to 1 on an out-of-range id
  int hidden, vocab;
  // One row only: when norm_w is set, the first RMSNorm's operand of the
  // row (the PRO_NQ prologue of gemv_core.h): Q8_0 codes of x*w, d' =
  // amax/127 and the sum of x^2 per 32-element block.  x_in set: the row is
  // x_in (copied to x) instead of an embedding.
  const float* norm_w;
  int8_t* xq;
  float* xd;
  float* xss;
  const float* x_in;
  // Batched decode (> 0): row y is sequence y, token tokens[y * batch_stride
  // + pos_ptr[y]]; 0: row y of a chunk, token tokens[*pos_ptr + y].
  int batch_stride;
  // Decode steps: the RoPE row of the position (of sequence y: at y * 2 * rope_mid)
  // copied to rope_now, so that the attention reads it without waiting for
  // the position; null: none.
  const float* rope_cos;
  const float* rope_sin;
  float* rope_now;
  int rope_mid, rope_rows;
};

// Prefill GEMM (prefill.hip): Y[t][r] = sum_b isum_b(t, r) * (d_w[r,b] * d_a[t,b])
// over M token rows of Q8_0 activation codes and an [N, K] quantised weight.
struct PrefillGemmArgs {
  const int8_t* xq;      // [M][K] activation codes
  const float* xd;       // [M][K/32] activation scales
  const uint8_t* wq;     // weight codes [N][nb][B]
  const void* ws;        // weight scales [N][nb]
  float* y;              // [M][ldy]: GEMM out (STORE, RESID) or m (SILU, may be null)
  const float* res;      // [M][N] residual (RESID; may alias y)
  int8_t* yq;            // SILU: [M][N/2] codes of m
  float* yd;             // SILU: [M][N/64] scales of m
  int M, N, K, ldy;
  // Tile order (0 = row-major).  Workgroups reach the 8 XCDs round-robin in
  // dispatch order; with group_m > 0 and a tile count divisible by 8, XCD x
  // takes the x-th contiguous eighth of the tiles, walked group_m token tiles
  // at a time, so the workgroups resident on one XCD share operand panels
  // in its L2.
  int group_m;
};

// Dynamic LDS of the prefill GEMM: two pipeline stages of 4 blocks, each
// activation and weight codes (int8) 2 x 128 x 128 B, f32 scales 2 x 4 x 132.
constexpr size_t gemm_lds_bytes() {
  return 2 * ((size_t)2 * 4 * 128 * 16 * 2 + (size_t)4 * 132 * 4 * 2);
}

// Prefill row kernels (prefill.hip).
struct PrefillRowArgs {
  const float* x;        // [M][dim] input rows
  const float* w;        // [dim] RMSNorm weight (null: plain Q8_0)
  int8_t* xq;            // [M][dim] codes (act_offset order `layout` within a row)
  float* xd;             // [M][dim/32] scales
  int M, dim;
  float eps;
  int layout;
};

// RoPE of the projections and K/V append for positions start_pos + t.
struct PrefillRopeArgs {
  const float* qkv;      // [M][qkv_rows] projections
  float* q;              // [M][nq*hd] rotated queries
  void* kc;              // layer K cache [nkv][max_seq][hd]
  void* vc;              // layer V cache
  const float* rope_cos; // [max_seq][hd/2]
  const float* rope_sin;
  int M, nq, nkv, hd, max_seq, start_pos, qkv_rows, kv16;
};

// Causal prefill attention: query rows t at positions start_pos + t attend to
// cache positions [0, start_pos + t].
struct PrefillAttnArgs {
  const float* q;        // [M][nq*hd] rotated queries
  const void* kc;        // layer K cache [nkv][max_seq][hd]
  const void* vc;
  float* ctx;            // [M][nq*hd] (may be null)
  int8_t* ctx_q;         // [M][nq*hd] Q8_0 codes of ctx
  float* ctx_d;          // [M][nq*hd/32]
  int M, nq, nkv, max_seq, start_pos;
  float scale;           // fl(1 / fl(sqrt(hd)))
  int ctx_layout;        // operand order of ctx_q within a row (act_offset)
};

// ints between the split tickets of two KV heads: each head's counter has a
// 256-byte line of its own, so the heads' atomics do not queue on one line.
constexpr int kTicketStride = 64;
// Reference-order decode kernels (exact.hip).
// One workgroup per row (grid.x rows, row r at offset r * n).
struct ExactNormArgs {
  const float* x;        // [rows][n] input rows
  const float* w;        // [n] RMSNorm weight
  int8_t* xq;            // [rows][n] Q8_0 codes of the normed rows (act_offset order `layout`)
  float* xd;             // [rows][n/32] their scales
  float* y;              // [rows][n] the normed rows (may be null)
  int n;
  float eps;
  int layout;
};

struct ExactGemvArgs {
  const uint8_t* wq;     // weight codes [n][nb][B]
  const void* ws;        // weight scales [n][nb]
  const int8_t* xq;      // [k] activation codes
  const float* xd;       // [k/32] activation scales
  float* y;              // [n] (may be null for the argmax epilogue; silu: [n/2] m as f32, may be null)
  const float* res;      // [n] residual (resid epilogue; may alias y)
  float* part_val;       // [gridDim.x] (argmax epilogue)
  int* part_idx;
  int n, k;
  int8_t* mq;            // silu epilogue: [n/2] Q8_0 codes of m = silu(g) * u
  float* md;             // [n/64]
};

struct ExactAttnArgs {
  const float* qkv;      // [nq*hd | nkv*hd | nkv*hd] projections of this token
  const int* pos_ptr;    // device position
  void* kc;              // layer K cache [nkv][max_seq][hd]
  void* vc;              // layer V cache (v_offset)
  const float* rope_cos; // [positions][hd/2]
  const float* rope_sin;
  float* ctx;            // [nq*hd]
  int8_t* ctx_q;         // [nq*hd]
  float* ctx_d;          // [nq*hd/32]
  int max_seq, nq, nkv;  // max_seq: cache rows per KV head (kv_rows)
  float scale;           // fl(1 / fl(sqrt(hd)))
};

// Positions per decode-attention tile (attn_core.h, attn_mfma.h).
constexpr int kAttnTile = 32;
constexpr int attn_tile(bool) { return kAttnTile; }
// Splits of one matrix-core decode-attention launch at most (its combine
// holds split s's (max, sum) in lane s of a wave).
constexpr int kMfmaAttnMaxSplits = 64;
// (max, sum) pairs per query head in the decode-attention partials: the
// split count rounded up to even, so the matrix-core combine reads them two
// per 16-byte load.
constexpr int ml_stride(int nsplit) { return (nsplit + 1) & ~1; }
// Positions allocated per KV head in a layer's cache: max_seq rounded up to
// whole tiles, so a tile load never leaves the buffer.
constexpr int kv_rows(int max_seq) { return (max_seq + kAttnTile - 1) / kAttnTile * kAttnTile; }
// Element offset of (position p, dim d) in one KV head's rows.  K, and a V
// cache in f32, are row-major [p][hd]; a V cache in f16 is blocked and
// transposed, [p/8][hd][p%8]: the 8 positions of a block are 16 contiguous
// bytes per dim, one matrix-core operand (attn_mfma.h).
constexpr size_t v_offset(size_t p, int d, int hd, bool f16) {
  return f16 ? ((p / 8) * (size_t)hd + (size_t)d) * 8 + p % 8 : p * (size_t)hd + (size_t)d;
}

// LDS bytes of one vector-ALU decode-attention work item (attn_core.h, f32
// caches: query heads, per stream a padded K tile and a V tile, the new row,
// the ticket); at most 8 query heads per KV head; `streams` tile streams per
// workgroup.
constexpr size_t attn_lds_bytes(int hd, bool kv16, int streams = 1) {
  const size_t es = kv16 ? 2 : 4, tile = (size_t)kAttnTile, kstride = (size_t)hd + (kv16 ? 2 : 1);
  const size_t kb = (es * tile * kstride + 15) / 16 * 16;
  const size_t stream = kb + es * tile * (size_t)hd;
  return 4 * 8 * (size_t)hd + (size_t)streams * stream + 4 * 2 * (size_t)hd + 16;
}

}  // namespace llmrs
