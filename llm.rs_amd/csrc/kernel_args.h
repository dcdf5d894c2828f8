// kernel_args.h - argument blocks of every gfx950 kernel.
//
// Included by the device code (csrc/kernels/*.hip) and by the host library
// (csrc/host/*.cpp), so the by-value kernel argument layout is defined once.
// Plain C structs: pointers, int32, float - identical layout on x86-64 and
// amdgcn.
#pragma once
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
  const int8_t* xq;      // [k] activation codes (PRO_Q8)
  const float* xd;       // [k/32] activation scales (PRO_Q8)
  float* y;              // [m][n]; EPI_SILU: [n/2] (may be null); EPI_ARGMAX: logits (may be null)
  const float* res;      // [m][n] residual (EPI_RESID; may alias y)
  int8_t* yq;            // [n/2] codes of silu(g)*u (EPI_SILU)
  float* yd;             // [n/64] scales of silu(g)*u (EPI_SILU)
  float* part_val;       // [gridDim.x] (EPI_ARGMAX)
  int* part_idx;         // [gridDim.x] (EPI_ARGMAX)
};

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

// Decode attention (attention.hip).
struct AttnArgs {
  const float* qkv;        // [nq*hd | nkv*hd | nkv*hd] projections of this token
  const int* pos_ptr;      // device position (the new token's index)
  void* kc;                // this layer's K cache [nkv][max_seq][hd]
  void* vc;                // this layer's V cache [nkv][max_seq][hd]
  const float* rope_cos;   // [max_seq][hd/2]
  const float* rope_sin;
  float* part_o;           // [nq][nsplit][hd]
  float* part_ml;          // [nq][nsplit][2]
  int* counters;           // [nkv] tickets, zero between launches
  float* ctx;              // [nq*hd]
  int8_t* ctx_q;           // [nq*hd]
  float* ctx_d;            // [nq*hd/32]
  int max_seq, nq, nkv, nsplit;
  float scale;             // fl(1 / fl(sqrt(hd))), layer.rs:258
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
};

}  // namespace llmrs
