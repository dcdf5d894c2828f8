/*
 * oracle.h - CPU restatement of the llm.rs reference CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing on the product path (the llmrs_hip
 * library, its kernels, bench.py's GPU leg) may include, link or call this.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * as the parity reference of the tests and as the timed CPU baseline.
 *
 * Every function follows a reference file:line (paths relative to the
 * reference root), stated at its definition in oracle.cpp.  Floating-point
 * order follows the reference exactly: this file is compiled with
 * -ffp-contract=off (Rust never fuses a*b+c), glibc libm supplies
 * expf/powf/sinf/cosf/sqrtf, roundf is ties-away like Rust's f32::round.
 *
 * How each part is pinned (tests/test_oracle.py):
 *   quantize_row_q8_0   closed form per block + brute force (amax=0, ties,
 *                       clamp) in numpy.
 *   Q4 format / GEMV    integer block sums vs numpy int64 brute force, and vs
 *                       a float64 dot over dequantised weights
 *                       (test/opencl.rs:237-258 tolerance 1e-3).
 *   rms_norm            KAT test/cpu.rs:197-212 + float64 closed form.
 *   rope                KAT test/cpu.rs:229-245 + rotation invariants.
 *   softmax             KAT test/cpu.rs:214-227 + float64 closed form.
 *   attention / KV      layer.rs:430-489 (causality, KV update) + float64
 *                       brute force; GQA row duplication == true GQA.
 *   model / token loop  batched prefill == sequential decode (bit-exact,
 *                       a property of the reference's arithmetic), layer
 *                       composition vs a numpy float64 restatement.
 * Parity unpinned at the bit level: expf/powf/sinf/cosf come from the host
 * glibc, as in the reference; no reference test pins them beyond 1e-5.
 */
#ifndef LLMRS_ORACLE_H
#define LLMRS_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_set_threads(int n);
int orc_get_threads(void);
/* Test-only: which build of the reference the arithmetic restates, 0 = x86-64
 * (default), 1 = aarch64 (NEON orders of cpu.rs:461-544,558-619,747-886). */
void orc_set_arch(int arch);
int orc_get_arch(void);
/* Test-only: attention scores, softmax and P.V summed in float64 (on != 0),
 * the rest of the reference arithmetic unchanged. */
void orc_set_attn_f64(int on);
/* Test-only: record every Q8_0 code produced (on != 0 clears the record);
 * orc_recorded_codes copies up to `cap` of them and returns the count. */
void orc_record_codes(int on);
int64_t orc_recorded_codes(int8_t* out, int64_t cap);
/* Test-only: while `codes` is set (null stops), quantize_row_q8_0 takes its
 * codes from it in call order instead of its own rounding - so a forward
 * pass can be replayed with another implementation's activation codes - and
 * checks each taken code against its own: a differing code must be one step
 * away with the product x*inv within `tol` (code units) of the rounding
 * midpoint between the two.  orc_injected_stats reports codes taken,
 * codes that differ, differing codes failing that check, and the largest
 * midpoint distance of a differing code. */
void orc_inject_codes(const int8_t* codes, int64_t n, float tol);
void orc_injected_stats(int64_t* taken, int64_t* differ, int64_t* bad, float* max_dist);

/* ---- cpu.rs primitives -------------------------------------------------- */
void orc_quantize_row_q8_0(const float* x, int64_t k, int8_t* q, float* d);
void orc_quantize_q4(const float* x, int64_t count, uint8_t* qs, float* scales);
void orc_dequantize_q4(const uint8_t* qs, const float* scales, int64_t count,
                       float* out);
int32_t orc_q4_block_isum(const uint8_t* q4, const int8_t* a);
int32_t orc_q4_block_isum_scalar(const uint8_t* q4, const int8_t* a);
void orc_matmul_transposed_q4(const float* a, int64_t m, int64_t k,
                              const uint8_t* qs, const float* scales,
                              int64_t n, float* out);
void orc_matmul_transposed_q8w(const float* a, int64_t m, int64_t k,
                               const int8_t* qs, const float* scales,
                               int64_t n, float* out);
void orc_matmul_transposed_f32(const float* a, int64_t m, int64_t k,
                               const float* b, int64_t n, float* out);
void orc_matmul(const float* a, int64_t m, int64_t k, const float* b,
                int64_t n, float* out);
void orc_matmul_slice(const float* a, int64_t m, int64_t k,
                      const float* other, int64_t rows, float* out);
void orc_add_assign(float* a, const float* b, int64_t n);
void orc_silu_mul(float* gate, const float* up, int64_t n);
/* f32::exp as the reference calls it (host libm expf), element-wise. */
void orc_expf(const float* x, int64_t n, float* out);
void orc_rope_inplace(float* x, int64_t count, int64_t head_dim,
                      int64_t start_pos);
void orc_rms_norm(const float* x, int64_t rows, int64_t dim, const float* w,
                  float eps, float* out);
void orc_softmax(const float* x, int64_t rows, int64_t dim, float* out);
void orc_scale(const float* x, int64_t n, float value, float* out);
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
int64_t orc_argmax(const float* x, int64_t n, float* margin);

/* ---- model (layer.rs / model.rs / main.rs) ------------------------------ */
typedef struct {
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
  float rms_eps, rope_theta;
  int32_t weight_dtype; /* 2 = Q4 (f32 scales), 3 = Q4_0, 4 = Q8_0 */
  int32_t kv_dtype;     /* 0 = f32, 1 = f16 */
} orc_config;

typedef struct orc_model orc_model;
orc_model* orc_model_create(const orc_config* cfg);
void orc_model_free(orc_model* m);
/* Weights are borrowed: the caller keeps the arrays alive. */
int orc_model_set_embedding(orc_model* m, const float* table);
int orc_model_set_norm(orc_model* m, int layer, int slot, const float* w);
int orc_model_set_linear_q4(orc_model* m, int layer, int slot,
                            const uint8_t* qs, const float* scales);
int orc_model_set_linear_q8(orc_model* m, int layer, int slot,
                            const int8_t* qs, const float* scales);
int orc_model_kv_write(orc_model* m, int layer, int kv_head, int64_t pos0,
                       int64_t n, const float* k, const float* v);
int orc_model_kv_read(orc_model* m, int layer, int kv_head, int64_t pos0,
                      int64_t n, float* k, float* v);
/* LlamaModel::forward over `n` tokens at start_pos, batched like the
 * reference prefill.  logits: [n][vocab] if all_rows else [vocab] (last
 * row); trace: [n][n_layers+1][hidden] or NULL. */
int orc_model_forward(orc_model* m, const int32_t* tokens, int64_t n,
                      int64_t start_pos, float* logits, int all_rows,
                      float* trace);
/* Test probes: the block loop over already-quantised activation rows
 * (xq [m][k], xd [m][k/32]) with Q4 (q8w = 0) or Q8 weight codes; and the
 * attention of one layer given the Q|K|V projections of `seq` rows. */
void orc_gemv_codes(const int8_t* xq, const float* xd, int64_t m, int64_t k, const void* w,
                    const float* scales, int64_t n, int q8w, float* out);
int orc_model_attention(orc_model* m, int layer, const float* qkv, int64_t seq,
                        int64_t start_pos, float* ctx);
/* The token loop's sampling (main.rs:192-305) for the draw u in [0, 1):
 * returns the id; with candidate >= 0, *accept = 1 when the candidate id is
 * this one or within the rounding of the reference's f32 running sums. */
int32_t orc_sample(const float* logits, int64_t vocab, const int32_t* hist, int64_t n_hist,
                   float penalty, float temperature, float top_p, int64_t window, float u,
                   int32_t candidate, int32_t* accept);
/* Greedy token loop (main.rs:128-327 with argmax).  out: n_steps ids;
 * margins: top1-top2 logit gap per step (may be NULL). */
int orc_model_generate(orc_model* m, const int32_t* prompt, int64_t n_prompt,
                       int64_t n_steps, int32_t* out, float* margins);

#ifdef __cplusplus
}
#endif
#endif
