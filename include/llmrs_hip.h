/*
 * llmrs_hip.h - C ABI of the MI355X (gfx950) backend for llm.rs.
 *
 * This is the drop-in boundary.  The first group of entry points mirrors the
 * reference's operator plug-in interface, `trait Backend`
 * (src/backend.rs:15-40), one export per trait method, with the same argument
 * meaning.  The second group has no trait counterpart: it keeps the whole
 * decode loop resident in HBM (KV cache, attention, embedding gather, greedy
 * argmax, whole-step graph replay), because the reference's layer code reads
 * device tensors on the host (src/core/layer.rs:41,166,191-195,219-246;
 * src/main.rs:163), which only works on the mapped shared memory of a mobile
 * SoC.
 *
 * Conventions
 *  - Every function returns 0 on success or a negative LLMRS_E_* code.  The
 *    message of the last failure on the calling thread is returned by
 *    llmrs_last_error().  The reference panics instead (cpu.rs:37,46;
 *    Cargo.toml:60 panic="abort"); a Rust shim maps non-zero to panic!.
 *  - Tensors are opaque handles owned by the caller until llmrs_tensor_free
 *    (the reference's Arc<Storage> drop, src/core/tensor.rs:50-57).  Ops that
 *    return a tensor allocate it (like cpu.rs:150, opencl.rs:307).
 *  - All work runs on one HIP stream in issue order; host visibility is at
 *    llmrs_tensor_download / llmrs_sync / model calls that return host data,
 *    which matches the reference's synchronous op semantics
 *    (opencl.rs:290,389: queue.finish()).
 *  - Exports are serialised by one internal mutex, so calls from several host
 *    threads (rayon workers in the reference) are safe.
 *  - No torch types and no HIP types appear here: plain pointers and sizes.
 */
#ifndef LLMRS_HIP_H
#define LLMRS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes -------------------------------------------------------- */
#define LLMRS_OK 0
#define LLMRS_E_INVALID (-1)    /* bad argument / shape mismatch (cpu.rs:37) */
#define LLMRS_E_DTYPE (-2)      /* wrong storage kind for the op (cpu.rs:46) */
#define LLMRS_E_HIP (-3)        /* a HIP runtime call failed */
#define LLMRS_E_NOINIT (-4)     /* llmrs_init not called / failed */
#define LLMRS_E_MODULE (-5)     /* hsaco missing or kernel not found */
#define LLMRS_E_RANGE (-6)      /* position beyond max_seq, id beyond vocab */
#define LLMRS_E_OOM (-7)        /* device allocation failed */
#define LLMRS_E_FORMAT (-8)     /* unreadable or unsupported weight file */

/* ---- devices (src/backend.rs:7-12 plus the new Hip variant) ------------- */
#define LLMRS_DEVICE_CPU 0
#define LLMRS_DEVICE_OPENCL 1
#define LLMRS_DEVICE_QNN 2
#define LLMRS_DEVICE_HIP 3

/* ---- storage kinds (src/core/tensor.rs:13-44 plus extensions) ----------- */
#define LLMRS_F32 0   /* Storage::Cpu / Storage::Shared                      */
#define LLMRS_F16 1   /* KV cache only (extension)                           */
#define LLMRS_Q4 2    /* Storage::CpuQ4: 4-bit codes, f32 scale per 32 block */
#define LLMRS_Q4_0 3  /* Q4_0: 4-bit codes, fp16 scale per 32 block          */
#define LLMRS_Q8_0 4  /* Q8_0: int8 codes, fp16 scale per 32 block (ext.)    */

typedef struct llmrs_tensor llmrs_tensor;
typedef struct llmrs_model llmrs_model;

/* ---- context ------------------------------------------------------------ */
/* Select the HIP device, create the stream, hipModuleLoad every hsaco in
 * `hsaco_dir` (NULL = the directory of this shared library).  Replaces the
 * OpenCL context bring-up cl_context() (src/backend/opencl.rs:11-34). */
int llmrs_init(int device_ordinal, const char* hsaco_dir);
int llmrs_shutdown(void);
const char* llmrs_last_error(void);
/* Backend::device (src/backend.rs:17): always LLMRS_DEVICE_HIP. */
int llmrs_device(void);
/* Backend::name (src/backend.rs:18). */
const char* llmrs_name(void);
/* Wait for all queued work (the reference's queue.finish()). */
int llmrs_sync(void);
/* Number of compute units of the current device (0 before init). */
int llmrs_num_cus(void);

/* ---- tensors (Tensor::new / to_device / data / drop) -------------------- */
/* Cpu -> device upload of an f32 tensor (tensor.rs:232-253). */
int llmrs_tensor_upload_f32(const float* data, const size_t* dims, int ndim,
                            llmrs_tensor** out);
/* CpuQ4 -> device (tensor.rs:255-281).  `qs` is the reference's planar
 * nibble array [n][k/2] (byte i of a block = e[2i] | e[2i+1] << 4,
 * tensor.rs:125-131) and `scales` its f32 array [n][k/32].  The device copy
 * keeps fp16 scales when every scale is exactly representable in fp16, else
 * f32 scales; codes and scales are bit-preserved either way. */
int llmrs_tensor_upload_q4(const uint8_t* qs, const float* scales, size_t n,
                           size_t k, llmrs_tensor** out);
/* Q8_0 weights (extension): int8 codes [n][k], f32 scales [n][k/32] that are
 * exactly representable in fp16. */
int llmrs_tensor_upload_q8_0(const int8_t* qs, const float* scales, size_t n,
                             size_t k, llmrs_tensor** out);
int llmrs_tensor_zeros(const size_t* dims, int ndim, llmrs_tensor** out);
/* Tensor::data() / to_device(Cpu) for f32 tensors: copies `count` floats. */
int llmrs_tensor_download(const llmrs_tensor* t, float* out, size_t count);
int llmrs_tensor_ndim(const llmrs_tensor* t);
int llmrs_tensor_dims(const llmrs_tensor* t, size_t* dims);
int llmrs_tensor_dtype(const llmrs_tensor* t);
int llmrs_tensor_free(llmrs_tensor* t);

/* ---- trait Backend mirror (src/backend.rs:21-39) ------------------------ */
/* Backend::matmul (backend.rs:21): a[m,k] @ b[k,n], f32. */
int llmrs_matmul(const llmrs_tensor* a, const llmrs_tensor* b,
                 llmrs_tensor** out);
/* Backend::matmul_transposed (backend.rs:24): a[m,k] @ b[n,k]^T.  b is f32,
 * Q4, Q4_0 or Q8_0; for quantised b each row of a is first quantised to Q8_0
 * (cpu.rs:76-110, quantize_row_q8_0 cpu.rs:663-745). */
int llmrs_matmul_transposed(const llmrs_tensor* a, const llmrs_tensor* b,
                            llmrs_tensor** out);
/* Backend::matmul_slice (backend.rs:28): a[m,cols] @ other[rows,cols]^T,
 * `other_data` is a host slice that is uploaded (opencl.rs:396-419). */
int llmrs_matmul_slice(const llmrs_tensor* a, const float* other_data,
                       size_t rows, size_t cols, llmrs_tensor** out);
/* Backend::add_assign (backend.rs:31): a += b. */
int llmrs_add_assign(llmrs_tensor* a, const llmrs_tensor* b);
/* Backend::silu_mul (backend.rs:32): gate = gate/(1+exp(-gate)) * up. */
int llmrs_silu_mul(llmrs_tensor* gate, const llmrs_tensor* up);
/* Backend::rope_inplace (backend.rs:33): rotate-half RoPE, theta 500000,
 * rows of size dims[last] at positions start_pos + row (cpu.rs:326-357). */
int llmrs_rope_inplace(llmrs_tensor* x, size_t start_pos);
/* Backend::rms_norm (backend.rs:36). */
int llmrs_rms_norm(const llmrs_tensor* x, const llmrs_tensor* weight,
                   float eps, llmrs_tensor** out);
/* Backend::softmax (backend.rs:37), over the last dimension. */
int llmrs_softmax(const llmrs_tensor* x, llmrs_tensor** out);
/* Backend::scale (backend.rs:38). */
int llmrs_scale(const llmrs_tensor* x, float value, llmrs_tensor** out);
/* Backend::copy_from (backend.rs:39). */
int llmrs_copy_from(const llmrs_tensor* t, llmrs_tensor** out);
/* No counterpart in the reference: a self-check of the device arithmetic the
 * reference-order attention relies on.  For every f16 pattern h (both halves
 * of a word) and every value a of the f32 tensor x, the one-instruction
 * product (mixed-precision FMA with an addend of -0) is compared in bits with
 * a * (float)h; *out = an f32 tensor [65536] of mismatch counts per pattern
 * (NaN against NaN counts as equal).  All zero on a correct device. */
int llmrs_check_mul_f16(const llmrs_tensor* x, llmrs_tensor** out);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the product of llmrs_matmul_transposed written into `out`,
 * an f32 tensor of shape [m, n] the caller allocated beforehand, with no
 * device allocation.  Quantised b with m > 1 stages each row's Q8_0 codes in
 * a fixed per-device scratch of 16 MiB: m*k + 4*m*k/32 bytes must fit
 * (else LLMRS_E_RANGE).  Calls that overlap on one device race on that
 * scratch.  Results equal llmrs_matmul_transposed's. */
int llmrs_matmul_transposed_noalloc(const llmrs_tensor* a, const llmrs_tensor* b,
                                    llmrs_tensor* out);

/* Test probe (no reference counterpart): the device exponential used by
 * SiLU and softmax on n host values, out[i] = expf(x[i]) as the reference's
 * host libm (glibc) computes it, bit for bit. */
int llmrs_probe_expf(const float* x, size_t n, float* out);

/* ---- resident decode model (no trait counterpart) ----------------------- */
/* Mirrors LlamaConfig (src/core/config.rs:3-17) plus what the reference
 * hard-codes: head_dim (loader.rs:164 derives hidden/num_heads), max_seq
 * (loader.rs:165 fixes 2048), and the weight / KV storage kinds. */
typedef struct {
  int32_t n_layers;     /* num_hidden_layers   */
  int32_t hidden;       /* hidden_size         */
  int32_t n_heads;      /* num_attention_heads */
  int32_t n_kv_heads;   /* num_key_value_heads */
  int32_t head_dim;     /* hidden / n_heads in the reference */
  int32_t ffn;          /* intermediate_size   */
  int32_t vocab;        /* vocab_size          */
  int32_t max_seq;      /* KV capacity in positions */
  float rms_eps;        /* rms_norm_eps        */
  float rope_theta;     /* 500000 (hard-coded at cpu.rs:330) */
  int32_t weight_dtype; /* LLMRS_Q4 | LLMRS_Q4_0 | LLMRS_Q8_0 */
  int32_t kv_dtype;     /* LLMRS_F32 | LLMRS_F16 */
} llmrs_model_config;

/* Linear weight slots of one layer (loader.rs:113-150); LM_HEAD uses
 * layer = -1 (loader.rs:186-190). */
#define LLMRS_W_Q 0
#define LLMRS_W_K 1
#define LLMRS_W_V 2
#define LLMRS_W_O 3
#define LLMRS_W_GATE 4
#define LLMRS_W_UP 5
#define LLMRS_W_DOWN 6
#define LLMRS_W_LM_HEAD 7
/* Norm slots (loader.rs:153-159,183); FINAL uses layer = -1. */
#define LLMRS_N_INPUT 0
#define LLMRS_N_POST 1
#define LLMRS_N_FINAL 2

int llmrs_model_create(const llmrs_model_config* cfg, llmrs_model** out);
/* Frees the model; LLMRS_E_INVALID while batches created on it
 * (llmrs_batch_create) are alive, which hold its weights and must be freed
 * first. */
int llmrs_model_free(llmrs_model* m);
/* The configuration a model was created with (e.g. by a loader). */
int llmrs_model_get_config(const llmrs_model* m, llmrs_model_config* out);
/* embed_tokens (loader.rs:105): f32 [vocab][hidden]. */
int llmrs_model_set_embedding(llmrs_model* m, const float* table);
int llmrs_model_set_norm(llmrs_model* m, int layer, int slot, const float* w);
/* A linear weight in the reference CpuQ4 format (see llmrs_tensor_upload_q4)
 * for weight_dtype LLMRS_Q4 / LLMRS_Q4_0.  K/V take true-GQA shapes
 * [n_kv_heads*head_dim][hidden]; the reference duplicates those rows
 * (loader.rs:62-98), which gives bit-identical outputs per query head. */
int llmrs_model_set_linear_q4(llmrs_model* m, int layer, int slot,
                              const uint8_t* qs, const float* scales);
/* A linear weight in Q8_0 (weight_dtype LLMRS_Q8_0): int8 [n][k] + scales. */
int llmrs_model_set_linear_q8_0(llmrs_model* m, int layer, int slot,
                                const int8_t* qs, const float* scales);
/* Loading a model from weight files (Loader::load_model, loader.rs:100-198).
 * max_seq <= 0 takes the reference's 2048 positions (KVCache::new,
 * loader.rs:162-166); weight_dtype 0 takes the file's own (else it must
 * match); a NULL options pointer means {2048, LLMRS_F16, 0}. */
typedef struct {
  int32_t max_seq;
  int32_t kv_dtype;     /* LLMRS_F16 | LLMRS_F32 */
  int32_t weight_dtype; /* 0 | LLMRS_Q4 | LLMRS_Q4_0 | LLMRS_Q8_0 */
} llmrs_load_options;
/* A Hugging Face checkpoint: `path` is a directory holding config.json and
 * model.safetensors (or model.safetensors.index.json with its shards), or
 * a .safetensors file with config.json beside it.  F32/BF16 tensors (F16
 * too); every linear weight quantised with Tensor::quantize_q4
 * (tensor.rs:102-167) into LLMRS_Q4; lm_head, or the tied embedding when
 * the checkpoint has none (loader.rs:186-190).  Replaces Loader::new +
 * Loader::load_model (loader.rs:19-23,100-198). */
int llmrs_model_load_safetensors(const char* path, const llmrs_load_options* opt,
                                 llmrs_model** out);
/* A GGUF file of the llama architecture (no reference counterpart): Q4_0
 * and Q8_0 linear weights are uploaded as they are, in the model weight
 * dtype of the same name (all linear weights must share one), F32/F16/BF16
 * ones quantised as above; Q and K rows are put back from llama.cpp's
 * interleaved RoPE order into the rotate-half order; output.weight, or the
 * tied token_embd.weight, as lm_head. */
int llmrs_model_load_gguf(const char* path, const llmrs_load_options* opt, llmrs_model** out);
/* Write already-rotated K and V rows for positions [pos0, pos0+n) of one
 * layer and KV head (pre-filled caches); k, v are f32 [n][head_dim], stored
 * in the model's kv_dtype. */
int llmrs_model_kv_write(llmrs_model* m, int layer, int kv_head, size_t pos0,
                         size_t n, const float* k, const float* v);
/* Read back K and V rows (as f32) - for tests. */
int llmrs_model_kv_read(llmrs_model* m, int layer, int kv_head, size_t pos0,
                        size_t n, float* k, float* v);
/* One forward pass of `n` tokens at positions [start_pos, start_pos+n)
 * (LlamaModel::forward, src/core/model.rs:17-49, driven like
 * src/main.rs:134-190).  n > 1 runs the batched prefill kernels (every
 * linear layer as an exact int8 GEMM over Q8_0 rows, cpu.rs:90-110; causal
 * attention, layer.rs:248-326) in chunks of up to 2048 rows; n == 1 is one
 * decode step.  Environment LLMRS_PREFILL=0 processes the rows one decode
 * step at a time instead.  Outputs (each may be NULL):
 *   logits  f32 [vocab] of the last row;
 *   next    greedy argmax of the last row (lowest index on ties);
 *   trace   f32 [n][n_layers+1][hidden]: the residual stream entering each
 *           layer and the one leaving the last layer. */
int llmrs_model_forward(llmrs_model* m, const int32_t* tokens, size_t n,
                        size_t start_pos, float* logits, int32_t* next,
                        float* trace);
/* Greedy generation (src/main.rs:128-327 with argmax in place of sampling):
 * processes the prompt from position 0 (batched prefill, as in
 * llmrs_model_forward), then emits n_steps tokens into out_tokens.  Each
 * decode position runs as one replay of a captured HIP graph. */
int llmrs_model_generate(llmrs_model* m, const int32_t* prompt,
                         size_t n_prompt, size_t n_steps, int32_t* out_tokens);
/* ---- sampling (src/main.rs:192-305) ------------------------------------
 * The token loop's sampling in place of the greedy argmax: repetition
 * penalty, temperature, softmax, then nucleus (top_p < 1) or roulette
 * sampling, and the end-of-sequence stop.  The reference draws U from an
 * unseeded thread RNG (main.rs:123, rng.random::<f32>()); here the draw after
 * the token at position p uses U = (output p+1 of the SplitMix64 stream
 * seeded with `seed`) >> 40, times 2^-24 - 24 random bits, as the
 * reference's f32 draw - so a run repeats. */
#define LLMRS_MAX_EOS 8
typedef struct {
  float temperature;      /* logits / t unless |t - 1| <= 1e-6 (main.rs:214-220); finite, > 0 */
  float top_p;            /* < 1: nucleus over p > 1e-5 (main.rs:249-283); >= 1: roulette (main.rs:284-294) */
  float repeat_penalty;   /* > 1: the ids of the history window penalised (main.rs:193-212) */
  int32_t penalty_window; /* ids of the history penalised; <= 0: all of it */
  uint64_t seed;
  int32_t n_eos;          /* end-of-sequence ids (main.rs:121), up to LLMRS_MAX_EOS */
  int32_t eos[LLMRS_MAX_EOS];
} llmrs_sampling;
/* Sets (s != NULL) or clears (NULL: greedy argmax) the sampling of the
 * model's decode steps: llmrs_model_begin, decode_steps and generate, and
 * llmrs_model_forward's `next`.  The penalty history is the prompt plus the
 * ids produced.  A drawn end-of-sequence id ends the sequence (main.rs:
 * 308-310): it is not appended, and later steps leave the tokens as they are.
 * llmrs_model_generate then fills the rest of out_tokens with -1.
 * Vocabularies up to 262144 ids. */
int llmrs_model_set_sampling(llmrs_model* m, const llmrs_sampling* s);
/* Reference-order decode (on != 0; no trait counterpart; environment
 * LLMRS_EXACT=1 sets it at llmrs_model_create).  Single-sequence steps then
 * run kernels that add every f32 sum in the reference CPU path's order
 * (x86-64 build): the RMSNorm sum of squares (cpu.rs:381-389), each GEMV
 * output's block loop (kernel_avx2, cpu.rs:903-938), the attention's dots,
 * softmax sum and P.V (layer.rs:257-299, cpu.rs:395-423), and glibc's expf
 * for SiLU and softmax (layer.rs:75-79).  For the same weights and tokens,
 * logits and greedy tokens then equal the reference's bit for bit.  Prompts
 * run batched (the reference's batched prompt adds each row's sums in the
 * same orders).  Slower than the fast step (8B shape on MI355X: 2.17 vs
 * 1.35 ms per token at 512-600 positions); needs max_seq <= 16384.  Batches
 * (llmrs_batch_*) always use the fast kernels. */
int llmrs_model_set_exact(llmrs_model* m, int on);
/* Tokens produced since llmrs_model_begin (the first comes from the prompt's
 * last position) and whether an end-of-sequence id stopped the run. */
int llmrs_model_produced(llmrs_model* m, size_t* n, int32_t* stopped);
/* The sampler alone (test probe, no reference counterpart): the logits of
 * one step, the history the penalty window reads (input_ids, main.rs:
 * 195-203) and the position that selects U.  Writes the drawn id and U
 * (either may be NULL). */
int llmrs_sample_logits(const float* logits, int32_t vocab, const int32_t* history,
                        size_t n_history, const llmrs_sampling* s, uint64_t position,
                        int32_t* token, float* u);
/* Benchmark helpers: start a run (prompt processed, state resident),
 * then replay `n` more decode steps without host synchronisation. */
int llmrs_model_begin(llmrs_model* m, const int32_t* prompt, size_t n_prompt);
/* As llmrs_model_begin with the prompt at positions [start_pos, start_pos +
 * n_prompt): the cache below start_pos is taken as already filled (the
 * reference's chunk at cur_pos > 0, main.rs:134-138,313; llmrs_model_kv_write
 * fills it). */
int llmrs_model_begin_at(llmrs_model* m, const int32_t* prompt, size_t n_prompt, size_t start_pos);
int llmrs_model_decode_steps(llmrs_model* m, size_t n);
/* Tokens produced since llmrs_model_begin (count = n_prompt + steps). */
int llmrs_model_tokens(llmrs_model* m, int32_t* out, size_t count);
/* Per-kernel timing of one eager decode step at the current position, with
 * HIP events on the model's stream.  `names` receives up to `cap` entries of
 * 32 chars; `ms` and `bytes` the duration and algorithmic bytes of each
 * launch.  Returns the number of launches recorded (>= 0) or an error. */
int llmrs_model_profile_step(llmrs_model* m, char* names, float* ms,
                             double* bytes, int cap);
/* Mean duration of one decode GEMV launch: the `slot` GEMV (LLMRS_W_Q = the
 * stacked Q|K|V rows, LLMRS_W_O, LLMRS_W_GATE = gate|up, LLMRS_W_DOWN) of
 * every layer in turn, `reps` times back to back between two HIP events on
 * the model's stream (each launch streams a different layer's weights, as
 * in decoding).  Uses the decode activation buffers as they are (scratch
 * that the next step recomputes).  Also returns the launch's algorithmic
 * bytes.  Requires llmrs_model_begin. */
int llmrs_model_time_linear(llmrs_model* m, int slot, int reps, double* us_per_launch,
                            double* bytes_per_launch);
/* Per-kernel timing of one batched prefill of `n` tokens (n at most one
 * chunk, 2048 rows by default) at positions [start_pos, start_pos+n), as in
 * llmrs_model_forward.  Same outputs as llmrs_model_profile_step, with
 * `work` = FLOPs for the GEMM and attention launches (2 per multiply-add) and
 * bytes for the others. */
int llmrs_model_profile_prefill(llmrs_model* m, const int32_t* tokens, size_t n,
                                size_t start_pos, char* names, float* ms,
                                double* work, int cap);
/* ---- batched decode (no reference counterpart) ---------------------------
 * B sequences of one model decoding together (greedy), each with its own K/V
 * cache, position and history.  The reference decodes one sequence; its
 * layer code takes any number of rows (layer.rs:175-333), and each row's
 * values depend only on that row and its own cache.  Every linear layer runs
 * the B rows as one exact int8 GEMM (the prefill path's, cpu.rs:90-110 per
 * row); the decode attention runs one slice per sequence.  A batch shares the
 * model's weights; it holds B caches of the model's max_seq positions. */
typedef struct llmrs_batch llmrs_batch;
int llmrs_batch_create(llmrs_model* m, int32_t batch, llmrs_batch** out);
int llmrs_batch_free(llmrs_batch* b);
/* Prefills slot `slot` with a prompt (the model's prefill kernels, into the
 * slot's cache) and takes its first greedy token.  Uses the model's own
 * sequence state as scratch (a later llmrs_model_decode_steps needs a new
 * llmrs_model_begin).  The model's sampling must be cleared. */
int llmrs_batch_begin(llmrs_batch* b, int32_t slot, const int32_t* prompt, size_t n_prompt);
/* n greedy steps of every slot (each slot must have been begun), one HIP
 * graph replay per step. */
int llmrs_batch_decode_steps(llmrs_batch* b, size_t n);
/* The ids of slot `slot` from position 0: its prompt, then what it produced. */
int llmrs_batch_tokens(llmrs_batch* b, int32_t slot, int32_t* out, size_t count);
/* The logits of the last step, f32 [B][vocab] (tests). */
int llmrs_batch_logits(llmrs_batch* b, float* out);
/* Per-launch timing of one eager batched step (as llmrs_model_profile_step). */
int llmrs_batch_profile_step(llmrs_batch* b, char* names, float* ms, double* work, int cap);

/* ---- test probes (no reference counterpart) ------------------------------
 * One layer's kernels run on inputs given by the host, with every
 * intermediate the kernels produce copied back, so each kernel can be held to
 * the reference arithmetic on its own inputs.  Every pointer of the probe
 * may be NULL (not copied).  Decode rows are 1, prefill rows n. */
typedef struct {
  float* qkv;     /* [rows][(n_heads+2*n_kv_heads)*head_dim] Q|K|V before RoPE */
  int8_t* xq;     /* [rows][hidden] Q8_0 codes of RMSNorm(x) (Q|K|V input) */
  float* xd;      /* [rows][hidden/32] their scales */
  float* ctx;     /* [rows][n_heads*head_dim] attention output */
  int8_t* ctx_q;  /* [rows][n_heads*head_dim] its Q8_0 codes (O input) */
  float* ctx_d;   /* [rows][n_heads*head_dim/32] */
  float* h;       /* [rows][hidden] x + O.ctx (layer.rs:386) */
  int8_t* hq;     /* [rows][hidden] Q8_0 codes of RMSNorm(h) (gate|up input) */
  float* hd;      /* [rows][hidden/32] */
  float* m;       /* [rows][ffn] silu(gate)*up (layer.rs:75-79) */
  int8_t* m_q;    /* [rows][ffn] its Q8_0 codes (down input) */
  float* m_d;     /* [rows][ffn/32] */
  float* out;     /* [rows][hidden] h + down.m (layer.rs:403) */
} llmrs_layer_probe;
/* One decode step of `layer` at position `pos` on the row x[hidden]: the
 * Q|K|V GEMV, the decode attention (which appends K/V at pos; the cache below
 * pos is taken as filled), O, gate|up and down GEMVs, as in the decode loop. */
int llmrs_model_probe_decode_layer(llmrs_model* m, int layer, size_t pos,
                                   const float* x, llmrs_layer_probe* out);
/* Final RMSNorm + lm_head GEMV + greedy argmax of the row x[hidden]: the
 * prologue's Q8_0 operand (xq[hidden], xd[hidden/32]), the logits and the
 * argmax (each may be NULL). */
int llmrs_model_probe_head(llmrs_model* m, const float* x, int8_t* xq,
                           float* xd, float* logits, int32_t* next);
/* The batched prefill kernels of `layer` on rows x[n][hidden] at positions
 * [start_pos, start_pos+n), n at most one prefill chunk. */
int llmrs_model_probe_prefill_layer(llmrs_model* m, int layer, size_t start_pos,
                                    size_t n, const float* x,
                                    llmrs_layer_probe* out);

/* Profiling (no reference counterpart): one eager decode step in which the
 * decode GEMV of `slot` (LLMRS_W_Q = Q|K|V, LLMRS_W_O, LLMRS_W_GATE =
 * gate|up, LLMRS_W_DOWN), or with slot -2 the decode attention, of `layer`
 * records per-workgroup stamps.  Per workgroup 9 values: 7 stamps in us from
 * the launch's earliest start (-1 = not recorded; GEMV: start, operand
 * ready, unit loop done, end, input arrived, norm factor known, operand
 * quantised; attention, items (KV head, split) in head-major order:
 * start, projections loaded, first tile staged, tiles done, partials
 * written, ticket taken, splits combined), the XCC id and HW_ID.  Returns
 * the count written. */
int llmrs_model_profile_stamps(llmrs_model* m, int layer, int slot, double* out,
                               int cap);
/* Algorithmic weight bytes streamed per decode token (all linear weights). */
double llmrs_model_weight_bytes(const llmrs_model* m);
/* How a single-sequence decode step runs its attention (no reference
 * counterpart; tests and the benchmark report it): out[0] splits per KV head
 * of the standalone attention launch, out[1] its tile waves (f16 caches) or
 * tile streams (f32), out[2] 1 when a KV head's splits exchange partials
 * through one XCD's L2, out[3] 1 when the model runs the reference-order
 * kernels (LLMRS_EXACT, see llmrs_model_create). */
int llmrs_model_decode_plan(const llmrs_model* m, int32_t out[4]);

/* ---- seeded synthetic inputs (benchmark and test data) ------------------ */
/* Counter-based SplitMix64 generator keyed by (seed, tensor_id, index).
 * Q4 codes uniform in 0..15 packed in the reference nibble order, scales
 * fp16-rounded uniform in [lo, hi); Q8 codes uniform in [-127, 127];
 * normals via Box-Muller; token ids uniform in [0, vocab).  Filled with
 * `threads` host threads (0 = all cores). */
int llmrs_synth_q4(uint64_t seed, uint64_t tensor_id, size_t n, size_t k,
                   float lo, float hi, uint8_t* qs, float* scales, int threads);
int llmrs_synth_q8(uint64_t seed, uint64_t tensor_id, size_t n, size_t k,
                   float lo, float hi, int8_t* qs, float* scales, int threads);
int llmrs_synth_normal(uint64_t seed, uint64_t tensor_id, size_t count,
                       float mean, float stddev, float* out, int threads);
int llmrs_synth_tokens(uint64_t seed, uint64_t tensor_id, size_t count,
                       int32_t vocab, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* LLMRS_HIP_H */
