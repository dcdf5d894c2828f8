// oracle.cpp - CPU restatement of the llm.rs reference CPU path.
//
// TEST INFRASTRUCTURE ONLY (the tests' parity reference and the timed CPU baseline); the
// product library never links it.  Compiled with -ffp-contract=off so that
// every a*b+c rounds twice, as Rust code does.  Reference citations are
// relative to the reference repository root.
#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// Fork-join pool.  Plays the role rayon has in the reference: every output
// element / row / head is computed by one task in a fixed sequential order,
// so results do not depend on the thread count (no cross-thread reductions,
// src/backend/cpu.rs:81,92,205 of layer.rs).
// ---------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(int n) { resize(n); }
  ~Pool() { stop(); }

  void resize(int n) {
    stop();
    if (n <= 0) n = (int)std::max(1u, std::thread::hardware_concurrency());
    nthreads_ = n;
    quit_ = false;
    for (int i = 1; i < n; ++i) workers_.emplace_back([this] { loop(); });
  }
  int size() const { return nthreads_; }

  void run(int64_t count, const std::function<void(int64_t)>& fn) {
    if (count <= 0) return;
    // Nested parallel regions (a task that calls run again) execute inline.
    if (nthreads_ == 1 || count == 1 || in_task()) {
      for (int64_t i = 0; i < count; ++i) fn(i);
      return;
    }
    std::lock_guard<std::mutex> outer(run_mu_);
    {
      std::unique_lock<std::mutex> lk(mu_);
      job_ = &fn;
      total_ = count;
      next_.store(0);
      pending_ = (int)workers_.size();
      ++gen_;
    }
    cv_.notify_all();
    work(fn, count);
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [this] { return pending_ == 0; });
    job_ = nullptr;
  }

 private:
  static bool& in_task() {
    static thread_local bool flag = false;
    return flag;
  }
  void work(const std::function<void(int64_t)>& fn, int64_t count) {
    in_task() = true;
    for (;;) {
      int64_t i = next_.fetch_add(1);
      if (i >= count) break;
      fn(i);
    }
    in_task() = false;
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int64_t)>* job;
      int64_t count;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return quit_ || gen_ != seen; });
        if (quit_) return;
        seen = gen_;
        job = job_;
        count = total_;
      }
      work(*job, count);
      std::unique_lock<std::mutex> lk(mu_);
      if (--pending_ == 0) done_cv_.notify_all();
    }
  }
  void stop() {
    {
      std::unique_lock<std::mutex> lk(mu_);
      quit_ = true;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
    workers_.clear();
  }

  std::vector<std::thread> workers_;
  std::mutex run_mu_;  // one parallel region at a time
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int64_t)>* job_ = nullptr;
  int64_t total_ = 0;
  std::atomic<int64_t> next_{0};
  int pending_ = 0;
  uint64_t gen_ = 0;
  bool quit_ = false;
  int nthreads_ = 1;
};

Pool& pool() {
  static Pool p(0);
  return p;
}

// Which build of the reference the arithmetic restates (orc_set_arch):
// 0 = x86-64 (the default; the timed host), 1 = aarch64, the reference's
// primary target (Android), whose NEON paths sum in other orders: the Q4
// GEMV adds four blocks before the running total (kernel_neon_sdot,
// cpu.rs:747-886), simd_dot_f32 keeps 32 fused multiply-add lanes
// (cpu.rs:461-544) and simd_saxpy fuses (cpu.rs:558-619).  Test-only: it
// measures how far the reference's own two builds disagree.
std::atomic<int> g_arch{0};

// Rust's `iter().zip().map(|(x, y)| x * y).sum()`: sequential from zero
// (cpu.rs:546-549, the non-aarch64 simd_dot_f32).
inline float dot_seq(const float* a, const float* b, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s = s + a[i] * b[i];
  return s;
}

// simd_dot_f32 on aarch64 (cpu.rs:461-544): eight 4-lane accumulators over
// 32-element steps with fused multiply-add, combined as
// ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)) lane-wise, 4-element leftovers fused
// into that, the lanes summed pairwise ((l0+l1)+(l2+l3), vaddvq_f32), then
// scalar leftovers unfused.
inline float dot_neon(const float* a, const float* b, int64_t n) {
  float acc[8][4] = {};
  int64_t i = 0;
  for (; i + 32 <= n; i += 32)
    for (int j = 0; j < 8; ++j)
      for (int l = 0; l < 4; ++l) acc[j][l] = std::fma(a[i + 4 * j + l], b[i + 4 * j + l], acc[j][l]);
  float v[4];
  for (int l = 0; l < 4; ++l)
    v[l] = ((acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l])) +
           ((acc[4][l] + acc[5][l]) + (acc[6][l] + acc[7][l]));
  for (; i + 4 <= n; i += 4)
    for (int l = 0; l < 4; ++l) v[l] = std::fma(a[i + l], b[i + l], v[l]);
  float sum = (v[0] + v[1]) + (v[2] + v[3]);
  for (; i < n; ++i) sum = sum + a[i] * b[i];
  return sum;
}

// simd_dot_f32 of the selected build.
inline float dot_ref(const float* a, const float* b, int64_t n) {
  return g_arch.load(std::memory_order_relaxed) ? dot_neon(a, b, n) : dot_seq(a, b, n);
}

// simd_saxpy of the selected build (y += alpha * x): unfused on x86
// (cpu.rs:620-625); on aarch64 fused over whole 32-element steps and unfused
// for the leftovers (cpu.rs:558-619).
inline void saxpy_ref(float alpha, const float* x, float* y, int64_t n) {
  int64_t i = 0;
  if (g_arch.load(std::memory_order_relaxed))
    for (const int64_t n32 = n / 32 * 32; i < n32; ++i) y[i] = std::fma(alpha, x[i], y[i]);
  for (; i < n; ++i) y[i] = y[i] + alpha * x[i];
}

// Test-only: attention sums in float64 (orc_set_attn_f64), to measure how
// far the reference's own f32 attention sums move its results.
std::atomic<int> g_attn_f64{0};

// Test-only record of every Q8_0 code quantize_row_q8_0 produces, in call
// order (orc_record_codes), so two runs can be compared code by code.
std::atomic<int> g_record{0};
std::mutex g_record_mu;
std::vector<int8_t> g_recorded;

// Test-only substitution of Q8_0 codes (orc_inject_codes), guarded by
// g_record_mu.
std::atomic<int> g_inject{0};
std::vector<int8_t> g_inject_codes;
int64_t g_inject_pos = 0, g_inject_differ = 0, g_inject_bad = 0;
float g_inject_tol = 0.0f, g_inject_max_dist = 0.0f;

// Exact integer sum over one Q4 block: sum_i (q_i - 8) * a_i, with the
// reference nibble order (element 2i = low nibble of byte i, element 2i+1 =
// high nibble; tensor.rs:125-131).  Any evaluation order gives the same
// int32 (|sum| <= 32 * 8 * 127), which is what cpu.rs:914-930 computes.
inline int32_t q4_isum_avx2(const uint8_t* q4, const int8_t* a) {
  const __m128i m4 = _mm_set1_epi8(0x0F);
  __m128i b = _mm_loadu_si128((const __m128i*)q4);
  __m128i lo = _mm_and_si128(b, m4);
  __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), m4);
  __m128i e0 = _mm_unpacklo_epi8(lo, hi);  // elements 0..15
  __m128i e1 = _mm_unpackhi_epi8(lo, hi);  // elements 16..31
  const __m256i eight = _mm256_set1_epi16(8);
  __m256i w0 = _mm256_sub_epi16(_mm256_cvtepu8_epi16(e0), eight);
  __m256i w1 = _mm256_sub_epi16(_mm256_cvtepu8_epi16(e1), eight);
  __m256i a0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)a));
  __m256i a1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + 16)));
  __m256i p = _mm256_add_epi32(_mm256_madd_epi16(w0, a0), _mm256_madd_epi16(w1, a1));
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(p), _mm256_extracti128_si256(p, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
}

inline int32_t q8_isum_avx2(const int8_t* w, const int8_t* a) {
  __m256i w0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)w));
  __m256i w1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(w + 16)));
  __m256i a0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)a));
  __m256i a1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + 16)));
  __m256i p = _mm256_add_epi32(_mm256_madd_epi16(w0, a0), _mm256_madd_epi16(w1, a1));
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(p), _mm256_extracti128_si256(p, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
}

// The f32 block accumulation of one output row from its exact block sums.
// x86 (kernel_avx2, cpu.rs:903-938): sequential over blocks from 0.0,
// total += isum * (d_w * d_a).  aarch64 (kernel_neon_sdot, cpu.rs:771-877):
// four blocks at a time, total += ((p0 + p1) + p2) + p3 with p = isum *
// (d_a * d_w), then the remaining blocks one by one.
template <class ISum>
inline float block_row(const float* srow, const float* ad, int64_t nb, ISum isum) {
  float total = 0.0f;
  int64_t b = 0;
  if (g_arch.load(std::memory_order_relaxed)) {
    for (; b + 4 <= nb; b += 4) {
      float p[4];
      for (int j = 0; j < 4; ++j) p[j] = (float)isum(b + j) * (ad[b + j] * srow[b + j]);
      total = total + (((p[0] + p[1]) + p[2]) + p[3]);
    }
  }
  for (; b < nb; ++b) {
    float scale = srow[b] * ad[b];
    float blk = (float)isum(b);
    total = total + blk * scale;
  }
  return total;
}

// One Q4 output row (cpu.rs:903-938, or the aarch64 order).
inline float q4_row(const uint8_t* qrow, const float* srow, const int8_t* aq,
                    const float* ad, int64_t nb) {
  return block_row(srow, ad, nb, [&](int64_t b) { return q4_isum_avx2(qrow + 16 * b, aq + 32 * b); });
}

inline float q8_row(const int8_t* wrow, const float* srow, const int8_t* aq,
                    const float* ad, int64_t nb) {
  return block_row(srow, ad, nb, [&](int64_t b) { return q8_isum_avx2(wrow + 32 * b, aq + 32 * b); });
}

// f32 -> binary16, IEEE round-to-nearest-even (F16C).
inline uint16_t to_half(float x) { return _cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT); }
inline float from_half(uint16_t h) { return _cvtsh_ss(h); }

}  // namespace

extern "C" {

void orc_set_threads(int n) { pool().resize(n); }

void orc_set_arch(int arch) { g_arch.store(arch ? 1 : 0); }
int orc_get_arch(void) { return g_arch.load(); }

void orc_set_attn_f64(int on) { g_attn_f64.store(on ? 1 : 0); }

void orc_record_codes(int on) {
  std::lock_guard<std::mutex> lk(g_record_mu);
  g_record.store(on ? 1 : 0);
  if (on) g_recorded.clear();
}

int64_t orc_recorded_codes(int8_t* out, int64_t cap) {
  std::lock_guard<std::mutex> lk(g_record_mu);
  const int64_t n = (int64_t)g_recorded.size();
  if (out) std::memcpy(out, g_recorded.data(), (size_t)std::min(n, cap));
  return n;
}

int orc_get_threads(void) { return pool().size(); }

// cpu.rs:724-743 (x86 path of quantize_row_q8_0).  amax by strict '>' fold
// from 0, d = amax/127, inv = 1/d, q = round-half-away(x*inv) clamped to
// [-127,127]; amax == 0 gives d = 0 and q = 0.  A NaN product saturates to
// 0, as Rust's `as i8` does.
void orc_quantize_row_q8_0(const float* x, int64_t k, int8_t* q, float* d) {
  const int64_t nb = k / 32;
  for (int64_t b = 0; b < nb; ++b) {
    const float* src = x + 32 * b;
    int8_t* qb = q + 32 * b;
    float max_abs = 0.0f;
    for (int i = 0; i < 32; ++i)
      if (std::fabs(src[i]) > max_abs) max_abs = std::fabs(src[i]);
    if (max_abs == 0.0f) {
      d[b] = 0.0f;
      std::memset(qb, 0, 32);
    } else {
      float scale = max_abs / 127.0f;
      d[b] = scale;
      float inv = 1.0f / scale;
      for (int i = 0; i < 32; ++i) {
        float r = std::round(src[i] * inv);
        if (std::isnan(r)) r = 0.0f;
        r = std::min(127.0f, std::max(-127.0f, r));
        qb[i] = (int8_t)r;
      }
    }
  }
  if (g_record.load(std::memory_order_relaxed)) {
    std::lock_guard<std::mutex> lk(g_record_mu);
    g_recorded.insert(g_recorded.end(), q, q + nb * 32);
  }
  if (g_inject.load(std::memory_order_relaxed)) {
    std::lock_guard<std::mutex> lk(g_record_mu);
    for (int64_t b = 0; b < nb; ++b) {
      const float inv = d[b] == 0.0f ? 0.0f : 1.0f / d[b];
      for (int i = 0; i < 32; ++i) {
        const int64_t e = 32 * b + i;
        if (g_inject_pos >= (int64_t)g_inject_codes.size()) {
          ++g_inject_bad;  // more codes asked for than given
          continue;
        }
        const int8_t c = g_inject_codes[g_inject_pos++];
        if (c == q[e]) continue;
        ++g_inject_differ;
        // midpoint between the two codes, in code units
        const float p = x[e] * inv, mid = 0.5f * ((float)c + (float)q[e]);
        const float dist = std::fabs(p - mid);
        g_inject_max_dist = std::max(g_inject_max_dist, dist);
        if (std::abs((int)c - (int)q[e]) != 1 || !(dist <= g_inject_tol)) ++g_inject_bad;
        q[e] = c;
      }
    }
  }
}

void orc_inject_codes(const int8_t* codes, int64_t n, float tol) {
  std::lock_guard<std::mutex> lk(g_record_mu);
  g_inject_codes.assign(codes ? codes : nullptr, codes ? codes + n : nullptr);
  g_inject_pos = g_inject_differ = g_inject_bad = 0;
  g_inject_tol = tol;
  g_inject_max_dist = 0.0f;
  g_inject.store(codes ? 1 : 0);
}

void orc_injected_stats(int64_t* taken, int64_t* differ, int64_t* bad, float* max_dist) {
  std::lock_guard<std::mutex> lk(g_record_mu);
  *taken = g_inject_pos;
  *differ = g_inject_differ;
  *bad = g_inject_bad;
  *max_dist = g_inject_max_dist;
}

// Tensor::quantize_q4 (tensor.rs:102-167): d = amax/7, q = trunc(clamp(x/d +
// 8.5, 0, 15)) with inv = 1/d, two codes per byte (low = even element);
// d == 0 fills 0x88.  `count` must be a multiple of 32.
void orc_quantize_q4(const float* x, int64_t count, uint8_t* qs, float* scales) {
  const int64_t nb = count / 32;
  for (int64_t b = 0; b < nb; ++b) {
    const float* c = x + 32 * b;
    float max_abs = 0.0f;
    for (int i = 0; i < 32; ++i) max_abs = std::fmax(max_abs, std::fabs(c[i]));
    float scale = max_abs / 7.0f;
    scales[b] = scale;
    uint8_t* out = qs + 16 * b;
    if (scale == 0.0f) {
      std::memset(out, 0x88, 16);
      continue;
    }
    float inv = 1.0f / scale;
    for (int i = 0; i < 16; ++i) {
      float v0 = c[2 * i] * inv + 8.5f;
      float v1 = c[2 * i + 1] * inv + 8.5f;
      v0 = std::min(15.0f, std::max(0.0f, v0));
      v1 = std::min(15.0f, std::max(0.0f, v1));
      out[i] = (uint8_t)((uint8_t)v0 | ((uint8_t)v1 << 4));
    }
  }
}

// dequantize_q4_to_f32 (src/test/opencl.rs:182-235): (q - 8) * d.
void orc_dequantize_q4(const uint8_t* qs, const float* scales, int64_t count,
                       float* out) {
  for (int64_t i = 0; i < count / 2; ++i) {
    float s = scales[(2 * i) / 32];
    out[2 * i] = ((float)(qs[i] & 0x0F) - 8.0f) * s;
    out[2 * i + 1] = ((float)(qs[i] >> 4) - 8.0f) * s;
  }
}

int32_t orc_q4_block_isum(const uint8_t* q4, const int8_t* a) { return q4_isum_avx2(q4, a); }

int32_t orc_q4_block_isum_scalar(const uint8_t* q4, const int8_t* a) {
  int32_t s = 0;
  for (int i = 0; i < 16; ++i) {
    s += ((int32_t)(q4[i] & 0x0F) - 8) * a[2 * i];
    s += ((int32_t)(q4[i] >> 4) - 8) * a[2 * i + 1];
  }
  return s;
}

// CpuBackend::matmul_transposed, Q4 branch (cpu.rs:49-111): quantise each
// row of `a` to Q8 (cpu.rs:79,98-100), then one sequential block loop per
// output column (kernel_avx2 cpu.rs:888-941), columns in 512 chunks
// (cpu.rs:74,81).
//
// Loop order: every output is one q4_row call, whatever the order, so the
// values equal the reference's row-parallel loop (cpu.rs:91-110).  The
// rows are quantised first, then 512-column chunks run in parallel, each
// taking every row in turn while its weights stay in cache.
void orc_matmul_transposed_q4(const float* a, int64_t m, int64_t k,
                              const uint8_t* qs, const float* scales,
                              int64_t n, float* out) {
  const int64_t nb = k / 32;
  std::vector<int8_t> aq(m * k);
  std::vector<float> ad(m * nb);
  for (int64_t i = 0; i < m; ++i) orc_quantize_row_q8_0(a + i * k, k, &aq[i * k], &ad[i * nb]);
  orc_gemv_codes(aq.data(), ad.data(), m, k, qs, scales, n, 0, out);
}

// Q8_0-weight GEMV: no reference function (the reference has only F32 and
// Q4, tensor.rs:13-44); it extends cpu.rs:49-111 with int8 weight codes and
// the same scale-and-accumulate order.
void orc_matmul_transposed_q8w(const float* a, int64_t m, int64_t k,
                               const int8_t* qs, const float* scales,
                               int64_t n, float* out) {
  const int64_t nb = k / 32;
  std::vector<int8_t> aq(m * k);
  std::vector<float> ad(m * nb);
  for (int64_t i = 0; i < m; ++i) orc_quantize_row_q8_0(a + i * k, k, &aq[i * k], &ad[i * nb]);
  orc_gemv_codes(aq.data(), ad.data(), m, k, qs, scales, n, 1, out);
}

// matmul_transposed, f32 branch (cpu.rs:114-146): sequential dot per output.
void orc_matmul_transposed_f32(const float* a, int64_t m, int64_t k,
                               const float* b, int64_t n, float* out) {
  pool().run(m, [&](int64_t i) {
    for (int64_t j = 0; j < n; ++j) out[i * n + j] = dot_ref(a + i * k, b + j * k, k);
  });
}

// CpuBackend::matmul (cpu.rs:157-224): SAXPY over p, skipping exact zeros,
// y += alpha * x sequential (simd_saxpy non-aarch64, cpu.rs:620-625).
void orc_matmul(const float* a, int64_t m, int64_t k, const float* b,
                int64_t n, float* out) {
  std::fill(out, out + m * n, 0.0f);
  pool().run(m, [&](int64_t i) {
    float* res = out + i * n;
    for (int64_t p = 0; p < k; ++p) {
      float val = a[i * k + p];
      if (val == 0.0f) continue;
      saxpy_ref(val, b + p * n, res, n);
    }
  });
}

// CpuBackend::matmul_slice (cpu.rs:230-269): out[i][j] = dot(a_i, other_j).
void orc_matmul_slice(const float* a, int64_t m, int64_t k,
                      const float* other, int64_t rows, float* out) {
  pool().run(m, [&](int64_t i) {
    for (int64_t j = 0; j < rows; ++j) out[i * rows + j] = dot_ref(a + i * k, other + j * k, k);
  });
}

// cpu.rs:274-296
void orc_add_assign(float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] = a[i] + b[i];
}

// cpu.rs:298-324 (also layer.rs:75-79): g = g/(1+exp(-g)) * u.
void orc_silu_mul(float* gate, const float* up, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float v = gate[i];
    float silu = v / (1.0f + std::exp(-v));
    gate[i] = silu * up[i];
  }
}

// f32::exp (layer.rs:75-79, cpu.rs:410): the host libm's expf.
void orc_expf(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = std::exp(x[i]);
}

// cpu.rs:326-357: rotate-half; chunk i (of head_dim) sits at start_pos + i;
// theta = 1 / 500000^(2j/hd) in f32 via powf; sin/cos of pos*theta.
void orc_rope_inplace(float* x, int64_t count, int64_t head_dim, int64_t start_pos) {
  const int64_t mid = head_dim / 2;
  const float base = 500000.0f;
  const int64_t rows = count / head_dim;
  for (int64_t i = 0; i < rows; ++i) {
    float* c = x + i * head_dim;
    int64_t pos = start_pos + i;
    for (int64_t j = 0; j < mid; ++j) {
      float freq_idx = ((float)j * 2.0f) / (float)head_dim;
      float theta = 1.0f / std::pow(base, freq_idx);
      float m_theta = (float)pos * theta;
      float s = std::sin(m_theta), co = std::cos(m_theta);
      float re = c[j], im = c[j + mid];
      c[j] = re * co - im * s;
      c[j + mid] = re * s + im * co;
    }
  }
}

// cpu.rs:359-393: ss = fold(0, acc + v*v); rms = sqrt(ss/n + eps);
// s = 1/rms; y = x * s * w.
void orc_rms_norm(const float* x, int64_t rows, int64_t dim, const float* w,
                  float eps, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * dim;
    float ss = 0.0f;
    for (int64_t i = 0; i < dim; ++i) ss = ss + in[i] * in[i];
    float rms = std::sqrt(ss / (float)dim + eps);
    float scale = 1.0f / rms;
    for (int64_t i = 0; i < dim; ++i) out[r * dim + i] = in[i] * scale * w[i];
  }
}

// cpu.rs:395-423: max from f32::MIN, e = exp(x - max), sequential sum,
// inv = 1/sum, p = e * inv.
void orc_softmax(const float* x, int64_t rows, int64_t dim, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * dim;
    float* o = out + r * dim;
    float mx = -3.40282347e+38f;
    for (int64_t j = 0; j < dim; ++j) mx = std::fmax(mx, in[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j < dim; ++j) {
      float e = std::exp(in[j] - mx);
      o[j] = e;
      sum = sum + e;
    }
    float inv = 1.0f / sum;
    for (int64_t j = 0; j < dim; ++j) o[j] = o[j] * inv;
  }
}

// cpu.rs:425-435
void orc_scale(const float* x, int64_t n, float value, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] * value;
}

uint16_t orc_f32_to_f16(float x) { return to_half(x); }
float orc_f16_to_f32(uint16_t h) { return from_half(h); }

// Greedy choice replacing sampling (main.rs:192-305): the first index of the
// maximum (strict '>' scan).  margin = top1 - top2 over the other indices.
int64_t orc_argmax(const float* x, int64_t n, float* margin) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  if (margin) {
    float second = -INFINITY;
    for (int64_t i = 0; i < n; ++i)
      if (i != best && x[i] > second) second = x[i];
    *margin = x[best] - second;
  }
  return best;
}

namespace {

// Walk of the draw (main.rs:275-281 / 286-292): the first entry, in walk
// order, at which r minus the running f32 sum reaches <= 0; `fallback` when
// none does.
int64_t walk_f32(const std::vector<std::pair<float, int64_t>>& c, size_t n, float r, int64_t fallback) {
  for (size_t k = 0; k < n; ++k) {
    r -= c[k].first;
    if (r <= 0.0f) return c[k].second;
  }
  return fallback;
}

// Whether `token` is the entry at which the exact (double) running sum of
// the first n walk entries crosses some r' within tol of r, or the fallback
// when the exact total may fall short of r (within tol).
bool walk_accepts(const std::vector<std::pair<float, int64_t>>& c, size_t n, double r, double tol,
                  int64_t fallback, int64_t token) {
  double acc = 0.0;
  for (size_t k = 0; k < n; ++k) {
    const double lo = acc;
    acc += c[k].first;
    if (c[k].second == token && lo <= r + tol && acc >= r - tol) return true;
  }
  return token == fallback && acc <= r + tol;
}

}  // namespace

// The token loop's sampling (main.rs:192-305) for a given draw U: repetition
// penalty over the distinct ids of the last `window` history entries (<= 0:
// all; only when penalty > 1; a logit below 0 multiplied by the penalty,
// else divided; main.rs:193-212), temperature (logits / t unless |t - 1| <=
// 1e-6; main.rs:214-220), softmax (max folded from f32::MIN, exp(l - max),
// f32 sum in index order, p /= sum; main.rs:237-246), then top-p
// (main.rs:249-283: ids with p > 1e-5 - every id when none is - in
// descending p, cut at the first prefix whose f32 sum exceeds top_p, r = U *
// (f32 sum of the cut), walk) or, with top_p >= 1, the roulette walk over
// every id in index order with r = U (main.rs:284-294).  sort_unstable_by
// leaves equal probabilities in an unspecified order; this takes them in
// index order, as the GPU sampler does.
//
// `candidate` (>= 0) is another implementation's draw, judged acceptable
// (*accept = 1) when it equals this one or when the draw lies within the
// rounding of the reference's f32 sums: the candidate's interval of the
// exact running sum meets r +- tol.  tol = the largest gap between the f32
// and the exact running sums, plus 1e-6 of the total, plus - where the
// normalisation does not cancel (the roulette's r = U, the top-p cut, the
// 1e-5 threshold) - the relative error of the f32 softmax sum (another
// implementation normalises by its own sum).  Alternative top-p cuts whose
// exact prefix lies within tol of top_p are tried too.
int32_t orc_sample(const float* logits, int64_t vocab, const int32_t* hist, int64_t n_hist, float penalty,
                   float temperature, float top_p, int64_t window, float u, int32_t candidate,
                   int32_t* accept) {
  std::vector<float> l(logits, logits + vocab);
  if (penalty > 1.0f) {
    const int64_t w0 = window > 0 && n_hist > window ? n_hist - window : 0;
    std::vector<char> seen(vocab, 0);
    for (int64_t j = w0; j < n_hist; ++j) {
      const int64_t id = hist[j];
      if (id < 0 || id >= vocab || seen[id]) continue;
      seen[id] = 1;
      l[id] = l[id] < 0.0f ? l[id] * penalty : l[id] / penalty;
    }
  }
  if (std::fabs(temperature - 1.0f) > 1e-6f)
    for (float& v : l) v /= temperature;
  float mx = -FLT_MAX;
  for (float v : l) mx = std::max(mx, v);  // f32::max ignores NaN like fmaxf
  std::vector<float> p(vocab);
  float sum = 0.0f;
  for (int64_t i = 0; i < vocab; ++i) {
    p[i] = expf(l[i] - mx);
  }
  double sum_exact = 0.0;
  for (int64_t i = 0; i < vocab; ++i) {
    sum += p[i];
    sum_exact += p[i];
  }
  for (float& v : p) v /= sum;
  // relative error of the f32 softmax sum, plus room for another order's
  const double delta = std::fabs((double)sum - sum_exact) / sum_exact + 1e-6;

  std::vector<std::pair<float, int64_t>> c;
  int64_t token;
  int ok = 0;
  if (top_p < 1.0f) {
    for (int64_t i = 0; i < vocab; ++i)
      if (p[i] > 1e-5f) c.emplace_back(p[i], i);
    int64_t near_threshold = 0;  // ids whose membership a rounding of p could change
    for (int64_t i = 0; i < vocab; ++i)
      if (std::fabs((double)p[i] - 1e-5) <= (delta + 1e-6) * 1e-5) ++near_threshold;
    if (c.empty())
      for (int64_t i = 0; i < vocab; ++i) c.emplace_back(p[i], i);
    std::stable_sort(c.begin(), c.end(), [](const std::pair<float, int64_t>& a, const std::pair<float, int64_t>& b) {
      return a.first > b.first;
    });
    size_t cut = c.size() - 1;
    float cum = 0.0f;
    double exact = 0.0, gap = 0.0;
    std::vector<double> prefix(c.size());
    for (size_t k = 0; k < c.size(); ++k) {
      exact += c[k].first;
      prefix[k] = exact;
    }
    for (size_t k = 0; k < c.size(); ++k) {
      cum += c[k].first;
      gap = std::max(gap, std::fabs((double)cum - prefix[k]));
      if (cum > top_p) {
        cut = k;
        break;
      }
    }
    float total = 0.0f;
    for (size_t k = 0; k <= cut; ++k) total += c[k].first;
    const float r = u * total;
    token = walk_f32(c, cut + 1, r, c[0].second);
    if (candidate >= 0) {
      double g2 = 0.0, acc = 0.0;
      float cum2 = 0.0f;
      for (size_t k = 0; k < c.size(); ++k) {
        cum2 += c[k].first;
        acc += c[k].first;
        g2 = std::max(g2, std::fabs((double)cum2 - acc));
      }
      const double tol = std::max(gap, g2) + 1e-6 * prefix.back() + near_threshold * 1.1e-5;
      const double tol_cut = tol + delta * std::max(0.0f, top_p);
      ok = candidate == token;
      // every cut whose boundary the rounding could move: prefixes within
      // tol_cut of top_p, plus the reference's own
      for (size_t k = 0; k < c.size() && !ok; ++k) {
        const bool cand_cut = k == cut || std::fabs(prefix[k] - (double)top_p) <= tol_cut ||
                              (k > 0 && std::fabs(prefix[k - 1] - (double)top_p) <= tol_cut);
        if (!cand_cut) continue;
        const double tot = prefix[k];
        ok = walk_accepts(c, k + 1, (double)u * tot, tol, c[0].second, candidate);
      }
    }
  } else {
    for (int64_t i = 0; i < vocab; ++i) c.emplace_back(p[i], i);
    token = walk_f32(c, c.size(), u, 0);
    if (candidate >= 0) {
      double acc = 0.0, gap = 0.0;
      float cum = 0.0f;
      for (size_t k = 0; k < c.size(); ++k) {
        cum += c[k].first;
        acc += c[k].first;
        gap = std::max(gap, std::fabs((double)cum - acc));
      }
      ok = candidate == token || walk_accepts(c, c.size(), u, gap + 1e-6 * acc + delta * u, 0, candidate);
    }
  }
  if (accept) *accept = ok;
  return (int32_t)token;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Model: layer.rs / model.rs / loader.rs transforms with true-GQA KV.
// ---------------------------------------------------------------------------
struct OrcLinear {
  const uint8_t* q4 = nullptr;
  const int8_t* q8 = nullptr;
  const float* scales = nullptr;
  int64_t n = 0, k = 0;
};

struct OrcLayer {
  OrcLinear w[7];  // q k v o gate up down
  const float* norm[2] = {nullptr, nullptr};
  std::vector<float> k32, v32;       // kv_dtype f32: [nkv][max_seq][hd]
  std::vector<uint16_t> k16, v16;    // kv_dtype f16
};

struct orc_model {
  orc_config c;
  const float* embed = nullptr;
  const float* final_norm = nullptr;
  OrcLinear lm_head;
  std::vector<OrcLayer> layers;
};

namespace {

void linear_forward(const orc_model* m, const OrcLinear& w, const float* x,
                    int64_t rows, float* out) {
  if (m->c.weight_dtype == 4)
    orc_matmul_transposed_q8w(x, rows, w.k, w.q8, w.scales, w.n, out);
  else
    orc_matmul_transposed_q4(x, rows, w.k, w.q4, w.scales, w.n, out);
}

inline float kv_load(const OrcLayer& L, bool f16, bool is_k, int64_t idx) {
  if (f16) return from_half(is_k ? L.k16[idx] : L.v16[idx]);
  return is_k ? L.k32[idx] : L.v32[idx];
}
inline void kv_store(OrcLayer& L, bool f16, bool is_k, int64_t idx, float v) {
  if (f16) {
    (is_k ? L.k16 : L.v16)[idx] = to_half(v);
  } else {
    (is_k ? L.k32 : L.v32)[idx] = v;
  }
}

// LlamaAttention::forward (layer.rs:175-333) with the KV cache stored once
// per KV head.  The reference duplicates K/V projection rows per query head
// (loader.rs:62-98), so query head h reads KV head h / n_rep; the duplicated
// rows produce identical cache contents, hence identical results.
// The attention of layer li given the projections of `seq` rows (q_all
// [seq][nq*hd], k_all / v_all [seq][nkv*hd], before RoPE): RoPE, K/V append
// at start_pos.., scores, softmax and P.V (layer.rs:216-326).  ctx_out rows
// have stride ctx_stride.
void attention_core(orc_model* m, int li, const float* q_all, const float* k_all, const float* v_all,
                    int64_t seq, int64_t start_pos, float* ctx_out, int64_t ctx_stride) {
  const orc_config& c = m->c;
  OrcLayer& L = m->layers[li];
  const int64_t hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads;
  const int64_t qdim = nq * hd, kvdim = nkv * hd, ms = c.max_seq;
  const int64_t n_rep = nq / nkv;
  const bool f16 = c.kv_dtype == 1;
  const int64_t total = start_pos + seq;

  // KV update (layer.rs:219-246): rope k per head (layer.rs:217), store k
  // and v at pos = start_pos + i.
  pool().run(nkv, [&](int64_t g) {
    std::vector<float> kh(seq * hd);
    for (int64_t i = 0; i < seq; ++i)
      std::memcpy(&kh[i * hd], &k_all[i * kvdim + g * hd], hd * sizeof(float));
    orc_rope_inplace(kh.data(), seq * hd, hd, start_pos);
    for (int64_t i = 0; i < seq; ++i) {
      int64_t base = (g * ms + start_pos + i) * hd;
      for (int64_t d = 0; d < hd; ++d) {
        kv_store(L, f16, true, base + d, kh[i * hd + d]);
        kv_store(L, f16, false, base + d, v_all[i * kvdim + g * hd + d]);
      }
    }
  });

  const float inv_sqrt = 1.0f / std::sqrt((float)hd);  // layer.rs:258
  pool().run(nq, [&](int64_t h) {
    const int64_t g = h / n_rep;
    std::vector<float> qh(seq * hd);
    for (int64_t i = 0; i < seq; ++i)
      std::memcpy(&qh[i * hd], &q_all[i * qdim + h * hd], hd * sizeof(float));
    orc_rope_inplace(qh.data(), seq * hd, hd, start_pos);  // layer.rs:216
    // K and V rows of this head as f32 (the reference reads them in place).
    std::vector<float> kr(total * hd), vr(total * hd);
    for (int64_t t = 0; t < total; ++t)
      for (int64_t d = 0; d < hd; ++d) {
        kr[t * hd + d] = kv_load(L, f16, true, (g * ms + t) * hd + d);
        vr[t * hd + d] = kv_load(L, f16, false, (g * ms + t) * hd + d);
      }
    if (g_attn_f64.load(std::memory_order_relaxed)) {
      // Test-only: the same attention with every sum in float64 (scores,
      // softmax, P.V), rounded to f32 once at the end.
      std::vector<double> sc(total);
      for (int64_t i = 0; i < seq; ++i) {
        const int64_t last = seq > 1 ? start_pos + i : total - 1;
        double mx = -INFINITY;
        for (int64_t t = 0; t <= last; ++t) {
          double d = 0.0;
          for (int64_t e = 0; e < hd; ++e) d += (double)qh[i * hd + e] * (double)kr[t * hd + e];
          sc[t] = d * (double)inv_sqrt;
          mx = std::max(mx, sc[t]);
        }
        double sum = 0.0;
        for (int64_t t = 0; t <= last; ++t) sum += (sc[t] = std::exp(sc[t] - mx));
        for (int64_t e = 0; e < hd; ++e) {
          double acc = 0.0;
          for (int64_t t = 0; t <= last; ++t) acc += sc[t] * (double)vr[t * hd + e];
          ctx_out[i * ctx_stride + h * hd + e] = (float)(acc / sum);
        }
      }
      return;
    }
    std::vector<float> scores(seq * total), probs(seq * total);
    orc_matmul_slice(qh.data(), seq, hd, kr.data(), total, scores.data());  // layer.rs:257
    for (auto& s : scores) s = s * inv_sqrt;                                 // layer.rs:258
    if (seq > 1) {                                                           // layer.rs:260-269
      for (int64_t i = 0; i < seq; ++i)
        for (int64_t j = 0; j < total; ++j)
          if (j > start_pos + i) scores[i * total + j] = -INFINITY;
    }
    orc_softmax(scores.data(), seq, total, probs.data());  // layer.rs:270
    if (seq == 1) {
      // layer.rs:276-299: ctx[d] = sum_t p_t * V[d][t], sequential over t.
      for (int64_t d = 0; d < hd; ++d) {
        float s = 0.0f;
        for (int64_t t = 0; t < total; ++t) s = s + probs[t] * vr[t * hd + d];
        ctx_out[h * hd + d] = s;
      }
    } else {
      // layer.rs:300-326: probs.matmul(v_hist) (cpu.rs:202-221).
      std::vector<float> ctx(seq * hd, 0.0f);
      for (int64_t i = 0; i < seq; ++i) {
        float* res = &ctx[i * hd];
        for (int64_t p = 0; p < total; ++p) {
          float val = probs[i * total + p];
          if (val == 0.0f) continue;
          saxpy_ref(val, &vr[p * hd], res, hd);
        }
      }
      for (int64_t i = 0; i < seq; ++i)
        std::memcpy(&ctx_out[i * ctx_stride + h * hd], &ctx[i * hd], hd * sizeof(float));
    }
  });
}

void attention_forward(orc_model* m, int li, const float* hn, int64_t seq,
                       int64_t start_pos, float* ctx_out) {
  const orc_config& c = m->c;
  OrcLayer& L = m->layers[li];
  const int64_t qdim = (int64_t)c.n_heads * c.head_dim, kvdim = (int64_t)c.n_kv_heads * c.head_dim;
  std::vector<float> q_all(seq * qdim), k_all(seq * kvdim), v_all(seq * kvdim);
  linear_forward(m, L.w[0], hn, seq, q_all.data());  // layer.rs:177
  linear_forward(m, L.w[1], hn, seq, k_all.data());  // layer.rs:178
  linear_forward(m, L.w[2], hn, seq, v_all.data());  // layer.rs:179
  attention_core(m, li, q_all.data(), k_all.data(), v_all.data(), seq, start_pos, ctx_out, qdim);
}

}  // namespace

extern "C" {

orc_model* orc_model_create(const orc_config* cfg) {
  if (!cfg || cfg->n_layers <= 0 || cfg->hidden % 32 || cfg->ffn % 32) return nullptr;
  if (cfg->n_heads * cfg->head_dim != cfg->hidden) return nullptr;
  if (cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads) return nullptr;
  auto* m = new orc_model();
  m->c = *cfg;
  m->layers.resize(cfg->n_layers);
  const size_t kv = (size_t)cfg->n_kv_heads * cfg->max_seq * cfg->head_dim;
  for (auto& L : m->layers) {
    if (cfg->kv_dtype == 1) {
      L.k16.assign(kv, 0);
      L.v16.assign(kv, 0);
    } else {
      L.k32.assign(kv, 0.0f);
      L.v32.assign(kv, 0.0f);
    }
  }
  return m;
}

void orc_model_free(orc_model* m) { delete m; }

int orc_model_set_embedding(orc_model* m, const float* table) {
  m->embed = table;
  return 0;
}

int orc_model_set_norm(orc_model* m, int layer, int slot, const float* w) {
  if (layer < 0) {
    m->final_norm = w;
    return 0;
  }
  if (layer >= m->c.n_layers || slot < 0 || slot > 1) return -1;
  m->layers[layer].norm[slot] = w;
  return 0;
}

static int shape_of(const orc_model* m, int slot, int64_t* n, int64_t* k) {
  const orc_config& c = m->c;
  switch (slot) {
    case 0: *n = (int64_t)c.n_heads * c.head_dim; *k = c.hidden; return 0;
    case 1: case 2: *n = (int64_t)c.n_kv_heads * c.head_dim; *k = c.hidden; return 0;
    case 3: *n = c.hidden; *k = (int64_t)c.n_heads * c.head_dim; return 0;
    case 4: case 5: *n = c.ffn; *k = c.hidden; return 0;
    case 6: *n = c.hidden; *k = c.ffn; return 0;
    case 7: *n = c.vocab; *k = c.hidden; return 0;
  }
  return -1;
}

int orc_model_set_linear_q4(orc_model* m, int layer, int slot,
                            const uint8_t* qs, const float* scales) {
  OrcLinear w;
  if (shape_of(m, slot, &w.n, &w.k)) return -1;
  w.q4 = qs;
  w.scales = scales;
  if (slot == 7 || layer < 0) { m->lm_head = w; return 0; }
  if (layer >= m->c.n_layers || slot > 6) return -1;
  m->layers[layer].w[slot] = w;
  return 0;
}

int orc_model_set_linear_q8(orc_model* m, int layer, int slot,
                            const int8_t* qs, const float* scales) {
  OrcLinear w;
  if (shape_of(m, slot, &w.n, &w.k)) return -1;
  w.q8 = qs;
  w.scales = scales;
  if (slot == 7 || layer < 0) { m->lm_head = w; return 0; }
  if (layer >= m->c.n_layers || slot > 6) return -1;
  m->layers[layer].w[slot] = w;
  return 0;
}

int orc_model_kv_write(orc_model* m, int layer, int kv_head, int64_t pos0,
                       int64_t n, const float* k, const float* v) {
  const orc_config& c = m->c;
  if (layer < 0 || layer >= c.n_layers || kv_head < 0 || kv_head >= c.n_kv_heads) return -1;
  if (pos0 < 0 || pos0 + n > c.max_seq) return -1;
  OrcLayer& L = m->layers[layer];
  const bool f16 = c.kv_dtype == 1;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t d = 0; d < c.head_dim; ++d) {
      int64_t idx = ((int64_t)kv_head * c.max_seq + pos0 + i) * c.head_dim + d;
      kv_store(L, f16, true, idx, k[i * c.head_dim + d]);
      kv_store(L, f16, false, idx, v[i * c.head_dim + d]);
    }
  return 0;
}

int orc_model_kv_read(orc_model* m, int layer, int kv_head, int64_t pos0,
                      int64_t n, float* k, float* v) {
  const orc_config& c = m->c;
  if (layer < 0 || layer >= c.n_layers || kv_head < 0 || kv_head >= c.n_kv_heads) return -1;
  if (pos0 < 0 || pos0 + n > c.max_seq) return -1;
  OrcLayer& L = m->layers[layer];
  const bool f16 = c.kv_dtype == 1;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t d = 0; d < c.head_dim; ++d) {
      int64_t idx = ((int64_t)kv_head * c.max_seq + pos0 + i) * c.head_dim + d;
      k[i * c.head_dim + d] = kv_load(L, f16, true, idx);
      v[i * c.head_dim + d] = kv_load(L, f16, false, idx);
    }
  return 0;
}

// Test probes: one kernel's arithmetic on given inputs.
// The block loop of matmul_transposed (kernel_avx2 cpu.rs:888-941, or the
// aarch64 order) over `m` rows of already-quantised activations: xq [m][k]
// codes, xd [m][k/32] scales; weights Q4 (q8w == 0: reference nibble order)
// or Q8 codes.
void orc_gemv_codes(const int8_t* xq, const float* xd, int64_t m, int64_t k, const void* w,
                    const float* scales, int64_t n, int q8w, float* out) {
  const int64_t nb = k / 32;
  const int64_t chunks = (n + 511) / 512;
  pool().run(chunks, [&](int64_t c) {
    const int64_t j0 = c * 512, j1 = std::min(n, j0 + 512);
    for (int64_t i = 0; i < m; ++i) {
      const int8_t* aq = xq + i * k;
      const float* ad = xd + i * nb;
      float* res = out + i * n;
      for (int64_t j = j0; j < j1; ++j)
        res[j] = q8w ? q8_row((const int8_t*)w + j * k, scales + j * nb, aq, ad, nb)
                     : q4_row((const uint8_t*)w + j * (k / 2), scales + j * nb, aq, ad, nb);
    }
  });
}

// The attention of `layer` for `seq` rows given their Q|K|V projections
// qkv [seq][(nq + 2 nkv) hd] (before RoPE), at positions start_pos..: the K/V
// rows are appended to the oracle's cache, ctx [seq][nq hd] is written.
int orc_model_attention(orc_model* m, int layer, const float* qkv, int64_t seq, int64_t start_pos,
                        float* ctx) {
  const orc_config& c = m->c;
  if (layer < 0 || layer >= c.n_layers || seq <= 0 || start_pos < 0 || start_pos + seq > c.max_seq)
    return -1;
  const int64_t qdim = (int64_t)c.n_heads * c.head_dim, kvdim = (int64_t)c.n_kv_heads * c.head_dim;
  const int64_t rows = qdim + 2 * kvdim;
  std::vector<float> q_all(seq * qdim), k_all(seq * kvdim), v_all(seq * kvdim);
  for (int64_t i = 0; i < seq; ++i) {
    std::memcpy(&q_all[i * qdim], qkv + i * rows, qdim * sizeof(float));
    std::memcpy(&k_all[i * kvdim], qkv + i * rows + qdim, kvdim * sizeof(float));
    std::memcpy(&v_all[i * kvdim], qkv + i * rows + qdim + kvdim, kvdim * sizeof(float));
  }
  attention_core(m, layer, q_all.data(), k_all.data(), v_all.data(), seq, start_pos, ctx, qdim);
  return 0;
}

// LlamaModel::forward (model.rs:17-49) over LlamaBlock::forward
// (layer.rs:373-406) and LlamaMLP::forward (layer.rs:37-97); the embedding
// gather is main.rs:159-167.
int orc_model_forward(orc_model* m, const int32_t* tokens, int64_t n,
                      int64_t start_pos, float* logits, int all_rows,
                      float* trace) {
  const orc_config& c = m->c;
  if (n <= 0 || start_pos < 0 || start_pos + n > c.max_seq) return -1;
  if (!m->embed || !m->final_norm || !m->lm_head.scales) return -1;
  const int64_t H = c.hidden, F = c.ffn;
  std::vector<float> x(n * H), hn(n * H), attn(n * H), h2(n * H);
  std::vector<float> gate(n * F), up(n * F), mlp(n * H);
  for (int64_t i = 0; i < n; ++i) {
    if (tokens[i] < 0 || tokens[i] >= c.vocab) return -1;
    std::memcpy(&x[i * H], m->embed + (int64_t)tokens[i] * H, H * sizeof(float));
  }
  auto record = [&](int li) {
    if (!trace) return;
    for (int64_t i = 0; i < n; ++i)
      std::memcpy(trace + (i * (c.n_layers + 1) + li) * H, &x[i * H], H * sizeof(float));
  };
  for (int li = 0; li < c.n_layers; ++li) {
    OrcLayer& L = m->layers[li];
    record(li);
    orc_rms_norm(x.data(), n, H, L.norm[0], c.rms_eps, hn.data());     // layer.rs:377
    attention_forward(m, li, hn.data(), n, start_pos, attn.data());     // layer.rs:382 (ctx)
    std::vector<float> o(n * H);
    linear_forward(m, L.w[3], attn.data(), n, o.data());               // layer.rs:332
    orc_add_assign(o.data(), x.data(), n * H);                         // layer.rs:386
    orc_rms_norm(o.data(), n, H, L.norm[1], c.rms_eps, h2.data());     // layer.rs:393
    linear_forward(m, L.w[4], h2.data(), n, gate.data());              // layer.rs:40 rows [0,F)
    linear_forward(m, L.w[5], h2.data(), n, up.data());                // layer.rs:40 rows [F,2F)
    orc_silu_mul(gate.data(), up.data(), n * F);                       // layer.rs:75-79
    linear_forward(m, L.w[6], gate.data(), n, mlp.data());             // layer.rs:93-96
    orc_add_assign(mlp.data(), o.data(), n * H);                       // layer.rs:403
    x.swap(mlp);
  }
  record(c.n_layers);
  // model.rs:39-47: final norm, then lm_head.  The reference evaluates every
  // row; main.rs:189 reads only the last.
  const int64_t r0 = all_rows ? 0 : n - 1;
  const int64_t nr = n - r0;
  std::vector<float> fn(nr * H);
  orc_rms_norm(&x[r0 * H], nr, H, m->final_norm, c.rms_eps, fn.data());
  if (logits) linear_forward(m, m->lm_head, fn.data(), nr, logits);
  return 0;
}

// main.rs:128-327 with greedy argmax (no penalty, no temperature, no EOS
// stop): step 0 prefills the whole prompt at position 0, every later step
// feeds the last token at cur_pos.
int orc_model_generate(orc_model* m, const int32_t* prompt, int64_t n_prompt,
                       int64_t n_steps, int32_t* out, float* margins) {
  const orc_config& c = m->c;
  if (n_prompt <= 0 || n_prompt + n_steps > c.max_seq + 1) return -1;
  std::vector<float> logits(c.vocab);
  std::vector<int32_t> ids(prompt, prompt + n_prompt);
  int64_t cur = 0;
  for (int64_t s = 0; s < n_steps; ++s) {
    int rc;
    if (cur == 0) {
      rc = orc_model_forward(m, ids.data(), (int64_t)ids.size(), 0, logits.data(), 0, nullptr);
      cur = (int64_t)ids.size();
    } else {
      rc = orc_model_forward(m, &ids.back(), 1, cur, logits.data(), 0, nullptr);
      cur += 1;
    }
    if (rc) return rc;
    float mg = 0.0f;
    int32_t t = (int32_t)orc_argmax(logits.data(), c.vocab, &mg);
    out[s] = t;
    if (margins) margins[s] = mg;
    ids.push_back(t);
  }
  return 0;
}

}  // extern "C"
