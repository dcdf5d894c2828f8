// synth.cpp - seeded synthetic weights, caches and prompts.
//
// Counter-based so any element can be generated independently (parallel
// host threads, identical results for any thread count):
//   mix(z)        = SplitMix64 finaliser of z + 0x9E3779B97F4A7C15
//   key(seed, t)  = mix(seed ^ mix(t ^ 0xA0761D6478BD642F))
//   draw(key, i)  = mix(key + i * 0x9E3779B97F4A7C15)
// Q4 codes: element e is nibble (e mod 16) of draw(key, e / 16), so bytes
//   8w..8w+7 of the reference-order packed array are word w (little endian).
// Q4/Q8 scales: block j, u = (draw(key', j) >> 40) * 2^-24 with
//   key' = key(seed, t + 2^32); d = fp16_rne(lo + u * (hi - lo)) (in double).
// Q8 codes: element e, c = 16-bit field (e mod 4) of draw(key, e / 4),
//   code = (c * 255 >> 16) - 127, uniform over [-127, 127].
// Normals: pair p = e / 2 from draw(key, p): u1 = ((w >> 40) + 1) * 2^-24,
//   u2 = ((w >> 16) & 0xFFFFFF) * 2^-24, Box-Muller in double.
// Token ids: draw(key, i) mod vocab.
#include <cmath>
#include <cstring>

#include "internal.h"

using namespace llmrs;

namespace {

inline uint64_t mix(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline uint64_t key_of(uint64_t seed, uint64_t tid) { return mix(seed ^ mix(tid ^ 0xA0761D6478BD642Full)); }
inline uint64_t draw(uint64_t key, uint64_t i) { return mix(key + i * 0x9E3779B97F4A7C15ull); }

void fill_scales(uint64_t seed, uint64_t tid, size_t nblocks, float lo, float hi, float* out,
                 int threads) {
  const uint64_t key = key_of(seed, tid + (1ull << 32));
  parallel_for(nblocks, threads, [&](size_t b0, size_t b1) {
    for (size_t j = b0; j < b1; ++j) {
      const double u = (double)(draw(key, j) >> 40) * (1.0 / 16777216.0);
      const double d = (double)lo + u * ((double)hi - (double)lo);
      out[j] = host_h2f(host_f2h((float)d));
    }
  });
}

}  // namespace

extern "C" {

int llmrs_synth_q4(uint64_t seed, uint64_t tensor_id, size_t n, size_t k, float lo, float hi,
                   uint8_t* qs, float* scales, int threads) {
  if (!qs || !scales || k % 32) return LLMRS_E_INVALID;
  const uint64_t key = key_of(seed, tensor_id);
  const size_t words = n * k / 16;  // 16 codes = 8 bytes per word
  parallel_for(words, threads, [&](size_t w0, size_t w1) {
    for (size_t w = w0; w < w1; ++w) {
      const uint64_t v = draw(key, w);
      std::memcpy(qs + 8 * w, &v, 8);
    }
  });
  fill_scales(seed, tensor_id, n * k / 32, lo, hi, scales, threads);
  return LLMRS_OK;
}

int llmrs_synth_q8(uint64_t seed, uint64_t tensor_id, size_t n, size_t k, float lo, float hi,
                   int8_t* qs, float* scales, int threads) {
  if (!qs || !scales || k % 32) return LLMRS_E_INVALID;
  const uint64_t key = key_of(seed, tensor_id);
  const size_t words = n * k / 4;
  parallel_for(words, threads, [&](size_t w0, size_t w1) {
    for (size_t w = w0; w < w1; ++w) {
      const uint64_t v = draw(key, w);
      for (int f = 0; f < 4; ++f) {
        const uint32_t c = (uint32_t)((v >> (16 * f)) & 0xFFFF);
        qs[4 * w + f] = (int8_t)((int)((c * 255u) >> 16) - 127);
      }
    }
  });
  fill_scales(seed, tensor_id, n * k / 32, lo, hi, scales, threads);
  return LLMRS_OK;
}

int llmrs_synth_normal(uint64_t seed, uint64_t tensor_id, size_t count, float mean, float stddev,
                       float* out, int threads) {
  if (!out) return LLMRS_E_INVALID;
  const uint64_t key = key_of(seed, tensor_id);
  const size_t pairs = (count + 1) / 2;
  parallel_for(pairs, threads, [&](size_t p0, size_t p1) {
    for (size_t p = p0; p < p1; ++p) {
      const uint64_t w = draw(key, p);
      const double u1 = (double)((w >> 40) + 1) * (1.0 / 16777216.0);
      const double u2 = (double)((w >> 16) & 0xFFFFFF) * (1.0 / 16777216.0);
      const double r = std::sqrt(-2.0 * std::log(u1));
      const double a = 6.283185307179586 * u2;
      const size_t e = 2 * p;
      out[e] = (float)(mean + stddev * r * std::cos(a));
      if (e + 1 < count) out[e + 1] = (float)(mean + stddev * r * std::sin(a));
    }
  });
  return LLMRS_OK;
}

int llmrs_synth_tokens(uint64_t seed, uint64_t tensor_id, size_t count, int32_t vocab, int32_t* out) {
  if (!out || vocab <= 0) return LLMRS_E_INVALID;
  const uint64_t key = key_of(seed, tensor_id);
  for (size_t i = 0; i < count; ++i) out[i] = (int32_t)(draw(key, i) % (uint64_t)vocab);
  return LLMRS_OK;
}

}  // extern "C"
