// sample.hip - device-side sampling of the next token for gfx950.
//
// Reference: the token loop's sampling (src/main.rs:192-305): repetition
// penalty over the last `window` ids (a logit below 0 is multiplied by the
// penalty, else divided; each distinct id once; only when penalty > 1),
// temperature (logits divided by t unless |t - 1| <= 1e-6), softmax
// (max folded from f32::MIN, exp(l - max), sum, p = e / sum), then either
// top-p - the ids with p > 1e-5 (all of them when none is) in descending
// probability, cut at the first prefix whose sum exceeds top_p, one drawn
// with r = U * (sum of the cut), subtracting probabilities in that order
// until r <= 0 - or, with top_p >= 1, one drawn over all ids in index order
// with r = U (main.rs:282-292).  An id of the end-of-sequence list stops
// the sequence (main.rs:308-310).  The reference draws U from an unseeded
// thread RNG (main.rs:123); here U = the high 24 bits of the SplitMix64
// output of (seed, position) divided by 2^24, so a run repeats.
//
// MI355X design: the vocabulary is spread over the whole chip - workgroups
// of 256 threads, 512 consecutive ids each - and the launches hand over
// through a small device state, each launch's last workgroup (a ticket, no
// waiting) reducing what the others published:
//   sample_prep    penalty (the window's ids as an LDS bitmap of the slice),
//                  temperature, per-workgroup max and sum of exp; the last
//                  workgroup forms the softmax max and sum.
//   sample_probs   p = exp(l - max) / sum; a histogram of the probabilities'
//                  top bits (counts and fixed-point sums) merged across the
//                  chip; the last workgroup finds the bin of the top-p cut
//                  (or of the draw), or for the roulette the workgroup whose
//                  running sum reaches U.
//   sample_refine  (4 launches) the next 10 bits inside the selected bin;
//                  after two levels the cut's value and tie count are exact,
//                  which fixes r = U * total, and the draw's selection starts.
//   sample_pick    the drawn value's k-th occurrence in index order (ties by
//                  index), or the roulette's id, and the step's bookkeeping.
// Instead of sorting (which the reference does on the host), the cut and
// the draw are radix selects over the probabilities' bit patterns (positive
// floats order like their patterns).  Sums are fixed point (p * 2^40 in 64
// bits), so the result does not depend on the order the threads add in.
// What one launch's workgroups hand to its last workgroup moves with
// device-scope stores, loads and atomics (the XCDs' L2s are not coherent).
#include "common.h"
#include "../kernel_args.h"

using namespace llmrs;

namespace {

constexpr int kT = kSampleThreads;
constexpr int kWaves = kT / 64;
constexpr int kPT = kSamplePerThread;
constexpr float kFixOne = 1099511627776.0f;  // 2^40
constexpr unsigned kLo = 0x3727C5ADu;        // the smallest pattern above 1e-5f (0x3727C5AC)
constexpr int kLoKey = (int)(kLo >> 20);     // 0x372
constexpr int kCandRanks = 2048 - kLoKey;    // first-level ranks of the candidates
constexpr int kNone = 0x7FFFFFFF;

__device__ __forceinline__ unsigned long long to_fix(float p) { return (unsigned long long)(p * kFixOne); }

// floor(t * u / 2^24) for u < 2^24 without 128-bit products
__device__ __forceinline__ unsigned long long scale24(unsigned long long t, unsigned u) {
  return (t >> 24) * u + (((t & 0xFFFFFFull) * u) >> 24);
}

__device__ __forceinline__ unsigned long long splitmix64(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ int step_pos(const SampleArgs& a) { return a.pos ? *a.pos : 0; }

// 24 random bits of the draw after the token at the step's position
__device__ __forceinline__ unsigned draw_u24(const SampleArgs& a) {
  const unsigned long long step =
      a.step_override >= 0 ? (unsigned long long)a.step_override : (unsigned long long)step_pos(a);
  return (unsigned)(splitmix64(a.seed + (step + 1ull) * 0x9E3779B97F4A7C15ull) >> 40);
}

// First-level bin of a probability pattern (bits 30..20; 2048 = the part of
// 1e-5's bin at or below 1e-5) and the bins' descending order: keys 2047 ..
// kLoKey, then 2048, then kLoKey-1 .. 0.  Ranks below kCandRanks hold the
// candidates (p > 1e-5).
__device__ __forceinline__ int l1_key(unsigned bits) {
  const int k = (int)(bits >> 20);
  return (k == kLoKey && bits < kLo) ? 2048 : k;
}
__device__ __forceinline__ int l1_rank_key(int r) {
  if (r < kCandRanks) return 2047 - r;
  if (r == kCandRanks) return 2048;
  return 2047 - (r - 1);
}
__device__ __forceinline__ unsigned key_bits(int key) { return (unsigned)(key == 2048 ? kLoKey : key) << 20; }

// device-scope 64-bit store / load
__device__ __forceinline__ void dev_st64(void* base, int byte_off, unsigned long long v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(dev_u32x2, v), dev_rsrc(base), byte_off, 0, kSc1);
}
__device__ __forceinline__ unsigned long long dev_ld64(const void* base, int byte_off) {
  return __builtin_bit_cast(unsigned long long, dev_ld8(base, byte_off));
}
template <class T>
__device__ __forceinline__ int off_of(const SampleState* st, const T* field) {
  return (int)((const char*)field - (const char*)st);
}

struct Shared {
  unsigned n[kSampleL1Bins + 3];
  unsigned long long s[kSampleL1Bins + 3];
  unsigned bitmap[kSampleSlice / 32];
  unsigned long long red_s[kWaves];
  float red_f[kWaves];
  int found, lastnz, choice;
  unsigned last;
  unsigned long long above;
};

__device__ float block_max(float v, Shared& sh) {
  v = wave_max(v);
  if (lane_id() == 0) sh.red_f[wave_id()] = v;
  __syncthreads();
  float r = sh.red_f[0];
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, sh.red_f[w]);
  __syncthreads();
  return r;
}

// f32 sum in a fixed order: butterfly per wave, then the waves in order
__device__ float block_sum(float v, Shared& sh) {
  v = wave_sum(v);
  if (lane_id() == 0) sh.red_f[wave_id()] = v;
  __syncthreads();
  float r = sh.red_f[0];
  for (int w = 1; w < kWaves; ++w) r = r + sh.red_f[w];
  __syncthreads();
  return r;
}

__device__ unsigned long long block_sum_u64(unsigned long long v, Shared& sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if (lane_id() == 0) sh.red_s[wave_id()] = v;
  __syncthreads();
  unsigned long long r = 0;
  for (int w = 0; w < kWaves; ++w) r += sh.red_s[w];
  __syncthreads();
  return r;
}

// exclusive prefix over the threads in thread order
__device__ unsigned long long block_excl_scan(unsigned long long v, Shared& sh) {
  unsigned long long incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long t = __shfl_up(incl, o);
    if (lane_id() >= o) incl += t;
  }
  if (lane_id() == 63) sh.red_s[wave_id()] = incl;
  __syncthreads();
  unsigned long long base = 0;
  for (int w = 0; w < wave_id(); ++w) base += sh.red_s[w];
  __syncthreads();
  return base + incl - v;
}

// Publish, then take the launch's ticket: true in the last workgroup, whose
// device-scope reads then see every workgroup's results.
__device__ bool last_group(unsigned* ticket, int groups, Shared& sh) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) sh.last = atomicAdd(ticket, 1u) == (unsigned)groups - 1;
  __syncthreads();
  return sh.last != 0;
}

// Over ranks [0, nr) of (count, sum) pairs in LDS, walking down from
// `base`: the first rank at which the running sum exceeds T (strict) or
// reaches it at a non-empty rank; the last non-empty rank if none does.
// *above = the running sum before that rank.
__device__ int find_crossing(const unsigned* rn, const unsigned long long* rs, int nr, unsigned long long T,
                             bool strict, unsigned long long base, unsigned long long* above, Shared& sh) {
  const int tid = threadIdx.x;
  const int chunk = (nr + kT - 1) / kT;
  const int r0 = min(nr, tid * chunk), r1 = min(nr, r0 + chunk);
  unsigned long long local = 0;
  for (int r = r0; r < r1; ++r) local += rs[r];
  unsigned long long acc = base + block_excl_scan(local, sh);
  if (tid == 0) {
    sh.found = kNone;
    sh.lastnz = -1;
    sh.above = base;
  }
  __syncthreads();
  int mine = -1, nz = -1;
  unsigned long long mine_above = 0, nz_above = 0;
  for (int r = r0; r < r1; ++r) {
    const unsigned long long nxt = acc + rs[r];
    if (mine < 0 && (strict ? nxt > T : (rn[r] != 0 && nxt >= T))) {
      mine = r;
      mine_above = acc;
    }
    if (rn[r] != 0) {
      nz = r;
      nz_above = acc;
    }
    acc = nxt;
  }
  if (mine >= 0) atomicMin(&sh.found, mine);
  if (nz >= 0) atomicMax(&sh.lastnz, nz);
  __syncthreads();
  const int found = sh.found, lastnz = sh.lastnz;
  if (found != kNone) {
    if (mine == found) sh.above = mine_above;
  } else if (nz >= 0 && nz == lastnz) {
    sh.above = nz_above;
  }
  __syncthreads();
  *above = sh.above;
  __syncthreads();
  return found != kNone ? found : max(lastnz, 0);
}

// The first-level histogram in rank order into LDS (device-scope reads).
__device__ void load_l1(SampleState* st, Shared& sh) {
  for (int r = threadIdx.x; r < kSampleL1Bins; r += kT) {
    const int k = l1_rank_key(r);
    sh.n[r] = dev_ldu(st, off_of(st, &st->l1_n[k]));
    sh.s[r] = dev_ld64(st, off_of(st, &st->l1_s[k]));
  }
  __syncthreads();
}

// Starts the draw's selection at the first level over ranks [0, nr) in LDS
// (the cut bin's sum already replaced by what the cut keeps), r = st->r.
__device__ void start_draw(SampleState* st, unsigned long long r, int nr, Shared& sh) {
  unsigned long long above;
  const int rd = find_crossing(sh.n, sh.s, nr, r, false, 0, &above, sh);
  if (threadIdx.x == 0) {
    st->mode = 2;
    st->level = 1;
    st->bin1 = l1_rank_key(rd);
    st->above = above;
    st->target = r;
  }
}

// The ids of the history window in this workgroup's slice, as a bitmap.
__device__ void penalty_bitmap(const SampleArgs& a, int s0, int s1, Shared& sh) {
  for (int w = threadIdx.x; w < kSampleSlice / 32; w += kT) sh.bitmap[w] = 0;
  __syncthreads();
  if (a.penalty > 1.0f) {
    const int* hist = a.hist ? a.hist : a.tokens;
    const int len = a.hist ? a.n_hist : step_pos(a) + 1;
    const int w0 = a.window > 0 && len > a.window ? len - a.window : 0;
    for (int j = w0 + threadIdx.x; j < len; j += kT) {
      const int id = hist[j];
      if (id >= s0 && id < s1) atomicOr(&sh.bitmap[(id - s0) / 32], 1u << ((id - s0) % 32));
    }
  }
  __syncthreads();
}

// The step's result: probe outputs, end-of-sequence stop or the next token
// (as argmax_final does for greedy decoding).  Thread 0 of one workgroup.
__device__ void finish(const SampleArgs& a, int chosen) {
  if (a.out_token) a.out_token[0] = chosen;
  if (a.out_u) a.out_u[0] = (float)draw_u24(a) * (1.0f / 16777216.0f);
  if (!a.pos) return;
  const int pos = *a.pos;
  // only a draw after the last prompt token can end the sequence
  bool eos = false;
  if (pos + 1 >= *a.n_prompt)
    for (int e = 0; e < a.n_eos; ++e) eos = eos || a.eos[e] == chosen;
  if (eos) {
    *a.stopped = 1;  // main.rs:308-310: the id is not appended
    return;
  }
  if (pos + 1 < a.cap) {
    a.gen[pos + 1] = chosen;
    if (pos + 1 >= *a.n_prompt) a.tokens[pos + 1] = chosen;
  }
  *a.pos = pos + 1;
}

}  // namespace

// Penalty, temperature, per-workgroup max and sum of exp; the last
// workgroup forms the softmax max and sum.
extern "C" __global__ __launch_bounds__(kT) void sample_prep(SampleArgs a) {
  __shared__ Shared sh;
  if (a.stopped && *a.stopped) return;  // an end-of-sequence id was drawn earlier
  SampleState* st = a.st;
  const int tid = threadIdx.x, g = blockIdx.x;
  const int s0 = g * kSampleSlice, s1 = min(a.vocab, s0 + kSampleSlice);
  penalty_bitmap(a, s0, s1, sh);
  const bool temper = fabsf(a.temperature - 1.0f) > 1e-6f;
  float l[kPT];
  float mx = -3.40282347e38f;  // f32::MIN
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = s0 + tid + e * kT;
    l[e] = 0.0f;
    if (i < s1) {
      float v = a.logits[i];
      if ((sh.bitmap[(i - s0) / 32] >> ((i - s0) % 32)) & 1u) v = v < 0.0f ? v * a.penalty : v / a.penalty;
      if (temper) v = v / a.temperature;
      l[e] = v;
      a.probs[i] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = block_max(mx, sh);
  float es = 0.0f;
#pragma unroll
  for (int e = 0; e < kPT; ++e)
    if (s0 + tid + e * kT < s1) es += expf(l[e] - mx);
  es = block_sum(es, sh);
  if (tid == 0) {
    dev_stf(st, off_of(st, &st->wg_max[g]), mx);
    dev_stf(st, off_of(st, &st->wg_sum[g]), es);
  }
  if (!last_group(&st->ticket[0], a.groups, sh)) return;
  // the softmax max, and the sum rescaled to it in a fixed order
  constexpr int J = kSampleMaxGroups / kT;
  float m = -3.40282347e38f, w_m[J], w_s[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int w = tid * J + j;
    w_m[j] = w < a.groups ? dev_ldf(st, off_of(st, &st->wg_max[w])) : 0.0f;
    w_s[j] = w < a.groups ? dev_ldf(st, off_of(st, &st->wg_sum[w])) : 0.0f;
    if (w < a.groups) m = fmaxf(m, w_m[j]);
  }
  m = block_max(m, sh);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (tid * J + j < a.groups) s = s + w_s[j] * expf(w_m[j] - m);
  s = block_sum(s, sh);
  if (tid == 0) {
    st->M = m;
    st->S = s;
    st->ticket[0] = 0;
  }
}

// p = exp(l - max) / sum; the first-level histogram or (roulette) the
// workgroups' sums.  The last workgroup starts the top-p cut's selection,
// or the draw's when nothing is cut, or finds the roulette's workgroup.
extern "C" __global__ __launch_bounds__(kT) void sample_probs(SampleArgs a) {
  __shared__ Shared sh;
  if (a.stopped && *a.stopped) return;
  SampleState* st = a.st;
  const int tid = threadIdx.x, g = blockIdx.x;
  const int s0 = g * kSampleSlice, s1 = min(a.vocab, s0 + kSampleSlice);
  const float M = st->M, S = st->S;
  const bool roulette = !(a.top_p < 1.0f);
  if (!roulette) {
    for (int b = tid; b < kSampleL1Bins; b += kT) {
      sh.n[b] = 0;
      sh.s[b] = 0;
    }
    __syncthreads();
  }
  // roulette: thread t owns ids s0 + 2t, s0 + 2t + 1 (index order by thread)
  unsigned long long fsum = 0;
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = s0 + tid + e * kT;
    if (i < s1) {
      const float p = expf(a.probs[i] - M) / S;
      a.probs[i] = p;
      if (roulette) {
        fsum += to_fix(p);
      } else {
        const int k = l1_key(__float_as_uint(p));
        atomicAdd(&sh.n[k], 1u);
        atomicAdd(&sh.s[k], to_fix(p));
      }
    }
  }
  if (roulette) {
    fsum = block_sum_u64(fsum, sh);
    if (tid == 0) dev_st64(st, off_of(st, &st->wg_fix[g]), fsum);
  } else {
    __syncthreads();
    for (int b = tid; b < kSampleL1Bins; b += kT)
      if (sh.n[b]) {
        atomicAdd(&st->l1_n[b], sh.n[b]);
        atomicAdd(&st->l1_s[b], sh.s[b]);
      }
  }
  if (!last_group(&st->ticket[1], a.groups, sh)) return;

  const unsigned u24 = draw_u24(a);
  if (roulette) {
    // the workgroup whose running sum (index order) reaches r = U
    const unsigned long long r = scale24(to_fix(1.0f), u24);
    for (int w = tid; w < a.groups; w += kT) {
      sh.n[w] = 1;
      sh.s[w] = dev_ld64(st, off_of(st, &st->wg_fix[w]));
    }
    __syncthreads();
    unsigned long long tot = 0;
    for (int w = tid; w < a.groups; w += kT) tot += sh.s[w];
    tot = block_sum_u64(tot, sh);
    unsigned long long above;
    const int w = find_crossing(sh.n, sh.s, a.groups, r, false, 0, &above, sh);
    if (tid == 0) {
      st->r = r;
      st->pick = r > tot ? -1 : w;  // r never reached (rounding): id 0, as main.rs:286-292
      st->pick_base = above;
      st->ticket[1] = 0;
    }
    return;
  }
  load_l1(st, sh);
  unsigned long long cand = 0;
  for (int r = tid; r < kCandRanks; r += kT) cand += sh.n[r];
  const int nr = block_sum_u64(cand, sh) ? kCandRanks : kSampleL1Bins;  // none above 1e-5: every id
  unsigned long long tot = 0;
  for (int r = tid; r < nr; r += kT) tot += sh.s[r];
  tot = block_sum_u64(tot, sh);
  const unsigned long long tp = a.top_p > 0.0f ? (unsigned long long)(a.top_p * kFixOne) : 0ull;
  if (tot > tp) {
    unsigned long long above;
    const int rc = find_crossing(sh.n, sh.s, nr, tp, true, 0, &above, sh);
    if (tid == 0) {
      st->mode = 1;
      st->level = 1;
      st->bin1 = l1_rank_key(rc);
      st->cut_rank = rc;
      st->cut_base = above;
      st->above = above;
      st->target = tp;
    }
  } else {
    // no cut: every candidate, ties and all
    const unsigned long long r = scale24(tot, u24);
    if (tid == 0) {
      st->cut_rank = -1;
      st->vcut = 0;
      st->ktie = 0xFFFFFFFFu;
      st->total = tot;
      st->r = r;
    }
    start_draw(st, r, nr, sh);
  }
  if (tid == 0) st->ticket[1] = 0;
}

// One refine level of the selection in progress: the next 10 bits of the
// value inside the selected bin.  Nothing to do once the draw is resolved.
extern "C" __global__ __launch_bounds__(kT) void sample_refine(SampleArgs a) {
  __shared__ Shared sh;
  if (a.stopped && *a.stopped) return;
  SampleState* st = a.st;
  if (st->mode == 0) return;
  const int tid = threadIdx.x, g = blockIdx.x;
  const int s0 = g * kSampleSlice, s1 = min(a.vocab, s0 + kSampleSlice);
  const int level = st->level, bin1 = st->bin1;
  const unsigned digit2 = st->digit2;
  for (int b = tid; b < kSampleRBins; b += kT) {
    sh.n[b] = 0;
    sh.s[b] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = s0 + tid + e * kT;
    if (i < s1) {
      const float p = a.probs[i];
      const unsigned bits = __float_as_uint(p);
      if (l1_key(bits) == bin1 && (level == 1 || ((bits >> 10) & 1023u) == digit2)) {
        const int d = level == 1 ? (int)((bits >> 10) & 1023u) : (int)(bits & 1023u);
        atomicAdd(&sh.n[d], 1u);
        atomicAdd(&sh.s[d], to_fix(p));
      }
    }
  }
  __syncthreads();
  for (int b = tid; b < kSampleRBins; b += kT)
    if (sh.n[b]) {
      atomicAdd(&st->r_n[b], sh.n[b]);
      atomicAdd(&st->r_s[b], sh.s[b]);
    }
  if (!last_group(&st->ticket[2], a.groups, sh)) return;

  // descending digits as ranks; the global histogram cleared for the next level
  for (int r = tid; r < kSampleRBins; r += kT) {
    const int d = kSampleRBins - 1 - r;
    sh.n[r] = dev_ldu(st, off_of(st, &st->r_n[d]));
    sh.s[r] = dev_ld64(st, off_of(st, &st->r_s[d]));
  }
  __syncthreads();
  for (int d = tid; d < kSampleRBins; d += kT) {
    dev_stu(st, off_of(st, &st->r_n[d]), 0u);
    dev_st64(st, off_of(st, &st->r_s[d]), 0ull);
  }
  const int mode = st->mode;
  unsigned long long above;
  const int rank = find_crossing(sh.n, sh.s, kSampleRBins, st->target, mode == 1, st->above, &above, sh);
  const unsigned d = (unsigned)(kSampleRBins - 1 - rank);
  if (level == 1) {
    if (tid == 0) {
      st->digit2 = d;
      st->level = 2;
      st->above = above;
      st->ticket[2] = 0;
    }
    return;
  }
  const unsigned v = key_bits(bin1) | (digit2 << 10) | d;
  const unsigned long long fv = to_fix(__uint_as_float(v));
  if (mode == 1) {
    // the cut: ties at v in index order up to the first count whose sum
    // exceeds top_p; then the draw over what the cut keeps
    const unsigned long long tp = st->target;
    const unsigned ktie = fv && tp >= above ? (unsigned)((tp - above) / fv + 1) : 1u;
    const unsigned long long total = above + (unsigned long long)ktie * fv;
    const unsigned long long r = scale24(total, draw_u24(a));
    const int cr = st->cut_rank;
    const unsigned long long keep = above - st->cut_base + (unsigned long long)ktie * fv;
    if (tid == 0) {
      st->vcut = v;
      st->ktie = ktie;
      st->cut_above = above;
      st->total = total;
      st->r = r;
    }
    load_l1(st, sh);
    if (tid == 0) sh.s[cr] = keep;  // the cut bin: its part above v plus ktie ties
    __syncthreads();
    start_draw(st, r, cr + 1, sh);
  } else {
    // the draw: the k-th tie (index order) with the first running sum >= r
    const unsigned long long r = st->target;
    unsigned k = fv ? (unsigned)((r > above ? r - above + fv - 1 : 0) / fv) : 1u;
    k = max(k, 1u);
    if (v == st->vcut) k = min(k, st->ktie);
    if (tid == 0) {
      st->vsel = v;
      st->ksel = k;
      st->mode = 0;
    }
  }
  if (tid == 0) st->ticket[2] = 0;
}

// The drawn id - the k-th id (index order) of the selected value, or the
// roulette's id inside its workgroup - and the step's bookkeeping.
extern "C" __global__ __launch_bounds__(kT) void sample_pick(SampleArgs a) {
  __shared__ Shared sh;
  if (a.stopped && *a.stopped) return;
  SampleState* st = a.st;
  const int tid = threadIdx.x, g = blockIdx.x;
  if (!(a.top_p < 1.0f)) {
    const int pick = st->pick;
    if (g != max(pick, 0)) return;
    int chosen = 0;
    if (pick >= 0) {
      const int s0 = g * kSampleSlice, s1 = min(a.vocab, s0 + kSampleSlice);
      unsigned long long f[kPT], loc = 0;
#pragma unroll
      for (int e = 0; e < kPT; ++e) {
        const int i = s0 + kPT * tid + e;
        f[e] = i < s1 ? to_fix(a.probs[i]) : 0ull;
        loc += f[e];
      }
      unsigned long long acc = st->pick_base + block_excl_scan(loc, sh);
      if (tid == 0) sh.choice = kNone;
      __syncthreads();
      const unsigned long long r = st->r;
#pragma unroll
      for (int e = 0; e < kPT; ++e) {
        const int i = s0 + kPT * tid + e;
        acc += f[e];
        if (i < s1 && acc >= r) {
          atomicMin(&sh.choice, i);
          break;
        }
      }
      __syncthreads();
      chosen = sh.choice == kNone ? 0 : sh.choice;
    }
    if (tid == 0) finish(a, chosen);
    return;
  }
  // count the selected value in this slice
  const unsigned v = st->vsel;
  const int s0 = g * kSampleSlice, s1 = min(a.vocab, s0 + kSampleSlice);
  unsigned long long c = 0;
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = s0 + tid + e * kT;
    if (i < s1) c += __float_as_uint(a.probs[i]) == v;
  }
  c = block_sum_u64(c, sh);
  if (tid == 0) dev_st64(st, off_of(st, &st->wg_fix[g]), c);
  if (!last_group(&st->ticket[3], a.groups, sh)) return;
  for (int w = tid; w < a.groups; w += kT) {
    sh.s[w] = dev_ld64(st, off_of(st, &st->wg_fix[w]));
    sh.n[w] = sh.s[w] != 0;
  }
  __syncthreads();
  const unsigned k = st->ksel;
  unsigned long long before;
  const int w = find_crossing(sh.n, sh.s, a.groups, k, false, 0, &before, sh);
  // the (k - before)-th occurrence inside workgroup w's slice, index order
  const int w0 = w * kSampleSlice, w1 = min(a.vocab, w0 + kSampleSlice);
  unsigned cnt = 0;
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = w0 + kPT * tid + e;
    cnt += i < w1 && __float_as_uint(a.probs[i]) == v;
  }
  unsigned long long seen = before + block_excl_scan(cnt, sh);
  if (tid == 0) sh.choice = kNone;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kPT; ++e) {
    const int i = w0 + kPT * tid + e;
    if (i < w1 && __float_as_uint(a.probs[i]) == v && ++seen == k) atomicMin(&sh.choice, i);
  }
  // the first-level histogram cleared for the next step
  for (int b = tid; b < kSampleL1Bins; b += kT) {
    dev_stu(st, off_of(st, &st->l1_n[b]), 0u);
    dev_st64(st, off_of(st, &st->l1_s[b]), 0ull);
  }
  __syncthreads();
  if (tid == 0) {
    finish(a, sh.choice == kNone ? 0 : sh.choice);
    st->ticket[3] = 0;
  }
}
