// attention.hip - batch-1 decode attention over the KV cache for gfx950.
//
// Reference: LlamaAttention::forward, seq == 1 (layer.rs:175-299): per query
// head, RoPE on q and k (layer.rs:216-217, cpu.rs:326-357), K/V append at
// pos (layer.rs:219-246), scores = q.K_t * (1/sqrt(hd)) (layer.rs:257-258),
// softmax (cpu.rs:395-423), ctx = sum_t p_t V_t (layer.rs:276-299).
//
// MI355X design: one workgroup per (KV head, sequence split).  The group's
// n_rep query heads share every K/V tile (true GQA: the reference instead
// duplicates K/V rows per query head, loader.rs:62-98, which gives the same
// numbers).  K/V tiles of 64 positions are staged through LDS with 16-byte
// loads; each lane owns one position for the q.K dot (sequential over d, as
// the reference's dot is) and two head dimensions for P.V; softmax is online
// (running max and sum).  The workgroup owning position `pos` rotates the
// new k and appends k and v to the cache.  Partials (m, l, acc) go to global
// memory; the last workgroup of a KV head (atomic ticket) combines them and
// writes ctx as f32 and as Q8_0 codes for the O projection.
//
// RoPE uses cos/sin tables [max_seq][hd/2] computed on the host with the
// reference's own f32 formula and glibc, so rotation is bit-exact.
#include "common.h"
#include "../kernel_args.h"

using namespace llmrs;


template <bool KV16>
struct KvType;
template <>
struct KvType<true> {
  typedef uint16_t T;
};
template <>
struct KvType<false> {
  typedef float T;
};

template <bool KV16>
__device__ __forceinline__ float kv_to_f(typename KvType<KV16>::T v) {
  if constexpr (KV16) return h2f(v);
  else return v;
}

template <int HD, bool KV16>
__device__ __forceinline__ void attn_decode_impl(const AttnArgs& a) {
  typedef typename KvType<KV16>::T kv_t;
  constexpr int TILE = (HD == 128 && !KV16) ? 32 : 64;
  constexpr int KP = HD + 1;  // padded K rows: lane-per-position reads are conflict-free
  constexpr int MID = HD / 2;
  constexpr int DPL = HD / LLMRS_WAVE;  // head dims per lane in P.V
  constexpr int MAXREP = 8;             // query heads per KV head supported
  constexpr int SLOTS = MAXREP / 4;     // heads per wave

  __shared__ float s_q[MAXREP][HD];
  __shared__ float s_k[TILE][KP];
  __shared__ kv_t s_v[TILE][HD];
  __shared__ float s_p[4][LLMRS_WAVE];
  __shared__ float s_new[2][HD];
  __shared__ int s_ticket;

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int g = blockIdx.y, split = blockIdx.x;
  const int pos = *a.pos_ptr;
  const int T = pos + 1;
  const int n_rep = a.nq / a.nkv;
  const int chunk = (T + a.nsplit - 1) / a.nsplit;
  const int start = split * chunk;
  const int end = min(T, start + chunk);
  const int qdim = a.nq * HD;
  const float* rc = a.rope_cos + (size_t)pos * MID;
  const float* rs = a.rope_sin + (size_t)pos * MID;
  kv_t* kc = (kv_t*)a.kc + (size_t)g * a.max_seq * HD;
  kv_t* vc = (kv_t*)a.vc + (size_t)g * a.max_seq * HD;

  // Rotated query heads of this group (cpu.rs:351-354).
  for (int i = tid; i < n_rep * MID; i += blockDim.x) {
    const int hr = i / MID, j = i % MID;
    const float* q = a.qkv + (size_t)(g * n_rep + hr) * HD;
    const float re = q[j], im = q[j + MID], c = rc[j], s = rs[j];
    s_q[hr][j] = re * c - im * s;
    s_q[hr][j + MID] = re * s + im * c;
  }
  // The owner of position pos rotates k and appends k, v (layer.rs:219-246).
  const bool owner = pos >= start && pos < end;
  if (owner) {
    const float* kr = a.qkv + qdim + (size_t)g * HD;
    const float* vr = a.qkv + qdim + (size_t)a.nkv * HD + (size_t)g * HD;
    for (int j = tid; j < MID; j += blockDim.x) {
      const float re = kr[j], im = kr[j + MID], c = rc[j], s = rs[j];
      const float k0 = re * c - im * s, k1 = re * s + im * c;
      if constexpr (KV16) {
        const uint16_t h0 = f2h(k0), h1 = f2h(k1);
        kc[(size_t)pos * HD + j] = h0;
        kc[(size_t)pos * HD + j + MID] = h1;
        s_new[0][j] = h2f(h0);
        s_new[0][j + MID] = h2f(h1);
      } else {
        kc[(size_t)pos * HD + j] = k0;
        kc[(size_t)pos * HD + j + MID] = k1;
        s_new[0][j] = k0;
        s_new[0][j + MID] = k1;
      }
    }
    for (int d = tid; d < HD; d += blockDim.x) {
      const float v = vr[d];
      if constexpr (KV16) {
        const uint16_t h = f2h(v);
        vc[(size_t)pos * HD + d] = h;
        s_new[1][d] = h2f(h);
      } else {
        vc[(size_t)pos * HD + d] = v;
        s_new[1][d] = v;
      }
    }
  }

  float m[SLOTS], l[SLOTS], acc[SLOTS][DPL];
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[j][e] = 0.0f;
  }

  for (int t0 = start; t0 < end; t0 += TILE) {
    __syncthreads();  // previous tile fully consumed; s_q / s_new written
    // Stage K (as f32) and V (as stored) rows [t0, t0+TILE) with 16-byte loads.
    constexpr int EPC = 16 / sizeof(kv_t);  // elements per 16-byte chunk
    constexpr int CPR = HD / EPC;           // chunks per row
    for (int c = tid; c < TILE * CPR; c += blockDim.x) {
      const int r = c / CPR, col = (c % CPR) * EPC;
      const int t = t0 + r;
      float kf[EPC];
      kv_t vv[EPC];
      // Rows past `end` are zero-filled: they belong to the next split
      // (possibly the owner of pos, whose s_new this workgroup never wrote)
      // and a 0 * NaN from stale LDS would poison P.V.
      if (t < end && t != pos) {
        const uint4 kraw = *(const uint4*)(kc + (size_t)t * HD + col);
        const uint4 vraw = *(const uint4*)(vc + (size_t)t * HD + col);
        const kv_t* kp = (const kv_t*)&kraw;
        const kv_t* vp = (const kv_t*)&vraw;
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          kf[e] = kv_to_f<KV16>(kp[e]);
          vv[e] = vp[e];
        }
      } else if (t < end) {  // t == pos: this workgroup is the owner
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          kf[e] = s_new[0][col + e];
          if constexpr (KV16) vv[e] = f2h(s_new[1][col + e]);
          else vv[e] = s_new[1][col + e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          kf[e] = 0.0f;
          vv[e] = (kv_t)0;
        }
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        s_k[r][col + e] = kf[e];
        s_v[r][col + e] = vv[e];
      }
    }
    __syncthreads();

#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int hr = 4 * j + wave;
      const bool active = hr < n_rep;
      float sc = -INFINITY;
      const int t = t0 + lane;
      if (active && lane < TILE && t < end) {
        float s = 0.0f;
        for (int d = 0; d < HD; ++d) s = s + s_q[hr][d] * s_k[lane][d];  // cpu.rs:548
        sc = s * a.scale;
      }
      const float tmax = group_max(sc);
      const float mnew = fmaxf(m[j], tmax);
      const float p = (sc == -INFINITY) ? 0.0f : expf(sc - mnew);
      const float corr = (m[j] == -INFINITY) ? 0.0f : expf(m[j] - mnew);
      l[j] = l[j] * corr + group_sum(p);
      m[j] = mnew;
      s_p[wave][lane] = p;
      __syncthreads();
      if (active) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          const int d = lane + LLMRS_WAVE * e;
          float o = acc[j][e] * corr;
          for (int u = 0; u < TILE; ++u) o = o + s_p[wave][u] * kv_to_f<KV16>(s_v[u][d]);
          acc[j][e] = o;
        }
      }
      __syncthreads();
    }
  }

  // Partials of this split.
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    const int hr = 4 * j + wave;
    if (hr < n_rep) {
      const int h = g * n_rep + hr;
      const size_t idx = (size_t)h * a.nsplit + split;
      if (lane == 0) {
        a.part_ml[2 * idx] = m[j];
        a.part_ml[2 * idx + 1] = l[j];
      }
#pragma unroll
      for (int e = 0; e < DPL; ++e) a.part_o[idx * HD + lane + LLMRS_WAVE * e] = acc[j][e];
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_ticket = atomicAdd(&a.counters[g], 1);
  __syncthreads();
  if (s_ticket != a.nsplit - 1) return;
  __threadfence();

  // Last workgroup of this KV head: combine the splits.
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    const int hr = 4 * j + wave;
    if (hr >= n_rep) continue;
    const int h = g * n_rep + hr;
    const size_t base = (size_t)h * a.nsplit;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, __builtin_nontemporal_load(&a.part_ml[2 * (base + s)]));
    float L = 0.0f, o[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[e] = 0.0f;
    for (int s = 0; s < a.nsplit; ++s) {
      const float ms = __builtin_nontemporal_load(&a.part_ml[2 * (base + s)]);
      if (ms == -INFINITY) continue;
      const float w = expf(ms - M);
      L = L + __builtin_nontemporal_load(&a.part_ml[2 * (base + s) + 1]) * w;
#pragma unroll
      for (int e = 0; e < DPL; ++e)
        o[e] = o[e] + __builtin_nontemporal_load(&a.part_o[(base + s) * HD + lane + LLMRS_WAVE * e]) * w;
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + LLMRS_WAVE * e;
      const float v = o[e] / L;
      a.ctx[(size_t)h * HD + d] = v;
      float dq;
      const int q = q8_group32(v, &dq);  // lanes 0-31 / 32-63 hold one 32-block each
      a.ctx_q[(size_t)h * HD + d] = (int8_t)q;
      if ((lane & 31) == 0) a.ctx_d[((size_t)h * HD + d) / 32] = dq;
    }
  }
  if (tid == 0) a.counters[g] = 0;
}

#define LLMRS_ATTN(name, HD, KV16)                                           \
  extern "C" __global__ __launch_bounds__(256) void name(AttnArgs a) {      \
    attn_decode_impl<HD, KV16>(a);                                          \
  }

LLMRS_ATTN(attn_decode_hd64_f32, 64, false)
LLMRS_ATTN(attn_decode_hd64_f16, 64, true)
LLMRS_ATTN(attn_decode_hd128_f32, 128, false)
LLMRS_ATTN(attn_decode_hd128_f16, 128, true)
