// attn_core.h - batch-1 decode attention over the KV cache for gfx950
// (instantiated by attention.hip).
//
// Reference: LlamaAttention::forward, seq == 1 (layer.rs:175-299): per query
// head, RoPE on q and k (layer.rs:216-217, cpu.rs:326-357), K/V append at
// pos (layer.rs:219-246), scores = q.K_t * (1/sqrt(hd)) (layer.rs:257-258),
// softmax (cpu.rs:395-423), ctx = sum_t p_t V_t (layer.rs:276-299).
//
// MI355X design: one workgroup per (KV head, sequence split), 4 waves.  The
// group's n_rep query heads share every K/V tile (true GQA: the reference
// instead duplicates K/V rows per query head, loader.rs:62-98, which gives
// the same numbers).  Splits take 32-position tiles round-robin.  Per tile:
//  - the K and V rows are requested with 16-byte loads for the whole tile at
//    once (and the next tile's loads are issued before this tile is used),
//    then staged through LDS, K rows padded so lane-per-position reads are
//    conflict-free;
//  - wave w owns query heads w, w+4: lanes p and p+32 form the score of
//    position p over the first and second half of the head dims (q
//    broadcast from LDS, f32 accumulate of f32 q times the stored K), so
//    every lane works and a tile costs half the instructions of a 64-lane
//    row walk over all dims;
//  - softmax is online per head (running max and sum, DPP wave reductions);
//  - for P.V lane l owns head dims 2l, 2l+1 (HD=128) or l (HD=64); the
//    probabilities are broadcast from the lane that holds them.
// The workgroup owning position `pos` rotates the new k and appends k and v
// to the cache.  Partials (m, l, acc) go to global memory; the last
// workgroup of a KV head (atomic ticket; partials move with device-scope
// stores and loads) combines them and writes ctx as f32 and as Q8_0 codes
// for the O projection.
//
// RoPE uses cos/sin tables [max_seq][hd/2] computed on the host with the
// reference's own f32 formula and glibc, so rotation is bit-exact.
#pragma once
#include "common.h"
#include "../kernel_args.h"

namespace llmrs {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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


template <bool DEV>
__device__ __forceinline__ float ld_qkv(const float* base, size_t idx) {
  if (DEV) return dev_ldf(base, (int)(idx * 4));
  return base[idx];
}
template <bool DEV>
__device__ __forceinline__ float ld_part(const float* base, size_t idx) {
  if (DEV) return dev_ldf(base, (int)(idx * 4));
  return __builtin_nontemporal_load(base + idx);
}
// Cache element store: `p` is the group's row base (plain path), `base` the
// layer buffer with element index `idx` (device-scope path).
template <bool DEV>
__device__ __forceinline__ void st_kv(uint16_t* p, void* base, size_t idx, uint16_t v) {
  if (DEV) dev_st_u16(base, (int)(idx * 2), v);
  else ((uint16_t*)base)[idx] = v;
}
template <bool DEV>
__device__ __forceinline__ void st_kv(float* p, void* base, size_t idx, float v) {
  if (DEV) dev_stf(base, (int)(idx * 4), v);
  else ((float*)base)[idx] = v;
}

template <int HD, bool KV16>
struct AttnCfg {
  typedef typename KvType<KV16>::T kv_t;
  static constexpr int TILE = attn_tile(KV16);            // positions per tile (32)
  static constexpr int EPC = 16 / (int)sizeof(kv_t);      // elements per 16 B
  static constexpr int CPR = HD / EPC;                    // 16 B chunks per row
  static constexpr int CHUNKS = TILE * CPR;               // per tile, K or V
  static constexpr int CPT = CHUNKS / 256;                // chunks per thread
  static constexpr int KSTRIDE = HD + (KV16 ? 2 : 1);     // padded K row (elements)
  static constexpr int MAXREP = 8;                        // query heads per KV head
  static constexpr int HPW = MAXREP / 4;                  // heads per wave
  static constexpr int DPL = HD / LLMRS_WAVE;             // head dims per lane in P.V
  static_assert(CHUNKS % 256 == 0, "tile must split evenly over 256 threads");
  static_assert(TILE == LLMRS_WAVE / 2, "two lanes (half rows) per position");
};

// LDS carve-up of one work item (bytes): s_q, then per stream a padded K
// tile and a V tile, s_new, ticket.
template <int HD, bool KV16, int S = 1>
struct AttnLds {
  typedef AttnCfg<HD, KV16> C;
  typedef typename C::kv_t kv_t;
  static constexpr size_t Q = 0;
  static constexpr size_t KBYTES = ((sizeof(kv_t) * C::TILE * C::KSTRIDE + 15) / 16) * 16;
  static constexpr size_t STREAM = KBYTES + sizeof(kv_t) * C::TILE * HD;
  static constexpr size_t K0 = Q + sizeof(float) * C::MAXREP * HD;
  static constexpr size_t NEW = K0 + S * STREAM;
  static constexpr size_t TICKET = NEW + sizeof(float) * 2 * HD;
  static constexpr size_t BYTES = TICKET + 16;
  static constexpr size_t K(int st) { return K0 + (size_t)st * STREAM; }
  static constexpr size_t V(int st) { return K(st) + KBYTES; }
  // stream merge area (reuses the tiles): per stream, head, dims + (m, l)
  static constexpr size_t MERGE_BYTES = sizeof(float) * S * C::MAXREP * (HD + 2);
  static_assert(S == 1 || MERGE_BYTES <= S * STREAM, "merge area fits in the tiles");
  static_assert(BYTES == attn_lds_bytes(HD, KV16, S), "host LDS size formula out of date");
};

struct NoWait {
  __device__ __forceinline__ bool operator()() const { return true; }
};

// `wait` runs after the first K/V tile has been requested and before the
// projections are read: a launch that also computes the projections waits
// there for them (returning false abandons the item).  Returns true for the
// workgroup that combined the splits of KV head g (ctx written).
//
// S > 1 runs S streams of 4 waves in one workgroup (256 * S threads): stream
// st takes every S-th tile of the split, with its own online softmax, and
// the streams merge through LDS before the partials are written, so a long
// context needs S times fewer splits for the same parallelism (and the
// combine reads S times fewer partials).
template <int HD, bool KV16, bool DEV, int S = 1, bool LOCAL = false, class Wait = NoWait>
__device__ __forceinline__ bool attn_item(const AttnArgs& a, int g, int split, int pos, uint8_t* lds,
                                          const Wait& wait = Wait()) {
  typedef AttnCfg<HD, KV16> C;
  typedef AttnLds<HD, KV16, S> LY;
  typedef typename C::kv_t kv_t;
  constexpr int TILE = C::TILE, MID = HD / 2, HPW = C::HPW, DPL = C::DPL;
  constexpr int ES = (int)sizeof(kv_t);

  const int tid = threadIdx.x, lane = lane_id();
  const int stm = wave_id() / 4, wave = wave_id() % 4;  // stream, wave within the stream
  // LOCAL: all splits of KV head g run on one XCD (the caller's mapping)
  // and exchange partials through its L2; otherwise with device-scope
  // operations that bypass the per-XCD L2 copies.
  constexpr bool loc = LOCAL;
  const int ltid = tid % 256;                           // thread within the stream
  float (*s_q)[HD] = (float (*)[HD])(lds + LY::Q);
  kv_t* s_k = (kv_t*)(lds + LY::K(stm));
  kv_t* s_v = (kv_t*)(lds + LY::V(stm));
  float (*s_new)[HD] = (float (*)[HD])(lds + LY::NEW);
  int& s_ticket = *(int*)(lds + LY::TICKET);

  // Profiling stamps, kept in registers and stored when the item ends (a
  // store issued mid-kernel would make the next reuse of its data registers
  // wait for every outstanding load).
  const bool prof = a.ts != nullptr;
  unsigned long long st[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto stamp = [&](int k) {
    if (prof) st[k] = __builtin_amdgcn_s_memrealtime();
  };
  auto flush_stamps = [&]() {
    if (prof && tid == 0) {
      unsigned long long* dst = a.ts + ((size_t)g * a.nsplit + split) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = st[i];
    }
  };
  stamp(0);
  if (prof)  // where it ran: XCC id << 32 | HW_ID
    st[7] = ((unsigned long long)__builtin_amdgcn_s_getreg((15 << 11) | 20) << 32) |
            (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);
  const int n_rep = a.nq / a.nkv;
  // Tiles are dealt to the splits round-robin: stream st of split s takes
  // tiles (it * S + st) * nsplit + s, it = 0, 1, ...  The first tile of every
  // stream is therefore known without the position, and its loads are
  // requested before the position has arrived; rows past the context are
  // clamped to the cache and masked.
  const int first = (stm * a.nsplit + split) * TILE;  // this stream's first tile
  const int stride = S * a.nsplit * TILE;             // and the distance to its next one
  const int qdim = a.nq * HD;
  const size_t gbase = (size_t)g * a.max_seq * HD;  // elements
  kv_t* kc = (kv_t*)a.kc + gbase;
  kv_t* vc = (kv_t*)a.vc + gbase;

  // Tile loader: chunk c of the tile = row c / CPR, columns (c % CPR) * EPC.
  u32x4 pk[C::CPT], pv[C::CPT];
  auto issue = [&](int t0) {
#pragma unroll
    for (int i = 0; i < C::CPT; ++i) {
      const int c = ltid + 256 * i;
      const int t = min(t0 + c / C::CPR, a.max_seq - 1);  // clamped: rows past the context are masked
      const int col = (c % C::CPR) * C::EPC;
      if (DEV) {
        const int off = (int)((gbase + (size_t)t * HD + col) * ES);
        pk[i] = dev_ld16(a.kc, off);
        pv[i] = dev_ld16(a.vc, off);
      } else {
        pk[i] = *(const u32x4*)(kc + (size_t)t * HD + col);
        pv[i] = *(const u32x4*)(vc + (size_t)t * HD + col);
      }
    }
  };
  issue(first);
  // Keep the position's uses (and the wait for it) below the tile requests.
  __builtin_amdgcn_sched_barrier(0);
  const int T = pos + 1;
  const float* rc = a.rope_cos + (size_t)pos * MID;
  const float* rs = a.rope_sin + (size_t)pos * MID;
  if (!wait()) return false;

  // Rotated query heads of this group (cpu.rs:351-354) and, for the owner
  // of position pos, the rotated k and the v it appends (layer.rs:219-246).
  // Every projection and table value is loaded first, in one batch, so the
  // section costs one memory round trip.
  const bool owner = (pos / TILE) % a.nsplit == split;  // holds the new position's tile
  const bool qthr = tid < 256;  // the projections are read by the first 256 threads
  constexpr int QPT = (C::MAXREP * MID + 255) / 256;  // query pairs per thread
  const size_t kr = qdim + (size_t)g * HD;
  const size_t vr = qdim + (size_t)a.nkv * HD + (size_t)g * HD;
  float qre[QPT], qim[QPT], qc[QPT], qs[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = min(tid + 256 * u, n_rep * MID - 1);  // clamped: extra ones unused
    const int hr = i / MID, j = i % MID;
    const size_t q = (size_t)(g * n_rep + hr) * HD;
    qre[u] = ld_qkv<DEV>(a.qkv, q + j);
    qim[u] = ld_qkv<DEV>(a.qkv, q + j + MID);
    qc[u] = rc[j];
    qs[u] = rs[j];
  }
  const bool kown = owner && tid < MID, vown = owner && tid < HD;  // tid < 256
  float kre = 0.0f, kim = 0.0f, kcs = 0.0f, ksn = 0.0f, vv = 0.0f;
  if (kown) {
    kre = ld_qkv<DEV>(a.qkv, kr + tid);
    kim = ld_qkv<DEV>(a.qkv, kr + tid + MID);
    kcs = rc[tid];
    ksn = rs[tid];
  }
  if (vown) vv = ld_qkv<DEV>(a.qkv, vr + tid);
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = tid + 256 * u;
    if (qthr && i < n_rep * MID) {
      const int hr = i / MID, j = i % MID;
      s_q[hr][j] = qre[u] * qc[u] - qim[u] * qs[u];
      s_q[hr][j + MID] = qre[u] * qs[u] + qim[u] * qc[u];
    }
  }
  // The owner keeps the stored values in s_new: its own tile loads may have
  // been issued before these stores.
  if (kown) {
    const int j = tid;
    const float k0 = kre * kcs - kim * ksn, k1 = kre * ksn + kim * kcs;
    if constexpr (KV16) {
      const uint16_t h0 = f2h(k0), h1 = f2h(k1);
      st_kv<DEV>(kc, a.kc, gbase + (size_t)pos * HD + j, h0);
      st_kv<DEV>(kc, a.kc, gbase + (size_t)pos * HD + j + MID, h1);
      s_new[0][j] = h2f(h0);
      s_new[0][j + MID] = h2f(h1);
    } else {
      st_kv<DEV>(kc, a.kc, gbase + (size_t)pos * HD + j, k0);
      st_kv<DEV>(kc, a.kc, gbase + (size_t)pos * HD + j + MID, k1);
      s_new[0][j] = k0;
      s_new[0][j + MID] = k1;
    }
  }
  if (vown) {
    const int d = tid;
    if constexpr (KV16) {
      const uint16_t h = f2h(vv);
      st_kv<DEV>(vc, a.vc, gbase + (size_t)pos * HD + d, h);
      s_new[1][d] = h2f(h);
    } else {
      st_kv<DEV>(vc, a.vc, gbase + (size_t)pos * HD + d, vv);
      s_new[1][d] = vv;
    }
  }

  float m[HPW], l[HPW], acc[HPW][DPL];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[j][e] = 0.0f;
  }

  stamp(1);
  for (int it = 0; (it * S * a.nsplit + split) * TILE < T; ++it) {
    const int t0 = first + it * stride;  // this stream's tile
    const bool have = t0 < T;            // uniform per stream
    __syncthreads();  // previous tile consumed; s_q / s_new written
    if (have) {
      // Stage the tile (already loaded into registers) into LDS: V rows with
      // 16-byte stores, padded K rows with 4-byte stores.
#pragma unroll
      for (int i = 0; i < C::CPT; ++i) {
        const int c = ltid + 256 * i;
        const int r = c / C::CPR, col = (c % C::CPR) * C::EPC;
        u32x4 kw = pk[i], vw = pv[i];
        if (t0 + r == pos) {  // owner only: the row it just wrote
          kv_t* kp = (kv_t*)&kw;
          kv_t* vp = (kv_t*)&vw;
#pragma unroll
          for (int e = 0; e < C::EPC; ++e) {
            if constexpr (KV16) {
              kp[e] = f2h(s_new[0][col + e]);
              vp[e] = f2h(s_new[1][col + e]);
            } else {
              kp[e] = s_new[0][col + e];
              vp[e] = s_new[1][col + e];
            }
          }
        }
        unsigned* kd = (unsigned*)(s_k + r * C::KSTRIDE + col);
        kd[0] = kw.x;
        kd[1] = kw.y;
        kd[2] = kw.z;
        kd[3] = kw.w;
        *(u32x4*)(s_v + r * HD + col) = vw;
      }
    }
    if (t0 + stride < T) issue(t0 + stride);  // next tile in flight during this one
    __syncthreads();
    if (it == 0) stamp(2);
    if (!have) continue;

    const int tvalid = min(TILE, T - t0);
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const int hr = wave + 4 * j;
      if (hr >= n_rep) continue;  // uniform per wave
      // Score of position t0 + (lane % 32): lanes 32..63 sum the second half
      // of the head dims and the halves are added across the wave.  Four
      // partial sums (d mod 4) per half instead of the reference's one
      // sequential sum (cpu.rs:548): with one wave per SIMD nothing hides the
      // latency of a single dependent FMA chain.  Lanes 32..63 then carry
      // -inf, so each position enters the softmax once.
      float sc = -INFINITY;
      {
        const int prow = lane & (TILE - 1), dbase = (lane >> 5) * (HD / 2);
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        // 32-bit LDS reads of the padded row: bank (prow*KSTRIDE/2 + i) mod 32
        // differs across the 32 lanes of each half.
        const unsigned* krow = (const unsigned*)(s_k + prow * C::KSTRIDE);
#pragma unroll 8
        for (int i = 0; i < HD / 2; i += 4) {
          const int d = dbase + i;
          const f32x4 q4 = *(const f32x4*)&s_q[hr][d];
          float k0, k1, k2, k3;
          if constexpr (KV16) {
            const unsigned w0 = krow[d / 2], w1 = krow[d / 2 + 1];
            k0 = h2f((uint16_t)(w0 & 0xFFFF));
            k1 = h2f((uint16_t)(w0 >> 16));
            k2 = h2f((uint16_t)(w1 & 0xFFFF));
            k3 = h2f((uint16_t)(w1 >> 16));
          } else {
            k0 = __uint_as_float(krow[d]);
            k1 = __uint_as_float(krow[d + 1]);
            k2 = __uint_as_float(krow[d + 2]);
            k3 = __uint_as_float(krow[d + 3]);
          }
          s0 = __builtin_fmaf(q4.x, k0, s0);
          s1 = __builtin_fmaf(q4.y, k1, s1);
          s2 = __builtin_fmaf(q4.z, k2, s2);
          s3 = __builtin_fmaf(q4.w, k3, s3);
        }
        float sp = (s0 + s1) + (s2 + s3);
        sp = sp + __shfl_xor(sp, 32);
        if (lane < TILE && prow < tvalid) sc = sp * a.scale;
      }
      const float mnew = fmaxf(m[j], wave_max(sc));
      const float p = (sc == -INFINITY) ? 0.0f : expf(sc - mnew);
      const float corr = (m[j] == -INFINITY) ? 0.0f : expf(m[j] - mnew);
      l[j] = l[j] * corr + wave_sum(p);
      m[j] = mnew;
      // P.V over the tile's positions in four independent partial sums
      // (position mod 4); a full tile is unrolled so the LDS reads of
      // successive rows overlap.  p of position u sits in lane u.
      float pt[4][DPL];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < DPL; ++e) pt[c][e] = 0.0f;
      auto pv_row = [&](int u, int c) {
        const float pu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), u));
        const kv_t* vrow = s_v + u * HD + DPL * lane;
        if constexpr (KV16 && DPL == 2) {
          const unsigned w = *(const unsigned*)vrow;
          pt[c][0] = __builtin_fmaf(pu, h2f((uint16_t)(w & 0xFFFF)), pt[c][0]);
          pt[c][1] = __builtin_fmaf(pu, h2f((uint16_t)(w >> 16)), pt[c][1]);
        } else {
#pragma unroll
          for (int e = 0; e < DPL; ++e) pt[c][e] = __builtin_fmaf(pu, kv_to_f<KV16>(vrow[e]), pt[c][e]);
        }
      };
      if (tvalid == TILE) {
#pragma unroll
        for (int u = 0; u < TILE; u += 4) {
          pv_row(u, 0);
          pv_row(u + 1, 1);
          pv_row(u + 2, 2);
          pv_row(u + 3, 3);
        }
      } else {
        for (int u = 0; u < tvalid; ++u) pv_row(u, 0);
      }
#pragma unroll
      for (int e = 0; e < DPL; ++e)
        acc[j][e] = acc[j][e] * corr + ((pt[0][e] + pt[1][e]) + (pt[2][e] + pt[3][e]));
    }
  }

  stamp(3);
  if constexpr (S > 1) {
    // Merge the streams into stream 0 (every stream covered the same heads
    // with its own running max): through LDS, reusing the tiles.
    float* mg = (float*)(lds + LY::K(0));
    __syncthreads();  // tiles consumed
    if (stm > 0) {
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        const int hr = wave + 4 * j;
        if (hr >= n_rep) continue;
        float* dst = mg + ((size_t)stm * C::MAXREP + hr) * (HD + 2);
#pragma unroll
        for (int e = 0; e < DPL; ++e) dst[DPL * lane + e] = acc[j][e];
        if (lane == 0) {
          dst[HD] = m[j];
          dst[HD + 1] = l[j];
        }
      }
    }
    __syncthreads();
    if (stm == 0) {
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        const int hr = wave + 4 * j;
        if (hr >= n_rep) continue;
        float M = m[j];
        for (int q = 1; q < S; ++q) M = fmaxf(M, mg[((size_t)q * C::MAXREP + hr) * (HD + 2) + HD]);
        const float c0 = m[j] == -INFINITY ? 0.0f : expf(m[j] - M);
        float Ls = l[j] * c0, av[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) av[e] = acc[j][e] * c0;
        for (int q = 1; q < S; ++q) {
          const float* src = mg + ((size_t)q * C::MAXREP + hr) * (HD + 2);
          const float mq = src[HD];
          const float cq = mq == -INFINITY ? 0.0f : expf(mq - M);
          Ls = Ls + src[HD + 1] * cq;
#pragma unroll
          for (int e = 0; e < DPL; ++e) av[e] = av[e] + src[DPL * lane + e] * cq;
        }
        m[j] = M;
        l[j] = Ls;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = av[e];
      }
    }
  }
  // Partials of this split (stream 0's waves).
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int hr = wave + 4 * j;
    if (stm == 0 && hr < n_rep) {
      const int h = g * n_rep + hr;
      const size_t idx = (size_t)h * a.nsplit + split;
      if (loc) {
        if (lane == 0) {
          a.part_ml[2 * idx] = m[j];
          a.part_ml[2 * idx + 1] = l[j];
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) a.part_o[idx * HD + DPL * lane + e] = acc[j][e];
      } else {
        if (lane == 0) {
          st_act<true>(a.part_ml, 2 * idx, m[j]);
          st_act<true>(a.part_ml, 2 * idx + 1, l[j]);
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) st_act<true>(a.part_o, idx * HD + DPL * lane + e, acc[j][e]);
      }
    }
  }
  // Publish the partials, then take a ticket; the last workgroup combines.
  // The stores only need to have completed before the ticket: no agent-scope
  // fence (a write-back and invalidate of the whole L2, microseconds under
  // contention) is needed.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  stamp(4);
  if (tid == 0)
    s_ticket = loc ? __hip_atomic_fetch_add(&a.counters[g * kTicketStride], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP)
                   : atomicAdd(&a.counters[g * kTicketStride], 1);
  __syncthreads();
  stamp(5);
  if (s_ticket != a.nsplit - 1) {
    flush_stamps();
    return false;
  }

  // Last workgroup of this KV head: combine the splits, one query head per
  // wave over all 4 * S waves of the workgroup (with 4 streams, 16 waves for
  // at most 8 heads, so no wave combines two heads one after the other).
#pragma unroll
  for (int j = 0; j < (HPW + S - 1) / S; ++j) {
    const int hr = wave_id() + 4 * S * j;
    if (hr >= n_rep) continue;
    const int h = g * n_rep + hr;
    const size_t base = (size_t)h * a.nsplit;
    // Device-scope loads in batches: (m, l) of split `lane` (8 bytes) with
    // this lane's dims of the first PF splits' partial O, then PF splits at a
    // time, so a combine costs one memory round trip per PF splits (every
    // split writes its partials; an empty one has m = -inf, l = 0, o = 0).
    constexpr int PF = 32;
    float opf[PF][DPL];
    auto load_chunk = [&](int c0) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int uu = min(c0 + u, a.nsplit - 1);  // clamped; weighted by 0 past nsplit
        const int off = (int)(((base + uu) * HD + DPL * lane) * 4);
        if constexpr (DPL == 2) {
          const dev_u32x2 t = loc ? xcd_ld8(a.part_o, off) : dev_ld8(a.part_o, off);
          opf[u][0] = __uint_as_float(t.x);
          opf[u][1] = __uint_as_float(t.y);
        } else {
          opf[u][0] = loc ? xcd_ldf(a.part_o, off) : dev_ldf(a.part_o, off);
        }
      }
    };
    auto ld_ml = [&](int sp) {
      const int off = (int)(2 * (base + sp) * 4);
      return loc ? xcd_ld8(a.part_ml, off) : dev_ld8(a.part_ml, off);
    };
    load_chunk(0);
    float ms, ls;
    {
      const int sp = min(lane, a.nsplit - 1);
      const dev_u32x2 t = ld_ml(sp);
      ms = lane < a.nsplit ? __uint_as_float(t.x) : -INFINITY;
      ls = lane < a.nsplit ? __uint_as_float(t.y) : 0.0f;
    }
    float M = wave_max(ms);
    for (int s0 = LLMRS_WAVE; s0 < a.nsplit; s0 += LLMRS_WAVE) {
      const int sp = min(s0 + lane, a.nsplit - 1);
      const dev_u32x2 t = ld_ml(sp);
      M = fmaxf(M, wave_max(s0 + lane < a.nsplit ? __uint_as_float(t.x) : -INFINITY));
    }
    float L = 0.0f, o[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[e] = 0.0f;
    for (int s0 = 0; s0 < a.nsplit; s0 += LLMRS_WAVE) {
      if (s0 > 0) {
        const int sp = min(s0 + lane, a.nsplit - 1);
        const dev_u32x2 t = ld_ml(sp);
        ms = s0 + lane < a.nsplit ? __uint_as_float(t.x) : -INFINITY;
        ls = s0 + lane < a.nsplit ? __uint_as_float(t.y) : 0.0f;
      }
      // w is 0 in lanes past nsplit, so clamped extra loads add 0
      const float w = ms == -INFINITY ? 0.0f : expf(ms - M);
      L = L + wave_sum(ls * w);
#pragma unroll
      for (int half = 0; half < LLMRS_WAVE / PF; ++half) {
        const int c0 = s0 + PF * half;
        if (c0 >= a.nsplit) break;
        if (c0 > 0) load_chunk(c0);
#pragma unroll
        for (int u = 0; u < PF; ++u) {
          const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), PF * half + u));
#pragma unroll
          for (int e = 0; e < DPL; ++e) o[e] = o[e] + opf[u][e] * wu;
        }
      }
    }
    // ctx as f32 and as Q8_0 (32-dim blocks: 16 lanes x 2 dims, or 32 lanes x 1).
    constexpr int LPB = 32 / DPL;  // lanes per Q8 block
    float amax = 0.0f;
    float v[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      v[e] = o[e] / L;
      amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = max16(amax);  // DPP within the 16-lane row
    if (LPB == 32) amax = fmaxf(amax, __shfl_xor(amax, 16, 32));
    const float d = amax / 127.0f;
    const float inv = amax == 0.0f ? 0.0f : 1.0f / d;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int dd = DPL * lane + e;
      st_act<true>(a.ctx, (size_t)h * HD + dd, v[e]);
      const int8_t q = amax == 0.0f ? (int8_t)0 : (int8_t)q8_code(v[e], inv);
      dev_st8(a.ctx_q, act_offset((int)((size_t)h * HD + dd), a.ctx_layout), q);
    }
    if ((lane % LPB) == 0) st_act<true>(a.ctx_d, ((size_t)h * HD + DPL * lane) / 32, amax == 0.0f ? 0.0f : d);
  }
  if (tid == 0) {
    if (loc) xcd_stu(a.counters, 4 * g * kTicketStride, 0u);
    else dev_stu(a.counters, 4 * g * kTicketStride, 0u);
  }
  stamp(6);
  flush_stamps();
  return true;
}

}  // namespace llmrs

