// attn_mfma.h - batch-1 decode attention on the matrix cores, f16 KV cache
// (instantiated by attention.hip).
//
// Reference: LlamaAttention::forward, seq == 1 (layer.rs:175-299): per query
// head, RoPE on q and k (layer.rs:216-217, cpu.rs:326-357), K/V append at
// pos (layer.rs:219-246), scores = q.K_t * (1/sqrt(hd)) (layer.rs:257-258),
// softmax (cpu.rs:395-423), ctx = sum_t p_t V_t (layer.rs:276-299).  Query
// head h reads KV head h / n_rep (the reference duplicates the K/V rows per
// query head, loader.rs:62-98, which gives the same numbers).
//
// One workgroup of max(4, TW) waves per (KV head g, split); TW of them (1,
// 4 or 8) take tiles.  The KV head's tiles of 32 positions are dealt over
// (split, tile wave): tile (i * TW + wave) * nsplit + split for i = 0, 1,
// ...  TW = 1 spreads a short context's tiles over the most CUs (a tile's
// 16 KB of loads per CU); TW = 4 or 8 keeps that many tiles in flight per CU
// for long contexts.  A
// wave takes a whole tile for all n_rep query heads of the group with
// v_mfma_f32_16x16x32_f16 (A 16 x 32, B 32 x 16; the 16 columns are query
// heads, at most 16):
//   S^T = K Q^T    A = K: 16 positions x 32 dims, 16 bytes per lane straight
//                  from the cache; B = the rotated q, scaled per head by a
//                  power of two that puts its largest |q| in [2^14, 2^15)
//                  and split into f16 hi + lo, so the products carry ~22 bits
//                  of q as f32 products do;
//   softmax        online per query head: lane (column c, group r) holds
//                  positions 8r .. 8r+7 of the tile (the rows of the two
//                  16-position blocks are ordered so), exp2 of
//                  log2(e)-scaled scores;
//   O^T += V^T P^T A = V^T: 16 dims x 32 positions; the f16 V cache is kept
//                  blocked and transposed, [p/8][hd][p%8] (v_offset), so
//                  these are again 16 contiguous bytes per lane; B = p * 2^14
//                  split into f16 hi + lo.
// K and V never pass through LDS, and a wave's next tile is loaded while the
// current one is computed.  The tile waves' (max, sum, O) merge through LDS
// into the split's partials; the last workgroup of the KV head (atomic
// ticket; partials move with device-scope stores and loads) combines the
// splits and writes ctx as f32 and as Q8_0 codes for the O projection.
//
// v_mfma_f32_16x16x32_f16 lane layout: lane l holds A[l%16][8(l/16) + e],
// B[8(l/16) + e][l%16] (e = 0..7) and D[4(l/16) + i][l%16] (i = 0..3).
#pragma once
#include "common.h"
#include "../kernel_args.h"

namespace llmrs {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ h16x8 as_h16x8(u32x4 v) { return __builtin_bit_cast(h16x8, v); }

__device__ __forceinline__ f32x4 mfma16(h16x8 a, h16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LDS of one work item: with TW > 1 the tile waves' O^T blocks as the
// matrix core leaves them ([wave][block][i][lane]) and their (max, sum) per
// column; with TW == 1 the operands wave 1 prepares for wave 0 (per lane the
// q hi and lo operands and the new K row's operand, per column the score
// scale, per (V block, column) the new V element); the ticket.
template <int HD, int TW>
struct MfmaAttnLds {
  static constexpr int NS = HD / 32, NB = HD / 16;
  static constexpr size_t O = 0;
  static constexpr size_t ML = O + (TW > 1 ? sizeof(float) * TW * NB * 4 * 64 : 0);
  static constexpr size_t QOP = ML + (TW > 1 ? sizeof(float) * TW * 16 * 2 : 0);
  static constexpr size_t KNEW = QOP + (TW == 1 ? 16 * 64 * NS * 2 : 0);
  static constexpr size_t SL2 = KNEW + (TW == 1 ? 16 * 64 * NS : 0);
  static constexpr size_t VNEW = SL2 + (TW == 1 ? 4 * 16 : 0);
  static constexpr size_t TICKET = VNEW + (TW == 1 ? 2 * 16 * NB : 0);
  static constexpr size_t BYTES = TICKET + 16;
};

// `pos` (the new token's position) is read by the caller at kernel entry, so
// it arrives through the scalar cache while the vector loads below are in
// flight.
template <int HD, int TW, bool LOCAL>
__device__ __forceinline__ void attn_mfma_item(const AttnArgs& a, int pos, uint8_t* lds) {
  constexpr int NS = HD / 32, NB = HD / 16, MID = HD / 2, TILE = kAttnTile;
  constexpr float kLog2e = 1.4426950408889634f;
  constexpr float kP = 16384.0f;  // p is scaled by 2^14 before its hi/lo split
  typedef MfmaAttnLds<HD, TW> LY;
  static_assert(TILE == 32, "two 16-position blocks per tile");
  static_assert(TW == 1 || TW == 4 || TW == 8, "one, four or eight tile waves");
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int c = lane & 15, r = lane >> 4;  // MFMA column (query head of the group), lane group
  // LOCAL: KV head = linear workgroup index % nkv, so with nkv = 8 all
  // splits of a head run on one XCD and exchange partials through its L2.
  constexpr bool loc = LOCAL;
  const int lin = blockIdx.x + blockIdx.y * gridDim.x;
  const int g = loc ? lin % a.nkv : blockIdx.y, split = loc ? lin / a.nkv : blockIdx.x;
  const int n_rep = a.nq / a.nkv;
  const size_t hrow = (size_t)g * a.max_seq * HD;  // first element of this KV head
  const uint16_t* kc = (const uint16_t*)a.kc + hrow;
  const uint16_t* vc = (const uint16_t*)a.vc + hrow;

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

  // A operands of the tile at t0: K rows of block b (row c = position
  // t0 + 8(c/4) + 4b + c%4, dims 32s + 8r ..) and V^T rows (dim 16b + c,
  // positions t0 + 8r .. t0 + 8r + 7).
  struct Ops {
    u32x4 k[2][NS];
    u32x4 v[NB];
  };
  auto fetch = [&](Ops& o, int t0) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint16_t* kr = kc + (size_t)(t0 + 8 * (c >> 2) + 4 * b + (c & 3)) * HD + 8 * r;
#pragma unroll
      for (int s = 0; s < NS; ++s) o.k[b][s] = *(const u32x4*)(kr + 32 * s);
    }
    const uint16_t* vr = vc + v_offset((size_t)t0 + 8 * r, c, HD, true);
#pragma unroll
    for (int b = 0; b < NB; ++b) o.v[b] = *(const u32x4*)(vr + (size_t)16 * 8 * b);
  };
  // The tile holding pos belongs to one wave of one split: that wave's
  // operands of the tile take the new k (rotated, layer.rs:216-217) and v,
  // whose loads may have been requested before they are appended to the
  // cache (layer.rs:219-246).
  const int T = pos + 1;
  const int town = pos & ~(TILE - 1), dl = pos - town;
  const int own_wave = (town / TILE / a.nsplit) % TW;
  const bool own_split = (town / TILE) % a.nsplit == split;
  const int kb_own = (dl >> 2) & 1, kc_own = 4 * (dl >> 3) + (dl & 3);  // K block and row of pos
  const int vr_own = dl >> 3, vs_own = dl & 7;                            // V lane group and slot
  const bool col_on = c < n_rep;  // columns past the group stay zero

  // Operands of the query heads (B of S^T = K Q^T) and the score scale: q of
  // query head g * n_rep + c, dims 32s + 8r + e, and the RoPE row of pos
  // (neither needs the position: requested first; `prefetch` runs next).
  // The partner of dim d < hd/2 is d + hd/2, held by the same lane in step
  // s + NS/2.
  h16x8 qh[NS], ql[NS];
  float sl2;
  // The RoPE row of pos (rope_now: copied by the step's embedding launch, so
  // its loads need no position).
  auto load_rope = [&](float (&cs)[NS / 2][8], float (&sn)[NS / 2][8]) {
    const float* rc = a.rope_now + 8 * r;
    const float* rs = a.rope_now + MID + 8 * r;
#pragma unroll
    for (int s = 0; s < NS / 2; ++s) {
      const f32x4 c0 = *(const f32x4*)(rc + 32 * s), c1 = *(const f32x4*)(rc + 32 * s + 4);
      const f32x4 s0 = *(const f32x4*)(rs + 32 * s), s1 = *(const f32x4*)(rs + 32 * s + 4);
      cs[s][0] = c0.x; cs[s][1] = c0.y; cs[s][2] = c0.z; cs[s][3] = c0.w;
      cs[s][4] = c1.x; cs[s][5] = c1.y; cs[s][6] = c1.z; cs[s][7] = c1.w;
      sn[s][0] = s0.x; sn[s][1] = s0.y; sn[s][2] = s0.z; sn[s][3] = s0.w;
      sn[s][4] = s1.x; sn[s][5] = s1.y; sn[s][6] = s1.z; sn[s][7] = s1.w;
    }
  };
  // dims 32s + 8r + e of the row at `src` (q of a head, or the new k)
  auto load_row = [&](float (&x)[NS][8], const float* src) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const f32x4 x0 = *(const f32x4*)(src + 32 * s), x1 = *(const f32x4*)(src + 32 * s + 4);
      x[s][0] = x0.x; x[s][1] = x0.y; x[s][2] = x0.z; x[s][3] = x0.w;
      x[s][4] = x1.x; x[s][5] = x1.y; x[s][6] = x1.z; x[s][7] = x1.w;
    }
  };
  // x0' = x0 c - x1 s, x1' = x0 s + x1 c (cpu.rs:351-354)
  auto rotate = [&](float (&x)[NS][8], const float (&cs)[NS / 2][8], const float (&sn)[NS / 2][8]) {
#pragma unroll
    for (int s = 0; s < NS / 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float re = x[s][e], im = x[s + NS / 2][e];
        x[s][e] = re * cs[s][e] - im * sn[s][e];
        x[s + NS / 2][e] = re * sn[s][e] + im * cs[s][e];
      }
  };
  // cs, sn: the RoPE row, requested by the caller.
  auto q_prologue = [&](auto&& prefetch, const float (&cs)[NS / 2][8], const float (&sn)[NS / 2][8]) {
    float qv[NS][8];
    load_row(qv, a.qkv + (size_t)(g * n_rep + min(c, n_rep - 1)) * HD + 8 * r);
    __builtin_amdgcn_sched_barrier(0);
    prefetch();
    __builtin_amdgcn_sched_barrier(0);
    rotate(qv, cs, sn);
    // Per-head power-of-two scale 2^ex: max |q| * 2^ex in [2^14, 2^15).
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[s][e]));
    amax = fmaxf(amax, xor16(amax));
    amax = fmaxf(amax, xor32(amax));
    int fe = 0;
    (void)frexpf(amax, &fe);
    const int ex = amax > 0.0f ? 15 - fe : 0;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = col_on ? ldexpf(qv[s][e], ex) : 0.0f;
        const _Float16 hi = (_Float16)x;
        qh[s][e] = hi;
        ql[s][e] = (_Float16)(x - (float)hi);
      }
    // score in log2 units per matrix-core unit: fl(1/sqrt(hd)) * log2(e) * 2^-ex
    sl2 = ldexpf(a.scale * kLog2e, -ex);
  };
  // The new row as operands: k rotated and in f16, per lane dims 32s + 8r +
  // e (for the K row of pos); v in f16, per lane dims 16b + c.  Its loads
  // (RoPE row included) need no position; `owner` is only needed once they
  // are back.
  u32x4 knew[NS];
  uint16_t vnew[NB];
  auto row_prologue = [&](auto&& is_owner, const float (&cs)[NS / 2][8], const float (&sn)[NS / 2][8]) {
    float kv[NS][8], vraw[NB];
    load_row(kv, a.qkv + (size_t)a.nq * HD + (size_t)g * HD + 8 * r);
    const float* vr = a.qkv + (size_t)(a.nq + a.nkv) * HD + (size_t)g * HD + c;
#pragma unroll
    for (int b = 0; b < NB; ++b) vraw[b] = vr[16 * b];
    if (!is_owner()) return;
#pragma unroll
    for (int b = 0; b < NB; ++b) vnew[b] = f2h(vraw[b]);
    rotate(kv, cs, sn);
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        knew[s][w] = (unsigned)f2h(kv[s][2 * w]) | ((unsigned)f2h(kv[s][2 * w + 1]) << 16);
  };
  // The owner's append of the new row (read by later launches only).
  auto append = [&]() {
    uint16_t* kdst = (uint16_t*)a.kc + hrow + (size_t)pos * HD + 8 * r;
    if (c == kc_own) {
#pragma unroll
      for (int s = 0; s < NS; ++s) *(u32x4*)(kdst + 32 * s) = knew[s];
    }
    if (r == vr_own) {
#pragma unroll
      for (int b = 0; b < NB; ++b) ((uint16_t*)a.vc)[hrow + v_offset(pos, 16 * b + c, HD, true)] = vnew[b];
    }
  };
  // This wave's first tile is known without the position.
  const int first = wave < TW ? (wave * a.nsplit + split) * TILE : a.max_seq;  // other waves: none
  const int stride = TW * a.nsplit * TILE;
  Ops A, B;
  auto prefetch_first = [&]() {
    if (first < a.max_seq) fetch(A, first);  // max_seq: whole tiles of cache rows
  };
  const bool owner = own_split && own_wave == wave;
  if constexpr (TW == 1) {
    // Waves 1 (q) and 2 (new row) prepare the operands while wave 0 waits
    // for its tile.
    uint8_t* qop = lds + LY::QOP;
    float cs[NS / 2][8], sn[NS / 2][8];  // the RoPE row (waves 1 and 2)
    if (wave == 0) prefetch_first();
    else if (wave <= 2) load_rope(cs, sn);
    if (wave == 1) {
      q_prologue([] {}, cs, sn);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        *(h16x8*)(qop + ((s * 2) * 64 + lane) * 16) = qh[s];
        *(h16x8*)(qop + ((s * 2 + 1) * 64 + lane) * 16) = ql[s];
      }
      if (r == 0) ((float*)(lds + LY::SL2))[c] = sl2;
    } else if (wave == 2) {
      row_prologue([&] { return own_split; }, cs, sn);
      if (own_split) {
#pragma unroll
        for (int s = 0; s < NS; ++s) *(u32x4*)(lds + LY::KNEW + (s * 64 + lane) * 16) = knew[s];
        if (r == 0) {
#pragma unroll
          for (int b = 0; b < NB; ++b) ((uint16_t*)(lds + LY::VNEW))[b * 16 + c] = vnew[b];
        }
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        qh[s] = *(const h16x8*)(qop + ((s * 2) * 64 + lane) * 16);
        ql[s] = *(const h16x8*)(qop + ((s * 2 + 1) * 64 + lane) * 16);
      }
      sl2 = ((const float*)(lds + LY::SL2))[c];
      if (owner) {
#pragma unroll
        for (int s = 0; s < NS; ++s) knew[s] = *(const u32x4*)(lds + LY::KNEW + (s * 64 + lane) * 16);
#pragma unroll
        for (int b = 0; b < NB; ++b) vnew[b] = ((const uint16_t*)(lds + LY::VNEW))[b * 16 + c];
      }
    } else if (wave == 2 && own_split) {
      append();  // after the handoff: the barrier does not wait for these stores
    }
  } else {
    float cs[NS / 2][8], sn[NS / 2][8];
    load_rope(cs, sn);
    q_prologue(prefetch_first, cs, sn);
    if (owner) {
      row_prologue([] { return true; }, cs, sn);
      append();
    }
  }
  // Put the new row into the operands of the tile holding pos.  kb_own and
  // the V word are uniform: scalar branches pick the registers.
  auto patch = [&](Ops& o) {
#pragma unroll
    for (int b = 0; b < 2; ++b)  // constant indices keep the operands in registers
      if (b == kb_own) {
#pragma unroll
        for (int s = 0; s < NS; ++s) o.k[b][s] = c == kc_own ? knew[s] : o.k[b][s];
      }
    const int w = vs_own >> 1;
    const bool upper = vs_own & 1;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2)
      if (w2 == w) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const unsigned x = o.v[b][w2];
          const unsigned y = upper ? (x & 0xFFFFu) | ((unsigned)vnew[b] << 16) : (x & 0xFFFF0000u) | vnew[b];
          o.v[b][w2] = r == vr_own ? y : x;
        }
      }
  };
  stamp(1);

  // Running max (log2 units) and sum of this lane's query head, and O^T:
  // o[b][i] = 2^14 * O[head c][dim 16b + 4r + i].
  float m = -INFINITY, l = 0.0f;
  bool started = false;  // wave-uniform: a tile has been accumulated
  f32x4 o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) o[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto process = [&](const Ops& op, int t0) {
    f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, s2 = s0, s3 = s0;  // block 0/1 x hi/lo
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      s0 = mfma16(as_h16x8(op.k[0][s]), qh[s], s0);
      s1 = mfma16(as_h16x8(op.k[1][s]), qh[s], s1);
      s2 = mfma16(as_h16x8(op.k[0][s]), ql[s], s2);
      s3 = mfma16(as_h16x8(op.k[1][s]), ql[s], s3);
    }
    // sv[j]: position t0 + 8r + j (j < 4 from block 0, else block 1)
    float sv[8];
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float raw = j < 4 ? s0[j] + s2[j] : s1[j - 4] + s3[j - 4];
      sv[j] = t0 + 8 * r + j < T ? raw * sl2 : -INFINITY;
      mt = fmaxf(mt, sv[j]);
    }
    mt = fmaxf(mt, xor16(mt));
    mt = fmaxf(mt, xor32(mt));
    const float mn = fmaxf(m, mt);  // finite: position t0 < T is in the tile
    const float corr = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first tile
    float ls = 0.0f;
    h16x8 ph, pl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = __builtin_amdgcn_exp2f(sv[j] - mn);
      ls += p;
      const float x = p * kP;
      const _Float16 hi = (_Float16)x;
      ph[j] = hi;
      pl[j] = (_Float16)(x - (float)hi);
    }
    ls += xor16(ls);
    ls += xor32(ls);
    l = l * corr + ls;
    m = mn;
    // all hi products, then all lo: a block's two products are NB apart
    if (started) {
#pragma unroll
      for (int b = 0; b < NB; ++b) o[b] = o[b] * corr;
    }
    started = true;
#pragma unroll
    for (int b = 0; b < NB; ++b) o[b] = mfma16(as_h16x8(op.v[b]), ph, o[b]);
#pragma unroll
    for (int b = 0; b < NB; ++b) o[b] = mfma16(as_h16x8(op.v[b]), pl, o[b]);
  };
  // Tiles of this wave: with up to four tile waves, two register sets in
  // turn (the next tile loads while one is computed); with eight, two waves
  // per SIMD share the registers, so one set, and a wave rarely has a second
  // tile.
  int t0 = first;
  if constexpr (TW <= 4) {
    while (t0 < T) {
      int t1 = t0 + stride;
      if (t1 < T) fetch(B, t1);
      if (owner && t0 == town) patch(A);
      process(A, t0);
      if (t0 == first) stamp(2);
      t0 = t1;
      if (t0 >= T) break;
      t1 = t0 + stride;
      if (t1 < T) fetch(A, t1);
      if (owner && t0 == town) patch(B);
      process(B, t0);
      t0 = t1;
    }
  } else {
    for (; t0 < T; t0 += stride) {
      if (t0 != first) fetch(A, t0);
      if (owner && t0 == town) patch(A);
      process(A, t0);
      if (t0 == first) stamp(2);
    }
  }
  stamp(3);

  // The split's partials: with one tile wave its own (max, sum, O); with
  // more, merged through LDS, wave w writing O blocks w, w + TW, ...
  auto pst16 = [&](float* base, int off, dev_u32x4 v) {
    if (loc) xcd_st16(base, off, v);
    else dev_st16(base, off, v);
  };
  auto pstml = [&](size_t mi, float mv, float lv) {
    if (loc) {
      __builtin_amdgcn_raw_buffer_store_b64(dev_u32x2{__float_as_uint(mv), __float_as_uint(lv)},
                                            dev_rsrc(a.part_ml), (int)(8 * mi), 0, 0);
    } else {
      dev_stf(a.part_ml, (int)(8 * mi), mv);
      dev_stf(a.part_ml, (int)(8 * mi + 4), lv);
    }
  };
  const size_t pidx = (size_t)(g * n_rep + c) * a.nsplit + split;
  const size_t midx = (size_t)(g * n_rep + c) * ml_stride(a.nsplit) + split;
  if constexpr (TW == 1) {
    if (wave == 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
        if (col_on)
          pst16(a.part_o, (int)((pidx * HD + 16 * b + 4 * r) * 4),
                __builtin_bit_cast(dev_u32x4, o[b] * (1.0f / kP)));
      if (r == 0 && col_on) {
        pstml(midx, m, l);
      }
    }
  } else {
    float* so = (float*)(lds + LY::O);
    float* sml = (float*)(lds + LY::ML);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) so[((wave * NB + b) * 4 + i) * 64 + lane] = o[b][i];
    if (r == 0) {
      sml[(wave * 16 + c) * 2] = m;
      sml[(wave * 16 + c) * 2 + 1] = l;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < TW; ++w) M = fmaxf(M, sml[(w * 16 + c) * 2]);
    float cw[TW], L = 0.0f;
#pragma unroll
    for (int w = 0; w < TW; ++w) {
      const float mw = sml[(w * 16 + c) * 2];
      cw[w] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      L = L + cw[w] * sml[(w * 16 + c) * 2 + 1];
    }
#pragma unroll
    for (int b = wave; b < NB; b += TW) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < TW; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] + cw[w] * so[((w * NB + b) * 4 + i) * 64 + lane];
      acc = acc * (1.0f / kP);
      if (col_on) pst16(a.part_o, (int)((pidx * HD + 16 * b + 4 * r) * 4), __builtin_bit_cast(dev_u32x4, acc));
    }
    if (wave == 0 && r == 0 && col_on) {
      pstml(midx, M, L);
    }
  }
  // Publish the partials (device scope: they bypass the per-XCD L2), then
  // take a ticket; the last workgroup of the KV head combines.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  stamp(4);
  int* s_ticket = (int*)(lds + LY::TICKET);
  if (tid == 0)
    *s_ticket = loc ? __hip_atomic_fetch_add(&a.counters[g * kTicketStride], 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_WORKGROUP)
                    : atomicAdd(&a.counters[g * kTicketStride], 1);
  __syncthreads();
  stamp(5);
  if (*s_ticket != a.nsplit - 1) {
    flush_stamps();
    return;
  }

  // Combine: wave w takes query heads w, w + nw, ... of the group.  Lane s
  // loads split s's (max, sum) (one 8-byte load), so the maximum M is one
  // wave reduction, lane s forms the split's weight 2^(m_s - M) and the
  // total sum is one wave sum of weight * sum (a fixed DPP tree); the
  // weights reach every lane through the wave's own 256 bytes at the start
  // of the LDS (free once every wave has passed the ticket's barrier), read
  // back four at a time.  Lane l owns dims DPL*l .. DPL*l + DPL-1 and adds
  // the live splits' partial O in split order, loaded in batches of 8, 16
  // or 32 (the live split count rounded up) through a descriptor that ends
  // at the head's last live split, so loads past it read zero with no
  // memory access and need no per-load select.  Splits past the context
  // hold no tile (split s starts at tile s): their partials (max -inf, sum
  // 0) would add exact zeros, so they are not read.
  constexpr int DPL = HD / 64;  // dims per lane
  // waves of the launch (its launch bounds; the block size read at run time
  // would be a memory load)
  constexpr int nw = TW > 4 ? TW : 4;
  const int ns = a.nsplit, ns2 = ml_stride(ns);
  const int nlive = min(ns, (T + TILE - 1) / TILE);
  float* wsl = (float*)lds + LLMRS_WAVE * wave;  // this wave's split weights, split s at [s]
  static_assert(LY::TICKET >= (size_t)4 * LLMRS_WAVE * nw, "the combine's weight slots overlap the ticket");
  constexpr int pol = loc ? kSc0 : kSc1;
  // hr is wave-uniform: made a scalar so the descriptors below stay in SGPRs
  for (int hr = __builtin_amdgcn_readfirstlane(wave); hr < n_rep; hr += nw) {
    const size_t obase = (size_t)(g * n_rep + hr) * ns, mbase = (size_t)(g * n_rep + hr) * ns2;
    // The head's live splits only: loads past them read zero, no memory access.
    const __amdgpu_buffer_rsrc_t ro = span_rsrc(a.part_o + obase * HD, nlive * HD * 4);
    float Lx = 0.0f, Ox[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) Ox[i] = 0.0f;
    // NL partial-O loads from split s0, issued together; `ml` also requests
    // the (max, sum) loads with the first batch and forms the weights, so
    // nothing waits between the two requests.
    auto batch = [&](auto nl_tag, int s0, bool ml) {
      constexpr int NL = decltype(nl_tag)::value;
      dev_u32x2 mlv = {0u, 0u};
      if (ml) mlv = __builtin_amdgcn_raw_buffer_load_b64(span_rsrc(a.part_ml + 2 * mbase, nlive * 8), 8 * lane, 0, pol);
      float po[NL][DPL];
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int off = ((s0 + u) * HD + DPL * lane) * 4;
        if constexpr (DPL == 2) {
          const dev_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(ro, off, 0, pol);
          po[u][0] = __uint_as_float(v.x);
          po[u][1] = __uint_as_float(v.y);
        } else {
          po[u][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ro, off, 0, pol));
        }
      }
      if (ml) {
        const float ms = lane < nlive ? __uint_as_float(mlv.x) : -INFINITY;  // split 0 holds position 0
        const float ls = lane < nlive ? __uint_as_float(mlv.y) : 0.0f;
        const float M = wave_max(ms);
        const float wl = __builtin_amdgcn_exp2f(ms - M);  // 0 past the live splits
        Lx = wave_sum(wl * ls);
        wsl[lane] = wl;
      }
      float w[NL];
#pragma unroll
      for (int u = 0; u < NL; u += 4) {
        const f32x4 t = *(const f32x4*)(wsl + s0 + u);
        w[u] = t.x; w[u + 1] = t.y; w[u + 2] = t.z; w[u + 3] = t.w;
      }
#pragma unroll
      for (int u = 0; u < NL; ++u)
#pragma unroll
        for (int i = 0; i < DPL; ++i) Ox[i] = Ox[i] + po[u][i] * w[u];
    };
    if (nlive <= 8) batch(std::integral_constant<int, 8>{}, 0, true);
    else if (nlive <= 16) batch(std::integral_constant<int, 16>{}, 0, true);
    else batch(std::integral_constant<int, 32>{}, 0, true);
    for (int s0 = 32; s0 < nlive; s0 += 32) batch(std::integral_constant<int, 32>{}, s0, false);
    // ctx as f32 and as Q8_0: a 32-dim block is 32 / DPL lanes.
    float v[DPL], bmax = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      v[i] = Ox[i] / Lx;
      bmax = fmaxf(bmax, fabsf(v[i]));
    }
    bmax = max16(bmax);
    if (DPL == 1) bmax = fmaxf(bmax, xor16(bmax));
    const float d = bmax / 127.0f;
    const float inv = bmax == 0.0f ? 0.0f : 1.0f / d;
    const size_t e = (size_t)(g * n_rep + hr) * HD + DPL * lane;
    unsigned codes = 0;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int q8 = bmax == 0.0f ? 0 : q8_code(v[i], inv);
      codes |= ((unsigned)q8 & 0xFFu) << (8 * i);
    }
    const int qo = act_offset((int)e, a.ctx_layout);  // aligned runs of 4 stay together
    if constexpr (DPL == 2) {
      *(float2*)(a.ctx + e) = make_float2(v[0], v[1]);
      *(uint16_t*)(a.ctx_q + qo) = (uint16_t)codes;
    } else {
      a.ctx[e] = v[0];
      a.ctx_q[qo] = (int8_t)codes;
    }
    if (lane % (32 / DPL) == 0) a.ctx_d[e / 32] = bmax == 0.0f ? 0.0f : d;
  }
  if (tid == 0) {  // every split has taken its ticket: the ticket restarts
    if (loc) xcd_stu(a.counters, 4 * g * kTicketStride, 0u);
    else dev_stu(a.counters, 4 * g * kTicketStride, 0u);
  }
  stamp(6);
  flush_stamps();
}

}  // namespace llmrs
