// sgemm.hip - skinny GEMM of batched decode for gfx950.
//
// Reference: the Q4/Q8 x Q8_0 block loop of CpuBackend::matmul_transposed
// per activation row (cpu.rs:90-110; kernel_avx2 cpu.rs:888-941):
// y[t][n] = sum over blocks b of fl(isum_b * fl(d_w[n,b] * d_a[t,b])), isum_b
// the exact int32 dot of the block's weight and activation codes.
//
// MI355X design: M <= 64 activation rows (the sequences of a batch) against
// a weight streamed once.  One v_mfma_i32_16x16x32_i8 per block gives the 16
// rows x 16 tokens of exact block sums, and one v_mfma_f32_16x16x1_4b_f32 per
// four blocks every scale product d_w * d_a of the 16 x 16 tile as a single
// IEEE product (lane 16 b + i supplies row / token i of block b; block b's
// products sit in registers 4 b .. 4 b + 3 in the layout of the block sums);
// the epilogue then multiplies and adds in f32 as the reference does.  Lane (r, g) of a wave (r = lane % 16, g = lane / 16) loads 16
// bytes: one Q4 block of weight row r (four blocks per lane group), so each
// load instruction reads 64 contiguous bytes of each of 16 rows; a 4x4 dword
// transpose across the lane groups (v_permlane32_swap, v_permlane16_swap)
// then gives lane group g dword g of each of the four blocks - its MFMA
// operand (the nibbles unpacked to q - 8 in four instructions; the device
// Q4 layout is the same for both Q4 storages, only their scales differ).
// The activation codes are stored in the matching operand order
// (act_offset), so a lane reads its four blocks' operands as 32 contiguous
// bytes.
//
// Batched decode: a wave takes RT 16-row tiles, which share its activation
// operands (the activation bytes a group loads are twice its weight bytes
// per tile): two, or one for the residual projections, whose few rows would
// leave too few workgroups.  A workgroup holds RS row sets of RT tiles and
// splits the blocks of each over KP waves in contiguous parts, partial sums
// added in part order.  STORE / RESID: one row set, KP = 4.  SILU: 64 rows
// per workgroup - a run of 32 gate and 32 up rows, one row set each, KP = 2;
// m = silu(gate) * up and its Q8_0 codes (one 32-element block per run) in
// the operand order of the down projection.  (Same box, 8B: eight waves per
// workgroup with twice the parts were slower at B = 16 and 64, e.g. the
// SwiGLU launch 42.8 vs 39.7 us; plain instead of streaming weight loads
// changed nothing.)
//
// EXACT launches (prompt prefill) give each output row's blocks to one wave
// in order, as the reference adds them, so the result is bit-identical to
// the reference's for the same activation codes: STORE / RESID run one wave
// (16 rows) per workgroup, SILU four (the run's 64 rows).
//
// Each wave keeps PF groups of loads in flight (a ring of register sets, the
// loop unrolled by PF so every set has a fixed place).
#include "common.h"
#include "exact_math.h"
#include "gemv_core.h"
#include "../kernel_args.h"

using namespace llmrs;

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

// q - 8 for four nibbles held one per byte (0..15): (v + 0x78) ^ 0x80 per
// byte, no carry between bytes.
__device__ __forceinline__ unsigned nib_s8(unsigned v) { return (v + 0x78787878u) ^ 0x80808080u; }

// In: lane group g holds the four dwords of its block g.  Out: x[j] = dword
// g of block j.  v_permlane32_swap(a, b) exchanges the upper half of a with
// the lower half of b; v_permlane16_swap the odd 16-lane rows of a with the
// even rows of b.
__device__ __forceinline__ void transpose4(unsigned x[4]) {
  auto p = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
  x[0] = p[0];
  x[2] = p[1];
  p = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
  x[1] = p[0];
  x[3] = p[1];
  p = __builtin_amdgcn_permlane16_swap(x[0], x[1], false, false);
  x[0] = p[0];
  x[1] = p[1];
  p = __builtin_amdgcn_permlane16_swap(x[2], x[3], false, false);
  x[2] = p[0];
  x[3] = p[1];
}

// What one 128-element group needs in registers.
template <int WT, int TT, int RT>
struct Group {
  u32x4 w[RT];          // Q4: this lane's block of each row tile (transposed after arrival)
  unsigned w8[RT][4][2];  // Q8: dwords g and g + 4 of each block
  unsigned dw[RT];       // raw scale of (row lane % 16, block lane / 16) per row tile
  u32x4 x[TT][2];       // activation operands of 4 blocks, per token tile
  float da[TT];         // scale of (token lane % 16, block lane / 16) per token tile
};

// Loads of group q for the wave's rows n0 .. n0 + 16 RT - 1.
template <int WT, int TT, int RT>
__device__ __forceinline__ void load_group(Group<WT, TT, RT>& G, const SgemmArgs& a, int q, int n0, int tok, int nb,
                                           int g) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int wrow = min(n0 + 16 * rt + tok, a.N - 1);
    if (WT == WT_Q8H) {
      const unsigned* base = (const unsigned*)(a.wq + ((size_t)wrow * nb + 4 * q) * 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        G.w8[rt][j][0] = __builtin_nontemporal_load(base + 8 * j + g);
        G.w8[rt][j][1] = __builtin_nontemporal_load(base + 8 * j + g + 4);
      }
    } else {
      G.w[rt] = __builtin_nontemporal_load((const u32x4*)(a.wq + ((size_t)wrow * nb + 4 * q + g) * 16));
    }
    G.dw[rt] = load_wscale_raw<WT>(a.ws, (size_t)wrow * nb + 4 * q + g);
  }
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const int t = min(16 * tt + tok, a.M - 1);
    const u32x4* xp = (const u32x4*)(a.xq + (size_t)t * a.K + (size_t)q * 128 + g * 32);
    G.x[tt][0] = xp[0];
    G.x[tt][1] = xp[1];
    G.da[tt] = a.xd[(size_t)t * nb + 4 * q + g];
  }
}

// One group's MFMAs and epilogue into acc[rt][tt][i] (output row n0 + 16 rt
// + 4 g + i, token 16 tt + tok).
template <int WT, int TT, int RT>
__device__ __forceinline__ void compute_group(Group<WT, TT, RT>& G, f32x4 (&acc)[RT][TT]) {
  long op_a[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (WT == WT_Q8H) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        op_a[rt][j] = (long)((unsigned long long)G.w8[rt][j][0] | ((unsigned long long)G.w8[rt][j][1] << 32));
    } else {
      unsigned wd[4] = {G.w[rt][0], G.w[rt][1], G.w[rt][2], G.w[rt][3]};
      transpose4(wd);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned lo = nib_s8(wd[j] & 0x0F0F0F0Fu), hi = nib_s8((wd[j] >> 4) & 0x0F0F0F0Fu);
        op_a[rt][j] = (long)((unsigned long long)lo | ((unsigned long long)hi << 32));
      }
    }
  }
  // Per token tile every MFMA first, then the epilogue: an MFMA result read
  // right after its issue would stall the wave for the MFMA's latency.
  float dw[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) dw[rt] = wscale<WT>(G.dw[rt]);
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    v16f sc[RT];  // sc[rt][4 j + i] = fl(d_w * d_a) of block j, row 4 g + i, token tok
    i32x4 isum[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) sc[rt] = __builtin_amdgcn_mfma_f32_16x16x1f32(dw[rt], G.da[tt], v16f{}, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned b0 = G.x[tt][j >> 1][2 * (j & 1)], b1 = G.x[tt][j >> 1][2 * (j & 1) + 1];
      const long op_b = (long)((unsigned long long)b0 | ((unsigned long long)b1 << 32));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        isum[rt][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(op_a[rt][j], op_b, i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)  // cpu.rs:930-935
          acc[rt][tt][i] = acc[rt][tt][i] + (float)isum[rt][j][i] * sc[rt][4 * j + i];
  }
}

// Groups of loads in flight per wave (register sets of the ring).  Measured
// on 8B batched decode: with one token tile the SwiGLU launch is fastest with
// one group ahead (35.7 us against 37.6 with two and 39.5 with four), the
// others with two (B = 16 step 3.35 ms with these depths, 3.63 with four
// throughout, 4.09 with eight); the exact launches walk every block of a row
// in one wave and keep deeper rings.
template <int EPI, int TT, bool EXACT>
constexpr int prefetch_depth() {
  if (EXACT) return TT == 1 ? 4 : TT == 2 ? 3 : 2;
  return TT == 1 && EPI == EPI_SILU ? 1 : 2;
}

// The rows' partial sums over groups [q0, q1) in group order, PF groups of
// loads ahead (addresses past the range clamped to its last group).
template <int WT, int TT, int RT, int PF>
__device__ __forceinline__ void run_groups(const SgemmArgs& a, int q0, int q1, int n0, int tok, int nb, int g,
                                           f32x4 (&acc)[RT][TT]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[rt][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // Wave-uniform bounds (they derive from the wave index): the loop and its
  // tail test become scalar branches, which the memory counter is tracked
  // through; a per-lane (exec-mask) loop would make every iteration wait for
  // all outstanding loads, ring included.
  q0 = __builtin_amdgcn_readfirstlane(q0);
  q1 = __builtin_amdgcn_readfirstlane(q1);
  if (q0 >= q1) return;
  Group<WT, TT, RT> ring[PF];
#pragma unroll
  for (int s = 0; s < PF; ++s) load_group<WT, TT, RT>(ring[s], a, min(q0 + s, q1 - 1), n0, tok, nb, g);
  // Whole rounds of PF groups without a branch (one block the scheduler can
  // interleave), then the last partial round from the ring.
  int q = q0;
  for (; q + PF <= q1; q += PF) {
#pragma unroll
    for (int s = 0; s < PF; ++s) {
      compute_group<WT, TT, RT>(ring[s], acc);
      load_group<WT, TT, RT>(ring[s], a, min(q + s + PF, q1 - 1), n0, tok, nb, g);
    }
  }
#pragma unroll
  for (int s = 0; s < PF - 1; ++s)
    if (q + s < q1) compute_group<WT, TT, RT>(ring[s], acc);
}

// Workgroup shape: RS row sets of RT 16-row tiles, each row set's blocks
// split over KP waves (EXACT: KP = 1, every output's blocks in order in one
// wave, as the reference adds them - bit-identical to it for the same
// activation codes; prompt prefill).
template <int EPI, bool EXACT, int KP>
struct SgemmShape {
  static constexpr int RT = EXACT || EPI == EPI_RESID ? 1 : 2;
  static constexpr int RS = EPI == EPI_SILU ? 64 / (16 * RT) : 1;
  static constexpr int WAVES = RS * KP;
  static constexpr int THREADS = 64 * WAVES;
  static_assert(!EXACT || KP == 1, "exact launches keep every output's blocks in one wave");
};

template <int WT, int EPI, int TT, bool EXACT, int KP>
__device__ __forceinline__ void sgemm_impl(const SgemmArgs& a) {
  typedef SgemmShape<EPI, EXACT, KP> S;
  constexpr int RT = S::RT, RS = S::RS;
  __shared__ f32x4 s_acc[S::WAVES][RT][TT][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nb = a.K >> 5, ngroups = nb >> 2;
  const int rs = w / KP, kp = w % KP;
  f32x4 acc[RT][TT];
  // row set rs: rows n0 .. n0 + 16 RT - 1 (SILU: the run's gate rows, then its up rows)
  const int n0 = blockIdx.x * (16 * RT * RS) + 16 * RT * rs;
  run_groups<WT, TT, RT, prefetch_depth<EPI, TT, EXACT>()>(a, kp * ngroups / KP, (kp + 1) * ngroups / KP, n0, r,
                                                          nb, g, acc);

  if (EPI != EPI_SILU && EXACT) {
    const int row0 = n0 + 4 * g;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = 16 * tt + r;
      if (t < a.M) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + i;
          if (row < a.N) {
            float o = acc[0][tt][i];
            if (EPI == EPI_RESID) o = o + a.res[(size_t)t * a.N + row];  // layer.rs:386,403
            a.y[(size_t)t * a.ldy + row] = o;
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) s_acc[w][rt][tt][lane] = acc[rt][tt];
  __syncthreads();

  if (EPI == EPI_SILU) {
    // m = silu(gate) * up (layer.rs:72-79) for 8 tokens x 32 elements per
    // pass; Q8_0 of the 32 elements of a token (one block of m)
    const int run = blockIdx.x;
    const int j = tid & 31;
    // gate row j of the run: row set, row tile, lane group, register; the
    // matching up row sits RS / 2 row sets later
    const int gs = j / (16 * RT), rt = (j >> 4) % RT, gg = (j & 15) >> 2, ii = j & 3;
    for (int t0 = tid >> 5; t0 < 16 * TT; t0 += S::THREADS / 32) {
      const int tt = t0 >> 4, l = 16 * gg + (t0 & 15);
      float gv = s_acc[gs * KP][rt][tt][l][ii], uv = s_acc[(RS / 2 + gs) * KP][rt][tt][l][ii];
#pragma unroll
      for (int k = 1; k < KP; ++k) {
        gv = gv + s_acc[gs * KP + k][rt][tt][l][ii];
        uv = uv + s_acc[(RS / 2 + gs) * KP + k][rt][tt][l][ii];
      }
      const float mv = (gv / (1.0f + exact_expf(-gv))) * uv;  // glibc expf (exact_math.h)
      float amax = fabsf(mv);
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
      const float d = amax / 127.0f;
      const float inv = amax == 0.0f ? 0.0f : 1.0f / d;
      if (t0 < a.M) {
        const int F = a.N / 2;
        if (a.y) a.y[(size_t)t0 * a.ldy + 32 * run + j] = mv;  // the f32 product (test probes)
        a.yq[(size_t)t0 * F + act_offset(32 * run + j, a.layout)] =
            amax == 0.0f ? (int8_t)0 : (int8_t)q8_code(mv, inv);
        if (j == 0) a.yd[(size_t)t0 * (F / 32) + run] = amax == 0.0f ? 0.0f : d;
      }
    }
    return;
  }
  if (w != 0) return;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row0 = n0 + 16 * rt + 4 * g;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = 16 * tt + r;
      f32x4 v = s_acc[0][rt][tt][lane];
#pragma unroll
      for (int k = 1; k < KP; ++k) v = v + s_acc[k][rt][tt][lane];
      if (t < a.M) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + i;
          if (row < a.N) {
            float o = v[i];
            if (EPI == EPI_RESID) o = o + a.res[(size_t)t * a.N + row];  // layer.rs:386,403
            a.y[(size_t)t * a.ldy + row] = o;
          }
        }
      }
    }
  }
}

}  // namespace

// Kernels: sgemm_<weights>_<epilogue>_t<token tiles>[_exact].
#define LLMRS_SGEMM(name, WT, EPI, TT, EXACT, KP)                                               \
  extern "C" __global__ __launch_bounds__((SgemmShape<EPI, EXACT, KP>::THREADS)) void name(SgemmArgs a) { \
    sgemm_impl<WT, EPI, TT, EXACT, KP>(a);                                                        \
  }
#define LLMRS_SGEMM_TILES(tag, WT, EPI, KP)                            \
  LLMRS_SGEMM(sgemm_##tag##_t1, WT, EPI, 1, false, KP)                 \
  LLMRS_SGEMM(sgemm_##tag##_t2, WT, EPI, 2, false, KP)                 \
  LLMRS_SGEMM(sgemm_##tag##_t4, WT, EPI, 4, false, KP)                 \
  LLMRS_SGEMM(sgemm_##tag##_t1_exact, WT, EPI, 1, true, 1)             \
  LLMRS_SGEMM(sgemm_##tag##_t2_exact, WT, EPI, 2, true, 1)             \
  LLMRS_SGEMM(sgemm_##tag##_t4_exact, WT, EPI, 4, true, 1)
LLMRS_SGEMM_TILES(q4h_store, WT_Q4H, EPI_STORE, 4)
LLMRS_SGEMM_TILES(q4h_resid, WT_Q4H, EPI_RESID, 4)
LLMRS_SGEMM_TILES(q4h_silu, WT_Q4H, EPI_SILU, 2)
LLMRS_SGEMM_TILES(q4f_store, WT_Q4F, EPI_STORE, 4)
LLMRS_SGEMM_TILES(q4f_resid, WT_Q4F, EPI_RESID, 4)
LLMRS_SGEMM_TILES(q4f_silu, WT_Q4F, EPI_SILU, 2)
LLMRS_SGEMM_TILES(q8h_store, WT_Q8H, EPI_STORE, 4)
LLMRS_SGEMM_TILES(q8h_resid, WT_Q8H, EPI_RESID, 4)
LLMRS_SGEMM_TILES(q8h_silu, WT_Q8H, EPI_SILU, 2)
