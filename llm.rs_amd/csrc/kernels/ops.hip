// ops.hip - the remaining trait Backend operators (src/backend.rs:21-39) and
// the embedding gather, for gfx950.
//
// Every operator keeps the reference's f32 operation order, so its results
// are bit-identical to the reference CPU backend's (x86-64 build): the f32
// matmuls sum each output sequentially (one lane per output element,
// cpu.rs:157-269), RMSNorm and softmax fold their row sums in index order
// (cpu.rs:381, 410-415), and SiLU and softmax use glibc's expf
// (exact_math.h).  They are off the quantised decode hot path.
#include "common.h"
#include "exact_math.h"
#include "../kernel_args.h"

using namespace llmrs;


// Backend::add_assign (cpu.rs:274-296): a += b.
extern "C" __global__ __launch_bounds__(256) void add_assign_f32(EwArgs e) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < e.n; i += (long)gridDim.x * blockDim.x)
    e.a[i] = e.a[i] + e.b[i];
}

// Backend::silu_mul (cpu.rs:298-324): g = g/(1+exp(-g)) * u.
extern "C" __global__ __launch_bounds__(256) void silu_mul_f32(EwArgs e) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < e.n; i += (long)gridDim.x * blockDim.x) {
    const float v = e.a[i];
    e.a[i] = (v / (1.0f + exact_expf(-v))) * e.b[i];
  }
}

// Backend::scale (cpu.rs:425-435).
extern "C" __global__ __launch_bounds__(256) void scale_f32(EwArgs e) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < e.n; i += (long)gridDim.x * blockDim.x)
    e.out[i] = e.a[i] * e.value;
}


// Self-check of mul_f16lo / mul_f16hi (the reference-order attention's f16
// products): thread h takes f16 pattern h in both halves of a word and
// counts the values e.a[0 .. e.n) for which either mixed product differs in
// bits from the conversion and multiply (NaN against NaN counts as equal);
// the count goes to e.out[h].  Grid 256 x 256: every f16 pattern once.
extern "C" __global__ __launch_bounds__(256) void check_mul_f16(EwArgs e) {
  const unsigned h = blockIdx.x * 256u + threadIdx.x;
  const unsigned w = h | (h << 16);
  const float b = h2f((uint16_t)h);
  unsigned bad = 0;
  for (long i = 0; i < e.n; ++i) {
    const float a = e.a[i], r = a * b, lo = mul_f16lo(a, w), hi = mul_f16hi(a, w);
    const bool rn = r != r;
    bad += (rn ? lo == lo : __float_as_uint(lo) != __float_as_uint(r)) ? 1u : 0u;
    bad += (rn ? hi == hi : __float_as_uint(hi) != __float_as_uint(r)) ? 1u : 0u;
  }
  e.out[h] = (float)bad;
}

// Backend::rope_inplace (cpu.rs:326-357) with host-made sin/cos tables.
extern "C" __global__ __launch_bounds__(256) void rope_f32(RopeArgs r) {
  const int mid = r.hd / 2;
  const long total = (long)r.rows * mid;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long row = i / mid;
    const int j = (int)(i % mid);
    float* c = r.x + row * r.hd;
    const float re = c[j], im = c[j + mid];
    const float co = r.cos_t[i], s = r.sin_t[i];
    c[j] = re * co - im * s;
    c[j + mid] = re * s + im * co;
  }
}


// Row sums in index order: the row is staged through LDS in chunks of
// kChunk floats and lane 0 of the workgroup folds acc = acc + f(v).
constexpr int kChunk = 2048;

// Backend::rms_norm (cpu.rs:359-393); one workgroup per row:
// ss = fold(0, acc + v*v), rms = sqrt(ss/n + eps), y = (x * (1/rms)) * w.
extern "C" __global__ __launch_bounds__(256) void rms_norm_f32(RowArgs r) {
  __shared__ float s_x[kChunk];
  __shared__ float s_scale;
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* x = r.x + (size_t)row * r.dim;
  float ss = 0.0f;  // lane 0's running sum
  for (int c0 = 0; c0 < r.dim; c0 += kChunk) {
    const int n = min(kChunk, r.dim - c0);
    for (int i = tid; i < n; i += blockDim.x) s_x[i] = x[c0 + i];
    __syncthreads();
    if (tid == 0)
      for (int i = 0; i < n; ++i) ss = ss + s_x[i] * s_x[i];
    __syncthreads();
  }
  if (tid == 0) {
    const float rms = __builtin_sqrtf(ss / (float)r.dim + r.eps);
    s_scale = 1.0f / rms;
  }
  __syncthreads();
  const float scale = s_scale;
  for (int i = tid; i < r.dim; i += blockDim.x) r.out[(size_t)row * r.dim + i] = x[i] * scale * r.w[i];
}

// Backend::softmax (cpu.rs:395-423): max from f32::MIN, e = exp(x - max),
// sum of the e in index order, p = e * (1/sum).  One workgroup per row.
extern "C" __global__ __launch_bounds__(256) void softmax_f32(RowArgs r) {
  __shared__ float s_red[8];
  __shared__ float s_x[kChunk];
  __shared__ float s_inv;
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* x = r.x + (size_t)row * r.dim;
  float* o = r.out + (size_t)row * r.dim;
  float mx = -3.40282347e+38f;
  for (int i = tid; i < r.dim; i += blockDim.x) mx = fmaxf(mx, x[i]);
  mx = group_max(mx);
  if (lane_id() == 0) s_red[wave_id()] = mx;
  __syncthreads();
  mx = s_red[0];
  for (int w = 1; w < (int)(blockDim.x / LLMRS_WAVE); ++w) mx = fmaxf(mx, s_red[w]);
  float sum = 0.0f;  // lane 0's running sum
  for (int c0 = 0; c0 < r.dim; c0 += kChunk) {
    const int n = min(kChunk, r.dim - c0);
    for (int i = tid; i < n; i += blockDim.x) {
      const float e = exact_expf(x[c0 + i] - mx);
      o[c0 + i] = e;
      s_x[i] = e;
    }
    __syncthreads();
    if (tid == 0)
      for (int i = 0; i < n; ++i) sum = sum + s_x[i];
    __syncthreads();
  }
  if (tid == 0) s_inv = 1.0f / sum;
  __syncthreads();
  const float inv = s_inv;
  for (int i = tid; i < r.dim; i += blockDim.x) o[i] = o[i] * inv;
}


// Backend::matmul (cpu.rs:157-224): out[i][j] = sum_p a[i][p] * b[p][j],
// sequential over p, exact zeros of a skipped (cpu.rs:192,211).
extern "C" __global__ __launch_bounds__(256) void matmul_f32(MatArgs g) {
  const long total = (long)g.m * g.n;
  for (long t = blockIdx.x * (long)blockDim.x + threadIdx.x; t < total; t += (long)gridDim.x * blockDim.x) {
    const int i = (int)(t / g.n), j = (int)(t % g.n);
    const float* ar = g.a + (size_t)i * g.k;
    float s = 0.0f;
    for (int p = 0; p < g.k; ++p) {
      const float v = ar[p];
      if (v == 0.0f) continue;
      s = s + v * g.b[(size_t)p * g.n + j];
    }
    g.out[t] = s;
  }
}

// matmul_transposed with f32 weights (cpu.rs:114-146) and matmul_slice
// (cpu.rs:230-269): out[i][j] = dot(a_i, b_j), sequential over k.
extern "C" __global__ __launch_bounds__(256) void matmul_t_f32(MatArgs g) {
  const long total = (long)g.m * g.n;
  for (long t = blockIdx.x * (long)blockDim.x + threadIdx.x; t < total; t += (long)gridDim.x * blockDim.x) {
    const int i = (int)(t / g.n), j = (int)(t % g.n);
    const float* ar = g.a + (size_t)i * g.k;
    const float* br = g.b + (size_t)j * g.k;
    float s = 0.0f;
    for (int p = 0; p < g.k; ++p) s = s + ar[p] * br[p];
    g.out[t] = s;
  }
}


// Embedding gather (main.rs:159-167) for the token at the device position,
// or a given row; with norm_w set, also the first RMSNorm's operand: per
// 32-element block (one half-wave), Q8_0 codes of x*w with d' = amax/127
// (cpu.rs:724-743) and the block's sum of x^2 (cpu.rs:381, summed per block).
// Threads of an embed_gather launch (its launch bounds; the block size read
// at run time would be a memory load).
constexpr int kEmbedThreads = 256;

extern "C" __global__ __launch_bounds__(kEmbedThreads) void embed_gather(EmbedArgs e) {
  if (e.rope_now && blockIdx.x == 0 && (e.batch_stride || blockIdx.y == 0)) {
    const int p = min(e.batch_stride ? e.pos_ptr[blockIdx.y] : *e.pos_ptr, e.rope_rows - 1);
    float* dst = e.rope_now + (size_t)blockIdx.y * 2 * e.rope_mid;
    for (int t = threadIdx.x; t < e.rope_mid; t += kEmbedThreads) {
      dst[t] = e.rope_cos[(size_t)p * e.rope_mid + t];
      dst[e.rope_mid + t] = e.rope_sin[(size_t)p * e.rope_mid + t];
    }
  }
  const float* row;
  if (e.x_in) {
    row = e.x_in;
  } else {
    // Row blockIdx.y of a chunk starting at *pos_ptr (one row when decoding),
    // or sequence blockIdx.y of a batch at its own position.
    int tok = e.batch_stride ? e.tokens[(size_t)blockIdx.y * e.batch_stride + e.pos_ptr[blockIdx.y]]
                             : e.tokens[*e.pos_ptr + blockIdx.y];
    if (tok < 0 || tok >= e.vocab) {
      if (threadIdx.x == 0 && blockIdx.x == 0) *e.err = 1;
      tok = 0;
    }
    row = e.table + (size_t)tok * e.hidden;
  }
  float* x = e.x + (size_t)blockIdx.y * e.hidden;
  for (int i0 = blockIdx.x * kEmbedThreads; i0 < e.hidden; i0 += gridDim.x * kEmbedThreads) {
    const int i = i0 + threadIdx.x;
    const bool ok = i < e.hidden;  // hidden is a multiple of 32: whole half-waves
    const float v = ok ? row[i] : 0.0f;
    if (ok) x[i] = v;
    if (e.norm_w) {
      const float z = ok ? v * e.norm_w[i] : 0.0f;
      float d;
      const int q = q8_group32(z, &d);
      const float ss = group_sum<32>(v * v);
      if (ok) {
        e.xq[i] = (int8_t)q;
        if ((i & 31) == 0) {
          e.xd[i / 32] = d;
          e.xss[i / 32] = ss;
        }
      }
    }
  }
}

// XCD (XCC id) each workgroup of a (gx, gy) grid runs on, at its linear index:
// lets the host check how workgroups are dealt to the XCDs.
extern "C" __global__ __launch_bounds__(64) void xcc_ids(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x + blockIdx.y * gridDim.x] = __builtin_amdgcn_s_getreg((15 << 11) | 20);
}

// The device exponential on n values: out[i] = exp(a[i]) as glibc's expf
// computes it (exact_math.h; test probe).
extern "C" __global__ __launch_bounds__(256) void expf_probe(EwArgs e) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < e.n; i += (long)gridDim.x * blockDim.x)
    e.out[i] = exact_expf(e.a[i]);
}
