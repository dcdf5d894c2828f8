// tensor.cpp - device tensors and the trait Backend mirror (src/backend.rs).
#include <cstring>
#include <memory>

#include "../kernel_args.h"
#include "internal.h"

using namespace llmrs;

namespace {

constexpr int kBlock = 256;

llmrs_tensor* new_tensor(int dtype, const std::vector<size_t>& dims) {
  auto* t = new llmrs_tensor();
  t->dtype = dtype;
  t->dims = dims;
  return t;
}

// Allocates an f32 tensor through the caching allocator.
llmrs_tensor* alloc_f32(const std::vector<size_t>& dims) {
  std::unique_ptr<llmrs_tensor> t(new_tensor(LLMRS_F32, dims));
  t->bytes = t->numel() * sizeof(float);
  t->data = ctx().alloc.alloc(t->bytes);
  return t.release();
}

void require_f32(const llmrs_tensor* t, const char* what) {
  LLMRS_REQUIRE(t, LLMRS_E_INVALID, std::string(what) + ": null tensor");
  LLMRS_REQUIRE(t->dtype == LLMRS_F32, LLMRS_E_DTYPE,
                std::string(what) + ": requires an f32 tensor");
}

std::vector<size_t> dims_of(const size_t* dims, int ndim) {
  LLMRS_REQUIRE(ndim >= 1 && ndim <= 8 && dims, LLMRS_E_INVALID, "ndim must be in 1..8");
  return std::vector<size_t>(dims, dims + ndim);
}

// (rows, last) view of a tensor: the reference's row-wise ops take the last
// dimension as the row length (cpu.rs:328,361,397).
void rows_last(const llmrs_tensor* t, size_t* rows, size_t* last) {
  *last = t->dims.back();
  *rows = *last ? t->numel() / *last : 0;
}

unsigned grid_for(size_t n) {
  size_t g = (n + kBlock - 1) / kBlock;
  return (unsigned)std::max<size_t>(1, std::min<size_t>(g, 65535));
}

void upload(void* dst, const void* src, size_t bytes) {
  if (!bytes) return;
  LLMRS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream));
  LLMRS_HIP(hipStreamSynchronize(ctx().stream));
}

// Quantised weight upload: codes + scales in the device layout, one
// allocation.
llmrs_tensor* upload_quant(int dtype, int wt, size_t n, size_t k,
                           const std::function<void(uint8_t*, uint8_t*)>& fill) {
  LLMRS_REQUIRE(n > 0 && k > 0 && k % 32 == 0, LLMRS_E_INVALID,
                "quantised tensor needs n > 0 and k a positive multiple of 32");
  const size_t nb = k / 32;
  const size_t code_bytes = n * nb * block_code_bytes(wt);
  const size_t scale_off = align_up(code_bytes, 256);
  const size_t total = scale_off + n * nb * block_scale_bytes(wt);
  std::vector<uint8_t> host(total, 0);
  fill(host.data(), host.data() + scale_off);
  std::unique_ptr<llmrs_tensor> t(new_tensor(dtype, {n, k}));
  t->wt = wt;
  t->bytes = total;
  t->data = ctx().alloc.alloc(total);
  t->scales = (uint8_t*)t->data + scale_off;
  upload(t->data, host.data(), total);
  return t.release();
}

}  // namespace

extern "C" {

int llmrs_tensor_upload_f32(const float* data, const size_t* dims, int ndim, llmrs_tensor** out) {
  return guard([&] {
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    std::unique_ptr<llmrs_tensor> t(alloc_f32(dims_of(dims, ndim)));
    if (t->numel()) {
      LLMRS_REQUIRE(data, LLMRS_E_INVALID, "data is null");
      upload(t->data, data, t->bytes);
    }
    *out = t.release();
  });
}

int llmrs_tensor_upload_q4(const uint8_t* qs, const float* scales, size_t n, size_t k,
                           llmrs_tensor** out) {
  return guard([&] {
    LLMRS_REQUIRE(out && qs && scales, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(k % 32 == 0, LLMRS_E_INVALID, "k must be a multiple of 32");
    const bool f16 = scales_fit_f16(scales, n * (k / 32));
    const int wt = f16 ? WT_Q4H : WT_Q4F;
    *out = upload_quant(f16 ? LLMRS_Q4_0 : LLMRS_Q4, wt, n, k, [&](uint8_t* c, uint8_t* s) {
      repack_q4_rows(qs, scales, n, k, wt, {}, c, s);
    });
  });
}

int llmrs_tensor_upload_q8_0(const int8_t* qs, const float* scales, size_t n, size_t k,
                             llmrs_tensor** out) {
  return guard([&] {
    LLMRS_REQUIRE(out && qs && scales, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(k % 32 == 0, LLMRS_E_INVALID, "k must be a multiple of 32");
    LLMRS_REQUIRE(scales_fit_f16(scales, n * (k / 32)), LLMRS_E_INVALID,
                  "Q8_0 scales must be exactly representable in fp16");
    *out = upload_quant(LLMRS_Q8_0, WT_Q8H, n, k, [&](uint8_t* c, uint8_t* s) {
      repack_q8_rows(qs, scales, n, k, {}, c, s);
    });
  });
}

int llmrs_tensor_zeros(const size_t* dims, int ndim, llmrs_tensor** out) {
  return guard([&] {
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    std::unique_ptr<llmrs_tensor> t(alloc_f32(dims_of(dims, ndim)));
    if (t->bytes) LLMRS_HIP(hipMemsetAsync(t->data, 0, t->bytes, ctx().stream));
    *out = t.release();
  });
}

int llmrs_tensor_download(const llmrs_tensor* t, float* out, size_t count) {
  return guard([&] {
    require_f32(t, "download");
    LLMRS_REQUIRE(count == t->numel(), LLMRS_E_INVALID, "download count != numel");
    LLMRS_REQUIRE(out || !count, LLMRS_E_INVALID, "out is null");
    if (count)
      LLMRS_HIP(hipMemcpyAsync(out, t->data, count * sizeof(float), hipMemcpyDeviceToHost,
                               ctx().stream));
    LLMRS_HIP(hipStreamSynchronize(ctx().stream));
  });
}

int llmrs_tensor_ndim(const llmrs_tensor* t) { return t ? (int)t->dims.size() : LLMRS_E_INVALID; }

int llmrs_tensor_dims(const llmrs_tensor* t, size_t* dims) {
  if (!t || !dims) return LLMRS_E_INVALID;
  for (size_t i = 0; i < t->dims.size(); ++i) dims[i] = t->dims[i];
  return LLMRS_OK;
}

int llmrs_tensor_dtype(const llmrs_tensor* t) { return t ? t->dtype : LLMRS_E_INVALID; }

int llmrs_tensor_free(llmrs_tensor* t) {
  return guard([&] {
    if (!t) return;
    if (t->data) ctx().alloc.release(t->data);
    delete t;
  });
}

// Backend::matmul (backend.rs:21; cpu.rs:157-224).
int llmrs_matmul(const llmrs_tensor* a, const llmrs_tensor* b, llmrs_tensor** out) {
  return guard([&] {
    require_f32(a, "matmul a");
    require_f32(b, "matmul b");
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    LLMRS_REQUIRE(a->dims.size() == 2 && b->dims.size() == 2, LLMRS_E_INVALID, "matmul: 2-D only");
    const size_t m = a->dims[0], k = a->dims[1], n = b->dims[1];
    LLMRS_REQUIRE(b->dims[0] == k, LLMRS_E_INVALID, "MatMul Dimension mismatch");
    std::unique_ptr<llmrs_tensor> o(alloc_f32({m, n}));
    if (m && n) {
      MatArgs g{(const float*)a->data, (const float*)b->data, (float*)o->data, (int)m, (int)k, (int)n};
      launch("matmul_f32", dim3(grid_for(m * n)), dim3(kBlock), 0, ctx().stream, g);
    }
    *out = o.release();
  });
}

// Backend::matmul_transposed (backend.rs:24; cpu.rs:31-151).
int llmrs_matmul_transposed(const llmrs_tensor* a, const llmrs_tensor* b, llmrs_tensor** out) {
  return guard([&] {
    require_f32(a, "matmul_transposed a");
    LLMRS_REQUIRE(b && out, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(a->dims.size() == 2 && b->dims.size() == 2, LLMRS_E_INVALID,
                  "matmul_transposed: 2-D only");
    const size_t m = a->dims[0], k = a->dims[1], n = b->dims[0];
    LLMRS_REQUIRE(b->dims[1] == k, LLMRS_E_INVALID, "MatMul Transposed dimensions mismatch");
    std::unique_ptr<llmrs_tensor> o(alloc_f32({m, n}));
    if (m == 0 || n == 0) {
      *out = o.release();
      return;
    }
    if (b->dtype == LLMRS_F32) {
      MatArgs g{(const float*)a->data, (const float*)b->data, (float*)o->data, (int)m, (int)k, (int)n};
      launch("matmul_t_f32", dim3(grid_for(m * n)), dim3(kBlock), 0, ctx().stream, g);
    } else if (m > 1) {
      // Several rows (cpu.rs:90-110): Q8_0 codes of each row, then the exact
      // int8 GEMM, whose outputs equal the reference's bit for bit.
      LLMRS_REQUIRE(b->wt >= 0, LLMRS_E_DTYPE, "Unsupported storage type for B in matmul_transposed");
      LLMRS_REQUIRE(k <= 32768, LLMRS_E_INVALID, "matmul_transposed: k is limited to 32768");
      LLMRS_REQUIRE(m <= 65535 * 128, LLMRS_E_INVALID, "matmul_transposed: too many rows");
      hipStream_t s = ctx().stream;
      int8_t* xq = (int8_t*)ctx().alloc.alloc(m * k);
      float* xd = (float*)ctx().alloc.alloc(m * (k / 32) * sizeof(float));
      PrefillRowArgs r{(const float*)a->data, nullptr, xq, xd, (int)m, (int)k, 0.0f, llmrs::kActNatural};
      launch("prefill_rows_q8", dim3((unsigned)m), dim3(kBlock), gemv_act_lds_host((int)k), s, r);
      PrefillGemmArgs g{xq, xd, (const uint8_t*)b->data, b->scales, (float*)o->data, nullptr,
                        nullptr, nullptr, (int)m, (int)n, (int)k, (int)n, gemm_group_m()};
      launch(std::string("gemm_") + wt_tag(b->wt) + "_store",
             dim3((unsigned)((n + 127) / 128), (unsigned)((m + 127) / 128)), dim3(kBlock),
             gemm_lds_bytes(), s, g);
      ctx().alloc.release(xd);  // stream-ordered reuse only
      ctx().alloc.release(xq);
    } else {
      LLMRS_REQUIRE(b->wt >= 0, LLMRS_E_DTYPE, "Unsupported storage type for B in matmul_transposed");
      GemvArgs g{};
      g.wq = (const uint8_t*)b->data;
      g.ws = b->scales;
      g.n = (int)n;
      g.k = (int)k;
      g.x = (const float*)a->data;
      g.y = (float*)o->data;
      LLMRS_REQUIRE(k <= 32768, LLMRS_E_INVALID, "matmul_transposed: k is limited to 32768");
      const GemvPlan p = gemv_plan(b->wt, "quant_store", (int)n, (int)k, ctx().num_cus);
      launch(p.name, dim3(p.grid, (unsigned)m), dim3(kBlock), p.lds, ctx().stream, g);
    }
    *out = o.release();
  });
}

// Backend::matmul_slice (backend.rs:28; cpu.rs:230-269): the host slice is
// uploaded first, as the OpenCL backend does (opencl.rs:396-419).
int llmrs_matmul_slice(const llmrs_tensor* a, const float* other_data, size_t rows, size_t cols,
                       llmrs_tensor** out) {
  return guard([&] {
    require_f32(a, "matmul_slice a");
    LLMRS_REQUIRE(out && (other_data || rows * cols == 0), LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(a->dims.size() == 2, LLMRS_E_INVALID, "matmul_slice: 2-D only");
    const size_t m = a->dims[0], k = a->dims[1];
    LLMRS_REQUIRE(k == cols, LLMRS_E_INVALID, "MatMul Slice mismatch");
    std::unique_ptr<llmrs_tensor> o(alloc_f32({m, rows}));
    if (m && rows) {
      void* tmp = ctx().alloc.alloc(rows * cols * sizeof(float));
      upload(tmp, other_data, rows * cols * sizeof(float));
      MatArgs g{(const float*)a->data, (const float*)tmp, (float*)o->data, (int)m, (int)k, (int)rows};
      launch("matmul_t_f32", dim3(grid_for(m * rows)), dim3(kBlock), 0, ctx().stream, g);
      ctx().alloc.release(tmp);  // stream-ordered reuse only
    }
    *out = o.release();
  });
}

// Backend::add_assign (backend.rs:31; cpu.rs:274-296).
int llmrs_add_assign(llmrs_tensor* a, const llmrs_tensor* b) {
  return guard([&] {
    require_f32(a, "add_assign a");
    require_f32(b, "add_assign b");
    LLMRS_REQUIRE(a->dims == b->dims, LLMRS_E_INVALID, "Shape mismatch");
    EwArgs e{(float*)a->data, (const float*)b->data, nullptr, 0.0f, (long)a->numel()};
    if (e.n) launch("add_assign_f32", dim3(grid_for(e.n)), dim3(kBlock), 0, ctx().stream, e);
  });
}

// Backend::silu_mul (backend.rs:32; cpu.rs:298-324).
int llmrs_silu_mul(llmrs_tensor* gate, const llmrs_tensor* up) {
  return guard([&] {
    require_f32(gate, "silu_mul gate");
    require_f32(up, "silu_mul up");
    LLMRS_REQUIRE(gate->dims == up->dims, LLMRS_E_INVALID, "Shape mismatch");
    EwArgs e{(float*)gate->data, (const float*)up->data, nullptr, 0.0f, (long)gate->numel()};
    if (e.n) launch("silu_mul_f32", dim3(grid_for(e.n)), dim3(kBlock), 0, ctx().stream, e);
  });
}

// The device exponential of the SiLU and softmax kernels on n host values
// (test probe): out[i] = expf(x[i]) as glibc computes it.
int llmrs_probe_expf(const float* x, size_t n, float* out) {
  return guard([&] {
    LLMRS_REQUIRE((x && out) || n == 0, LLMRS_E_INVALID, "null argument");
    if (!n) return;
    void* d = ctx().alloc.alloc(2 * n * sizeof(float));
    try {
      upload(d, x, n * sizeof(float));
      EwArgs e{(float*)d, nullptr, (float*)d + n, 0.0f, (long)n};
      launch("expf_probe", dim3(grid_for(e.n)), dim3(kBlock), 0, ctx().stream, e);
      LLMRS_HIP(hipMemcpyAsync(out, (float*)d + n, n * sizeof(float), hipMemcpyDeviceToHost, ctx().stream));
      LLMRS_HIP(hipStreamSynchronize(ctx().stream));
    } catch (...) {
      (void)hipStreamSynchronize(ctx().stream);
      ctx().alloc.release(d);
      throw;
    }
    ctx().alloc.release(d);
  });
}

// Backend::rope_inplace (backend.rs:33; cpu.rs:326-357).
int llmrs_rope_inplace(llmrs_tensor* x, size_t start_pos) {
  return guard([&] {
    require_f32(x, "rope_inplace");
    size_t rows, hd;
    rows_last(x, &rows, &hd);
    LLMRS_REQUIRE(hd % 2 == 0, LLMRS_E_INVALID, "rope: head_dim must be even");
    if (!rows || !hd) return;
    const size_t mid = hd / 2;
    std::vector<float> tab(2 * rows * mid);
    rope_table(start_pos, rows, (int)hd, 500000.0f, tab.data(), tab.data() + rows * mid);
    void* dt = ctx().alloc.alloc(tab.size() * sizeof(float));
    upload(dt, tab.data(), tab.size() * sizeof(float));
    RopeArgs r{(float*)x->data, (const float*)dt, (const float*)dt + rows * mid, (int)rows, (int)hd};
    launch("rope_f32", dim3(grid_for(rows * mid)), dim3(kBlock), 0, ctx().stream, r);
    ctx().alloc.release(dt);
  });
}

// Backend::rms_norm (backend.rs:36; cpu.rs:359-393).
int llmrs_rms_norm(const llmrs_tensor* x, const llmrs_tensor* weight, float eps, llmrs_tensor** out) {
  return guard([&] {
    require_f32(x, "rms_norm x");
    require_f32(weight, "rms_norm weight");
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    size_t rows, dim;
    rows_last(x, &rows, &dim);
    LLMRS_REQUIRE(weight->numel() >= dim, LLMRS_E_INVALID, "rms_norm: weight shorter than row");
    std::unique_ptr<llmrs_tensor> o(alloc_f32(x->dims));
    if (rows && dim) {
      RowArgs r{(const float*)x->data, (const float*)weight->data, (float*)o->data, (int)rows, (int)dim, eps};
      launch("rms_norm_f32", dim3((unsigned)rows), dim3(kBlock), 0, ctx().stream, r);
    }
    *out = o.release();
  });
}

// Backend::softmax (backend.rs:37; cpu.rs:395-423).
int llmrs_softmax(const llmrs_tensor* x, llmrs_tensor** out) {
  return guard([&] {
    require_f32(x, "softmax");
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    size_t rows, dim;
    rows_last(x, &rows, &dim);
    std::unique_ptr<llmrs_tensor> o(alloc_f32(x->dims));
    if (rows && dim) {
      RowArgs r{(const float*)x->data, nullptr, (float*)o->data, (int)rows, (int)dim, 0.0f};
      launch("softmax_f32", dim3((unsigned)rows), dim3(kBlock), 0, ctx().stream, r);
    }
    *out = o.release();
  });
}

// Backend::scale (backend.rs:38; cpu.rs:425-435).
int llmrs_scale(const llmrs_tensor* x, float value, llmrs_tensor** out) {
  return guard([&] {
    require_f32(x, "scale");
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    std::unique_ptr<llmrs_tensor> o(alloc_f32(x->dims));
    EwArgs e{(float*)x->data, nullptr, (float*)o->data, value, (long)x->numel()};
    if (e.n) launch("scale_f32", dim3(grid_for(e.n)), dim3(kBlock), 0, ctx().stream, e);
    *out = o.release();
  });
}

// Self-check with no counterpart in the reference: the reference-order
// attention's one-instruction f16 products against the conversion and
// multiply, for every f16 pattern and the values of x.
int llmrs_check_mul_f16(const llmrs_tensor* x, llmrs_tensor** out) {
  return guard([&] {
    require_f32(x, "check_mul_f16");
    LLMRS_REQUIRE(out, LLMRS_E_INVALID, "out is null");
    std::unique_ptr<llmrs_tensor> o(alloc_f32({65536}));
    EwArgs e{(float*)x->data, nullptr, (float*)o->data, 0.0f, (long)x->numel()};
    launch("check_mul_f16", dim3(256), dim3(256), 0, ctx().stream, e);
    *out = o.release();
  });
}

// Backend::copy_from (backend.rs:39; cpu.rs:437-446).
int llmrs_copy_from(const llmrs_tensor* t, llmrs_tensor** out) {
  return guard([&] {
    LLMRS_REQUIRE(t && out, LLMRS_E_INVALID, "null argument");
    std::unique_ptr<llmrs_tensor> o(new_tensor(t->dtype, t->dims));
    o->wt = t->wt;
    o->bytes = t->bytes;
    o->data = ctx().alloc.alloc(t->bytes);
    if (t->scales) o->scales = (uint8_t*)o->data + ((uint8_t*)t->scales - (uint8_t*)t->data);
    if (t->bytes)
      LLMRS_HIP(hipMemcpyAsync(o->data, t->data, t->bytes, hipMemcpyDeviceToDevice, ctx().stream));
    *out = o.release();
  });
}

}  // extern "C"
