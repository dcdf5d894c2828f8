// noalloc.hip - Backend::matmul_transposed into a caller-provided output,
// with no device allocation (llmrs_matmul_transposed_noalloc).
//
// For callers that cannot call hipMalloc (code under HIP graph capture,
// tight serving loops, harnesses that forbid it).  The per-row Q8_0
// activation codes the M > 1 path stages between its two kernels live in
// `scratch`, a fixed device array of this library's code object: every
// device the library runs on holds one copy until the process ends.  Host
// code never passes the array's name to a kernel (in host code it is a
// stand-in, not a device address): llmrs_init resolves the device address
// once per device with hipGetSymbolAddress, with that device current, and
// every kernel argument uses that address.
//
// Calls that overlap on one device share its scratch and race; the stream
// orders calls issued on it.  Nothing in the scratch has to start at zero:
// prefill_rows_q8 writes every code and scale the GEMM reads (its loads are
// clamped to the M rows written).
#include <hip/hip_runtime.h>

#include <memory>

#include "../kernel_args.h"
#include "internal.h"

namespace {

// codes [m][k] at offset 0, then scales [m][k/32] at the next 256-byte line
static __device__ __align__(256) uint8_t scratch[llmrs::kNoAllocScratchBytes];

size_t scratch_need(size_t m, size_t k, size_t* scale_off) {
  *scale_off = llmrs::align_up(m * k, 256);
  return *scale_off + m * (k / 32) * sizeof(float);
}

}  // namespace

namespace llmrs {

void* noalloc_scratch_address() {
  void* p = nullptr;
  LLMRS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  LLMRS_REQUIRE(p, LLMRS_E_HIP, "hipGetSymbolAddress(scratch) returned no address");
  return p;
}

}  // namespace llmrs

using namespace llmrs;

extern "C" int llmrs_matmul_transposed_noalloc(const llmrs_tensor* a, const llmrs_tensor* b,
                                               llmrs_tensor* out) {
  return guard([&] {
    LLMRS_REQUIRE(a && b && out, LLMRS_E_INVALID, "null argument");
    LLMRS_REQUIRE(a->dtype == LLMRS_F32 && out->dtype == LLMRS_F32, LLMRS_E_DTYPE,
                  "a and out must be f32 tensors");
    LLMRS_REQUIRE(a->dims.size() == 2 && b->dims.size() == 2, LLMRS_E_INVALID,
                  "matmul_transposed: 2-D only");
    const size_t m = a->dims[0], k = a->dims[1], n = b->dims[0];
    LLMRS_REQUIRE(b->dims[1] == k, LLMRS_E_INVALID, "MatMul Transposed dimensions mismatch");
    LLMRS_REQUIRE(out->dims.size() == 2 && out->dims[0] == m && out->dims[1] == n, LLMRS_E_INVALID,
                  "out must be an f32 tensor of shape [m, n]");
    if (m == 0 || n == 0) return;
    Context& cx = ctx();
    hipStream_t s = cx.stream;
    if (b->dtype == LLMRS_F32) {
      MatArgs g{(const float*)a->data, (const float*)b->data, (float*)out->data, (int)m, (int)k, (int)n};
      const size_t tot = m * n;
      launch("matmul_t_f32", dim3((unsigned)std::min<size_t>((tot + 255) / 256, 65535)), dim3(256), 0, s, g);
      return;
    }
    LLMRS_REQUIRE(b->wt >= 0, LLMRS_E_DTYPE, "Unsupported storage type for B in matmul_transposed");
    LLMRS_REQUIRE(k % 32 == 0 && k <= 32768, LLMRS_E_INVALID, "matmul_transposed: k must be a multiple of 32, at most 32768");
    if (m == 1) {  // the GEMV quantises its row in LDS: no scratch
      GemvArgs g{};
      g.wq = (const uint8_t*)b->data;
      g.ws = b->scales;
      g.n = (int)n;
      g.k = (int)k;
      g.x = (const float*)a->data;
      g.y = (float*)out->data;
      const GemvPlan p = gemv_plan(b->wt, "quant_store", (int)n, (int)k, cx.num_cus);
      launch(p.name, dim3(p.grid, 1), dim3(256), p.lds, s, g);
      return;
    }
    size_t scale_off = 0;
    const size_t need = scratch_need(m, k, &scale_off);
    LLMRS_REQUIRE(need <= kNoAllocScratchBytes, LLMRS_E_RANGE,
                  "matmul_transposed_noalloc: m*k*(1 + 4/32) bytes of activation codes exceed the " +
                      std::to_string(kNoAllocScratchBytes >> 20) + " MiB scratch (m=" + std::to_string(m) +
                      ", k=" + std::to_string(k) + ")");
    LLMRS_REQUIRE(m <= 65535 * 128, LLMRS_E_INVALID, "matmul_transposed: too many rows");
    LLMRS_REQUIRE(cx.noalloc_scratch, LLMRS_E_NOINIT,
                  "the scratch's device address was not resolved at init: " + cx.noalloc_error);
    int8_t* xq = (int8_t*)cx.noalloc_scratch;
    float* xd = (float*)((uint8_t*)cx.noalloc_scratch + scale_off);
    PrefillRowArgs r{(const float*)a->data, nullptr, xq, xd, (int)m, (int)k, 0.0f};
    launch("prefill_rows_q8", dim3((unsigned)m), dim3(256), gemv_act_lds_host((int)k), s, r);
    PrefillGemmArgs g{xq, xd, (const uint8_t*)b->data, b->scales, (float*)out->data, nullptr,
                      nullptr, nullptr, (int)m, (int)n, (int)k, (int)n, gemm_group_m()};
    launch(std::string("gemm_") + wt_tag(b->wt) + "_store",
           dim3((unsigned)((n + 127) / 128), (unsigned)((m + 127) / 128)), dim3(256), gemm_lds_bytes(), s, g);
  });
}
