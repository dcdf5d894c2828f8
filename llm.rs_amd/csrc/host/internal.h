// internal.h - shared declarations of the llmrs_hip host library.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "llmrs_hip.h"

// From libamdhip64 (declared in hip/hip_ext.h, whose C++ templates need the
// HIP compiler): a module launch whose start and stop events are recorded by
// the dispatch itself.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams, void** extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);

namespace llmrs {

// An error carried up to the C ABI, where it becomes a return code plus the
// thread-local message of llmrs_last_error().
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] void fail(int code, const std::string& msg);

#define LLMRS_HIP(expr)                                                              \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess)                                                            \
      ::llmrs::fail(LLMRS_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define LLMRS_REQUIRE(cond, code, msg) \
  do {                                 \
    if (!(cond)) ::llmrs::fail((code), (msg)); \
  } while (0)

// Size-bucketed caching allocator for operator outputs: the analogue of the
// reference's OpenCL scratch pool (opencl.rs:36-90), without its per-token
// reset - buffers return to their bucket when the tensor is freed.
class Allocator {
 public:
  void* alloc(size_t bytes);
  void release(void* p);
  void trim();  // hipFree every cached block
 private:
  std::multimap<size_t, void*> free_;
  std::map<void*, size_t> live_;
};

// Device scratch of llmrs_matmul_transposed_noalloc (noalloc.hip): a fixed
// array of the library's own code object, one per device.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
// Its device address on the current device (hipGetSymbolAddress).
void* noalloc_scratch_address();

// A loaded kernel and the most threads per workgroup it accepts.
struct KernelInfo {
  hipFunction_t f = nullptr;
  int max_threads = 0;
};

struct Context {
  int device = -1;
  hipStream_t stream = nullptr;
  int num_cus = 0;
  void* noalloc_scratch = nullptr;  // device address of the scratch on `device`
  std::string noalloc_error;        // why it is null
  std::vector<hipModule_t> modules;
  std::map<std::string, KernelInfo> kernels;
  Allocator alloc;
};

Context& ctx();  // fails with LLMRS_E_NOINIT before llmrs_init
std::recursive_mutex& api_mutex();
// The kernel `name`; fails (LLMRS_E_INVALID) when `block` exceeds the
// threads per workgroup it was compiled for (its launch bounds).
hipFunction_t kernel(const std::string& name, dim3 block = dim3(1));
// Whether the workgroups of a (gx, gy) launch whose linear indices agree mod 8
// run on one XCD (measured with one launch of xcc_ids).
bool xcd_dealt_mod8(unsigned gx, unsigned gy);

template <class Args>
void launch(const std::string& name, dim3 grid, dim3 block, size_t shmem, hipStream_t stream,
            const Args& args) {
  hipFunction_t f = kernel(name, block);
  void* params[] = {const_cast<Args*>(&args)};
  LLMRS_HIP(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                  (unsigned)shmem, stream, params, nullptr));
}

// A launch whose two events carry the dispatch packet's own start and end
// timestamps (hipExtModuleLaunchKernel), so their elapsed time is the
// kernel's execution time, as a kernel trace reports it, without the
// event packets' own latency.
template <class Args>
void launch_timed(const std::string& name, dim3 grid, dim3 block, size_t shmem, hipStream_t stream,
                  const Args& args, hipEvent_t start, hipEvent_t stop) {
  hipFunction_t f = kernel(name, block);
  void* params[] = {const_cast<Args*>(&args)};
  LLMRS_HIP(hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x,
                                     block.y, block.z, shmem, stream, params, nullptr, start, stop, 0));
}

// Runs `fn` and converts exceptions into a C return code.
template <class F>
int guard(F&& fn) {
  extern void set_last_error(const std::string&);
  try {
    std::lock_guard<std::recursive_mutex> lk(api_mutex());
    fn();
    return LLMRS_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return LLMRS_E_OOM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return LLMRS_E_INVALID;
  }
}
void set_last_error(const std::string& msg);

// ---- weight layouts ------------------------------------------------------
// Kernel weight types (must match the WT_* enumeration in gemv.hip).
enum { WT_Q4H = 0, WT_Q4F = 1, WT_Q8H = 2 };
const char* wt_tag(int wt);
// PrefillGemmArgs::group_m for every prefill GEMM launch (LLMRS_GEMM_GROUP).
int gemm_group_m();

// Launch plan of one GEMV: kernel name, grid and dynamic LDS bytes.
// `kind` is the prologue/epilogue pair of gemv.hip: quant_store,
// norm_store, q8_resid, norm_silu or norm_argmax.
struct GemvPlan {
  std::string name;
  unsigned grid = 1;
  unsigned threads = 256;
  size_t lds = 0;
};
GemvPlan gemv_plan(int wt, const std::string& kind, int n, int k, int num_cus);
// LDS bytes of a GEMV's activation area (codes, scales, Q4 offsets) for input length k.
inline size_t gemv_act_lds_host(int k) { return (size_t)k + 8 * (size_t)(k / 32); }

// Bytes of codes per 32-element block.
inline int block_code_bytes(int wt) { return wt == WT_Q8H ? 32 : 16; }
inline int block_scale_bytes(int wt) { return wt == WT_Q4F ? 4 : 2; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Host-side repack of rows of a reference-format matrix into the device
// layout: codes [rows][nb][B] then scales [rows][nb].  `dst_codes` /
// `dst_scales` are host staging areas indexed by device row; `row_map[i]`
// gives the device row of source row i.
void repack_q4_rows(const uint8_t* qs, const float* scales, size_t rows, size_t k, int wt,
                    const std::vector<size_t>& row_map, uint8_t* dst_codes, uint8_t* dst_scales);
void repack_q8_rows(const int8_t* qs, const float* scales, size_t rows, size_t k,
                    const std::vector<size_t>& row_map, uint8_t* dst_codes, uint8_t* dst_scales);
bool scales_fit_f16(const float* scales, size_t count);
uint16_t host_f2h(float f);
float host_h2f(uint16_t h);

// Parallel for over [0, n) chunks with host threads.
void parallel_for(size_t n, int threads, const std::function<void(size_t, size_t)>& fn);

// RoPE tables exactly as the reference computes them (cpu.rs:345-349):
// inv = 1 / powf(theta, fl(2j)/hd); a = fl(pos) * inv; sinf(a), cosf(a).
void rope_table(size_t pos0, size_t npos, int hd, float theta, float* cos_out, float* sin_out);

}  // namespace llmrs

struct llmrs_tensor {
  int dtype = LLMRS_F32;
  int wt = -1;                // kernel weight type for quantised tensors
  std::vector<size_t> dims;
  void* data = nullptr;       // f32 values, or codes of quantised tensors
  void* scales = nullptr;     // scales of quantised tensors (same allocation)
  size_t bytes = 0;
  size_t numel() const {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    return dims.empty() ? 0 : n;
  }
};
