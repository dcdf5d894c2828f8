// runtime.cpp - device context, module loading, allocator, errors, helpers.
#include <dlfcn.h>
#include <immintrin.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <functional>
#include <thread>

#include "../kernel_args.h"
#include "internal.h"

namespace llmrs {

namespace {
thread_local std::string g_last_error;
Context* g_ctx = nullptr;

std::string library_dir() {
  Dl_info info;
  if (dladdr((void*)&library_dir, &info) && info.dli_fname) {
    return std::filesystem::path(info.dli_fname).parent_path().string();
  }
  return ".";
}
}  // namespace

void fail(int code, const std::string& msg) { throw Error(code, msg); }
void set_last_error(const std::string& msg) { g_last_error = msg; }

std::recursive_mutex& api_mutex() {
  static std::recursive_mutex m;
  return m;
}

Context& ctx() {
  if (!g_ctx) fail(LLMRS_E_NOINIT, "llmrs_init has not been called");
  return *g_ctx;
}

hipFunction_t kernel(const std::string& name, dim3 block) {
  Context& c = ctx();
  auto it = c.kernels.find(name);
  if (it == c.kernels.end()) {
    for (hipModule_t m : c.modules) {
      KernelInfo k;
      if (hipModuleGetFunction(&k.f, m, name.c_str()) == hipSuccess && k.f) {
        LLMRS_HIP(hipFuncGetAttribute(&k.max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, k.f));
        it = c.kernels.emplace(name, k).first;
        break;
      }
    }
    if (it == c.kernels.end()) {
      (void)hipGetLastError();
      fail(LLMRS_E_MODULE, "kernel not found in any loaded hsaco: " + name);
    }
  }
  const long threads = (long)block.x * block.y * block.z;
  LLMRS_REQUIRE(threads <= it->second.max_threads, LLMRS_E_INVALID,
                name + ": " + std::to_string(threads) + " threads per workgroup, compiled for at most " +
                    std::to_string(it->second.max_threads));
  return it->second.f;
}

bool xcd_dealt_mod8(unsigned gx, unsigned gy) {
  const size_t n = (size_t)gx * gy;
  int* d = nullptr;
  LLMRS_HIP(hipMalloc(&d, n * sizeof(int)));
  std::vector<int> h(n);
  hipError_t e = hipSuccess;
  void* args[] = {&d};
  e = hipModuleLaunchKernel(kernel("xcc_ids", dim3(64)), gx, gy, 1, 64, 1, 1, 0, ctx().stream, args, nullptr);
  if (e == hipSuccess) e = hipMemcpyAsync(h.data(), d, n * sizeof(int), hipMemcpyDeviceToHost, ctx().stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
  (void)hipFree(d);
  LLMRS_HIP(e);
  for (size_t i = 8; i < n; ++i)
    if (h[i] != h[i % 8]) return false;
  return true;
}

int gemm_group_m() {
  // 4 token tiles per group: on the 8B shapes at M = 2048 this cuts the
  // gate|up GEMM's L2 fetches 2.7x against row-major (8 is close, 2 and 16
  // fetch 1.5x and 2.1x more than 4)
  static const int g = [] {
    const char* v = std::getenv("LLMRS_GEMM_GROUP");
    return (v && *v) ? std::atoi(v) : 4;
  }();
  return g;
}

const char* wt_tag(int wt) {
  switch (wt) {
    case WT_Q4H: return "q4h";
    case WT_Q4F: return "q4f";
    case WT_Q8H: return "q8h";
  }
  fail(LLMRS_E_DTYPE, "unknown weight type");
}

// Rows per wave-unit R and 64-block chunks per unit U follow the shape: U = 2
// when the row splits into whole 128-block chunks, R = 2 for the narrow
// (n <= 8192) projections so that more waves share them.  The SwiGLU tile is
// 64 rows per workgroup (8-wave workgroups looping over the tiles, one per
// CU, when the tiles outnumber the CUs); other kinds deal R-row groups to
// waves, capped at
// LLMRS_GEMV_WG_PER_CU (default 2, the best of 1/2/4/8 measured on the 8B
// decode) workgroups per CU, beyond which waves loop.
GemvPlan gemv_plan(int wt, const std::string& kind, int n, int k, int num_cus) {
  const int nb = k / 32;
  int U = (nb % 128 == 0) ? 2 : 1;
  const char* eu = std::getenv("LLMRS_GEMV_U");
  if (eu && (std::atoi(eu) == 1 || std::atoi(eu) == 2)) U = std::atoi(eu);
  int R = 4;
  if (kind == "norm_store" || kind == "q8_resid" || kind == "nq_store" || kind == "q8b_store" ||
      kind == "q8b_resid") {
    R = 2;
    const char* er = std::getenv("LLMRS_GEMV_R");
    if (er && (std::atoi(er) == 2 || std::atoi(er) == 4)) R = std::atoi(er);
  }
  int waves = 4;
  if (kind == "q8_nq") {  // 32-row tiles, one per 8-wave workgroup (gemv_w8.hip)
    R = 2;
    waves = 8;
  }
  // SwiGLU with the RMSNorm prologue, more 64-row tiles than CUs: 8-wave
  // workgroups, one per CU (LLMRS_GEMV_SILU_W8=0/1 forces either)
  const char* es = std::getenv("LLMRS_GEMV_SILU_W8");
  const bool silu_w8 = kind == "norm_silu" && (es && *es ? std::atoi(es) == 1 : n / 64 > num_cus);
  if (silu_w8) waves = 8;
  // Workgroups per CU (measured on MI355X): 1 for the RMSNorm-prologue
  // store GEMV (Q|K|V: 8B 14 MB, 70B 47 MB) and for matrices under 24 MB -
  // fewer, longer-lived workgroups keep the activation loads from queueing
  // behind as many weight requests - and 2 otherwise.
  const double wbytes = (double)n * k * (wt == WT_Q8H ? 34.0 : wt == WT_Q4F ? 20.0 : 18.0) / 32.0;
  const char* ew = std::getenv("LLMRS_GEMV_WG_PER_CU");
  const bool store = kind == "norm_store" || kind == "nq_store";
  const int per_cu = ew && *ew ? std::max(1, std::atoi(ew)) : (store || silu_w8 || wbytes < 24e6 ? 1 : 2);
  const long cap = (long)std::max(1, num_cus) * per_cu;
  GemvPlan p;
  p.name = std::string("gemv_") + wt_tag(wt) + "_" + kind + "_r" + std::to_string(R) + "u" +
           std::to_string(U) + (waves == 8 ? "_w8" : "");
  p.threads = 64 * waves;
  // tiled epilogues: whole 64-row SwiGLU tiles or 32-row next-norm tiles
  const int tile = (kind == "norm_silu" || kind == "nq_silu" || kind == "q8b_silu") ? 64 : kind == "q8_nq" ? 32 : 0;
  long wgs;
  if (tile) {
    wgs = (n + tile - 1) / tile;
  } else {
    const long nrg = (n + R - 1) / R;
    wgs = (nrg + waves - 1) / waves;
  }
  p.grid = (unsigned)std::max<long>(1, std::min(wgs, cap));
  p.lds = llmrs::gemv_lds_bytes(tile, n, k, R, (int)p.grid, waves);
  return p;
}

// ---- allocator -------------------------------------------------------------
void* Allocator::alloc(size_t bytes) {
  size_t sz = align_up(bytes ? bytes : 1, 256);
  if (sz > (1u << 20)) {  // round large requests to 1/8 octave to improve reuse
    size_t p = 1;
    while (p < sz) p <<= 1;
    size_t step = std::max<size_t>(p / 8, 256);
    sz = align_up(sz, step);
  }
  auto it = free_.find(sz);
  void* ptr = nullptr;
  if (it != free_.end()) {
    ptr = it->second;
    free_.erase(it);
  } else {
    hipError_t e = hipMalloc(&ptr, sz);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      trim();
      e = hipMalloc(&ptr, sz);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      fail(LLMRS_E_OOM, "hipMalloc of " + std::to_string(sz) + " bytes failed");
    }
  }
  live_[ptr] = sz;
  return ptr;
}

void Allocator::release(void* p) {
  if (!p) return;
  auto it = live_.find(p);
  if (it == live_.end()) return;
  free_.emplace(it->second, p);
  live_.erase(it);
}

void Allocator::trim() {
  for (auto& kv : free_) (void)hipFree(kv.second);
  free_.clear();
}

// ---- host helpers ----------------------------------------------------------
uint16_t host_f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
float host_h2f(uint16_t h) { return _cvtsh_ss(h); }

bool scales_fit_f16(const float* scales, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    float back = host_h2f(host_f2h(scales[i]));
    if (!(back == scales[i]) && !(std::isnan(back) && std::isnan(scales[i]))) return false;
  }
  return true;
}

void parallel_for(size_t n, int threads, const std::function<void(size_t, size_t)>& fn) {
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  if (n < 2 || threads == 1) {
    if (n) fn(0, n);
    return;
  }
  size_t nt = std::min<size_t>((size_t)threads, n);
  size_t chunk = (n + nt - 1) / nt;
  std::vector<std::thread> ts;
  for (size_t t = 0; t < nt; ++t) {
    size_t b = t * chunk, e = std::min(n, b + chunk);
    if (b >= e) break;
    ts.emplace_back(fn, b, e);
  }
  for (auto& t : ts) t.join();
}

// Reference nibble order: byte i of a block = e[2i] | e[2i+1] << 4
// (tensor.rs:125-131).  Device order: byte i = e[i] | e[i+16] << 4, so that
// the low nibbles of a dword are four consecutive elements.
void repack_q4_rows(const uint8_t* qs, const float* scales, size_t rows, size_t k, int wt,
                    const std::vector<size_t>& row_map, uint8_t* dst_codes, uint8_t* dst_scales) {
  const size_t nb = k / 32;
  parallel_for(rows, 0, [&](size_t r0, size_t r1) {
    uint8_t e[32];
    for (size_t r = r0; r < r1; ++r) {
      const size_t dr = row_map.empty() ? r : row_map[r];
      for (size_t b = 0; b < nb; ++b) {
        const uint8_t* src = qs + r * (k / 2) + b * 16;
        for (int i = 0; i < 16; ++i) {
          e[2 * i] = src[i] & 0x0F;
          e[2 * i + 1] = src[i] >> 4;
        }
        uint8_t* dst = dst_codes + (dr * nb + b) * 16;
        for (int i = 0; i < 16; ++i) dst[i] = (uint8_t)(e[i] | (e[i + 16] << 4));
        const float s = scales[r * nb + b];
        if (wt == WT_Q4F) {
          std::memcpy(dst_scales + (dr * nb + b) * 4, &s, 4);
        } else {
          const uint16_t h = host_f2h(s);
          std::memcpy(dst_scales + (dr * nb + b) * 2, &h, 2);
        }
      }
    }
  });
}

void repack_q8_rows(const int8_t* qs, const float* scales, size_t rows, size_t k,
                    const std::vector<size_t>& row_map, uint8_t* dst_codes, uint8_t* dst_scales) {
  const size_t nb = k / 32;
  parallel_for(rows, 0, [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) {
      const size_t dr = row_map.empty() ? r : row_map[r];
      std::memcpy(dst_codes + dr * k, qs + r * k, k);
      for (size_t b = 0; b < nb; ++b) {
        const uint16_t h = host_f2h(scales[r * nb + b]);
        std::memcpy(dst_scales + (dr * nb + b) * 2, &h, 2);
      }
    }
  });
}

void rope_table(size_t pos0, size_t npos, int hd, float theta, float* cos_out, float* sin_out) {
  const int mid = hd / 2;
  std::vector<float> inv(mid);
  for (int j = 0; j < mid; ++j) {
    float freq_idx = ((float)j * 2.0f) / (float)hd;
    inv[j] = 1.0f / std::pow(theta, freq_idx);
  }
  for (size_t p = 0; p < npos; ++p)
    for (int j = 0; j < mid; ++j) {
      float a = (float)(pos0 + p) * inv[j];
      cos_out[p * mid + j] = std::cos(a);
      sin_out[p * mid + j] = std::sin(a);
    }
}

}  // namespace llmrs

using namespace llmrs;

extern "C" {

const char* llmrs_last_error(void) { return g_last_error.c_str(); }

int llmrs_init(int device_ordinal, const char* hsaco_dir) {
  return guard([&] {
    if (g_ctx) return;
    int count = 0;
    LLMRS_HIP(hipGetDeviceCount(&count));
    LLMRS_REQUIRE(device_ordinal >= 0 && device_ordinal < count, LLMRS_E_INVALID,
                  "no such HIP device: " + std::to_string(device_ordinal));
    auto* c = new Context();
    try {
      c->device = device_ordinal;
      LLMRS_HIP(hipSetDevice(device_ordinal));
      hipDeviceProp_t prop;
      LLMRS_HIP(hipGetDeviceProperties(&prop, device_ordinal));
      c->num_cus = prop.multiProcessorCount;
      LLMRS_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      // the no-allocation entry point's scratch, resolved with the device
      // current; a failure is reported by that entry point, not by init
      try {
        c->noalloc_scratch = noalloc_scratch_address();
      } catch (const Error& e) {
        c->noalloc_scratch = nullptr;
        c->noalloc_error = e.what();
      }
      std::string dir = hsaco_dir ? std::string(hsaco_dir) : library_dir();
      for (const char* name : {"gemv", "gemv_w8", "attention", "exact", "ops", "prefill", "sample", "sgemm"}) {
        std::string path = dir + "/" + name + ".hsaco";
        LLMRS_REQUIRE(std::filesystem::exists(path), LLMRS_E_MODULE, "missing code object " + path);
        hipModule_t m = nullptr;
        hipError_t e = hipModuleLoad(&m, path.c_str());
        if (e != hipSuccess)
          fail(LLMRS_E_MODULE, "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
        c->modules.push_back(m);
      }
    } catch (...) {
      for (hipModule_t m : c->modules) (void)hipModuleUnload(m);
      if (c->stream) (void)hipStreamDestroy(c->stream);
      delete c;
      throw;
    }
    g_ctx = c;
  });
}

int llmrs_shutdown(void) {
  return guard([&] {
    if (!g_ctx) return;
    (void)hipStreamSynchronize(g_ctx->stream);
    g_ctx->alloc.trim();
    for (hipModule_t m : g_ctx->modules) (void)hipModuleUnload(m);
    (void)hipStreamDestroy(g_ctx->stream);
    delete g_ctx;
    g_ctx = nullptr;
  });
}

int llmrs_device(void) { return LLMRS_DEVICE_HIP; }
const char* llmrs_name(void) { return "Hip"; }

int llmrs_sync(void) {
  return guard([&] { LLMRS_HIP(hipStreamSynchronize(ctx().stream)); });
}

int llmrs_num_cus(void) { return g_ctx ? g_ctx->num_cus : 0; }

}  // extern "C"
