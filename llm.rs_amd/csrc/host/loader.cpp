// loader.cpp - decode models from weight files on disk.
//
// safetensors (Hugging Face checkpoints): Loader::load_model
// (src/core/loader.rs:100-198) - config.json (src/core/config.rs:3-21),
// bf16 or f32 tensors read from memory-mapped files (loader.rs:19-46), every
// linear weight quantised with Tensor::quantize_q4 (src/core/tensor.rs:102-
// 167), gate and up given separately (the model keeps them as one [2F][H]
// matrix, as loader.rs:128-146 concatenates them), lm_head or, when absent,
// the quantised embedding (loader.rs:186-190).  K and V keep their
// n_kv_heads rows: the reference duplicates them per query head
// (loader.rs:62-98), which gives the same outputs.
//
// GGUF (llama.cpp files, "llama" architecture): no reference counterpart.
// Q4_0 and Q8_0 blocks are taken as they are (the reference's own quantiser,
// amax/7, would change their codes); F32/F16/BF16 weights are quantised as
// above.  GGUF stores Q and K rows in the interleaved RoPE order of
// llama.cpp; they are put back in the rotate-half order of the reference
// (cpu.rs:326-357).
#include "internal.h"
#include "json.h"

#include <cmath>
#include <cstring>
#include <fcntl.h>
#include <fstream>
#include <sstream>
#include <sys/mman.h>
#include <sys/stat.h>
#include <thread>
#include <unistd.h>

using namespace llmrs;

namespace {

// A read-only memory map of a whole file.
struct MappedFile {
  const uint8_t* data = nullptr;
  size_t size = 0;
  int fd = -1;
  explicit MappedFile(const std::string& path) {
    fd = ::open(path.c_str(), O_RDONLY);
    LLMRS_REQUIRE(fd >= 0, LLMRS_E_FORMAT, "cannot open " + path);
    struct stat st {};
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
      ::close(fd);
      fail(LLMRS_E_FORMAT, "cannot stat " + path + " (or it is empty)");
    }
    size = (size_t)st.st_size;
    void* p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      ::close(fd);
      fail(LLMRS_E_FORMAT, "cannot map " + path);
    }
    data = (const uint8_t*)p;
  }
  ~MappedFile() {
    if (data) munmap((void*)data, size);
    if (fd >= 0) ::close(fd);
  }
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
};

std::string read_text(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  LLMRS_REQUIRE(f.good(), LLMRS_E_FORMAT, "cannot read " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

bool is_dir(const std::string& p) {
  struct stat st {};
  return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}
bool exists(const std::string& p) {
  struct stat st {};
  return stat(p.c_str(), &st) == 0;
}
std::string dir_of(const std::string& p) {
  const size_t s = p.find_last_of('/');
  return s == std::string::npos ? "." : p.substr(0, s);
}

float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

int loader_threads() {
  const unsigned hw = std::thread::hardware_concurrency();
  return (int)std::max(1u, std::min(hw == 0 ? 1u : hw, 32u));
}

// Tensor::quantize_q4 (tensor.rs:102-167) of rows x [n][k], k a multiple of
// 32, into the reference CpuQ4 format: per 32-block d = amax / 7 (amax folds
// from 0 with f32::max, which skips NaN), codes trunc(clamp(x * (1/d) + 8.5,
// 0, 15)) two per byte (the lower element in the low nibble), d == 0 giving
// 0x88; a NaN product becomes code 0, as Rust's `as u8` does.
void quantize_q4_rows(const float* x, size_t n, size_t k, uint8_t* qs, float* scales) {
  const size_t nb = n * k / 32;
  parallel_for(nb, loader_threads(), [&](size_t b0, size_t b1) {
    for (size_t b = b0; b < b1; ++b) {
      const float* c = x + 32 * b;
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) {
        const float v = std::fabs(c[i]);
        if (v > amax) amax = v;  // f32::max from 0: a NaN |x| leaves amax as it is
      }
      const float d = amax / 7.0f;
      scales[b] = d;
      uint8_t* q = qs + 16 * b;
      if (d == 0.0f) {
        std::memset(q, 0x88, 16);
        continue;
      }
      const float inv = 1.0f / d;
      auto code = [&](float v) -> unsigned {
        float t = v * inv;
        t = t + 8.5f;
        if (t != t) return 0;
        t = std::min(15.0f, std::max(0.0f, t));
        return (unsigned)t;
      };
      for (int i = 0; i < 16; ++i) q[i] = (uint8_t)(code(c[2 * i]) | (code(c[2 * i + 1]) << 4));
    }
  });
}

// ---- safetensors ----------------------------------------------------------
struct StTensor {
  std::string dtype;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

// One safetensors file: u64 header length, JSON header {name: {dtype, shape,
// data_offsets}}, then the data.
struct StFile {
  std::unique_ptr<MappedFile> map;
  std::map<std::string, StTensor> tensors;
  explicit StFile(const std::string& path) : map(new MappedFile(path)) {
    LLMRS_REQUIRE(map->size >= 8, LLMRS_E_FORMAT, path + ": too short for a safetensors file");
    uint64_t hlen = 0;
    std::memcpy(&hlen, map->data, 8);
    LLMRS_REQUIRE(hlen <= map->size - 8, LLMRS_E_FORMAT, path + ": header length beyond the file");
    json::Value h;
    try {
      h = json::parse((const char*)map->data + 8, (size_t)hlen);
    } catch (const std::exception& e) {
      fail(LLMRS_E_FORMAT, path + ": " + e.what());
    }
    LLMRS_REQUIRE(h.kind == json::Value::Object, LLMRS_E_FORMAT, path + ": header is not an object");
    const uint8_t* base = map->data + 8 + hlen;
    const size_t avail = map->size - 8 - (size_t)hlen;
    for (const auto& kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      StTensor t;
      try {
        t.dtype = kv.second.at("dtype").string();
        for (const auto& d : kv.second.at("shape").arr) t.shape.push_back((int64_t)d.number());
        const auto& off = kv.second.at("data_offsets").arr;
        LLMRS_REQUIRE(off.size() == 2, LLMRS_E_FORMAT, path + ": bad data_offsets of " + kv.first);
        const size_t b0 = (size_t)off[0].number(), b1 = (size_t)off[1].number();
        LLMRS_REQUIRE(b0 <= b1 && b1 <= avail, LLMRS_E_FORMAT, path + ": data of " + kv.first + " beyond the file");
        t.data = base + b0;
        t.bytes = b1 - b0;
      } catch (const Error&) {
        throw;
      } catch (const std::exception& e) {
        fail(LLMRS_E_FORMAT, path + ": tensor " + kv.first + ": " + e.what());
      }
      tensors[kv.first] = t;
    }
  }
};

// A checkpoint: model.safetensors, or the shards of
// model.safetensors.index.json (weight_map), in a directory or given as a file.
struct Checkpoint {
  std::vector<std::unique_ptr<StFile>> files;
  std::map<std::string, const StTensor*> tensors;
  std::string dir;
  explicit Checkpoint(const std::string& path) {
    std::vector<std::string> paths;
    if (is_dir(path)) {
      dir = path;
      const std::string index = path + "/model.safetensors.index.json";
      if (exists(index)) {
        json::Value ix = json::parse(read_text(index));
        std::map<std::string, int> seen;
        for (const auto& kv : ix.at("weight_map").obj) {
          const std::string f = path + "/" + kv.second.string();
          if (!seen.count(f)) {
            seen[f] = 1;
            paths.push_back(f);
          }
        }
      } else {
        paths.push_back(path + "/model.safetensors");
      }
    } else {
      dir = dir_of(path);
      paths.push_back(path);
    }
    for (const auto& p : paths) {
      files.emplace_back(new StFile(p));
      for (const auto& kv : files.back()->tensors) tensors[kv.first] = &kv.second;
    }
  }
  const StTensor* find(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : it->second;
  }
  const StTensor& get(const std::string& name, int64_t rows, int64_t cols) const {
    const StTensor* t = find(name);
    LLMRS_REQUIRE(t, LLMRS_E_FORMAT, "tensor not found: " + name);
    const bool ok = cols == 0 ? (t->shape.size() == 1 && t->shape[0] == rows)
                              : (t->shape.size() == 2 && t->shape[0] == rows && t->shape[1] == cols);
    LLMRS_REQUIRE(ok, LLMRS_E_FORMAT, "tensor " + name + " has an unexpected shape");
    return *t;
  }
};

// read_tensor (loader.rs:25-46): F32 and BF16 as f32 (F16 accepted as well).
std::vector<float> to_f32(const StTensor& t, const std::string& name) {
  const size_t n = (size_t)t.numel();
  std::vector<float> out(n);
  if (t.dtype == "F32") {
    LLMRS_REQUIRE(t.bytes == 4 * n, LLMRS_E_FORMAT, name + ": size does not match its shape");
    std::memcpy(out.data(), t.data, 4 * n);
  } else if (t.dtype == "BF16" || t.dtype == "F16") {
    LLMRS_REQUIRE(t.bytes == 2 * n, LLMRS_E_FORMAT, name + ": size does not match its shape");
    const bool bf = t.dtype == "BF16";
    parallel_for(n, loader_threads(), [&](size_t i0, size_t i1) {
      for (size_t i = i0; i < i1; ++i) {
        uint16_t h;
        std::memcpy(&h, t.data + 2 * i, 2);
        out[i] = bf ? bf16_to_f32(h) : host_h2f(h);
      }
    });
  } else {
    fail(LLMRS_E_FORMAT, name + ": unsupported dtype " + t.dtype + " (F32, BF16 or F16)");
  }
  return out;
}

void set_q4_from_f32(llmrs_model* m, int layer, int slot, const std::vector<float>& w, size_t n, size_t k) {
  std::vector<uint8_t> qs(n * k / 2);
  std::vector<float> sc(n * k / 32);
  quantize_q4_rows(w.data(), n, k, qs.data(), sc.data());
  const int rc = llmrs_model_set_linear_q4(m, layer, slot, qs.data(), sc.data());
  if (rc != LLMRS_OK) throw Error(rc, "uploading linear weight: " + std::string(llmrs_last_error()));
}

int cfg_int(const json::Value& c, const char* key, int dflt = -1) {
  if (!c.has(key)) {
    LLMRS_REQUIRE(dflt >= 0, LLMRS_E_FORMAT, std::string("config.json: missing ") + key);
    return dflt;
  }
  return (int)c.at(key).number();
}

// ---- GGUF -------------------------------------------------------------------
enum GgmlType : uint32_t { G_F32 = 0, G_F16 = 1, G_Q4_0 = 2, G_Q8_0 = 8, G_BF16 = 30 };

struct GgufTensor {
  std::vector<uint64_t> ne;  // ne[0] = columns (innermost), ne[1] = rows
  uint32_t type = 0;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
};

struct GgufMeta {
  enum Kind { Int, Float, Str, Arr, Bool } kind = Int;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  uint64_t count = 0;  // arrays: element count
};

struct GgufFile {
  std::unique_ptr<MappedFile> map;
  std::map<std::string, GgufMeta> meta;
  std::map<std::string, GgufTensor> tensors;
  size_t cur = 0;
  std::string path;

  void need(uint64_t n) {  // written so that no sum can wrap: cur <= size always holds
    LLMRS_REQUIRE(n <= map->size - cur, LLMRS_E_FORMAT, path + ": truncated GGUF header");
  }
  template <class T>
  T rd() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, map->data + cur, sizeof(T));
    cur += sizeof(T);
    return v;
  }
  std::string rd_str() {
    const uint64_t n = rd<uint64_t>();
    need(n);
    std::string s((const char*)map->data + cur, (size_t)n);
    cur += n;
    return s;
  }
  // One value of GGUF type t (arrays: recorded by count, elements skipped).
  GgufMeta rd_value(uint32_t t, int depth = 0) {
    GgufMeta v;
    switch (t) {
      case 0: v.i = rd<uint8_t>(); break;
      case 1: v.i = rd<int8_t>(); break;
      case 2: v.i = rd<uint16_t>(); break;
      case 3: v.i = rd<int16_t>(); break;
      case 4: v.i = rd<uint32_t>(); break;
      case 5: v.i = rd<int32_t>(); break;
      case 6: v.kind = GgufMeta::Float; v.f = rd<float>(); break;
      case 7: v.kind = GgufMeta::Bool; v.i = rd<uint8_t>(); break;
      case 8: v.kind = GgufMeta::Str; v.s = rd_str(); break;
      case 9: {
        LLMRS_REQUIRE(depth < 4, LLMRS_E_FORMAT, path + ": nested GGUF arrays too deep");
        const uint32_t et = rd<uint32_t>();
        v.kind = GgufMeta::Arr;
        v.count = rd<uint64_t>();
        for (uint64_t k = 0; k < v.count; ++k) (void)rd_value(et, depth + 1);
        break;
      }
      case 10: v.i = (int64_t)rd<uint64_t>(); break;
      case 11: v.i = rd<int64_t>(); break;
      case 12: v.kind = GgufMeta::Float; v.f = rd<double>(); break;
      default: fail(LLMRS_E_FORMAT, path + ": unknown GGUF value type " + std::to_string(t));
    }
    if (v.kind == GgufMeta::Int) v.f = (double)v.i;
    return v;
  }

  explicit GgufFile(const std::string& p) : map(new MappedFile(p)), path(p) {
    LLMRS_REQUIRE(rd<uint32_t>() == 0x46554747u, LLMRS_E_FORMAT, path + ": not a GGUF file");
    const uint32_t version = rd<uint32_t>();
    LLMRS_REQUIRE(version == 2 || version == 3, LLMRS_E_FORMAT,
                  path + ": GGUF version " + std::to_string(version) + " (2 or 3 supported)");
    const uint64_t nt = rd<uint64_t>(), nkv = rd<uint64_t>();
    for (uint64_t k = 0; k < nkv; ++k) {
      const std::string key = rd_str();
      const uint32_t t = rd<uint32_t>();
      meta[key] = rd_value(t);
    }
    struct Info {
      std::string name;
      GgufTensor t;
      uint64_t off;
    };
    std::vector<Info> infos;
    for (uint64_t k = 0; k < nt; ++k) {
      Info in;
      in.name = rd_str();
      const uint32_t nd = rd<uint32_t>();
      LLMRS_REQUIRE(nd >= 1 && nd <= 4, LLMRS_E_FORMAT, path + ": tensor " + in.name + " has bad dims");
      for (uint32_t d = 0; d < nd; ++d) in.t.ne.push_back(rd<uint64_t>());
      in.t.type = rd<uint32_t>();
      in.off = rd<uint64_t>();
      infos.push_back(in);
    }
    const size_t align = meta.count("general.alignment") ? (size_t)meta["general.alignment"].i : 32;
    LLMRS_REQUIRE(align > 0, LLMRS_E_FORMAT, path + ": bad alignment");
    const size_t base = align_up(cur, align);
    LLMRS_REQUIRE(base <= map->size, LLMRS_E_FORMAT, path + ": tensor data beyond the file");
    const uint64_t avail = map->size - base;  // bytes of the data section
    for (auto& in : infos) {
      // element count and byte size, each bounded by the file before the
      // next multiplication, so no product can wrap
      uint64_t n = 1;
      for (uint64_t d : in.t.ne) {
        LLMRS_REQUIRE(d == 0 || n <= avail / d, LLMRS_E_FORMAT,
                      path + ": tensor " + in.name + " is larger than the file");
        n *= d;
      }
      uint64_t bytes = 0;
      switch (in.t.type) {
        case G_F32: bytes = n <= avail / 4 ? 4 * n : UINT64_MAX; break;
        case G_F16:
        case G_BF16: bytes = n <= avail / 2 ? 2 * n : UINT64_MAX; break;
        case G_Q4_0: bytes = n / 32 * 18; break;   // n <= avail, so n / 32 * 18 cannot wrap
        case G_Q8_0: bytes = n / 32 * 34; break;
        default: bytes = 0;  // unsupported types are rejected where they are used
      }
      LLMRS_REQUIRE(in.off <= avail && bytes <= avail - in.off, LLMRS_E_FORMAT,
                    path + ": data of " + in.name + " beyond the file");
      in.t.data = map->data + base + in.off;
      in.t.bytes = bytes;
      tensors[in.name] = in.t;
    }
  }
  const GgufMeta* find_meta(const std::string& k) const {
    auto it = meta.find(k);
    return it == meta.end() ? nullptr : &it->second;
  }
  const GgufTensor* find(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
  }
  const GgufTensor& get(const std::string& name, uint64_t rows, uint64_t cols) const {
    const GgufTensor* t = find(name);
    LLMRS_REQUIRE(t, LLMRS_E_FORMAT, path + ": tensor not found: " + name);
    const bool ok = cols == 0 ? (t->ne.size() == 1 && t->ne[0] == rows)
                              : (t->ne.size() == 2 && t->ne[0] == cols && t->ne[1] == rows);
    LLMRS_REQUIRE(ok, LLMRS_E_FORMAT, path + ": tensor " + name + " has an unexpected shape");
    return *t;
  }
};

const char* ggml_type_name(uint32_t t) {
  switch (t) {
    case G_F32: return "F32";
    case G_F16: return "F16";
    case G_BF16: return "BF16";
    case G_Q4_0: return "Q4_0";
    case G_Q8_0: return "Q8_0";
    default: return "unsupported";
  }
}
bool ggml_float(uint32_t t) { return t == G_F32 || t == G_F16 || t == G_BF16; }

std::vector<float> gguf_f32(const GgufTensor& t, const std::string& name) {
  uint64_t n = 1;
  for (uint64_t d : t.ne) n *= d;
  std::vector<float> out((size_t)n);
  parallel_for((size_t)n / 32 + (n % 32 != 0), loader_threads(), [&](size_t b0, size_t b1) {
    for (size_t b = b0; b < b1; ++b)
      for (size_t i = 32 * b; i < std::min<size_t>(32 * b + 32, (size_t)n); ++i) {
        switch (t.type) {
          case G_F32: std::memcpy(&out[i], t.data + 4 * i, 4); break;
          case G_F16:
          case G_BF16: {
            uint16_t h;
            std::memcpy(&h, t.data + 2 * i, 2);
            out[i] = t.type == G_F16 ? host_h2f(h) : bf16_to_f32(h);
            break;
          }
          case G_Q4_0: {  // (q - 8) * d, qs[j] = e[j] | e[j + 16] << 4
            const uint8_t* blk = t.data + (i / 32) * 18;
            uint16_t dh;
            std::memcpy(&dh, blk, 2);
            const int j = (int)(i % 32);
            const int q = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
            out[i] = (float)(q - 8) * host_h2f(dh);
            break;
          }
          case G_Q8_0: {
            const uint8_t* blk = t.data + (i / 32) * 34;
            uint16_t dh;
            std::memcpy(&dh, blk, 2);
            out[i] = (float)(int8_t)blk[2 + i % 32] * host_h2f(dh);
            break;
          }
          default: fail(LLMRS_E_FORMAT, name + ": unsupported tensor type " + std::to_string(t.type));
        }
      }
  });
  return out;
}

// Source row of destination row r of a Q or K matrix with `heads` heads of
// hd rows: GGUF row 2j + h of a head holds rotate-half row h * hd/2 + j.
size_t unpermute_row(size_t r, int hd) {
  const size_t head = r / (size_t)hd, i = r % (size_t)hd, half = (size_t)hd / 2;
  const size_t h = i / half, j = i % half;
  return head * (size_t)hd + 2 * j + h;
}

// Upload one linear weight of a GGUF file into a model of weight dtype wt.
void gguf_linear(llmrs_model* m, int layer, int slot, const GgufTensor& t, const std::string& name, size_t n,
                 size_t k, int wt, int rope_hd) {
  auto src_row = [&](size_t r) { return rope_hd ? unpermute_row(r, rope_hd) : r; };
  const size_t nb = k / 32;
  int rc = LLMRS_OK;
  if (t.type == G_Q4_0 && (wt == LLMRS_Q4_0 || wt == LLMRS_Q4)) {
    // ggml nibble order (e[j] | e[j+16] << 4) to the reference's (e[2i] | e[2i+1] << 4)
    std::vector<uint8_t> qs(n * k / 2);
    std::vector<float> sc(n * nb);
    parallel_for(n, loader_threads(), [&](size_t r0, size_t r1) {
      for (size_t r = r0; r < r1; ++r) {
        const uint8_t* row = t.data + src_row(r) * nb * 18;
        for (size_t b = 0; b < nb; ++b) {
          const uint8_t* blk = row + 18 * b;
          uint16_t dh;
          std::memcpy(&dh, blk, 2);
          sc[r * nb + b] = host_h2f(dh);
          uint8_t e[32];
          for (int j = 0; j < 16; ++j) {
            e[j] = blk[2 + j] & 15;
            e[j + 16] = blk[2 + j] >> 4;
          }
          uint8_t* q = qs.data() + (r * nb + b) * 16;
          for (int i = 0; i < 16; ++i) q[i] = (uint8_t)(e[2 * i] | (e[2 * i + 1] << 4));
        }
      }
    });
    rc = llmrs_model_set_linear_q4(m, layer, slot, qs.data(), sc.data());
  } else if (t.type == G_Q8_0 && wt == LLMRS_Q8_0) {
    std::vector<int8_t> qs(n * k);
    std::vector<float> sc(n * nb);
    parallel_for(n, loader_threads(), [&](size_t r0, size_t r1) {
      for (size_t r = r0; r < r1; ++r) {
        const uint8_t* row = t.data + src_row(r) * nb * 34;
        for (size_t b = 0; b < nb; ++b) {
          uint16_t dh;
          std::memcpy(&dh, row + 34 * b, 2);
          sc[r * nb + b] = host_h2f(dh);
          std::memcpy(&qs[(r * nb + b) * 32], row + 34 * b + 2, 32);
        }
      }
    });
    rc = llmrs_model_set_linear_q8_0(m, layer, slot, qs.data(), sc.data());
  } else if (ggml_float(t.type) || t.type == G_Q4_0 || t.type == G_Q8_0) {
    // another storage than the model's: through f32 and the model's own
    // quantiser (Q8_0: quantize_row_q8_0's formula, cpu.rs:724-743)
    const std::vector<float> all = gguf_f32(t, name);
    std::vector<float> w(n * k);
    for (size_t r = 0; r < n; ++r) std::memcpy(&w[r * k], &all[src_row(r) * k], 4 * k);
    if (wt == LLMRS_Q8_0) {
      std::vector<int8_t> qs(n * k);
      std::vector<float> sc(n * nb);
      parallel_for(n * nb, loader_threads(), [&](size_t b0, size_t b1) {
        for (size_t b = b0; b < b1; ++b) {
          float amax = 0.0f;
          for (int i = 0; i < 32; ++i) amax = std::fabs(w[32 * b + i]) > amax ? std::fabs(w[32 * b + i]) : amax;
          const float d = amax / 127.0f;
          sc[b] = amax == 0.0f ? 0.0f : d;
          const float inv = amax == 0.0f ? 0.0f : 1.0f / d;
          for (int i = 0; i < 32; ++i) {
            const float p = std::round(w[32 * b + i] * inv);
            qs[32 * b + i] = p != p ? (int8_t)0 : (int8_t)std::min(127.0f, std::max(-127.0f, p));
          }
        }
      });
      rc = llmrs_model_set_linear_q8_0(m, layer, slot, qs.data(), sc.data());
    } else {
      set_q4_from_f32(m, layer, slot, w, n, k);
    }
  } else {
    fail(LLMRS_E_FORMAT, name + ": unsupported tensor type " + std::string(ggml_type_name(t.type)) + " (" +
                             std::to_string(t.type) + ")");
  }
  if (rc != LLMRS_OK) throw Error(rc, "uploading " + name + ": " + std::string(llmrs_last_error()));
}

void apply_options(llmrs_model_config& cfg, const llmrs_load_options* opt) {
  cfg.max_seq = opt && opt->max_seq > 0 ? opt->max_seq : 2048;  // KVCache::new(.., 2048), loader.rs:162-166
  cfg.kv_dtype = opt ? opt->kv_dtype : LLMRS_F16;
}

}  // namespace

extern "C" {

int llmrs_model_load_safetensors(const char* path, const llmrs_load_options* opt, llmrs_model** out) {
  llmrs_model* m = nullptr;
  const int rc = guard([&] {
    LLMRS_REQUIRE(path && out, LLMRS_E_INVALID, "null argument");
    *out = nullptr;
    Checkpoint ck(path);
    const std::string cfg_path = ck.dir + "/config.json";
    json::Value c;
    try {
      c = json::parse(read_text(cfg_path));
    } catch (const Error&) {
      throw;
    } catch (const std::exception& e) {
      fail(LLMRS_E_FORMAT, cfg_path + ": " + e.what());
    }
    llmrs_model_config cfg{};
    cfg.hidden = cfg_int(c, "hidden_size");
    cfg.n_layers = cfg_int(c, "num_hidden_layers");
    cfg.n_heads = cfg_int(c, "num_attention_heads");
    cfg.n_kv_heads = cfg_int(c, "num_key_value_heads", cfg.n_heads);
    cfg.ffn = cfg_int(c, "intermediate_size");
    cfg.vocab = cfg_int(c, "vocab_size");
    LLMRS_REQUIRE(cfg.n_heads > 0 && cfg.hidden % cfg.n_heads == 0, LLMRS_E_FORMAT,
                  "config.json: hidden_size must be a multiple of num_attention_heads");
    cfg.head_dim = cfg.hidden / cfg.n_heads;  // loader.rs:164
    cfg.rms_eps = (float)c.at("rms_norm_eps").number();
    cfg.rope_theta = c.has("rope_theta") ? (float)c.at("rope_theta").number() : 500000.0f;  // config.rs:19-21
    cfg.weight_dtype = LLMRS_Q4;
    apply_options(cfg, opt);
    LLMRS_REQUIRE(!opt || opt->weight_dtype == 0 || opt->weight_dtype == LLMRS_Q4, LLMRS_E_DTYPE,
                  "safetensors checkpoints are quantised with the reference's Q4 quantiser (LLMRS_Q4)");
    int rc2 = llmrs_model_create(&cfg, &m);
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    const size_t H = cfg.hidden, F = cfg.ffn, V = cfg.vocab, hd = cfg.head_dim;
    const size_t qd = (size_t)cfg.n_heads * hd, kvd = (size_t)cfg.n_kv_heads * hd;
    const std::vector<float> embed = to_f32(ck.get("model.embed_tokens.weight", V, H), "model.embed_tokens.weight");
    rc2 = llmrs_model_set_embedding(m, embed.data());
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    for (int l = 0; l < cfg.n_layers; ++l) {
      const std::string p = "model.layers." + std::to_string(l);
      struct Lin {
        const char* name;
        int slot;
        size_t n, k;
      } lins[] = {{".self_attn.q_proj.weight", LLMRS_W_Q, qd, H},    {".self_attn.k_proj.weight", LLMRS_W_K, kvd, H},
                  {".self_attn.v_proj.weight", LLMRS_W_V, kvd, H},   {".self_attn.o_proj.weight", LLMRS_W_O, H, qd},
                  {".mlp.gate_proj.weight", LLMRS_W_GATE, F, H},     {".mlp.up_proj.weight", LLMRS_W_UP, F, H},
                  {".mlp.down_proj.weight", LLMRS_W_DOWN, H, F}};
      for (const auto& li : lins) {
        const std::string name = p + li.name;
        set_q4_from_f32(m, l, li.slot, to_f32(ck.get(name, li.n, li.k), name), li.n, li.k);
      }
      const std::string n0 = p + ".input_layernorm.weight", n1 = p + ".post_attention_layernorm.weight";
      rc2 = llmrs_model_set_norm(m, l, LLMRS_N_INPUT, to_f32(ck.get(n0, H, 0), n0).data());
      if (rc2 == LLMRS_OK) rc2 = llmrs_model_set_norm(m, l, LLMRS_N_POST, to_f32(ck.get(n1, H, 0), n1).data());
      if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    }
    rc2 = llmrs_model_set_norm(m, -1, LLMRS_N_FINAL, to_f32(ck.get("model.norm.weight", H, 0), "model.norm.weight").data());
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    if (ck.find("lm_head.weight"))
      set_q4_from_f32(m, -1, LLMRS_W_LM_HEAD, to_f32(ck.get("lm_head.weight", V, H), "lm_head.weight"), V, H);
    else
      set_q4_from_f32(m, -1, LLMRS_W_LM_HEAD, embed, V, H);  // tied (loader.rs:186-190)
    *out = m;
  });
  if (rc != LLMRS_OK && m) llmrs_model_free(m);
  return rc;
}

int llmrs_model_load_gguf(const char* path, const llmrs_load_options* opt, llmrs_model** out) {
  llmrs_model* m = nullptr;
  const int rc = guard([&] {
    LLMRS_REQUIRE(path && out, LLMRS_E_INVALID, "null argument");
    *out = nullptr;
    GgufFile g(path);
    const GgufMeta* arch = g.find_meta("general.architecture");
    LLMRS_REQUIRE(arch && arch->kind == GgufMeta::Str && arch->s == "llama", LLMRS_E_FORMAT,
                  std::string(path) + ": general.architecture must be \"llama\"");
    auto mi = [&](const char* key, int64_t dflt = -1) -> int64_t {
      const GgufMeta* v = g.find_meta(std::string("llama.") + key);
      if (!v) {
        LLMRS_REQUIRE(dflt >= 0, LLMRS_E_FORMAT, std::string(path) + ": missing llama." + key);
        return dflt;
      }
      return v->kind == GgufMeta::Float ? (int64_t)v->f : v->i;
    };
    auto mf = [&](const char* key, double dflt) -> double {
      const GgufMeta* v = g.find_meta(std::string("llama.") + key);
      return v ? v->f : dflt;
    };
    llmrs_model_config cfg{};
    cfg.n_layers = (int32_t)mi("block_count");
    cfg.hidden = (int32_t)mi("embedding_length");
    cfg.n_heads = (int32_t)mi("attention.head_count");
    cfg.n_kv_heads = (int32_t)mi("attention.head_count_kv", cfg.n_heads);
    cfg.ffn = (int32_t)mi("feed_forward_length");
    LLMRS_REQUIRE(cfg.n_heads > 0 && cfg.hidden % cfg.n_heads == 0, LLMRS_E_FORMAT,
                  std::string(path) + ": embedding_length must be a multiple of head_count");
    cfg.head_dim = cfg.hidden / cfg.n_heads;
    cfg.rms_eps = (float)mf("attention.layer_norm_rms_epsilon", 1e-5);
    cfg.rope_theta = (float)mf("rope.freq_base", 500000.0);
    const GgufTensor* emb = g.find("token_embd.weight");
    LLMRS_REQUIRE(emb && emb->ne.size() == 2, LLMRS_E_FORMAT, std::string(path) + ": token_embd.weight missing");
    cfg.vocab = (int32_t)emb->ne[1];
    // The model's weight storage from its linear weights: all Q4_0 -> Q4_0,
    // all Q8_0 -> Q8_0, floats -> the reference's Q4 quantiser.
    const char* lnames[] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    int n4 = 0, n8 = 0, nf = 0, other = 0;
    for (int l = 0; l < cfg.n_layers; ++l)
      for (const char* ln : lnames) {
        const GgufTensor* t = g.find("blk." + std::to_string(l) + "." + ln + ".weight");
        LLMRS_REQUIRE(t, LLMRS_E_FORMAT, std::string(path) + ": missing blk." + std::to_string(l) + "." + ln);
        if (t->type == G_Q4_0) ++n4;
        else if (t->type == G_Q8_0) ++n8;
        else if (ggml_float(t->type)) ++nf;
        else ++other;
      }
    LLMRS_REQUIRE(other == 0, LLMRS_E_FORMAT,
                  std::string(path) + ": linear weights must be F32, F16, BF16, Q4_0 or Q8_0");
    int wt = n4 && !n8 ? LLMRS_Q4_0 : n8 && !n4 ? LLMRS_Q8_0 : !n4 && !n8 ? LLMRS_Q4 : -1;
    LLMRS_REQUIRE(wt >= 0, LLMRS_E_FORMAT, std::string(path) + ": linear weights mix Q4_0 and Q8_0");
    if (opt && opt->weight_dtype != 0) {
      LLMRS_REQUIRE(opt->weight_dtype == wt, LLMRS_E_DTYPE,
                    std::string(path) + ": its weights load as weight dtype " + std::to_string(wt));
    }
    cfg.weight_dtype = wt;
    // Every other tensor's type and shape, before any device work: the
    // embedding and lm_head (float, Q4_0 or Q8_0) and the norms (float).
    {
      auto check = [&](const std::string& name, uint64_t rows, uint64_t cols, bool quant_ok) {
        const GgufTensor& t = g.get(name, rows, cols);
        LLMRS_REQUIRE(ggml_float(t.type) || (quant_ok && (t.type == G_Q4_0 || t.type == G_Q8_0)), LLMRS_E_FORMAT,
                      std::string(path) + ": " + name + " has ggml type " + std::to_string(t.type) + " (" +
                          ggml_type_name(t.type) + "); supported: F32, F16, BF16" + (quant_ok ? ", Q4_0, Q8_0" : ""));
      };
      const uint64_t Hc = (uint64_t)cfg.hidden, Vc = (uint64_t)cfg.vocab;
      check("token_embd.weight", Vc, Hc, true);
      if (g.find("output.weight")) check("output.weight", Vc, Hc, true);
      check("output_norm.weight", Hc, 0, false);
      for (int l = 0; l < cfg.n_layers; ++l)
        for (const char* nn : {"attn_norm", "ffn_norm"})
          check("blk." + std::to_string(l) + "." + nn + ".weight", Hc, 0, false);
    }
    apply_options(cfg, opt);
    int rc2 = llmrs_model_create(&cfg, &m);
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    const size_t H = cfg.hidden, F = cfg.ffn, V = cfg.vocab, hd = cfg.head_dim;
    const size_t qd = (size_t)cfg.n_heads * hd, kvd = (size_t)cfg.n_kv_heads * hd;
    const std::vector<float> embed = gguf_f32(g.get("token_embd.weight", V, H), "token_embd.weight");
    rc2 = llmrs_model_set_embedding(m, embed.data());
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    for (int l = 0; l < cfg.n_layers; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      struct Lin {
        const char* name;
        int slot;
        size_t n, k;
        bool rope;
      } lins[] = {{"attn_q", LLMRS_W_Q, qd, H, true},     {"attn_k", LLMRS_W_K, kvd, H, true},
                  {"attn_v", LLMRS_W_V, kvd, H, false},   {"attn_output", LLMRS_W_O, H, qd, false},
                  {"ffn_gate", LLMRS_W_GATE, F, H, false}, {"ffn_up", LLMRS_W_UP, F, H, false},
                  {"ffn_down", LLMRS_W_DOWN, H, F, false}};
      for (const auto& li : lins) {
        const std::string name = p + li.name + ".weight";
        gguf_linear(m, l, li.slot, g.get(name, li.n, li.k), name, li.n, li.k, wt, li.rope ? (int)hd : 0);
      }
      const std::string n0 = p + "attn_norm.weight", n1 = p + "ffn_norm.weight";
      rc2 = llmrs_model_set_norm(m, l, LLMRS_N_INPUT, gguf_f32(g.get(n0, H, 0), n0).data());
      if (rc2 == LLMRS_OK) rc2 = llmrs_model_set_norm(m, l, LLMRS_N_POST, gguf_f32(g.get(n1, H, 0), n1).data());
      if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    }
    rc2 = llmrs_model_set_norm(m, -1, LLMRS_N_FINAL, gguf_f32(g.get("output_norm.weight", H, 0), "output_norm.weight").data());
    if (rc2 != LLMRS_OK) throw Error(rc2, llmrs_last_error());
    const std::string head = g.find("output.weight") ? "output.weight" : "token_embd.weight";  // tied when absent
    gguf_linear(m, -1, LLMRS_W_LM_HEAD, g.get(head, V, H), head, V, H, wt, 0);
    *out = m;
  });
  if (rc != LLMRS_OK && m) llmrs_model_free(m);
  return rc;
}

}  // extern "C"
