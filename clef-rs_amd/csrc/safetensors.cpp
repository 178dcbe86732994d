// Safetensors reader and device loader: the on-disk weight format of the
// reference (models/weights.rs:26-104 Weights::load, :196-215 validate_header)
// restated for a C ABI.  A file is memory-mapped read-only; the header is
// parsed and checked before any tensor is used:
//   - 8-byte little-endian header length, at most 1 MiB (weights.rs:204-206);
//   - a JSON object of at most 2048 entries with no duplicate names (the
//     reference fails duplicates before the map could overwrite them,
//     weights.rs:213-214); "__metadata__" (string to string) is skipped;
//   - each tensor: dtype BF16, F16 or F32, a shape, data_offsets [b, e) with
//     e - b = elements x element size (overflow-checked, weights.rs:68-76);
//   - the tensors tile the data section exactly (sorted by offset, no gap and
//     no overlap), as the safetensors format requires.
// clef_st_load copies one tensor's bytes to the device and converts it there
// to f16 or f32 (BF16 -> F32 exact, BF16/F32 -> F16 round to nearest even),
// one tensor of staging at a time, so a loader never holds a second
// model-sized allocation (the concern of weights.rs:88-90).
#include <hip/hip_runtime.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/clef_hip.h"
#include "common.hpp"

namespace clef {
namespace {

struct StTensor {
  std::string name;
  int dtype = 0;  // CLEF_ST_BF16 / F16 / F32
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // within the data section
};

struct JsonCursor {
  const char* p;
  const char* e;
  int depth = 0;
  bool ok = true;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool str(std::string& out) {
    ws();
    if (p >= e || *p != '"') return ok = false;
    ++p;
    out.clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return ok = false;
        switch (*p) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {  // kept as the escape text: names compare byte-wise
            if (e - p < 5) return ok = false;
            out.append(p - 1, 6);
            p += 4;
            break;
          }
          default: return ok = false;
        }
        ++p;
      } else {
        if (static_cast<unsigned char>(*p) < 0x20) return ok = false;
        out += *p++;
      }
    }
    if (p >= e) return ok = false;
    ++p;
    return true;
  }
  bool uint(uint64_t& v) {
    ws();
    if (p >= e || *p < '0' || *p > '9') return ok = false;
    v = 0;
    while (p < e && *p >= '0' && *p <= '9') {
      const uint64_t d = static_cast<uint64_t>(*p - '0');
      if (v > (UINT64_MAX - d) / 10) return ok = false;
      v = v * 10 + d;
      ++p;
    }
    return true;
  }
  // any value, discarded (bounded depth)
  bool skip() {
    ws();
    if (p >= e || ++depth > 16) return ok = false;
    bool r = true;
    if (*p == '{') {
      ++p;
      if (!eat('}')) {
        do {
          std::string k;
          r = str(k) && eat(':') && skip();
        } while (r && eat(','));
        r = r && eat('}');
      }
    } else if (*p == '[') {
      ++p;
      if (!eat(']')) {
        do r = skip();
        while (r && eat(','));
        r = r && eat(']');
      }
    } else if (*p == '"') {
      std::string s;
      r = str(s);
    } else {
      const char* s = p;
      while (p < e && (std::strchr("+-.eE0123456789", *p) || (*p >= 'a' && *p <= 'z'))) ++p;
      r = p > s;
    }
    --depth;
    return r ? true : (ok = false);
  }
};

int dtype_size(int dt) { return dt == CLEF_ST_F32 ? 4 : 2; }

}  // namespace

struct SafeTensorsFile {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  const uint8_t* data = nullptr;  // start of the data section
  uint64_t data_size = 0;
  std::vector<StTensor> tensors;
  std::unordered_map<std::string, int> index;
  ~SafeTensorsFile() {
    if (map) munmap(const_cast<uint8_t*>(map), size);
    if (fd >= 0) close(fd);
  }
};

namespace {

int parse(SafeTensorsFile& f) {
  CLEF_REQUIRE(f.size >= 8, "safetensors: short file");
  uint64_t n = 0;
  std::memcpy(&n, f.map, 8);  // little-endian host (x86-64)
  CLEF_REQUIRE(n <= 1024 * 1024, "safetensors: header longer than 1 MiB");
  CLEF_REQUIRE(8 + n <= f.size, "safetensors: truncated header");
  f.data = f.map + 8 + n;
  f.data_size = f.size - 8 - n;
  JsonCursor c{reinterpret_cast<const char*>(f.map + 8), reinterpret_cast<const char*>(f.map + 8 + n)};
  CLEF_REQUIRE(c.eat('{'), "safetensors: header is not a JSON object");
  std::unordered_map<std::string, int> seen;
  if (!c.eat('}')) {
    do {
      std::string name;
      CLEF_REQUIRE(c.str(name) && c.eat(':'), "safetensors: malformed header");
      CLEF_REQUIRE(seen.emplace(name, 1).second, "safetensors: duplicate tensor name " + name);
      CLEF_REQUIRE(seen.size() <= 2048, "safetensors: more than 2048 header entries");
      if (name == "__metadata__") {
        CLEF_REQUIRE(c.skip(), "safetensors: malformed metadata");
        continue;
      }
      StTensor t;
      t.name = name;
      bool has_dtype = false, has_shape = false, has_offsets = false;
      CLEF_REQUIRE(c.eat('{'), "safetensors: tensor entry is not an object");
      if (!c.eat('}')) {
        do {
          std::string key;
          CLEF_REQUIRE(c.str(key) && c.eat(':'), "safetensors: malformed tensor entry");
          if (key == "dtype") {
            std::string d;
            CLEF_REQUIRE(c.str(d), "safetensors: malformed dtype");
            if (d == "BF16")
              t.dtype = CLEF_ST_BF16;
            else if (d == "F16")
              t.dtype = CLEF_ST_F16;
            else if (d == "F32")
              t.dtype = CLEF_ST_F32;
            else
              return fail(-1, "safetensors: unsupported dtype " + d + " for " + name);
            has_dtype = true;
          } else if (key == "shape") {
            CLEF_REQUIRE(c.eat('['), "safetensors: malformed shape");
            if (!c.eat(']')) {
              do {
                uint64_t v = 0;
                CLEF_REQUIRE(c.uint(v) && v <= (uint64_t(1) << 40), "safetensors: malformed shape");
                t.shape.push_back(static_cast<int64_t>(v));
              } while (c.eat(','));
              CLEF_REQUIRE(c.eat(']') && t.shape.size() <= 8, "safetensors: malformed shape");
            }
            has_shape = true;
          } else if (key == "data_offsets") {
            CLEF_REQUIRE(c.eat('[') && c.uint(t.begin) && c.eat(',') && c.uint(t.end) && c.eat(']'),
                         "safetensors: malformed data_offsets");
            has_offsets = true;
          } else {
            CLEF_REQUIRE(c.skip(), "safetensors: malformed tensor entry");
          }
        } while (c.eat(','));
        CLEF_REQUIRE(c.eat('}'), "safetensors: malformed tensor entry");
      }
      CLEF_REQUIRE(has_dtype && has_shape && has_offsets, "safetensors: incomplete entry for " + name);
      uint64_t elems = 1;
      for (int64_t d : t.shape) {
        CLEF_REQUIRE(d == 0 || elems <= UINT64_MAX / static_cast<uint64_t>(d), "safetensors: dimension overflow");
        elems *= static_cast<uint64_t>(d);
      }
      CLEF_REQUIRE(elems <= UINT64_MAX / 4, "safetensors: dimension overflow");
      CLEF_REQUIRE(t.begin <= t.end && t.end <= f.data_size, "safetensors: data offsets outside the file for " + name);
      CLEF_REQUIRE(t.end - t.begin == elems * dtype_size(t.dtype), "safetensors: tensor bytes for " + name);
      f.tensors.push_back(std::move(t));
    } while (c.eat(','));
    CLEF_REQUIRE(c.eat('}'), "safetensors: malformed header");
  }
  c.ws();
  CLEF_REQUIRE(c.ok && c.p == c.e, "safetensors: trailing bytes after the header object");
  // the tensors tile the data section: no gap, no overlap
  std::vector<const StTensor*> by_off;
  for (const auto& t : f.tensors) by_off.push_back(&t);
  std::sort(by_off.begin(), by_off.end(), [](const StTensor* a, const StTensor* b) {
    return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
  });
  uint64_t at = 0;
  for (const StTensor* t : by_off) {
    CLEF_REQUIRE(t->begin == at, "safetensors: tensor data overlaps or leaves a gap at " + t->name);
    at = t->end;
  }
  CLEF_REQUIRE(at == f.data_size, "safetensors: data section longer than its tensors");
  for (size_t i = 0; i < f.tensors.size(); ++i) f.index.emplace(f.tensors[i].name, static_cast<int>(i));
  return 0;
}

// ---- device conversion ------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__global__ void convert_kernel(const void* src, int sdt, void* dst, int ddt, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v;
  if (sdt == CLEF_ST_BF16)
    v = bf16_to_f32(static_cast<const uint16_t*>(src)[i]);
  else if (sdt == CLEF_ST_F16)
    v = static_cast<float>(static_cast<const half_t*>(src)[i]);
  else
    v = static_cast<const float*>(src)[i];
  if (ddt == CLEF_F16)
    static_cast<half_t*>(dst)[i] = static_cast<half_t>(v);  // round to nearest even
  else
    static_cast<float*>(dst)[i] = v;
}

}  // namespace
}  // namespace clef

using clef::fail;
using clef::SafeTensorsFile;

extern "C" int clef_st_open(const char* path, clef_safetensors** out) {
  CLEF_REQUIRE(path && out, "safetensors: null argument");
  *out = nullptr;
  auto* f = new (std::nothrow) SafeTensorsFile();
  CLEF_REQUIRE(f, "safetensors: out of host memory");
  f->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (f->fd < 0) {
    delete f;
    return fail(-2, std::string("safetensors: cannot open ") + path);
  }
  struct stat st;
  if (fstat(f->fd, &st) != 0 || st.st_size < 8) {
    delete f;
    return fail(-1, std::string("safetensors: short file ") + path);
  }
  f->size = static_cast<size_t>(st.st_size);
  void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
  if (m == MAP_FAILED) {
    delete f;
    return fail(-2, std::string("safetensors: cannot map ") + path);
  }
  f->map = static_cast<const uint8_t*>(m);
  if (int rc = clef::parse(*f)) {
    delete f;
    return rc;
  }
  *out = reinterpret_cast<clef_safetensors*>(f);
  return 0;
}

extern "C" void clef_st_close(clef_safetensors* f) { delete reinterpret_cast<SafeTensorsFile*>(f); }

extern "C" int clef_st_count(const clef_safetensors* f) {
  return f ? static_cast<int>(reinterpret_cast<const SafeTensorsFile*>(f)->tensors.size()) : -1;
}

extern "C" int clef_st_info(const clef_safetensors* f, int i, const char** name, int* dtype, int* rank,
                            int64_t* shape8) {
  CLEF_REQUIRE(f, "safetensors: null file");
  const auto* s = reinterpret_cast<const SafeTensorsFile*>(f);
  CLEF_REQUIRE(i >= 0 && i < static_cast<int>(s->tensors.size()), "safetensors: tensor index");
  const clef::StTensor& t = s->tensors[i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype;
  if (rank) *rank = static_cast<int>(t.shape.size());
  if (shape8)
    for (size_t d = 0; d < t.shape.size(); ++d) shape8[d] = t.shape[d];
  return 0;
}

extern "C" int clef_st_find(const clef_safetensors* f, const char* name) {
  if (!f || !name) return -1;
  const auto* s = reinterpret_cast<const SafeTensorsFile*>(f);
  auto it = s->index.find(name);
  return it == s->index.end() ? -1 : it->second;
}

extern "C" int clef_st_load(const clef_safetensors* f, int i, int dtype_out, void* dst, size_t dst_bytes,
                            void* stream) {
  CLEF_REQUIRE(f && dst, "safetensors: null argument");
  const auto* s = reinterpret_cast<const SafeTensorsFile*>(f);
  CLEF_REQUIRE(i >= 0 && i < static_cast<int>(s->tensors.size()), "safetensors: tensor index");
  CLEF_REQUIRE(dtype_out == CLEF_F16 || dtype_out == CLEF_F32, "safetensors: output dtype f16 or f32");
  const clef::StTensor& t = s->tensors[i];
  const uint64_t bytes = t.end - t.begin;
  const int64_t n = static_cast<int64_t>(bytes / clef::dtype_size(t.dtype));
  CLEF_REQUIRE(dst_bytes >= static_cast<size_t>(n) * (dtype_out == CLEF_F16 ? 2 : 4),
               "safetensors: destination smaller than the tensor");
  if (n == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool same = (t.dtype == CLEF_ST_F16 && dtype_out == CLEF_F16) || (t.dtype == CLEF_ST_F32 && dtype_out == CLEF_F32);
  auto hip_fail = [](hipError_t e, const char* what) {
    return fail(static_cast<int>(e), std::string("safetensors: ") + what + ": " + hipGetErrorString(e));
  };
  if (same) {
    hipError_t e = hipMemcpyAsync(dst, s->data + t.begin, bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : hip_fail(e, "upload");
  }
  void* staging = nullptr;
  if (hipError_t e0 = hipMalloc(&staging, bytes); e0 != hipSuccess) return hip_fail(e0, "staging allocation");
  hipError_t e = hipMemcpyAsync(staging, s->data + t.begin, bytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(clef::convert_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, staging,
                       t.dtype, dst, dtype_out, n);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(staging);
  return e == hipSuccess ? 0 : hip_fail(e, "load");
}
