// Host-side helpers shared by the engine and the codec decoder: error reporting (Failure /
// fail, checked HIP calls), bf16 conversion, device allocation and the safetensors reader.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/q3t.h"
#include "q3t_json.h"

namespace q3t {

struct Failure {
  int code;
  std::string msg;
};

[[noreturn]] inline void fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Failure{code, buf};
}

inline void hip_check(hipError_t e, const char *call) {
  if (e != hipSuccess) fail(Q3T_ERR_HIP, "%s failed: %s (%d)", call, hipGetErrorString(e), (int)e);
}
#define HIPC(x) ::q3t::hip_check((x), #x)

inline uint16_t f32_to_bf16_host(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
inline float bf16_to_f32_host(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// ------------------------------------------------------------------------------------
// safetensors (BF16 or F32 tensors; F32 is rounded to bf16 on load)
// ------------------------------------------------------------------------------------
class SafeTensors {
 public:
  // The file stays mapped for the object's lifetime.  A constructor that throws releases the
  // mapping and the descriptor itself (the destructor does not run then).
  explicit SafeTensors(const std::string &path) : path_(path) {
    fd_ = open(path.c_str(), O_RDONLY);
    if (fd_ < 0) fail(Q3T_ERR_NOT_FOUND, "cannot open %s", path.c_str());
    try {
      struct stat sb;
      if (fstat(fd_, &sb) != 0) fail(Q3T_ERR_INVALID, "cannot stat %s", path.c_str());
      size_ = (size_t)sb.st_size;
      if (size_ < 8) fail(Q3T_ERR_INVALID, "%s is not a safetensors file", path.c_str());
      void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
      if (m == MAP_FAILED) fail(Q3T_ERR_INVALID, "mmap of %s failed", path.c_str());
      base_ = (const uint8_t *)m;
      uint64_t hlen;
      memcpy(&hlen, base_, 8);
      if (hlen > size_ - 8) fail(Q3T_ERR_INVALID, "%s: header length out of range", path.c_str());
      header_ = json::parse(std::string((const char *)base_ + 8, (size_t)hlen));
      data_ = base_ + 8 + hlen;
      data_size_ = size_ - 8 - (size_t)hlen;
      validate_header();
    } catch (...) {
      release();
      throw;
    }
  }
  ~SafeTensors() { release(); }
  SafeTensors(const SafeTensors &) = delete;
  SafeTensors &operator=(const SafeTensors &) = delete;

  // Appends the tensor (as bf16) to out, checking its shape.
  void append_bf16(const std::string &name, const std::vector<int64_t> &shape, std::vector<uint16_t> &out) const {
    const auto [ptr, dtype, n] = view(name, shape);
    const size_t at = out.size();
    out.resize(at + n);
    if (dtype == "BF16") {
      memcpy(out.data() + at, ptr, n * 2);
    } else {
      for (size_t i = 0; i < n; ++i) {
        float f;
        memcpy(&f, ptr + 4 * i, 4);  // data offsets need not be 4-byte aligned
        out[at + i] = f32_to_bf16_host(f);
      }
    }
  }
  std::vector<float> f32(const std::string &name, const std::vector<int64_t> &shape) const {
    const auto [ptr, dtype, n] = view(name, shape);
    std::vector<float> out(n);
    if (dtype == "BF16") {
      for (size_t i = 0; i < n; ++i) {
        uint16_t b;
        memcpy(&b, ptr + 2 * i, 2);
        out[i] = bf16_to_f32_host(b);
      }
    } else {
      memcpy(out.data(), ptr, n * 4);
    }
    return out;
  }
  bool has(const std::string &name) const { return header_.has(name); }
  std::vector<int64_t> shape(const std::string &name) const {
    std::vector<int64_t> out;
    for (const json::Value &d : header_.at(name).at("shape").arr) out.push_back(d.integer());
    return out;
  }

 private:
  struct View {
    const uint8_t *ptr;
    std::string dtype;
    size_t n;
  };
  View view(const std::string &name, const std::vector<int64_t> &shape) const {
    if (!header_.has(name)) fail(Q3T_ERR_NOT_FOUND, "tensor %s not found in %s", name.c_str(), path_.c_str());
    const json::Value &t = header_.at(name);
    const std::string dtype = t.at("dtype").str;
    if (dtype != "BF16" && dtype != "F32")
      fail(Q3T_ERR_INVALID, "%s has dtype %s, expected BF16 or F32", name.c_str(), dtype.c_str());
    const auto &sh = t.at("shape").arr;
    bool ok = sh.size() == shape.size();
    size_t n = 1;
    for (size_t i = 0; ok && i < sh.size(); ++i) {
      ok = sh[i].integer() == shape[i];
      n *= (size_t)shape[i];
    }
    if (!ok) {
      std::string want, got;
      for (auto d : shape) want += std::to_string(d) + ",";
      for (auto &d : sh) got += std::to_string(d.integer()) + ",";
      fail(Q3T_ERR_INVALID, "%s shape [%s] does not match expected [%s]", name.c_str(), got.c_str(), want.c_str());
    }
    const auto &off = t.at("data_offsets").arr;
    if (off.size() != 2) fail(Q3T_ERR_INVALID, "%s: data_offsets must hold two integers", name.c_str());
    const int64_t b = off[0].integer(), e = off[1].integer();
    const uint64_t esz = dtype == "BF16" ? 2 : 4;
    if (b < 0 || e < b || (uint64_t)e > (uint64_t)data_size_ || (uint64_t)(e - b) != (uint64_t)n * esz)
      fail(Q3T_ERR_INVALID, "%s: data offsets [%lld, %lld) do not hold %zu elements inside the %zu data bytes",
           name.c_str(), (long long)b, (long long)e, n, data_size_);
    return {data_ + b, dtype, n};
  }
  // Every entry of the header (the format's optional __metadata__ aside) must describe a
  // byte range inside the data section that holds exactly its shape's elements, so no later
  // view can point outside the mapping.
  void validate_header() const {
    if (header_.kind != json::Value::Object) fail(Q3T_ERR_INVALID, "%s: header is not an object", path_.c_str());
    for (const auto &kv : header_.obj) {
      if (kv.first == "__metadata__") continue;
      const json::Value &t = kv.second;
      const std::string &dtype = t.at("dtype").str;
      uint64_t esz = 0;
      if (dtype == "BF16" || dtype == "F16" || dtype == "I16" || dtype == "U16") esz = 2;
      else if (dtype == "F32" || dtype == "I32" || dtype == "U32") esz = 4;
      else if (dtype == "F64" || dtype == "I64" || dtype == "U64") esz = 8;
      else if (dtype == "BOOL" || dtype == "U8" || dtype == "I8") esz = 1;
      else fail(Q3T_ERR_INVALID, "%s: tensor %s has unknown dtype %s", path_.c_str(), kv.first.c_str(), dtype.c_str());
      uint64_t n = 1;
      for (const json::Value &d : t.at("shape").arr) {
        const int64_t x = d.integer();
        if (x < 0 || (x > 0 && n > (UINT64_MAX / 8) / (uint64_t)x))
          fail(Q3T_ERR_INVALID, "%s: tensor %s has an invalid shape", path_.c_str(), kv.first.c_str());
        n *= (uint64_t)x;
      }
      const auto &off = t.at("data_offsets").arr;
      if (off.size() != 2) fail(Q3T_ERR_INVALID, "%s: data_offsets must hold two integers", kv.first.c_str());
      const int64_t b = off[0].integer(), e = off[1].integer();
      if (b < 0 || e < b || (uint64_t)e > (uint64_t)data_size_ || (uint64_t)(e - b) != n * esz)
        fail(Q3T_ERR_INVALID, "%s: data offsets [%lld, %lld) do not hold %llu elements inside the %zu data bytes",
             kv.first.c_str(), (long long)b, (long long)e, (unsigned long long)n, data_size_);
    }
  }
  void release() {
    if (base_) munmap((void *)base_, size_);
    if (fd_ >= 0) close(fd_);
    base_ = nullptr;
    fd_ = -1;
  }

  std::string path_;
  int fd_ = -1;
  size_t size_ = 0;
  const uint8_t *base_ = nullptr;
  const uint8_t *data_ = nullptr;
  size_t data_size_ = 0;
  json::Value header_;
};

template <typename T>
T *dev_alloc(size_t n, int64_t &tally) {
  void *p = nullptr;
  if (n == 0) n = 1;
  HIPC(hipMalloc(&p, n * sizeof(T)));
  tally += (int64_t)(n * sizeof(T));
  return (T *)p;
}

}  // namespace q3t
