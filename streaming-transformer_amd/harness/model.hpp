// Checkpoint loading for the benchmark driver: the reference's on-disk format (manifest.json
// + tensors.bin; reference/export.py:31-43) with the loader's checks of Stream::Model
// (src/runtime/Model.cpp:15-139): format fields, archive and per-tensor SHA-256, contiguous
// bounds, FP16 decode for mixed checkpoints, and the exact shape of every tensor.
#pragma once

#include "json.hpp"
#include "sha256.hpp"
#include "st_runtime.h"

#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace stbench {

inline std::vector<char> read_bytes(const std::string& path) {
  std::ifstream file(path, std::ios::binary | std::ios::ate);
  if (!file) throw std::runtime_error("Cannot read " + path);
  const std::streamoff length = file.tellg();
  std::vector<char> bytes((size_t)length);
  file.seekg(0);
  if (length && !file.read(bytes.data(), (std::streamsize)bytes.size())) throw std::runtime_error("Short read " + path);
  return bytes;
}

inline Json load_json(const std::string& path) {
  const std::vector<char> b = read_bytes(path);
  return Json::parse(std::string(b.begin(), b.end()));
}

// IEEE binary16 to binary32 (exact: every half value is a float value).
inline float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);  // inf / nan
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {  // subnormal half: normalize
    int e = -1;
    uint32_t m = man;
    do {
      m <<= 1;
      e++;
    } while (!(m & 0x400u));
    bits = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3FFu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

struct Tensor {
  std::vector<int> shape;
  std::vector<float> data;
};

struct Model {
  st_config config{};
  bool mixed = false;
  Json manifest;
  std::map<std::string, Tensor> tensors;

  explicit Model(const std::string& dir) {
    manifest = load_json(dir + "/manifest.json");
    if (manifest.at("version") != Json(1) || manifest.at("byte_order") != Json("little") ||
        manifest.at("orientation") != Json("out_in"))
      throw std::runtime_error("Unsupported tensor format");
    const Json& c = manifest.at("config");
    config.layers = (int32_t)c.at("layers").integer();
    config.width = (int32_t)c.at("width").integer();
    config.heads = (int32_t)c.at("heads").integer();
    config.ffn = (int32_t)c.at("ffn").integer();
    config.window = (int32_t)c.at("window").integer();
    config.features = (int32_t)c.at("features").integer();
    config.epsilon = (float)c.at("epsilon").number();
    validate();
    const std::string mode = manifest.at("mode").str();
    if (mode != "fp32" && mode != "mixed") throw std::runtime_error("Unknown numerical mode");
    mixed = mode == "mixed";
    const std::vector<char> bytes = read_bytes(dir + "/tensors.bin");
    if (sha256(bytes.data(), bytes.size()) != manifest.at("sha256").str())
      throw std::runtime_error("Checkpoint hash mismatch");
    size_t end = 0;
    for (const Json& item : manifest.at("tensors").elements()) {
      Tensor t;
      size_t count = 1;
      for (const Json& d : item.at("shape").elements()) {
        const long long dim = d.integer();
        if (dim <= 0 || count > bytes.size() / (size_t)dim) throw std::runtime_error("Invalid tensor dimensions");
        t.shape.push_back((int)dim);
        count *= (size_t)dim;
      }
      const std::string dtype = item.at("dtype").str();
      const size_t size = dtype == "float32" ? 4 : dtype == "float16" ? 2 : 0;
      const size_t offset = (size_t)item.at("offset").uinteger(), nbytes = (size_t)item.at("nbytes").uinteger();
      if (!size || offset != end || nbytes != count * size || offset > bytes.size() || nbytes > bytes.size() - offset)
        throw std::runtime_error("Invalid tensor bounds");
      if (sha256(bytes.data() + offset, nbytes) != item.at("sha256").str())
        throw std::runtime_error("Tensor hash mismatch");
      t.data.resize(count);
      if (size == 4) {
        std::memcpy(t.data.data(), bytes.data() + offset, nbytes);
      } else {
        for (size_t i = 0; i < count; i++) {
          uint16_t h;
          std::memcpy(&h, bytes.data() + offset + 2 * i, 2);
          t.data[i] = half_to_float(h);
        }
      }
      if (!tensors.emplace(item.at("name").str(), std::move(t)).second) throw std::runtime_error("Duplicate tensor");
      end += nbytes;
    }
    if (end != bytes.size()) throw std::runtime_error("Trailing tensor bytes");
    const int d = config.width, f = config.ffn;
    check("input", {d, config.features});
    check("final_norm", {d});
    check("score", {1, d});
    for (int l = 0; l < config.layers; l++) {
      const std::string p = "layers." + std::to_string(l) + ".";
      check(p + "norm1", {d});
      check(p + "norm2", {d});
      for (const char* n : {"q", "k", "v", "out"}) check(p + n, {d, d});
      check(p + "gate", {f, d});
      check(p + "up", {f, d});
      check(p + "down", {d, f});
    }
  }

  // ModelConfig::validate (src/runtime/Model.cpp:22-29).
  void validate() const {
    const st_config& c = config;
    if (c.layers < 1 || c.layers > 16 || c.width < 1 || c.width > 1024 || c.heads < 1 || c.width % c.heads ||
        (c.width / c.heads) % 2 || c.ffn < 1 || c.ffn > 4096 || c.window < 1 || c.window > 4096 || c.features < 1 ||
        c.features > 1024 || !std::isfinite(c.epsilon) || c.epsilon <= 0)
      throw std::runtime_error("Invalid or unsupported model dimensions");
  }

  size_t cache_elements() const { return (size_t)config.layers * config.width * config.window; }

  // The C ABI's tensor views, in the checkpoint's order.
  std::vector<st_tensor> views() const {
    std::vector<st_tensor> out;
    for (const auto& [name, t] : tensors) {
      st_tensor s{};
      s.name = name.c_str();
      s.rank = (int32_t)t.shape.size();
      s.shape[0] = t.shape[0];
      s.shape[1] = t.shape.size() > 1 ? t.shape[1] : 0;
      s.data = t.data.data();
      out.push_back(s);
    }
    return out;
  }

 private:
  void check(const std::string& name, std::vector<int> shape) const {
    auto it = tensors.find(name);
    if (it == tensors.end() || it->second.shape != shape) throw std::runtime_error("Shape mismatch: " + name);
  }
};

}  // namespace stbench
