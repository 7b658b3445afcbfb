// Result accounting of the benchmark driver: nearest-rank latency percentiles and the
// per-quantity error accounting with the reference's thresholds and mixed-mode scales
// (bench/Main.cpp:50-84, include/Numerical.hpp).
#pragma once

#include "json.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

namespace stbench {

// Nearest-rank percentiles over microsecond samples (Main.cpp:50-56).
inline Json distribution(std::vector<double> v) {
  if (v.empty()) return Json::object();
  std::sort(v.begin(), v.end());
  auto pct = [&](double q) { return v[(size_t)std::ceil(q * (double)v.size()) - 1]; };
  Json j = Json::object();
  j["p50_us"] = pct(.5);
  j["p95_us"] = pct(.95);
  j["p99_us"] = pct(.99);
  j["p999_us_diagnostic"] = pct(.999);
  j["worst_us"] = v.back();
  return j;
}

// Error accounting of one compared quantity (Main.cpp:57-84): FP32 atol 1e-5 / rtol 1e-4;
// mixed atol 2e-3 * scale / rtol 2e-2; non-finite values always fail.
struct Errors {
  double max_abs = 0, sq_err = 0, sq_ref = 0;
  uint64_t count = 0, failed = 0, nonfinite = 0;
  Json examples = Json::array();
  void check(float actual, float expected, bool mixed, double scale = 1) {
    count++;
    if (!std::isfinite(actual) || !std::isfinite(expected)) {
      nonfinite++;
      failed++;
      return;
    }
    const double diff = std::fabs((double)actual - (double)expected);
    max_abs = std::max(max_abs, diff);
    sq_err += diff * diff;
    sq_ref += (double)expected * expected;
    if (diff > (mixed ? 2e-3 * scale : 1e-5) + (mixed ? 2e-2 : 1e-4) * std::fabs((double)expected)) {
      failed++;
      if (examples.size() < 16) {
        Json e = Json::object();
        e["index"] = count - 1;
        e["actual"] = (double)actual;
        e["expected"] = (double)expected;
        e["difference"] = diff;
        examples.push_back(e);
      }
    }
  }
  double normalized_rmse() const {
    const double n = (double)std::max<uint64_t>(1, count);
    return std::sqrt(sq_err / n) / std::max(1.0, std::sqrt(sq_ref / n));
  }
  Json json() const {
    Json j = Json::object();
    j["elements"] = count;
    j["max_abs"] = max_abs;
    j["relative_l2"] = std::sqrt(sq_err / std::max(1e-30, sq_ref));
    j["normalized_rmse"] = normalized_rmse();
    j["failed"] = failed;
    j["nonfinite"] = nonfinite;
    j["examples"] = examples;
    return j;
  }
};

// include/Numerical.hpp: vector RMS floored at 1, relative L2, and the mixed state scale.
inline double residual_scale(const float* r, size_t n) {
  double s = 0;
  for (size_t i = 0; i < n; i++) s += (double)r[i] * r[i];
  return std::max(1.0, std::sqrt(s / (double)n));
}
inline double relative_l2(const float* a, const float* r, size_t n) {
  double e = 0, s = 0;
  for (size_t i = 0; i < n; i++) {
    const double d = (double)a[i] - r[i];
    e += d * d;
    s += (double)r[i] * r[i];
  }
  return std::sqrt(e / std::max(1e-30, s));
}
inline double mixed_state_scale(const float* r, size_t n, int layer) { return (layer + 1) * residual_scale(r, n); }


}  // namespace stbench
