// A CPU stand-in for libstamd.so's single-stream runtime ABI (include/st_runtime.h), backed by
// the C oracle (oracle/stream_oracle.c). TEST INFRASTRUCTURE ONLY: it is built under
// tests/_build/cpu_runtime/ as libstamd.so and put first on LD_LIBRARY_PATH by the CPU tests of
// the benchmark driver (tests/test_harness.py), so that stream-bench's own logic (option table,
// reset schedules, archives and gates, the scheduled producer/consumer queue, result files and
// exit codes) runs end to end without a GPU. The product never loads it.
//
// Only what the drivers call is provided: create/destroy, step, reset, stop, snapshot,
// info_json, device_trace, trace_step (the oracle's per-operation trace, for stream-diagnose)
// and transport_bench (a stub report). A runtime created with max_events > 0 fails its step
// after that many RUN commands, as the persistent worker does.
#include "st_runtime.h"
#include "stream_oracle.h"

#include <chrono>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {
thread_local std::string last_error;

int fail(int code, const char* what) {
  last_error = what;
  return code;
}
}  // namespace

struct st_runtime {
  so_state* oracle = nullptr;
  st_config config{};
  uint64_t max_events = 0, runs = 0;
  bool stopped = false;
};

extern "C" {

void st_options_default(st_options* o) {
  std::memset(o, 0, sizeof *o);
  o->backend = ST_BACKEND_GRAPH;
  o->blocks = 1;
  o->idle_seconds = 30.0;
}

int st_runtime_create(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t count,
                      const st_options* options, st_runtime** out) {
  if (!config || !tensors || !options || !out) return fail(ST_ERR_INVALID, "null argument");
  std::map<std::string, const float*> byname;
  for (size_t i = 0; i < count; i++) byname[tensors[i].name] = tensors[i].data;
  std::vector<std::string> order{"input", "final_norm", "score"};
  for (int l = 0; l < config->layers; l++)
    for (const char* n : {"norm1", "norm2", "q", "k", "v", "out", "gate", "up", "down"})
      order.push_back("layers." + std::to_string(l) + "." + n);
  std::vector<const float*> ptrs;
  for (const std::string& n : order) {
    auto it = byname.find(n);
    if (it == byname.end()) return fail(ST_ERR_INVALID, "missing tensor");
    ptrs.push_back(it->second);
  }
  so_config c{config->layers, config->width, config->heads, config->ffn, config->window, config->features,
              config->epsilon};
  so_state* s = so_create(&c, mixed, 0, ptrs.data());
  if (!s) return fail(ST_ERR_INVALID, "Invalid or unsupported model dimensions");
  *out = new st_runtime{s, *config, options->max_events, 0, false};
  return ST_OK;
}

void st_runtime_destroy(st_runtime* r) {
  if (!r) return;
  so_destroy(r->oracle);
  delete r;
}

int st_runtime_step(st_runtime* r, const float* input, float* score) {
  if (r->stopped) return fail(ST_ERR_STATE, "Runtime stopped");
  if (r->max_events && r->runs >= r->max_events) return fail(ST_ERR_STATE, "Persistent sequence exhausted");
  r->runs++;
  *score = so_step(r->oracle, input);
  return ST_OK;
}

int st_runtime_reset(st_runtime* r) {
  if (r->stopped) return fail(ST_ERR_STATE, "Runtime stopped");
  so_reset(r->oracle);
  return ST_OK;
}

int st_runtime_stop(st_runtime* r) {
  r->stopped = true;
  return ST_OK;
}

int st_runtime_snapshot(st_runtime* r, uint64_t* position, float* keys, float* values, float* hidden) {
  *position = so_position(r->oracle);
  so_snapshot(r->oracle, keys, values, hidden);
  return ST_OK;
}

int st_runtime_info_json(st_runtime*, char* buffer, size_t cap, size_t* needed) {
  static const char text[] = "{\"environment\": {\"gpu\": \"none (CPU stand-in for driver tests)\"}}";
  *needed = sizeof text;
  if (buffer && cap >= sizeof text) std::memcpy(buffer, text, sizeof text);
  return ST_OK;
}

int st_runtime_device_trace(st_runtime* r, const float* inputs, size_t count, double* us_per_event, double*) {
  const auto t0 = std::chrono::steady_clock::now();
  for (size_t i = 0; i < count; i++) so_step(r->oracle, inputs + i * (size_t)r->config.features);
  *us_per_event = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / (double)count;
  return ST_OK;
}

// The oracle's trace in the ABI's layout: names as a JSON object {"name": [offset, count]},
// values concatenated in execution order.
int st_runtime_trace_step(st_runtime* r, const float* input, char* names, size_t names_cap, size_t* names_needed,
                          float* values, size_t values_cap, size_t* values_count) {
  struct Capture {
    std::string index = "{";
    std::vector<float> values;
  } cap;
  auto take = [](void* user, const char* name, const float* v, int n) {
    Capture* c = static_cast<Capture*>(user);
    if (c->index.size() > 1) c->index += ", ";
    c->index += "\"" + std::string(name) + "\": [" + std::to_string(c->values.size()) + ", " + std::to_string(n) + "]";
    c->values.insert(c->values.end(), v, v + n);
  };
  if (names_cap == 0 && values_cap == 0) {
    // Sizes only, no step: the entry layout follows from the configuration. Input projection
    // f + 3d; per layer 28d + 6F (norms 3d each; q, k, v 3d each plus their rotated values;
    // attention d; out 3d; attention_residual d; gate and up d + 2F each; activation F; down
    // F + 2d; hidden d); final norm 3d; score d + 2.
    const st_config& c = r->config;
    const size_t d = (size_t)c.width, F = (size_t)c.ffn;
    *values_count = (size_t)c.features + 7 * d + 2 + (size_t)c.layers * (28 * d + 6 * F);
    *names_needed = 64 * (10 + 34 * (size_t)c.layers);  // an upper bound: names are under 40 bytes
    return ST_OK;
  }
  if (r->stopped) return fail(ST_ERR_STATE, "Runtime stopped");
  so_step_trace(r->oracle, input, take, &cap);
  cap.index += "}";
  *names_needed = cap.index.size() + 1;
  *values_count = cap.values.size();
  if (names_cap < cap.index.size() + 1 || values_cap < cap.values.size())
    return fail(ST_ERR_INVALID, "trace buffers too small");
  std::memcpy(names, cap.index.c_str(), cap.index.size() + 1);
  std::memcpy(values, cap.values.data(), cap.values.size() * sizeof(float));
  return ST_OK;
}

int st_transport_bench(const char* mode, uint64_t, int32_t, const char*, char* report, size_t cap, size_t* needed) {
  const std::string text = std::string("{\"mode\": \"") + mode + "\", \"stand_in\": true}";
  *needed = text.size() + 1;
  if (report && cap >= *needed) std::memcpy(report, text.c_str(), *needed);
  return ST_OK;
}

const char* st_last_error(void) { return last_error.c_str(); }

}  // extern "C"
