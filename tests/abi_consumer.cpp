// A C++ consumer of include/st_runtime.h, written the way a maintainer would bind the library
// into the reference (a Stream::Runtime shim over the C ABI: status codes turned into
// std::runtime_error(st_last_error()), two-pass sizing of the JSON and trace outputs), driven
// through the lifecycle checks of the reference's tests/Lifecycle.cu:
//  - persistent: repeated resets and zero events, position after each step, restart with an
//    independent mailbox sequence, stop twice, calls after stop throw (Lifecycle.cu:17-50);
//  - persistent: finite (max_events) and idle exits (Lifecycle.cu:52-75);
//  - persistent: the last sequence ID reserved for STOP (Lifecycle.cu:77-92);
//  - staged: traceStep leaves exactly the state of plain steps and its score.linear entry is
//    the step's score (Lifecycle.cu:108-137);
//  - info() through the two-pass sizing; an invalid call leaves a message in st_last_error.
// Zero events give a score of exactly 0 (the reference's CPU step of a zero event).
//
// Usage: abi_consumer <small-fp32 dir> <small-mixed dir> <main-mixed dir>  (reference layout:
// manifest.json + tensors.bin [+ trace.bin]). Prints one line per check; exit 0 if all pass.
#include "json.hpp"
#include "model.hpp"
#include "st_runtime.h"

#include <chrono>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

using stbench::Json;
using stbench::Model;

void check(int status) {
  if (status != ST_OK) throw std::runtime_error(st_last_error());
}

struct Snapshot {
  uint64_t position = 0;
  std::vector<float> keys, values, hidden;
};

// The shim: Stream::Runtime over the C ABI.
class Runtime {
 public:
  Runtime(const Model& model, const st_options& options) : config_(model.config) {
    const std::vector<st_tensor> views = model.views();
    check(st_runtime_create(&model.config, model.mixed, views.data(), views.size(), &options, &handle_));
  }
  ~Runtime() { st_runtime_destroy(handle_); }
  Runtime(const Runtime&) = delete;
  Runtime& operator=(const Runtime&) = delete;

  float step(const float* input) {
    float score = 0;
    check(st_runtime_step(handle_, input, &score));
    return score;
  }
  void reset() { check(st_runtime_reset(handle_)); }
  void stop() { check(st_runtime_stop(handle_)); }
  Snapshot snapshot() {
    Snapshot s;
    const size_t cache = (size_t)config_.layers * config_.width * config_.window;
    s.keys.resize(cache);
    s.values.resize(cache);
    s.hidden.resize((size_t)config_.layers * config_.width);
    check(st_runtime_snapshot(handle_, &s.position, s.keys.data(), s.values.data(), s.hidden.data()));
    return s;
  }
  std::map<std::string, std::vector<float>> traceStep(const float* input) {
    size_t needed = 0, total = 0;
    check(st_runtime_trace_step(handle_, input, nullptr, 0, &needed, nullptr, 0, &total));  // sizes only
    std::string names(needed, '\0');
    std::vector<float> values(total);
    check(st_runtime_trace_step(handle_, input, names.data(), needed, &needed, values.data(), total, &total));
    std::map<std::string, std::vector<float>> trace;
    const Json table = Json::parse(names.c_str());
    for (const auto& [name, span] : table.items()) {
      const size_t offset = (size_t)span.at(0).uinteger(), count = (size_t)span.at(1).uinteger();
      trace[name].assign(values.begin() + (long)offset, values.begin() + (long)(offset + count));
    }
    return trace;
  }
  Json info() {
    size_t needed = 0;
    check(st_runtime_info_json(handle_, nullptr, 0, &needed));
    std::string buf(needed, '\0');
    check(st_runtime_info_json(handle_, buf.data(), needed, &needed));
    return Json::parse(buf.c_str());
  }

 private:
  st_runtime* handle_ = nullptr;
  st_config config_;
};

int failures = 0;

void expect(bool ok, const std::string& what) {
  if (!ok) {
    failures++;
    std::printf("FAIL %s\n", what.c_str());
  }
}

template <class F>
void expect_throw(F&& f, const std::string& what) {
  try {
    f();
  } catch (const std::runtime_error& e) {
    expect(std::strlen(e.what()) > 0 && std::strlen(st_last_error()) > 0, what + " (message)");
    return;
  }
  expect(false, what + " (no throw)");
}

void run(const std::string& name, const std::function<void()>& body) {
  const int before = failures;
  try {
    body();
  } catch (const std::exception& e) {
    failures++;
    std::printf("FAIL %s: unexpected exception: %s\n", name.c_str(), e.what());
  }
  std::printf("%s %s\n", failures == before ? "PASS" : "FAIL", name.c_str());
  std::fflush(stdout);
}

st_options persistent_options(int blocks) {
  st_options o;
  st_options_default(&o);
  o.backend = ST_BACKEND_PERSISTENT;
  o.blocks = blocks;
  return o;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) {
    std::fprintf(stderr, "usage: abi_consumer <small-fp32> <small-mixed> <main-mixed>\n");
    return 1;
  }
  const std::string small_fp32 = argv[1], small_mixed = argv[2], main_mixed = argv[3];

  run("persistent reset, repeated zero scores and restart", [&] {
    for (const std::string& dir : {small_fp32, small_mixed}) {
      const Model model(dir);
      const int window = model.config.window;
      for (int blocks : {1, 4}) {
        for (int restart = 0; restart < 2; restart++) {
          Runtime runtime(model, persistent_options(blocks));
          std::vector<float> event((size_t)model.config.features, 0.f);
          uint64_t position = 0;
          for (int i = 0; i < 3 * window + 9; i++) {
            if (i == 1 || i == window || i == 2 * window + 3) {
              runtime.reset();
              runtime.reset();
              position = 0;
              expect(runtime.snapshot().position == 0, "position 0 after reset");
            }
            expect(runtime.step(event.data()) == 0.f, "zero event scores exactly 0");
            expect(runtime.snapshot().position == ++position, "position advances by one per step");
          }
          runtime.stop();
          runtime.stop();
          expect_throw([&] { runtime.step(event.data()); }, "step after stop");
          expect_throw([&] { runtime.reset(); }, "reset after stop");
        }
      }
    }
  });

  run("persistent finite and idle exit", [&] {
    const Model model(small_fp32);
    std::vector<float> event((size_t)model.config.features, 0.f);
    for (int blocks : {1, 4}) {
      st_options o = persistent_options(blocks);
      o.max_events = 2;
      Runtime runtime(model, o);
      expect(runtime.step(event.data()) == 0.f, "first RUN");
      runtime.reset();
      expect(runtime.step(event.data()) == 0.f, "second RUN (RESET does not count)");
      expect_throw([&] { runtime.step(event.data()); }, "third RUN past max_events");
      runtime.stop();
    }
    st_options idle = persistent_options(1);
    idle.idle_seconds = .001;
    Runtime runtime(model, idle);
    std::this_thread::sleep_for(std::chrono::milliseconds(100));
    expect_throw([&] { runtime.step(event.data()); }, "step after the idle exit");
    runtime.stop();
  });

  run("persistent sequence exhaustion still allows stop", [&] {
    const Model model(small_fp32);
    std::vector<float> event((size_t)model.config.features, 0.f);
    for (int blocks : {1, 4}) {
      st_options o = persistent_options(blocks);
      o.initial_sequence = std::numeric_limits<uint64_t>::max() - 2;
      Runtime runtime(model, o);
      expect(runtime.step(event.data()) == 0.f, "the one RUN before exhaustion");
      expect_throw([&] { runtime.step(event.data()); }, "RUN past the last sequence ID");
      expect_throw([&] { runtime.reset(); }, "RESET past the last sequence ID");
      runtime.stop();
      runtime.stop();
    }
  });

  run("staged traceStep preserves execution", [&] {
    const Model model(main_mixed);
    st_options o;
    st_options_default(&o);
    o.backend = ST_BACKEND_CUDA;
    o.blocks = 4;
    Runtime runtime(model, o);
    const std::vector<char> bytes = stbench::read_bytes(main_mixed + "/trace.bin");
    const size_t f = (size_t)model.config.features;
    std::vector<float> event(f), scores;
    for (int i = 0; i < 12; i++) {
      std::memcpy(event.data(), bytes.data() + (size_t)i * f * 4, f * 4);
      scores.push_back(runtime.step(event.data()));
    }
    const Snapshot state = runtime.snapshot();
    runtime.reset();
    for (int i = 0; i < 12; i++) {
      std::memcpy(event.data(), bytes.data() + (size_t)i * f * 4, f * 4);
      const auto trace = runtime.traceStep(event.data());
      expect(trace.at("layers.0.attention").size() == (size_t)model.config.width, "attention entry size");
      expect(trace.at("score.linear").size() == 1 && scores[(size_t)i] == trace.at("score.linear")[0],
             "score.linear equals the plain step's score");
    }
    const Snapshot traced = runtime.snapshot();
    expect(state.position == traced.position, "position");
    expect(state.keys == traced.keys && state.values == traced.values && state.hidden == traced.hidden,
           "state after traced steps equals the state after plain steps");
  });

  run("info sizing and error messages", [&] {
    const Model model(small_fp32);
    st_options o;
    st_options_default(&o);
    o.backend = ST_BACKEND_FUSED;
    o.blocks = 0;
    Runtime runtime(model, o);
    const Json info = runtime.info();
    expect(info.contains("backend") && info.contains("environment"), "info() carries backend and environment");
    st_options bad;
    st_options_default(&bad);
    bad.backend = 99;
    const std::vector<st_tensor> views = model.views();
    st_runtime* handle = nullptr;
    expect(st_runtime_create(&model.config, 0, views.data(), views.size(), &bad, &handle) == ST_ERR_INVALID,
           "unknown backend rejected with ST_ERR_INVALID");
    expect(handle == nullptr && std::strlen(st_last_error()) > 0, "no handle and a message on failure");
    st_runtime_destroy(nullptr);  // never fails
  });

  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
