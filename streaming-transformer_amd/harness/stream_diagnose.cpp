// stream-diagnose: per-operation snapshots of a fixture's whole event stream through the GPU's
// staged backend, written as the reference's diagnostic archive (bench/Diagnose.cpp:12-68):
//   OUTPUT/stages.bin     float32, event-major: for every event the trace entries back to back,
//                         in the order of their names (the reference's std::map order);
//   OUTPUT/manifest.json  version, dtype, layout "event_major", events, event_elements, stages
//                         [{name, offset_elements, elements}], backend, checkpoint_sha256,
//                         compiler, trace_sha256, resets, provenance, sha256 of stages.bin.
// Usage: stream-diagnose FIXTURE OUTPUT_DIRECTORY [cuda]
// The fixture is a checkpoint directory with trace.bin and resets.json (the reset happens
// before each listed event). Every event runs through st_runtime_trace_step, which leaves
// the same state as an ordinary step. The reference's default backend, cpu, is its Eigen
// step; here the CPU side of a comparison is the test oracle's archive
// (oracle/stage_archive.py), so only cuda is accepted. The snapshots are diagnostics, never
// timing evidence. Exit 0 on success, 1 on any error.
#include "json.hpp"
#include "model.hpp"
#include "sha256.hpp"
#include "st_runtime.h"

#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <fstream>
#include <iostream>
#include <set>
#include <string>
#include <vector>

using namespace stbench;

namespace {

void ok(int status) {
  if (status != ST_OK) throw std::runtime_error(st_last_error());
}

void make_dirs(const std::string& dir) {
  std::string path;
  for (size_t i = 0; i <= dir.size(); i++) {
    if (i == dir.size() || (dir[i] == '/' && i > 0)) {
      path = dir.substr(0, i);
      struct stat st{};
      if (stat(path.c_str(), &st) != 0 && mkdir(path.c_str(), 0775) != 0)
        throw std::runtime_error("Cannot create " + path);
    }
  }
}

// One traced step: entry name -> (offset, count) into `values`.
struct Traced {
  Json index;
  std::vector<float> values;
};

Traced trace_event(st_runtime* rt, const float* event) {
  size_t names_needed = 0, count = 0;
  ok(st_runtime_trace_step(rt, event, nullptr, 0, &names_needed, nullptr, 0, &count));
  std::vector<char> names(names_needed + 1, '\0');
  Traced t;
  t.values.resize(count);
  ok(st_runtime_trace_step(rt, event, names.data(), names.size(), &names_needed, t.values.data(), t.values.size(),
                           &count));
  t.index = Json::parse(std::string(names.data()));
  return t;
}

int run(int argc, char** argv) {
  if (argc != 3 && argc != 4) throw std::runtime_error("Usage: stream-diagnose FIXTURE OUTPUT_DIRECTORY [cuda]");
  const std::string fixture = argv[1], output = argv[2], backend = argc == 4 ? argv[3] : "cuda";
  if (backend == "cpu")
    throw std::runtime_error("The CPU stages come from the test oracle (oracle/stage_archive.py); use cuda");
  if (backend != "cuda") throw std::runtime_error("Unknown diagnostic backend");
  Model model(fixture);
  const std::vector<char> trace_bytes = read_bytes(fixture + "/trace.bin");
  const size_t features = (size_t)model.config.features;
  if (trace_bytes.empty() || trace_bytes.size() % (features * sizeof(float)))
    throw std::runtime_error("Invalid trace size");
  std::vector<float> events(trace_bytes.size() / sizeof(float));
  std::memcpy(events.data(), trace_bytes.data(), trace_bytes.size());
  const size_t count = events.size() / features;
  const Json reset_list = load_json(fixture + "/resets.json");
  std::set<size_t> resets;
  for (const Json& r : reset_list.elements()) resets.insert((size_t)r.uinteger());

  st_options options;
  st_options_default(&options);
  options.backend = ST_BACKEND_CUDA;  // the staged backend: traceStep's only backend
  options.blocks = 4;
  const std::vector<st_tensor> views = model.views();
  st_runtime* rt = nullptr;
  ok(st_runtime_create(&model.config, model.mixed, views.data(), views.size(), &options, &rt));
  struct Owner {
    st_runtime* rt;
    ~Owner() { st_runtime_destroy(rt); }
  } owner{rt};

  make_dirs(output);
  std::ofstream data(output + "/stages.bin", std::ios::binary);
  if (!data) throw std::runtime_error("Cannot write " + output + "/stages.bin");
  Json layout = Json::array();
  size_t event_elements = 0;
  Sha256 digest;
  for (size_t i = 0; i < count; i++) {
    if (resets.count(i)) ok(st_runtime_reset(rt));
    const Traced t = trace_event(rt, events.data() + i * features);
    size_t written = 0;
    for (const auto& [name, where] : t.index.items()) {  // sorted by name
      const size_t at = (size_t)where.at(0).uinteger(), n = (size_t)where.at(1).uinteger();
      if (at > t.values.size() || n > t.values.size() - at) throw std::runtime_error("Invalid trace entry: " + name);
      if (i == 0) {
        Json stage = Json::object();
        stage["name"] = name;
        stage["offset_elements"] = (uint64_t)event_elements;
        stage["elements"] = (uint64_t)n;
        layout.push_back(stage);
        event_elements += n;
      }
      const char* bytes = reinterpret_cast<const char*>(t.values.data() + at);
      data.write(bytes, (std::streamsize)(n * sizeof(float)));
      digest.update(bytes, n * sizeof(float));
      written += n;
    }
    if (written != event_elements) throw std::runtime_error("Trace layout changed between events");
  }
  data.close();
  if (!data) throw std::runtime_error("Short write of stages.bin");

  Json manifest = Json::object();
  manifest["version"] = 1;
  manifest["dtype"] = "float32";
  manifest["layout"] = "event_major";
  manifest["events"] = (uint64_t)count;
  manifest["event_elements"] = (uint64_t)event_elements;
  manifest["stages"] = layout;
  manifest["backend"] = backend;
  manifest["checkpoint_sha256"] = model.manifest.at("sha256");
  manifest["compiler"] = std::string(__VERSION__);
  manifest["trace_sha256"] = sha256(trace_bytes.data(), trace_bytes.size());
  manifest["resets"] = reset_list;
  Json provenance = Json::object();
  char host[256] = {0};
  gethostname(host, sizeof host - 1);
  provenance["host"] = std::string(host);
  provenance["writer"] = "stream-diagnose (st_runtime_trace_step, staged backend, 4 workgroups)";
  manifest["provenance"] = provenance;
  manifest["sha256"] = digest.hex();
  std::ofstream(output + "/manifest.json") << manifest.dump(2) << '\n';
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::cerr << e.what() << '\n';
    return 1;
  }
}
