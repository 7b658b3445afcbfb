// The persistent backend's mailbox protocol on the CPU (test infrastructure), built plain, with
// AddressSanitizer + UndefinedBehaviorSanitizer and with ThreadSanitizer by
// tests/test_sanitizers.py.
//
// The host half is the runtime's own MailboxClient (streaming-transformer_amd/csrc/mailbox.hpp).
// The worker is a host thread that follows the resident kernel's side of the protocol
// (persistent_kernel in csrc/step_phases.hpp): acquire a new request word or leave after an idle
// budget; read the command; RUN computes a score from the event (here a checksum standing in
// for the model), RESET zeroes its position, PING reports a checksum of the event, STOP ends
// it; store the score and error words, then release the completion word; count RUN commands
// against max_events; on leaving, release exited = 1. The lifecycle checks follow the
// reference's tests/Lifecycle.cu:17-104: commands in order, STOP twice, a finite RUN budget, an
// idle exit, a worker that never answers (timeout), a worker whose launch ends without
// answering, the watchdog error word, and the last sequence IDs kept for STOP.
#include "mailbox.hpp"

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

using namespace stamd;

static int failures = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    failures++;
    std::printf("FAIL %s\n", what);
  }
}

struct WorkerOptions {
  uint64_t initial = 0;
  uint64_t max_events = 0;      // 0: unlimited
  double idle_seconds = 5.0;    // leave after this long without a request
  bool answer = true;           // false: read requests but never complete (a hung worker)
  bool end_silently = false;    // leave at the first request without answering or setting exited
  uint32_t error_bits = 0;      // reported with every completion (the device watchdog word)
};

// The worker thread: the resident kernel's side of the protocol, on ordinary host memory.
class FakeWorker {
 public:
  FakeWorker(Mailbox* mb, const float* event, int features, WorkerOptions o)
      : mb_(mb), event_(event), features_(features), o_(o) {
    thread_ = std::thread([this] { loop(); });
  }
  ~FakeWorker() {
    release();
    join();
  }
  // Ends the idle wait at once (a worker that never answers stays until released, however
  // slowly the host reaches its own timeout check).
  void release() { released_.store(true, std::memory_order_release); }
  void join() {
    if (thread_.joinable()) thread_.join();
  }
  bool finished() const { return done_.load(std::memory_order_acquire); }
  uint64_t position() const { return position_; }  // read after join()

 private:
  void loop() {
    uint64_t previous = o_.initial, processed = 0;
    while (true) {
      const auto start = std::chrono::steady_clock::now();
      uint64_t got = previous;
      int cmd = kCmdExit;
      while (true) {
        got = __atomic_load_n(&mb_->request, __ATOMIC_ACQUIRE);
        if (got != previous) {
          cmd = __atomic_load_n(&mb_->command, __ATOMIC_RELAXED);
          break;
        }
        if (released_.load(std::memory_order_acquire) ||
            std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() >= o_.idle_seconds)
          break;
        std::this_thread::yield();
      }
      if (cmd == kCmdExit) break;
      if (o_.end_silently) {
        done_.store(true, std::memory_order_release);
        return;  // the launch ends: no completion, no exited word
      }
      if (!o_.answer) {  // never completes; the host times out, and the worker idles out
        previous = got;
        continue;
      }
      if (cmd == kCmdRun) {
        uint32_t sum = 0;
        for (int i = 0; i < features_; i++) {
          uint32_t bits;
          std::memcpy(&bits, event_ + i, 4);
          sum = sum * 31u + bits;
        }
        float score = (float)(sum % 1000u) + (float)position_;
        __atomic_store(&mb_->score, &score, __ATOMIC_RELAXED);
        position_++;
      } else if (cmd == kCmdReset) {
        position_ = 0;
      } else if (cmd == kCmdPing) {
        unsigned long long sum = 0;
        for (int i = 0; i < features_; i++) {
          uint32_t bits;
          std::memcpy(&bits, event_ + i, 4);
          sum += bits;
        }
        __atomic_store_n(&mb_->checksum, sum, __ATOMIC_RELAXED);
      }
      __atomic_store_n(&mb_->error, o_.error_bits, __ATOMIC_RELAXED);
      __atomic_store_n(&mb_->completion, got, __ATOMIC_RELEASE);
      previous = got;
      if (cmd == kCmdRun) processed++;
      if (cmd == kCmdStop || (o_.max_events && processed >= o_.max_events)) break;
    }
    __atomic_store_n(&mb_->exited, 1ull, __ATOMIC_RELEASE);
    done_.store(true, std::memory_order_release);
  }

  Mailbox* mb_;
  const float* event_;
  int features_;
  WorkerOptions o_;
  uint64_t position_ = 0;
  std::atomic<bool> done_{false};
  std::atomic<bool> released_{false};
  std::thread thread_;
};

// The runtime's use of the client: check, then one round trip (Runtime::command / issue), and
// an idempotent stop that only sends STOP to a live worker, once (Runtime::stop).
struct Host {
  MailboxClient client;
  FakeWorker* worker = nullptr;
  double timeout = 5.0;
  bool running = true;
  MailboxError::Kind command(int cmd, bool* ok) {
    try {
      client.check(cmd);
      client.issue(cmd, true, timeout, [&] { return worker->finished(); });
      *ok = true;
      return MailboxError::kExhausted;  // unused when ok
    } catch (const MailboxError& e) {
      *ok = false;
      return e.kind;
    }
  }
  bool run(int cmd) {
    bool ok;
    command(cmd, &ok);
    return ok;
  }
  MailboxError::Kind fails_with(int cmd) {
    bool ok;
    MailboxError::Kind k = command(cmd, &ok);
    expect(!ok, "command was expected to fail");
    return k;
  }
  void stop() {
    if (!running) return;
    if (!client.exited()) run(kCmdStop);
    running = false;
  }
};

int main() {
  std::vector<float> event(32);
  for (int i = 0; i < 32; i++) event[i] = 0.25f * (float)i - 3.0f;
  Mailbox* mb = new Mailbox();

  {  // commands in order, scores from the worker's position, PING, RESET, STOP twice
    Host h;
    h.client.attach(mb, 1000);
    FakeWorker w(mb, event.data(), 32, WorkerOptions{1000});
    h.worker = &w;
    std::vector<float> scores;
    for (int i = 0; i < 50; i++) {
      expect(h.run(kCmdRun), "RUN");
      scores.push_back(h.client.score());
    }
    for (int i = 1; i < 50; i++) expect(scores[i] == scores[0] + (float)i, "RUN scores follow the worker's position");
    expect(h.run(kCmdPing), "PING");
    unsigned long long sum = 0;
    for (float v : event) {
      uint32_t bits;
      std::memcpy(&bits, &v, 4);
      sum += bits;
    }
    expect(h.client.checksum() == sum, "PING checksum of the event");
    expect(h.run(kCmdReset) && h.run(kCmdRun) && h.client.score() == scores[0], "RESET restarts the position");
    expect(h.client.sequence() == 1000 + 53, "one sequence ID per command");
    h.stop();
    h.stop();  // idempotent: no second STOP once the worker has exited
    w.join();
    expect(h.client.exited() && h.client.sequence() == 1000 + 54, "STOP ends the worker, once");
    expect(h.fails_with(kCmdRun) == MailboxError::kExited, "a command after STOP reports the exit");
  }
  {  // a finite RUN budget (max_events): the worker leaves after the last RUN it answers
    Host h;
    h.client.attach(mb, 0);
    FakeWorker w(mb, event.data(), 32, WorkerOptions{0, 3});
    h.worker = &w;
    expect(h.run(kCmdRun) && h.run(kCmdReset) && h.run(kCmdRun) && h.run(kCmdRun), "three RUNs within the budget");
    w.join();
    expect(h.fails_with(kCmdRun) == MailboxError::kExited, "the fourth RUN reports the exhausted budget");
    h.stop();  // nothing to stop
  }
  for (int round = 0; round < 20; round++) {  // the same, the next RUN sent at once: the worker
    // may not have raised `exited` yet, and the request then finds it gone
    Host h;
    h.client.attach(mb, 0);
    FakeWorker w(mb, event.data(), 32, WorkerOptions{0, 1});
    h.worker = &w;
    expect(h.run(kCmdRun), "the one RUN of the budget");
    expect(h.fails_with(kCmdRun) == MailboxError::kExited, "a RUN right after the budget reports the exit");
  }
  {  // idle exit
    Host h;
    h.client.attach(mb, 7);
    WorkerOptions o{7};
    o.idle_seconds = 0.05;
    FakeWorker w(mb, event.data(), 32, o);
    h.worker = &w;
    expect(h.run(kCmdRun), "RUN before the idle budget");
    w.join();
    expect(h.fails_with(kCmdPing) == MailboxError::kExited, "a command after the idle budget reports the exit");
  }
  {  // a worker that never answers: the host times out
    Host h;
    h.timeout = 0.2;
    h.client.attach(mb, 0);
    WorkerOptions o{0};
    o.answer = false;
    o.idle_seconds = 600.0;  // stays until released below
    FakeWorker w(mb, event.data(), 32, o);
    h.worker = &w;
    expect(h.fails_with(kCmdRun) == MailboxError::kTimeout, "an unanswered command times out");
    w.release();
    w.join();
  }
  {  // a launch that ends without answering
    Host h;
    h.client.attach(mb, 0);
    WorkerOptions o{0};
    o.end_silently = true;
    FakeWorker w(mb, event.data(), 32, o);
    h.worker = &w;
    expect(h.fails_with(kCmdRun) == MailboxError::kExitedBeforeCompletion, "the worker ended before completing");
  }
  {  // the device watchdog word arrives with the completion
    Host h;
    h.client.attach(mb, 0);
    WorkerOptions o{0};
    o.error_bits = 1;
    FakeWorker w(mb, event.data(), 32, o);
    h.worker = &w;
    expect(h.fails_with(kCmdRun) == MailboxError::kWatchdog, "watchdog error bits");
    h.stop();
    expect(h.client.exited(), "STOP still ends the worker");
  }
  {  // the last sequence IDs: RUN up to UINT64_MAX - 1, then only STOP
    const uint64_t m = ~0ull;
    Host h;
    h.client.attach(mb, m - 3);
    FakeWorker w(mb, event.data(), 32, WorkerOptions{m - 3});
    h.worker = &w;
    expect(h.run(kCmdRun) && h.run(kCmdRun), "RUN at UINT64_MAX - 2 and - 1");
    expect(h.fails_with(kCmdRun) == MailboxError::kExhausted, "no RUN with the last ID");
    expect(h.run(kCmdStop) && h.client.sequence() == m, "STOP takes the last ID");
    w.join();
    expect(h.fails_with(kCmdStop) == MailboxError::kExhausted, "nothing after the last ID");
  }
  delete mb;
  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
