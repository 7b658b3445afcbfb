// Host half of the persistent worker's mailbox protocol (src/cuda/Runtime.cu:398-428,466-474;
// docs/transport.md:9-16). No HIP types: the runtime drives it against the resident kernel,
// and the sanitizer tests drive it against a host-thread worker that follows the same
// protocol (tests/mailbox_selftest.cpp), under ThreadSanitizer and AddressSanitizer.
//
// Protocol. The request, completion and exited words sit on separate 64-byte lines; only
// naturally aligned 64-bit loads and stores cross the host/device boundary, never a
// read-modify-write. For each command the host writes the command word (and the event), then
// release-stores request = sequence + 1; the worker acquires the new request, runs the command,
// stores the score and error words, and release-stores completion = that sequence; the host
// acquires the completion before it reads them. The worker's last act is a release store of
// exited = 1 (after STOP, after max_events RUN commands, or when it sat idle for its budget).
// The last sequence ID is kept for STOP, so a runtime can always be stopped.
#pragma once

#include <chrono>
#include <cstdint>
#include <functional>
#include <limits>
#include <stdexcept>
#include <string>
#include <thread>

namespace stamd {

// Mailbox commands (the reference's Command enum, src/cuda/Primitives.cuh:14), plus the
// worker's own exit on an exhausted idle budget.
enum MailboxCommand : int { kCmdRun = 1, kCmdReset = 2, kCmdStop = 3, kCmdPing = 4, kCmdSnapshot = 5, kCmdExit = 64 };

// The mailbox in coherent host memory (src/cuda/Primitives.cuh:16-23).
struct alignas(64) Mailbox {
  alignas(64) unsigned long long request;
  alignas(64) unsigned long long completion;
  alignas(64) unsigned long long exited;
  alignas(64) int32_t command;
  float score;
  unsigned long long checksum;
  uint32_t error;
};

class MailboxError : public std::runtime_error {
 public:
  enum Kind { kExhausted, kExited, kExitedBeforeCompletion, kTimeout, kWatchdog };
  MailboxError(Kind k, const std::string& what) : std::runtime_error(what), kind(k) {}
  Kind kind;
};

class MailboxClient {
 public:
  MailboxClient() = default;
  // Start a sequence at `initial` (the worker starts with the same value as its "previous").
  void attach(Mailbox* mb, uint64_t initial) {
    mb_ = mb;
    sequence_ = initial;
    mb_->request = initial;
    mb_->completion = initial;
    mb_->exited = 0;
  }
  Mailbox* mailbox() const { return mb_; }
  uint64_t sequence() const { return sequence_; }
  bool exited() const { return __atomic_load_n(&mb_->exited, __ATOMIC_ACQUIRE) != 0; }

  // Refuse a command the sequence has no room for (the last ID is STOP's) or that no live
  // worker would answer.
  void check(int cmd) const {
    const uint64_t maximum = std::numeric_limits<uint64_t>::max();
    if (sequence_ == maximum || (sequence_ == maximum - 1 && cmd != kCmdStop))
      throw MailboxError(MailboxError::kExhausted, "Sequence exhausted; create a new runtime before wraparound");
    if (exited()) throw MailboxError(MailboxError::kExited, "Persistent worker exited: finite-event or idle budget reached");
  }

  // One round trip. `finished` tells whether the worker's launch has ended (it is asked every
  // 65,536 polls); `timeout_s` bounds the wait. With `backoff` the host yields between polls.
  void issue(int cmd, bool backoff, double timeout_s, const std::function<bool()>& finished) {
    mb_->command = cmd;
    __atomic_store_n(&mb_->request, ++sequence_, __ATOMIC_RELEASE);
    const auto start = std::chrono::steady_clock::now();
    uint64_t polls = 0;
    while (__atomic_load_n(&mb_->completion, __ATOMIC_ACQUIRE) != sequence_) {
      if (backoff) std::this_thread::yield();
      if ((++polls & 0xffff) == 0) {
        if (finished()) {
          // The completion may have landed just before the launch ended.
          if (__atomic_load_n(&mb_->completion, __ATOMIC_ACQUIRE) == sequence_) break;
          // A worker that ran out of its RUN or idle budget raises `exited` after its last
          // completion, so a request sent in between finds it gone: the same exit as check()'s.
          if (exited())
            throw MailboxError(MailboxError::kExited, "Persistent worker exited: finite-event or idle budget reached");
          throw MailboxError(MailboxError::kExitedBeforeCompletion, "Persistent worker exited before completion");
        }
        const double waited = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
        if (waited > timeout_s) throw MailboxError(MailboxError::kTimeout, "Persistent response timeout");
      }
    }
    if (mb_->error)
      throw MailboxError(MailboxError::kWatchdog, "Device watchdog tripped (error bits " + std::to_string(mb_->error) + ")");
  }

  float score() const { return mb_->score; }
  unsigned long long checksum() const { return mb_->checksum; }

 private:
  Mailbox* mb_ = nullptr;
  uint64_t sequence_ = 0;
};

}  // namespace stamd
