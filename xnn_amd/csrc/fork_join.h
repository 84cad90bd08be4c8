// Fork and join of independent launches of one entry point over side streams (per device,
// created once, default priority, non-blocking). The side streams start after everything
// enqueued so far on the caller's stream and the caller's stream waits for all of them at
// the end, so the entry point still behaves as one ordered step on the caller's stream (and
// a HIP-graph capture of that stream captures the fork and the join). While a ForkJoin is
// alive it holds a process-wide lock: the events are reused by every call.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>

namespace xnn {

constexpr int kSideStreams = 3;
constexpr int kMaxDevices = 64;

struct SideStreams {
  hipStream_t s[kSideStreams];
  hipEvent_t fork;
  hipEvent_t join[kSideStreams];
  bool ready;
};

inline std::mutex& fork_join_mutex() {
  static std::mutex m;
  return m;
}

inline SideStreams* side_streams_of(int dev) {
  static SideStreams table[kMaxDevices] = {};
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  SideStreams& S = table[dev];
  if (!S.ready) {
    bool ok = hipEventCreateWithFlags(&S.fork, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; ok && i < kSideStreams; ++i) {
      ok = hipStreamCreateWithFlags(&S.s[i], hipStreamNonBlocking) == hipSuccess &&
           hipEventCreateWithFlags(&S.join[i], hipEventDisableTiming) == hipSuccess;
    }
    if (!ok) return nullptr;
    S.ready = true;
  }
  return &S;
}

class ForkJoin {
 public:
  // Launches go to stream(i): i = 0 the caller's stream, i >= 1 a side stream. Without side
  // streams (they could not be made, or a capture is running and they do not exist yet)
  // every stream(i) is the caller's and the launches run in order.
  explicit ForkJoin(hipStream_t main) : lock_(fork_join_mutex()), main_(main) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(main, &cap) != hipSuccess) return;
    static bool created[kMaxDevices] = {};
    if (cap != hipStreamCaptureStatusNone && (dev >= kMaxDevices || !created[dev])) return;
    S_ = side_streams_of(dev);
    if (S_ == nullptr) return;
    created[dev] = true;
    if (hipEventRecord(S_->fork, main) != hipSuccess) {
      S_ = nullptr;
      return;
    }
  }

  hipStream_t stream(int i) {
    if (S_ == nullptr || i <= 0) return main_;
    const int k = (i - 1) % kSideStreams;
    if (!(used_ & (1u << k))) {
      if (hipStreamWaitEvent(S_->s[k], S_->fork, 0) != hipSuccess) return main_;
      used_ |= 1u << k;
    }
    return S_->s[k];
  }

  // the caller's stream waits for every side stream used; hipSuccess or the first error
  hipError_t join() {
    hipError_t err = hipSuccess;
    if (S_ == nullptr) return err;
    for (int k = 0; k < kSideStreams; ++k) {
      if (!(used_ & (1u << k))) continue;
      hipError_t e = hipEventRecord(S_->join[k], S_->s[k]);
      if (e == hipSuccess) e = hipStreamWaitEvent(main_, S_->join[k], 0);
      if (err == hipSuccess) err = e;
    }
    used_ = 0;
    return err;
  }

  ~ForkJoin() { (void)join(); }

 private:
  std::lock_guard<std::mutex> lock_;
  hipStream_t main_;
  SideStreams* S_ = nullptr;
  unsigned used_ = 0;
};

}  // namespace xnn
