// Opt-in per-kernel timing for benchmarks and diagnostics.
//
// When enabled, every kernel launch of the library is bracketed by two
// hipEvents recorded on the launch stream, so the elapsed time is that of the
// kernel on the stream it actually runs on (events recorded on another stream,
// such as a framework's current stream, would not see it).  Disabled (the
// default), a launch costs one relaxed atomic load.  The state is process-wide
// and guarded by a mutex; it holds only events and running totals, never
// device memory.
#include <atomic>
#include <mutex>
#include <vector>

#include "tsm_internal.hpp"

namespace tsm {

namespace {

const char* const kNames[kNumKernels] = {
    "scan_fwd_kernel",   "scan_bwd_kernel",      "verify_kernel",           "fwd_fixup_kernel",
    "bwd_fixup_kernel",  "apply_offsets_kernel", "marginal_kernel",         "finalize_rows_kernel",
    "finalize_shared_kernel", "checkpoints_kernel", "viterbi_kernel",       "backtrace_kernel",
    "retry_kernel",      "dense_prep_kernel",    "gold_kernels",
    "prologue_kernels",  "u_rows_kernel",        "trans_grad_kernel",       "fused_rows_kernel",
    "fused_shared_kernel", "coverage_kernels",
};

struct Pending {
  int id;
  hipEvent_t a, b;
};

std::mutex g_mu;
std::atomic<bool> g_on{false};
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_free;
double g_ms[kNumKernels];
int64_t g_count[kNumKernels];

hipEvent_t take_event() {
  if (!g_free.empty()) {
    hipEvent_t e = g_free.back();
    g_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Waits for every pending pair, adds its time (when `accumulate`) and recycles
// the events.  Caller holds g_mu.
int drain(bool accumulate) {
  int rc = 0;
  for (const Pending& p : g_pending) {
    float ms = 0.0f;
    hipError_t e = hipEventSynchronize(p.b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.a, p.b);
    if (e != hipSuccess) {
      rc = (int)e;
    } else if (accumulate) {
      g_ms[p.id] += ms;
      g_count[p.id] += 1;
    }
    g_free.push_back(p.a);
    g_free.push_back(p.b);
  }
  g_pending.clear();
  return rc;
}

}  // namespace

TimedLaunch::TimedLaunch(int id, hipStream_t s) : id_(-1), s_(s), a_(nullptr), b_(nullptr) {
  if (!g_on.load(std::memory_order_relaxed) || id < 0 || id >= kNumKernels) return;
  std::lock_guard<std::mutex> lk(g_mu);
  a_ = take_event();
  b_ = take_event();
  if (a_ == nullptr || b_ == nullptr || hipEventRecord(a_, s) != hipSuccess) {
    if (a_) g_free.push_back(a_);
    if (b_) g_free.push_back(b_);
    a_ = b_ = nullptr;
    return;
  }
  id_ = id;
}

TimedLaunch::~TimedLaunch() {
  if (id_ < 0) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (hipEventRecord(b_, s_) == hipSuccess) {
    g_pending.push_back(Pending{id_, a_, b_});
  } else {
    g_free.push_back(a_);
    g_free.push_back(b_);
  }
}

int timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int rc = drain(false);
  for (int i = 0; i < kNumKernels; ++i) {
    g_ms[i] = 0.0;
    g_count[i] = 0;
  }
  g_on.store(on != 0, std::memory_order_relaxed);
  return rc;
}

int timing_read(double* total_ms, int64_t* launches, int n) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int rc = drain(true);
  for (int i = 0; i < n && i < kNumKernels; ++i) {
    if (total_ms) total_ms[i] = g_ms[i];
    if (launches) launches[i] = g_count[i];
  }
  return rc;
}

const char* timing_name(int id) { return (id >= 0 && id < kNumKernels) ? kNames[id] : nullptr; }

}  // namespace tsm
