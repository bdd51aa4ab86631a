// Small utility kernels: the NaN/Inf guard (the reference's `sanity`,
// src/delta/path.rs:198-207, compiled in by its check-nan/check-inf features).

#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "dn_common.hpp"

namespace dn {
namespace {

template <class T>
__global__ __launch_bounds__(256) void nonfinite_kernel(const T* p, size_t n, int* flag) {
  bool bad = false;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    bad |= !isfinite(ld(p, i));
  // Every writer stores the same value, so the plain store needs no atomic.
  if (bad) *flag = 1;
}

}  // namespace

namespace {
// A second stream (default priority, non-blocking) and its fork / join
// events per (device, calling stream), created on first use and kept until
// the process ends. Keying by the calling stream keeps callers on different
// streams apart: their backward calls neither serialise on one side stream
// nor pull one another's work into a HIP graph that one of them captures
// (a side stream joins its calling stream's capture through the fork event).
struct Side {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex side_mu;
std::map<std::pair<int, hipStream_t>, Side> sides;
}  // namespace

hipError_t side_fork(hipStream_t main, hipStream_t* side) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(side_mu);
  Side& sd = sides[{dev, main}];
  if (!sd.s) {
    if ((e = hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&sd.join, hipEventDisableTiming)) != hipSuccess) return e;
  }
  if ((e = hipEventRecord(sd.fork, main)) != hipSuccess) return e;
  if ((e = hipStreamWaitEvent(sd.s, sd.fork, 0)) != hipSuccess) return e;
  *side = sd.s;
  return hipSuccess;
}

hipError_t side_join(hipStream_t main) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(side_mu);
  const auto it = sides.find({dev, main});
  if (it == sides.end() || !it->second.s) return hipErrorInvalidHandle;
  Side& sd = it->second;
  if ((e = hipEventRecord(sd.join, sd.s)) != hipSuccess) return e;
  return hipStreamWaitEvent(main, sd.join, 0);
}

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = -1;
  if (dev >= 0) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev < 0 ? 0 : dev) !=
          hipSuccess ||
      n <= 0)
    n = 256;
  if (dev >= 0) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

hipError_t launch_nonfinite_scan(const void* p, size_t n, int dtype, int* flag,
                                 hipStream_t stream) {
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (dtype == DN_BF16)
    hipLaunchKernelGGL(nonfinite_kernel<bf16>, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const bf16*>(p), n, flag);
  else
    hipLaunchKernelGGL(nonfinite_kernel<float>, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const float*>(p), n, flag);
  return hipGetLastError();
}

}  // namespace dn

// ---------------------------------------------------------------------------
// Per-kernel timing with HIP events.
// ---------------------------------------------------------------------------

#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace dn {
namespace {

struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
};

struct Profiler {
  std::mutex mu;
  bool on = false;
  std::vector<ProfRecord> pending;
  std::vector<hipEvent_t> free_events;
  std::map<std::string, std::pair<double, int64_t>> totals;

  hipEvent_t take() {
    if (!free_events.empty()) {
      hipEvent_t e = free_events.back();
      free_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }

  void flush() {
    for (ProfRecord& r : pending) {
      float ms = 0.f;
      if (r.start && r.stop && hipEventSynchronize(r.stop) == hipSuccess &&
          hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
        auto& t = totals[r.name];
        t.first += ms;
        t.second += 1;
      }
      if (r.start) free_events.push_back(r.start);
      if (r.stop) free_events.push_back(r.stop);
    }
    pending.clear();
  }
};

Profiler& prof() {
  static Profiler* p = new Profiler();  // never destroyed: events outlive static teardown
  return *p;
}

}  // namespace

ProfScope::ProfScope(const char* name, hipStream_t s) : slot(-1), stream(s) {
  Profiler& P = prof();
  std::lock_guard<std::mutex> lock(P.mu);
  if (!P.on) return;
  ProfRecord r{name, P.take(), nullptr};
  if (r.start) (void)hipEventRecord(r.start, stream);
  P.pending.push_back(r);
  slot = int(P.pending.size()) - 1;
}

ProfScope::~ProfScope() {
  if (slot < 0) return;
  Profiler& P = prof();
  std::lock_guard<std::mutex> lock(P.mu);
  if (slot >= int(P.pending.size())) return;
  hipEvent_t e = P.take();
  if (e) (void)hipEventRecord(e, stream);
  P.pending[size_t(slot)].stop = e;
}

}  // namespace dn

extern "C" int dn_profile_enable(int on) {
  dn::Profiler& P = dn::prof();
  std::lock_guard<std::mutex> lock(P.mu);
  P.flush();
  P.totals.clear();
  P.on = on != 0;
  return 0;
}

extern "C" int dn_profile_read(int index, char* name, size_t name_len, double* total_ms,
                               int64_t* launches) {
  dn::Profiler& P = dn::prof();
  std::lock_guard<std::mutex> lock(P.mu);
  P.flush();
  const int count = int(P.totals.size());
  if (index >= 0 && index < count) {
    auto it = P.totals.begin();
    std::advance(it, index);
    if (name && name_len) {
      std::strncpy(name, it->first.c_str(), name_len - 1);
      name[name_len - 1] = '\0';
    }
    if (total_ms) *total_ms = it->second.first;
    if (launches) *launches = it->second.second;
  }
  return count;
}
