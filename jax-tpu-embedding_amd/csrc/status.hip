// Error reporting and the optional launch-timing hooks shared by all libscemb
// entry points.
#include <mutex>
#include <string>
#include <vector>

#include "../../include/scemb.h"
#include "common.h"

namespace scemb {
namespace {
thread_local std::string g_last_error;

struct Span {
  std::string name;
  hipEvent_t start;
  hipEvent_t stop;
};

std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<Span> g_spans;
std::vector<hipEvent_t> g_free_events;

hipEvent_t TakeEvent() {
  if (!g_free_events.empty()) {
    hipEvent_t e = g_free_events.back();
    g_free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

void SetError(const std::string& msg) { g_last_error = msg; }

int Fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int ProfileBegin(const char* name, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (!g_prof_on) return -1;
  Span s{name, TakeEvent(), TakeEvent()};
  if (s.start == nullptr || s.stop == nullptr) return -1;
  if (hipEventRecord(s.start, stream) != hipSuccess) return -1;
  g_spans.push_back(s);
  return static_cast<int>(g_spans.size()) - 1;
}

void ProfileEnd(int token, hipStream_t stream) {
  if (token < 0) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (token < static_cast<int>(g_spans.size())) {
    (void)hipEventRecord(g_spans[token].stop, stream);
  }
}

namespace {
constexpr int kMaxSideDevices = 64;
struct SideState {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t join = nullptr;
};
std::mutex g_side_mu;
SideState g_side[kMaxSideDevices];

int SideOf(SideState** out) {
  int dev = 0;
  SCEMB_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxSideDevices) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "device index out of range");
  }
  SideState& st = g_side[dev];
  if (st.stream == nullptr) {
    SCEMB_HIP(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking));
    SCEMB_HIP(hipEventCreateWithFlags(&st.fork, hipEventDisableTiming));
    SCEMB_HIP(hipEventCreateWithFlags(&st.join, hipEventDisableTiming));
  }
  *out = &st;
  return 0;
}
}  // namespace

int ForkSide(hipStream_t stream, hipStream_t* side) {
  std::lock_guard<std::mutex> lock(g_side_mu);
  SideState* st = nullptr;
  const int rc = SideOf(&st);
  if (rc != 0) return rc;
  SCEMB_HIP(hipEventRecord(st->fork, stream));
  SCEMB_HIP(hipStreamWaitEvent(st->stream, st->fork, 0));
  *side = st->stream;
  return 0;
}

int JoinSide(hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_side_mu);
  SideState* st = nullptr;
  const int rc = SideOf(&st);
  if (rc != 0) return rc;
  SCEMB_HIP(hipEventRecord(st->join, st->stream));
  SCEMB_HIP(hipStreamWaitEvent(stream, st->join, 0));
  return 0;
}

}  // namespace scemb

extern "C" {

const char* scemb_last_error(void) { return scemb::g_last_error.c_str(); }

int scemb_version(void) { return (0 << 16) | 1; }

void scemb_profile_enable(int enable) {
  std::lock_guard<std::mutex> lock(scemb::g_prof_mu);
  scemb::g_prof_on = enable != 0;
}

int scemb_profile_collect(const char* name, double* total_ms,
                          int64_t* launches) {
  std::lock_guard<std::mutex> lock(scemb::g_prof_mu);
  double sum = 0.0;
  int64_t count = 0;
  std::vector<scemb::Span> keep;
  for (auto& s : scemb::g_spans) {
    if (name != nullptr && s.name != name) {
      keep.push_back(s);
      continue;
    }
    if (hipEventSynchronize(s.stop) != hipSuccess) {
      return scemb::Fail(SCEMB_ERR_DEVICE, "hipEventSynchronize failed");
    }
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, s.start, s.stop) != hipSuccess) {
      return scemb::Fail(SCEMB_ERR_DEVICE, "hipEventElapsedTime failed");
    }
    sum += ms;
    ++count;
    scemb::g_free_events.push_back(s.start);
    scemb::g_free_events.push_back(s.stop);
  }
  scemb::g_spans.swap(keep);
  if (total_ms != nullptr) *total_ms = sum;
  if (launches != nullptr) *launches = count;
  return SCEMB_OK;
}

}  // extern "C"
