// Host-side pass over row splits, built by the host compiler so that it can
// carry a vectorised clone for hosts with AVX2 (selected at load time).
#include <algorithm>
#include <cstdint>

namespace scemb {

// The longest row (returned) and the shortest (*least, at most 0) of host
// row splits [num_rows + 1], in one pass with independent accumulators.
__attribute__((target_clones("avx2", "default"))) int64_t RowLengthRange(
    const int64_t* sp, int64_t num_rows, int64_t* least) {
  int64_t hi[4] = {0, 0, 0, 0}, lo[4] = {0, 0, 0, 0};
  int64_t r = 0;
  for (; r + 4 <= num_rows; r += 4) {
    for (int j = 0; j < 4; ++j) {
      const int64_t d = sp[r + j + 1] - sp[r + j];
      hi[j] = d > hi[j] ? d : hi[j];
      lo[j] = d < lo[j] ? d : lo[j];
    }
  }
  for (; r < num_rows; ++r) {
    const int64_t d = sp[r + 1] - sp[r];
    hi[0] = d > hi[0] ? d : hi[0];
    lo[0] = d < lo[0] ? d : lo[0];
  }
  *least = std::min(std::min(lo[0], lo[1]), std::min(lo[2], lo[3]));
  return std::max(std::max(hi[0], hi[1]), std::max(hi[2], hi[3]));
}

}  // namespace scemb

namespace scemb {

// RowLengthRange that also copies the splits to dst (the same pass).
__attribute__((target_clones("avx2", "default"))) int64_t CopyRowLengthRange(
    const int64_t* sp, int64_t num_rows, int64_t* dst, int64_t* least) {
  int64_t hi[4] = {0, 0, 0, 0}, lo[4] = {0, 0, 0, 0};
  dst[0] = sp[0];
  int64_t r = 0;
  for (; r + 4 <= num_rows; r += 4) {
    for (int j = 0; j < 4; ++j) {
      const int64_t next = sp[r + j + 1];
      const int64_t d = next - sp[r + j];
      dst[r + j + 1] = next;
      hi[j] = d > hi[j] ? d : hi[j];
      lo[j] = d < lo[j] ? d : lo[j];
    }
  }
  for (; r < num_rows; ++r) {
    const int64_t d = sp[r + 1] - sp[r];
    dst[r + 1] = sp[r + 1];
    hi[0] = d > hi[0] ? d : hi[0];
    lo[0] = d < lo[0] ? d : lo[0];
  }
  *least = std::min(std::min(lo[0], lo[1]), std::min(lo[2], lo[3]));
  return std::max(std::max(hi[0], hi[1]), std::max(hi[2], hi[3]));
}

}  // namespace scemb

// ---------------------------------------------------------------------------
// Batched staging of many features' row splits over a few host threads.
// ---------------------------------------------------------------------------
#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/scemb.h"

namespace scemb {

int Fail(int code, const std::string& msg);

namespace {

// Worker threads that run the tasks of one batch alongside the calling
// thread. Created on first use and never destroyed (they wait on a condition
// variable between batches and end with the process); batches from several
// calling threads run one after another.
class HostPool {
 public:
  explicit HostPool(int workers) {
    for (int w = 0; w < workers; ++w) threads_.emplace_back([this] { Loop(); });
  }

  // fn(i) for every i in [0, n), on the calling thread and the workers.
  void Run(int n, const std::function<void(int)>& fn) {
    std::lock_guard<std::mutex> one_batch(run_mu_);
    {
      std::lock_guard<std::mutex> g(mu_);
      fn_ = &fn;
      n_ = n;
      next_.store(0);
      active_ = static_cast<int>(threads_.size());
      ++gen_;
    }
    cv_.notify_all();
    Work();
    std::unique_lock<std::mutex> g(mu_);
    done_.wait(g, [this] { return active_ == 0; });
    fn_ = nullptr;
  }

  static HostPool& Get() {
    static HostPool* pool = new HostPool(Workers());
    return *pool;
  }

 private:
  static int Workers() {
    const unsigned hc = std::thread::hardware_concurrency();
    return hc >= 8 ? 3 : (hc >= 2 ? static_cast<int>(hc) - 1 : 0);
  }

  void Work() {
    for (int i = next_.fetch_add(1); i < n_; i = next_.fetch_add(1)) (*fn_)(i);
  }

  void Loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> g(mu_);
        cv_.wait(g, [&] { return gen_ != seen; });
        seen = gen_;
      }
      Work();
      std::lock_guard<std::mutex> g(mu_);
      if (--active_ == 0) done_.notify_one();
    }
  }

  std::vector<std::thread> threads_;
  std::mutex run_mu_, mu_;
  std::condition_variable cv_, done_;
  const std::function<void(int)>* fn_ = nullptr;
  int n_ = 0;
  std::atomic<int> next_{0};
  int active_ = 0;
  uint64_t gen_ = 0;
};

// Rows per task: long enough that a task outweighs handing it out.
constexpr int64_t kStageChunkRows = int64_t{1} << 15;

struct StageTask {
  int feature;
  int64_t row0, row1;  // rows [row0, row1) of that feature
  int64_t most, least;
};

}  // namespace
}  // namespace scemb

extern "C" int scemb_stage_row_splits_batch(
    int32_t count, const int64_t* const* row_splits, const int64_t* num_rows,
    const int64_t* nnz, int64_t* const* dst, int64_t* max_row_length,
    int32_t* first_bad) {
  using scemb::StageTask;
  if (first_bad != nullptr) *first_bad = -1;
  if (count < 0 || (count > 0 && (row_splits == nullptr || num_rows == nullptr ||
                                  nnz == nullptr || dst == nullptr ||
                                  max_row_length == nullptr))) {
    return scemb::Fail(SCEMB_ERR_INVALID_ARGUMENT, "null row splits");
  }
  std::vector<StageTask> tasks;
  for (int f = 0; f < count; ++f) {
    if (row_splits[f] == nullptr || dst[f] == nullptr || num_rows[f] < 0) {
      if (first_bad != nullptr) *first_bad = f;
      return scemb::Fail(SCEMB_ERR_INVALID_ARGUMENT, "null row splits");
    }
    dst[f][0] = row_splits[f][0];
    for (int64_t r = 0; r < num_rows[f] || r == 0; r += scemb::kStageChunkRows) {
      const int64_t r1 = std::min(num_rows[f], r + scemb::kStageChunkRows);
      tasks.push_back(StageTask{f, r, r1, 0, 0});
    }
  }
  auto run = [&](int i) {
    StageTask& t = tasks[i];
    const int64_t* sp = row_splits[t.feature] + t.row0;
    t.most = scemb::CopyRowLengthRange(sp, t.row1 - t.row0,
                                       dst[t.feature] + t.row0, &t.least);
  };
  const int64_t total_rows = static_cast<int64_t>(tasks.size()) *
                             scemb::kStageChunkRows;
  if (tasks.size() > 1 && total_rows >= 4 * scemb::kStageChunkRows) {
    scemb::HostPool::Get().Run(static_cast<int>(tasks.size()), run);
  } else {
    for (size_t i = 0; i < tasks.size(); ++i) run(static_cast<int>(i));
  }
  for (int f = 0; f < count; ++f) max_row_length[f] = 0;
  std::vector<int64_t> least(count, 0);
  for (const StageTask& t : tasks) {
    max_row_length[t.feature] = std::max(max_row_length[t.feature], t.most);
    least[t.feature] = std::min(least[t.feature], t.least);
  }
  for (int f = 0; f < count; ++f) {
    if (row_splits[f][0] != 0 || row_splits[f][num_rows[f]] != nnz[f] ||
        least[f] < 0) {
      if (first_bad != nullptr) *first_bad = f;
      return scemb::Fail(SCEMB_ERR_INVALID_ARGUMENT,
                         "row_splits must start at 0, be non-decreasing and "
                         "end at the number of values.");
    }
  }
  return 0;
}
