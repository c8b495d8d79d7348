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
