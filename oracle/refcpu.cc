// refcpu: CPU restatement of jax-tpu-embedding's SparseCore hot path.
//
// TEST INFRASTRUCTURE ONLY. This file is the parity oracle and the CPU
// baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg load it, and only as a checker; the product path (libscemb.so) never
// links or calls it.
//
// It restates the reference algorithm stage by stage, so that every stage can
// be pinned separately against the reference's own known-answer tests:
//
//   extraction        jax_tpu_embedding/sparsecore/lib/core/
//                       input_preprocessing.cc:79-123, :312-436
//                       process_coo_tensors_impl.h:39-136
//                       coo_format.h:120-185
//   sort/group/dedupe sort_and_group_coo_tensors_impl.h:196-311, :349-646
//                       partitioned_coo_tensors.h:94-125
//   CSR fill          input_preprocessing_util.cc:73-208, :331-473
//   sizes/validation  input_preprocessing_util.cc:223-312, :490-522
//                       input_preprocessing.cc:757-786
//   minibatching      coo_format.h:31-49, :140-185 (HighwayHash buckets),
//                       minibatching_splits_impl.h:58-131 (split, merge tree)
//                       partitioned_coo_tensors.h:157-215 (bucket merge)
//                       sort_and_group_coo_tensors_impl.h:116-151, :349-646
//                       input_preprocessing.cc:238-310, :800-959 (passes)
//                       input_preprocessing_util.cc:135-143, :331-473 (fill)
//   lookup / update   primitives/sparse_dense_matmul_csr.py:171-201 (operand
//                       meaning), primitives/optimizers_computation.py:22-148,
//                       primitives/utils.py:24-59 (clip), and the numpy test
//                       oracles in primitives/tests/
//                       sparse_dense_matmul_grad_with_adagrad_test.py:356-400.
//   optimizers        the row-wise update bodies of primitives/
//                       sparse_dense_matmul_grad_with_adam.py:283-338,
//                       _adagrad_momentum.py:256-311, _ftrl.py:260-335,
//                       _laprop.py:282-340, _f2a.py:244-290.
//
// Numeric rules follow the C++ (not the Python reference): float gains,
// float sums in sorted order, std::pow(float,int) promoting to double in the
// weighted sqrtn divisor. Build with -ffp-contract=off.

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <thread>
#include <vector>

namespace {

enum Combiner : int { kSum = 0, kMean = 1, kSqrtn = 2 };

constexpr int kAlign = 8;           // TPU_VECTOR_REGISTER_ALIGNMENT_SIZE
constexpr uint32_t kDataBits = 26;  // coo_format.h:57-62
constexpr uint32_t kDataMask = (1u << kDataBits) - 1;
constexpr uint32_t kRotatedColIdOffset = kDataBits;

inline int64_t RoundUp(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
inline int Log2Exact(uint32_t v) {
  int b = 0;
  while ((1u << b) < v) ++b;
  return b;
}
inline uint32_t Rotr32(uint32_t x, int s) {
  s &= 31;
  return s == 0 ? x : ((x >> s) | (x << (32 - s)));
}
inline uint32_t Rotl32(uint32_t x, int s) {
  s &= 31;
  return s == 0 ? x : ((x << s) | (x >> (32 - s)));
}

// coo_format.h:120-135
inline int GetColId(int embedding_id, int col_shift, int col_offset,
                    int num_scs_mod) {
  return ((embedding_id + col_shift) & num_scs_mod) +
         (embedding_id & ~num_scs_mod) + col_offset;
}

// coo_format.h:154-185 (no minibatching buckets: bucket id is 0).
inline uint64_t GroupingKey(uint32_t col_id, uint32_t data, int num_scs_bit) {
  const uint32_t rotated = Rotr32(col_id, num_scs_bit);
  return (uint64_t{rotated} << kRotatedColIdOffset) | uint64_t{data};
}

struct Coo {
  int32_t row;
  int32_t col;
  float gain;
};

// ---------------------------------------------------------------------------
// HighwayHash-64. Third-party: google/highwayhash (the @highwayhash
// repository of XLA's workspace, third_party/xla/revision.bzl pins the XLA
// revision; absent here). The reference hashes the 4 bytes of an int column
// id with a fixed key through HighwayHashCatT (coo_format.h:31-49). Restated
// from the published algorithm (Alakuijala, Cox, Wassenberg, "Fast keyed hash
// / pseudo-random function using SIMD multiply and permute", 2016, and the
// project's portable C implementation): 256-bit state of four lanes
// (v0, v1, mul0, mul1), 32-byte packets, a remainder packet for the tail,
// four permute-and-update rounds at the end. Its output is fixed by the
// project's published test vectors (highwayhash_test.cc, key
// 0x0706050403020100..., data bytes 0, 1, 2, ...), which the tests check.
// ---------------------------------------------------------------------------

struct HhState {
  uint64_t v0[4], v1[4], mul0[4], mul1[4];
};

void HhReset(const uint64_t key[4], HhState* s) {
  static const uint64_t kInit0[4] = {0xdbe6d5d5fe4cce2full, 0xa4093822299f31d0ull,
                                     0x13198a2e03707344ull, 0x243f6a8885a308d3ull};
  static const uint64_t kInit1[4] = {0x3bd39e10cb0ef593ull, 0xc0acf169b5f18a8cull,
                                     0xbe5466cf34e90c6cull, 0x452821e638d01377ull};
  for (int i = 0; i < 4; ++i) {
    s->mul0[i] = kInit0[i];
    s->mul1[i] = kInit1[i];
    s->v0[i] = kInit0[i] ^ key[i];
    s->v1[i] = kInit1[i] ^ ((key[i] >> 32) | (key[i] << 32));
  }
}

// Byte shuffle of the lane pair (v1, v0) added into (add1, add0).
void HhZipperMergeAdd(uint64_t v1, uint64_t v0, uint64_t* add1,
                      uint64_t* add0) {
  *add0 += (((v0 & 0xff000000ull) | (v1 & 0xff00000000ull)) >> 24) |
           (((v0 & 0xff0000000000ull) | (v1 & 0xff000000000000ull)) >> 16) |
           (v0 & 0xff0000ull) | ((v0 & 0xff00ull) << 32) |
           ((v1 & 0xff00000000000000ull) >> 8) | (v0 << 56);
  *add1 += (((v1 & 0xff000000ull) | (v0 & 0xff00000000ull)) >> 24) |
           (v1 & 0xff0000ull) | ((v1 & 0xff0000000000ull) >> 16) |
           ((v1 & 0xff00ull) << 24) | ((v0 & 0xff000000000000ull) >> 8) |
           ((v1 & 0xffull) << 48) | (v0 & 0xff00000000000000ull);
}

void HhUpdate(const uint64_t lanes[4], HhState* s) {
  for (int i = 0; i < 4; ++i) {
    s->v1[i] += s->mul0[i] + lanes[i];
    s->mul0[i] ^= (s->v1[i] & 0xffffffffull) * (s->v0[i] >> 32);
    s->v0[i] += s->mul1[i];
    s->mul1[i] ^= (s->v0[i] & 0xffffffffull) * (s->v1[i] >> 32);
  }
  HhZipperMergeAdd(s->v1[1], s->v1[0], &s->v0[1], &s->v0[0]);
  HhZipperMergeAdd(s->v1[3], s->v1[2], &s->v0[3], &s->v0[2]);
  HhZipperMergeAdd(s->v0[1], s->v0[0], &s->v1[1], &s->v1[0]);
  HhZipperMergeAdd(s->v0[3], s->v0[2], &s->v1[3], &s->v1[2]);
}

void HhUpdatePacket(const uint8_t* p, HhState* s) {
  uint64_t lanes[4];
  for (int i = 0; i < 4; ++i) {
    uint64_t x = 0;
    for (int b = 7; b >= 0; --b) x = (x << 8) | p[8 * i + b];  // little endian
    lanes[i] = x;
  }
  HhUpdate(lanes, s);
}

// Tail of 1..31 bytes: the length enters v0 and rotates each 32-bit half of
// v1; whole 4-byte words are copied, the last 1-3 bytes (or the final 4
// bytes when 16 or more remain) go to fixed packet positions.
void HhUpdateRemainder(const uint8_t* bytes, size_t size_mod32, HhState* s) {
  const size_t size_mod4 = size_mod32 & 3;
  const uint8_t* remainder = bytes + (size_mod32 & ~size_t{3});
  uint8_t packet[32] = {0};
  for (int i = 0; i < 4; ++i) {
    s->v0[i] += (static_cast<uint64_t>(size_mod32) << 32) + size_mod32;
  }
  const uint32_t c = static_cast<uint32_t>(size_mod32);
  for (int i = 0; i < 4; ++i) {
    const uint32_t h0 = static_cast<uint32_t>(s->v1[i]);
    const uint32_t h1 = static_cast<uint32_t>(s->v1[i] >> 32);
    s->v1[i] = static_cast<uint64_t>((h0 << c) | (h0 >> (32 - c))) |
               (static_cast<uint64_t>((h1 << c) | (h1 >> (32 - c))) << 32);
  }
  for (size_t i = 0; i < static_cast<size_t>(remainder - bytes); ++i) {
    packet[i] = bytes[i];
  }
  if (size_mod32 & 16) {
    for (int i = 0; i < 4; ++i) packet[28 + i] = remainder[i + size_mod4 - 4];
  } else if (size_mod4) {
    packet[16] = remainder[0];
    packet[17] = remainder[size_mod4 >> 1];
    packet[18] = remainder[size_mod4 - 1];
  }
  HhUpdatePacket(packet, s);
}

void HhPermuteAndUpdate(HhState* s) {
  uint64_t p[4];
  p[0] = (s->v0[2] >> 32) | (s->v0[2] << 32);
  p[1] = (s->v0[3] >> 32) | (s->v0[3] << 32);
  p[2] = (s->v0[0] >> 32) | (s->v0[0] << 32);
  p[3] = (s->v0[1] >> 32) | (s->v0[1] << 32);
  HhUpdate(p, s);
}

uint64_t HighwayHash64(const uint8_t* data, size_t size,
                       const uint64_t key[4]) {
  HhState s;
  HhReset(key, &s);
  size_t i = 0;
  for (; i + 32 <= size; i += 32) HhUpdatePacket(data + i, &s);
  if ((size & 31) != 0) HhUpdateRemainder(data + i, size & 31, &s);
  for (int r = 0; r < 4; ++r) HhPermuteAndUpdate(&s);
  return s.v0[0] + s.v1[0] + s.mul0[0] + s.mul1[0];
}

// coo_format.h:31-36, :52-53, :140-145.
constexpr uint64_t kBucketHashKey[4] = {0x4451e30f87db9609ull,
                                        0xca7358a1fd2737f8ull,
                                        0x4b2c991fcee4fdeaull,
                                        0x0b2658e18326f6baull};
constexpr int kMaxBuckets = 64;
constexpr int kBucketIdOffset = kRotatedColIdOffset + 32;

uint32_t BucketOf(int32_t col_id) {
  uint8_t b[4];
  std::memcpy(b, &col_id, 4);
  return static_cast<uint32_t>(HighwayHash64(b, 4, kBucketHashKey) &
                               (kMaxBuckets - 1));
}

// ComputeMinibatchingSplit (minibatching_splits_impl.h:58-81): bottom-up over
// the bucket tree; a node whose children sum past the limit is split and
// keeps the larger child, otherwise it keeps the sum. Modifies `v`.
uint64_t ComputeSplit(int32_t* v, int n, int max_value) {
  uint64_t split = 0;
  int index = 0;
  for (int size = 2; size <= n; size *= 2) {
    for (int i = 0; i < n; i += size, ++index) {
      const int l = v[i], r = v[i + size / 2];
      if (l + r > max_value) {
        split |= uint64_t{1} << index;
        v[i] = std::max(l, r);
      } else {
        v[i] += r;
      }
    }
  }
  return split;
}

// MergeBuckets (minibatching_splits_impl.h:110-129): the (left, right)
// pairs whose tree node is not split, level by level.
template <typename Fn>
void ForEachMerge(uint64_t split, int n, Fn fn) {
  int index = 0;
  for (int size = 2; size <= n; size *= 2) {
    for (int i = 0; i < n; i += size, ++index) {
      if (((split >> index) & 1) == 0) fn(i, i + size / 2);
    }
  }
}

}  // namespace

extern "C" {

// One feature of a stacked table, in values + row-splits form. `weights` is
// null for unity weights (UnityWeightsStream, unity_weights_stream_impl.h).
struct RefFeature {
  const int32_t* ids;
  const int64_t* row_splits;  // num_rows + 1 entries
  const float* weights;       // null or parallel to ids
  int64_t num_rows;
  int32_t row_offset;
  int32_t col_offset;
  int32_t col_shift;
  int32_t pad_;
};

int ref_get_col_id(int embedding_id, int col_shift, int col_offset,
                   int num_scs_mod) {
  return GetColId(embedding_id, col_shift, col_offset, num_scs_mod);
}

uint64_t ref_grouping_key(uint32_t col_id, uint32_t data, int num_scs_bit) {
  return GroupingKey(col_id, data, num_scs_bit);
}

uint32_t ref_col_id_from_key(uint64_t key, int num_scs_bit) {
  return Rotl32(static_cast<uint32_t>(key >> kRotatedColIdOffset), num_scs_bit);
}

uint32_t ref_data_from_key(uint64_t key) {
  return static_cast<uint32_t>(key) & kDataMask;
}

// Gains of one row, following process_coo_tensors_impl.h:39-136.
// Unity weights: sum -> 1; mean -> 1.0f / float(n) (rematerialized from the
// token count, input_preprocessing_util.h:216-222); sqrtn -> 1.0f /
// sqrtf(float(n)) (process_coo_tensors_impl.h:48-49, :105-107).
// Variable weights: divisor = 1 | float running sum | sqrtf(float sum of
// double squares), gain = w / divisor (:54-74, :118).
static void RowGains(const float* w, int64_t n, int combiner, float* out) {
  if (w == nullptr) {
    float g = 1.0f;
    if (combiner == kMean) {
      g = 1.0f / static_cast<float>(static_cast<int>(n));
    } else if (combiner == kSqrtn) {
      const float divisor = std::sqrt(static_cast<float>(static_cast<int>(n)));
      g = 1.0f / divisor;
    }
    for (int64_t i = 0; i < n; ++i) out[i] = g;
    return;
  }
  float divisor = 1.0f;
  if (combiner == kMean) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) sum += w[i];
    divisor = sum;
  } else if (combiner == kSqrtn) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      // std::pow(float, int) is computed in double; the float accumulator
      // is promoted for the add and rounded back on assignment.
      sum = static_cast<float>(static_cast<double>(sum) +
                               static_cast<double>(w[i]) *
                                   static_cast<double>(w[i]));
    }
    divisor = std::sqrt(sum);
  }
  for (int64_t i = 0; i < n; ++i) out[i] = w[i] / divisor;
}

// ExtractCooTensors for one feature slice [slice_start, slice_end)
// (input_preprocessing.cc:79-123 with ProcessCooTensors). Appends to
// rows/cols/gains at *count. Returns 0.
int ref_extract_slice(const RefFeature* f, int slice_start, int slice_end,
                      int row_offset, int col_offset, int col_shift,
                      int num_scs, int combiner, int32_t* rows, int32_t* cols,
                      float* gains, int64_t* count) {
  const int num_scs_mod = num_scs - 1;
  std::vector<float> g;
  int64_t k = *count;
  for (int row = slice_start; row < slice_end; ++row) {
    const int sample_id = row - slice_start + row_offset;
    const int64_t b = f->row_splits[row];
    const int64_t n = f->row_splits[row + 1] - b;
    g.resize(static_cast<size_t>(n));
    RowGains(f->weights ? f->weights + b : nullptr, n, combiner, g.data());
    for (int64_t i = 0; i < n; ++i) {
      rows[k] = sample_id;
      cols[k] = GetColId(f->ids[b + i], col_shift, col_offset, num_scs_mod);
      gains[k] = g[static_cast<size_t>(i)];
      ++k;
    }
  }
  *count = k;
  return 0;
}

// ExtractCooTensorsForAllFeaturesPerLocalDevice (input_preprocessing.cc:
// 312-436). `features` must already be in row_offset order
// (pybind_input_preprocessing.cc:114-120). Output lists are concatenated SC by
// SC; sc_sizes[s] receives the per-SC counts. Returns 0, or 1 when the device
// batch is not divisible by num_sc_per_device / smaller than the number of
// feature slices (CHECK failures in the reference).
int ref_extract_device(const RefFeature* features, int n_features,
                       int local_device_id, int local_device_count,
                       int global_device_count, int num_sc_per_device,
                       int combiner, int32_t* rows, int32_t* cols,
                       float* gains, int64_t* sc_sizes,
                       int32_t* batch_size_for_device_out) {
  int batch_size_for_device = 0;
  for (int f = 0; f < n_features; ++f) {
    batch_size_for_device +=
        static_cast<int>(features[f].num_rows / local_device_count);
  }
  *batch_size_for_device_out = batch_size_for_device;
  if (batch_size_for_device % num_sc_per_device != 0) return 1;
  if (batch_size_for_device < num_sc_per_device * n_features) return 1;
  const int S = num_sc_per_device;
  const int num_scs = S * global_device_count;
  const int bps = (batch_size_for_device + S - 1) / S;
  int64_t k = 0;
  for (int s = 0; s < S; ++s) {
    const int64_t before = k;
    for (int f = 0; f < n_features; ++f) {
      const RefFeature& ft = features[f];
      const int num_samples = static_cast<int>(ft.num_rows);
      const int per_split = num_samples / (local_device_count * S);
      const int start = (local_device_id * S + s) * per_split;
      const int end = std::min(num_samples, start + per_split);
      const int row_offset_per_slice = ft.row_offset / (global_device_count * S);
      const int row_offset = s * bps + row_offset_per_slice;
      ref_extract_slice(&ft, start, end, row_offset, ft.col_offset,
                        ft.col_shift, num_scs, combiner, rows, cols, gains, &k);
    }
    sc_sizes[s] = k - before;
  }
  return 0;
}

// SortAndGroupCooTensorsPerLocalDevice without minibatching
// (sort_and_group_coo_tensors_impl.h:196-311, :349-646). Input: per-SC
// extraction-order lists. Output: per-SC grouped lists packed SC after SC
// (g_sizes[s] entries each; capacity = input size), stats in the reference's
// per-device layout:
//   max_ids[NS], max_unique[NS]  (max over local SCs of per-partition counts)
//   required[S]                  (sum over partitions of roundup8(ids))
// Returns 0 on success, 2 when a limit is exceeded and dropping is not allowed
// (LOG(FATAL) in the reference, :45-89).
int ref_sort_and_group(int num_sc_per_device, const int64_t* sc_sizes,
                       const int32_t* rows, const int32_t* cols,
                       const float* gains, int has_variable_weights,
                       int num_scs, int max_ids_per_partition,
                       int max_unique_ids_per_partition, int allow_id_dropping,
                       int32_t* g_rows, int32_t* g_cols, float* g_gains,
                       int64_t* g_sizes, int32_t* max_ids, int32_t* max_unique,
                       int32_t* required_buffer_size, int64_t* dropped) {
  const int S = num_sc_per_device;
  const int NS = num_scs;
  const int num_sc_bits = Log2Exact(static_cast<uint32_t>(NS));
  for (int p = 0; p < NS; ++p) max_ids[p] = max_unique[p] = 0;
  for (int s = 0; s < S; ++s) required_buffer_size[s] = 0;
  int64_t total_dropped = 0;
  int status = 0;
  int64_t in_base = 0;
  int64_t out_base = 0;  // grouped lists are written packed, SC after SC
  for (int s = 0; s < S; ++s) {
    const int64_t n = sc_sizes[s];
    const int32_t* r = rows + in_base;
    const int32_t* c = cols + in_base;
    const float* g = gains + in_base;
    // Keys: data = extraction index (variable weights) or row id (unity).
    std::vector<uint64_t> keys(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t data = has_variable_weights ? static_cast<uint32_t>(i)
                                                 : static_cast<uint32_t>(r[i]);
      keys[i] = GroupingKey(static_cast<uint32_t>(c[i]), data, num_sc_bits);
    }
    // Unity weights: gain is a function of the row id alone; recover it from
    // any entry with the same row (all equal by construction).
    std::vector<float> row_gain;
    if (!has_variable_weights) {
      int32_t max_row = -1;
      for (int64_t i = 0; i < n; ++i) max_row = std::max(max_row, r[i]);
      row_gain.assign(static_cast<size_t>(max_row + 1), 1.0f);
      for (int64_t i = 0; i < n; ++i) row_gain[r[i]] = g[i];
    }
    // hwy::VQSort(ascending) on uint64 keys: equal keys are bit-identical,
    // so any correct sort gives the same sequence.
    std::sort(keys.begin(), keys.end());

    std::vector<int32_t> obs_ids(NS, 0), obs_unique(NS, 0), kept_ids(NS, 0),
        kept_unique(NS, 0);
    const uint32_t kNone = std::numeric_limits<uint32_t>::max();
    uint32_t prev_col = kNone, prev_row = kNone;
    uint32_t dedup_col = kNone, dedup_row = kNone;
    bool dropping_current_col = false;
    const bool perform_dropping = allow_id_dropping != 0;
    int64_t out = 0;
    int32_t* orow = g_rows + out_base;
    int32_t* ocol = g_cols + out_base;
    float* ogain = g_gains + out_base;
    for (int64_t i = 0; i < n; ++i) {
      const uint64_t key = keys[i];
      const uint32_t col = ref_col_id_from_key(key, num_sc_bits);
      const uint32_t p = col & static_cast<uint32_t>(NS - 1);
      uint32_t row;
      float gain;
      if (has_variable_weights) {
        const uint32_t idx = ref_data_from_key(key);
        row = static_cast<uint32_t>(r[idx]);
        gain = g[idx];
      } else {
        row = ref_data_from_key(key);
        gain = row_gain[row];
      }
      // Merge with the last kept entry (partitioned_coo_tensors.h:102-113).
      if (row == dedup_row && col == dedup_col) {
        ogain[out - 1] += gain;
        continue;
      }
      // A repeat of a dropped entry is dropped too.
      if (perform_dropping && row == prev_row && col == prev_col) {
        ++total_dropped;
        continue;
      }
      const bool is_new_col = col != prev_col;
      obs_ids[p] += 1;
      if (is_new_col) obs_unique[p] += 1;
      bool add = true;
      if (perform_dropping) {
        const bool exceeds = (kept_ids[p] + 1) > max_ids_per_partition;
        if (is_new_col) {
          dropping_current_col =
              (kept_unique[p] + 1) > max_unique_ids_per_partition;
        }
        if (exceeds || dropping_current_col) {
          ++total_dropped;
          add = false;
        }
        kept_ids[p] += 1;
        if (is_new_col) kept_unique[p] += 1;
      }
      if (add) {
        orow[out] = static_cast<int32_t>(row);
        ocol[out] = static_cast<int32_t>(col);
        ogain[out] = gain;
        ++out;
        dedup_col = col;
        dedup_row = row;
      }
      prev_col = col;
      prev_row = row;
    }
    g_sizes[s] = out;
    int32_t obs_max_ids = 0, obs_max_unique = 0;
    int64_t req = 0;
    for (int p = 0; p < NS; ++p) {
      max_ids[p] = std::max(max_ids[p], obs_ids[p]);
      max_unique[p] = std::max(max_unique[p], obs_unique[p]);
      obs_max_ids = std::max(obs_max_ids, obs_ids[p]);
      obs_max_unique = std::max(obs_max_unique, obs_unique[p]);
      req += RoundUp(obs_ids[p], kAlign);
    }
    required_buffer_size[s] = static_cast<int32_t>(req);
    if (!allow_id_dropping && (obs_max_ids > max_ids_per_partition ||
                               obs_max_unique > max_unique_ids_per_partition)) {
      status = 2;
    }
    in_base += n;
    out_base += out;
  }
  *dropped = total_dropped;
  return status;
}

// FillLocalDeviceBufferAsync / FillBufferSegment without minibatching
// (input_preprocessing_util.cc:73-208, :331-473). Writes one device's CSR
// buffers: rp[S * rp_per_sc], eid/sid/gains[coo_size]. Positions past each
// segment's final index are left untouched (the reference leaves them
// uninitialised). Returns the statically dropped count in *dropped.
int ref_fill_device(int num_sc_per_device, const int64_t* g_sizes,
                    const int32_t* g_rows, const int32_t* g_cols,
                    const float* g_gains, int num_scs, int batch_size_per_sc,
                    int64_t coo_size, int rp_per_sc, int32_t* rp,
                    int32_t* eid, int32_t* sid, float* gains,
                    int64_t* dropped) {
  const int S = num_sc_per_device;
  const int NS = num_scs;
  const int64_t per_sc = coo_size / S;
  const float kNan = std::nanf("");
  int64_t total_dropped = 0;
  int64_t in_base = 0;
  for (int s = 0; s < S; ++s) {
    const int64_t K = g_sizes[s];
    const int32_t* r = g_rows + in_base;
    const int32_t* c = g_cols + in_base;
    const float* g = g_gains + in_base;
    int64_t coo_begin = std::min<int64_t>(s * per_sc, coo_size);
    const int64_t coo_end = coo_begin + per_sc;
    int rp_index = s * rp_per_sc;
    const int rp_end = rp_index + rp_per_sc;
    int64_t coo = coo_begin;
    int cur_p = 0;
    int64_t processed = 0;
    auto valid = [&]() {
      if (processed == K && coo == coo_end) return true;
      if (rp_index >= rp_end || coo >= coo_end) return false;
      return true;
    };
    auto advance = [&](int target) {
      while (cur_p < target) {
        if (!valid()) return;
        rp[rp_index++] = static_cast<int32_t>(coo - coo_begin);
        while (coo % kAlign != 0 && coo < coo_end) {
          eid[coo] = INT_MAX;
          sid[coo] = INT_MAX;
          gains[coo] = kNan;
          ++coo;
        }
        ++cur_p;
      }
    };
    for (int64_t i = 0; i < K; ++i) {
      const int target = static_cast<int>(c[i] % NS);
      advance(target);
      if (!valid()) {
        total_dropped += K - processed;
        break;
      }
      eid[coo] = c[i] / NS;
      sid[coo] = r[i] % batch_size_per_sc;
      gains[coo] = g[i];
      ++coo;
      ++processed;
    }
    advance(NS);
    while (rp_index < rp_end) rp[rp_index++] = static_cast<int32_t>(coo - coo_begin);
    in_base += K;
  }
  *dropped = total_dropped;
  return 0;
}

// Full preprocessing of one stacked table for all local devices
// (input_preprocessing.cc:800-959 restricted to one stack, no minibatching).
// features must be in row_offset order. Outputs (leading dimension L):
//   rp[L * S * rp_per_sc], eid/sid/gains[L * coo_size_per_device],
//   max_ids/max_unique[L * NS], required[L * S], *dropped (all devices).
// Returns 0, 1 (invalid batch split), 2 (limit exceeded without dropping).
int ref_preprocess_stack(const RefFeature* features, int n_features,
                         int local_device_count, int global_device_count,
                         int num_sc_per_device, int combiner,
                         int has_variable_weights, int max_ids_per_partition,
                         int max_unique_ids_per_partition,
                         int allow_id_dropping, int64_t coo_size_per_device,
                         int32_t* rp, int32_t* eid, int32_t* sid,
                         float* gains, int32_t* max_ids, int32_t* max_unique,
                         int32_t* required, int64_t* dropped) {
  const int L = local_device_count;
  const int S = num_sc_per_device;
  const int NS = S * global_device_count;
  const int rp_per_sc = std::max(NS, kAlign);
  int64_t total_ids = 0;
  for (int f = 0; f < n_features; ++f) {
    total_ids += features[f].row_splits[features[f].num_rows];
  }
  std::vector<int32_t> rows(total_ids), cols(total_ids), grows(total_ids),
      gcols(total_ids);
  std::vector<float> gn(total_ids), ggn(total_ids);
  std::vector<int64_t> sizes(S), gsizes(S);
  int64_t all_dropped = 0;
  int status = 0;
  for (int d = 0; d < L; ++d) {
    int32_t bfd = 0;
    if (ref_extract_device(features, n_features, d, L, global_device_count, S,
                           combiner, rows.data(), cols.data(), gn.data(),
                           sizes.data(), &bfd) != 0) {
      return 1;
    }
    int64_t drop_group = 0, drop_fill = 0;
    const int st = ref_sort_and_group(
        S, sizes.data(), rows.data(), cols.data(), gn.data(),
        has_variable_weights, NS, max_ids_per_partition,
        max_unique_ids_per_partition, allow_id_dropping, grows.data(),
        gcols.data(), ggn.data(), gsizes.data(), max_ids + d * NS,
        max_unique + d * NS, required + d * S, &drop_group);
    if (st != 0) status = st;
    const int bps = (bfd + S - 1) / S;
    ref_fill_device(S, gsizes.data(), grows.data(), gcols.data(), ggn.data(),
                    NS, bps, coo_size_per_device, rp_per_sc,
                    rp + static_cast<int64_t>(d) * S * rp_per_sc,
                    eid + d * coo_size_per_device,
                    sid + d * coo_size_per_device,
                    gains + d * coo_size_per_device, &drop_fill);
    all_dropped += drop_group + drop_fill;
  }
  *dropped = all_dropped;
  return status;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Minibatching (enable_minibatching), single host: the first pass groups
// without buckets and decides whether a limit is exceeded; if so, a second
// pass groups by (bucket, column), the per-partition bucket counts give the
// split of the 64 buckets into minibatches, and the buckets of one minibatch
// are merged partition by partition before the CSR is written minibatch by
// minibatch (input_preprocessing.cc:800-959).
// ---------------------------------------------------------------------------

namespace {

// One local SparseCore's grouped entries in bucket order with the bucket
// offsets (PartitionedCooTensors, partitioned_coo_tensors.h:30-215).
struct ScGroups {
  std::vector<Coo> coos;
  std::vector<int> offsets;  // buckets + 1, minibatches + 1 after MergeAll
};

struct GroupOut {
  std::vector<int32_t> obs_ids;     // [NS * buckets]
  std::vector<int32_t> obs_unique;  // [NS * buckets]
  int64_t dropped = 0;
};

// GroupAndDeduplicateCooTensorsForLocalSparseCore with buckets
// (sort_and_group_coo_tensors_impl.h:196-311) for one SC's extraction-order
// list. The first minibatching pass (create_buckets false) never drops.
void GroupSc(const int32_t* r, const int32_t* c, const float* g, int64_t n,
             bool has_w, int NS, bool create_buckets, bool enable_minibatching,
             int max_ids, int max_unique, bool allow_dropping, ScGroups* out,
             GroupOut* go) {
  const int B = create_buckets ? kMaxBuckets : 1;
  const int nsb = Log2Exact(static_cast<uint32_t>(NS));
  std::vector<uint64_t> keys(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t data =
        has_w ? static_cast<uint32_t>(i) : static_cast<uint32_t>(r[i]);
    const uint64_t bucket = create_buckets ? BucketOf(c[i]) : 0;
    keys[i] = (bucket << kBucketIdOffset) |
              GroupingKey(static_cast<uint32_t>(c[i]), data, nsb);
  }
  std::vector<float> row_gain;
  if (!has_w) {
    int32_t max_row = -1;
    for (int64_t i = 0; i < n; ++i) max_row = std::max(max_row, r[i]);
    row_gain.assign(static_cast<size_t>(max_row + 1), 1.0f);
    for (int64_t i = 0; i < n; ++i) row_gain[r[i]] = g[i];
  }
  std::sort(keys.begin(), keys.end());
  go->obs_ids.assign(static_cast<size_t>(NS) * B, 0);
  go->obs_unique.assign(static_cast<size_t>(NS) * B, 0);
  std::vector<int32_t> kept_ids(static_cast<size_t>(NS) * B, 0),
      kept_unique(static_cast<size_t>(NS) * B, 0);
  const bool can_drop = !enable_minibatching || create_buckets;
  const bool perform_dropping = allow_dropping && can_drop;
  const uint32_t kNone = std::numeric_limits<uint32_t>::max();
  uint32_t prev_col = kNone, prev_row = kNone, prev_bucket = 0;
  uint32_t dedup_col = kNone, dedup_row = kNone;
  bool dropping_current_col = false;
  out->coos.clear();
  out->offsets.assign(1, 0);
  int cur_bucket = 0;
  auto advance_buckets = [&](int target) {
    while (cur_bucket < target) {
      out->offsets.push_back(static_cast<int>(out->coos.size()));
      ++cur_bucket;
    }
  };
  for (const uint64_t key : keys) {
    const uint32_t bucket =
        create_buckets ? static_cast<uint32_t>(key >> kBucketIdOffset) : 0;
    const uint32_t col = Rotl32(
        static_cast<uint32_t>(key >> kRotatedColIdOffset), nsb);
    const uint32_t p = col & static_cast<uint32_t>(NS - 1);
    const size_t cell = static_cast<size_t>(p) * B + bucket;
    uint32_t row;
    float gain;
    if (has_w) {
      const uint32_t idx = static_cast<uint32_t>(key) & kDataMask;
      row = static_cast<uint32_t>(r[idx]);
      gain = g[idx];
    } else {
      row = static_cast<uint32_t>(key) & kDataMask;
      gain = row_gain[row];
    }
    if (row == dedup_row && col == dedup_col) {  // MaybeMerge
      out->coos.back().gain += gain;
      continue;
    }
    if (perform_dropping && row == prev_row && col == prev_col) {
      ++go->dropped;
      continue;
    }
    bool is_new_col = col != prev_col;
    if (create_buckets) is_new_col = is_new_col || bucket != prev_bucket;
    go->obs_ids[cell] += 1;
    if (is_new_col) go->obs_unique[cell] += 1;
    bool add = true;
    if (perform_dropping) {
      const bool exceeds = (kept_ids[cell] + 1) > max_ids;
      if (is_new_col) {
        dropping_current_col = (kept_unique[cell] + 1) > max_unique;
      }
      if (exceeds || dropping_current_col) {
        ++go->dropped;
        add = false;
      }
      kept_ids[cell] += 1;
      if (is_new_col) kept_unique[cell] += 1;
    }
    if (add) {  // PartitionedCooTensors::Add
      advance_buckets(static_cast<int>(bucket));
      out->coos.push_back({static_cast<int32_t>(row), static_cast<int32_t>(col),
                           gain});
      dedup_col = col;
      dedup_row = row;
    }
    prev_col = col;
    prev_row = row;
    prev_bucket = bucket;
  }
  advance_buckets(B);  // FillRemainingScBuckets
}

// PartitionedCooTensors::Merge (partitioned_coo_tensors.h:157-215): for each
// tree node that is not split, the last unmerged bucket of its left subtree
// is merged with the first unmerged bucket of its right subtree, stably by
// partition (std::inplace_merge); then the offsets of the unmerged buckets
// become the minibatch offsets.
void MergeSc(uint64_t split, int NS, ScGroups* sg, int N = kMaxBuckets) {
  std::vector<bool> merged(N, false);
  std::vector<int>& off = sg->offsets;
  ForEachMerge(split, N, [&](int left, int right) {
    const int size = right - left;
    int i = right - 1, j = right;
    while (i > left && merged[i]) --i;
    while (j < right + size && merged[j]) ++j;
    const int pl = off[i], pr = off[j], pe = off[j + 1];
    std::inplace_merge(sg->coos.begin() + pl, sg->coos.begin() + pr,
                       sg->coos.begin() + pe,
                       [NS](const Coo& a, const Coo& b) {
                         return (a.col & (NS - 1)) < (b.col & (NS - 1));
                       });
    off[i + 1] = pl;
    off[j] = pl;
    merged[i] = true;
  });
  int mb = 0;
  for (int b = 0; b < N - 1; ++b) {
    if (!merged[b]) off[1 + mb++] = off[1 + b];
  }
  const int minibatches = mb + 1;
  off[minibatches] = off[N];
  off.resize(1 + minibatches);
}

// FillLocalDeviceBufferAsync + FillBufferSegment with minibatching
// (input_preprocessing_util.cc:135-143, :167-208, :331-473): segments are
// (SC, minibatch) in that order, each with its own rp_per_bucket row
// pointers; row pointers hold positions in the device buffer; every segment
// may use the whole buffer. One minibatch: SC s starts at the sum of the
// required buffer sizes of the SCs before it; several: each segment starts
// where the previous one ended.
int64_t FillMinibatchingDevice(const std::vector<ScGroups>& scs, int NS,
                               int bps, int64_t coo_size, int rp_per_bucket,
                               const int32_t* required, int32_t* rp,
                               int32_t* eid, int32_t* sid, float* gains) {
  const int S = static_cast<int>(scs.size());
  const int nmb = static_cast<int>(scs[0].offsets.size()) - 1;
  const float kNan = std::nanf("");
  int64_t dropped = 0;
  int64_t chained = 0;
  int64_t packed = 0;
  int rp_begin = 0;
  for (int s = 0; s < S; ++s) {
    for (int m = 0; m < nmb; ++m) {
      int64_t coo_begin;
      if (nmb == 1) {
        coo_begin = std::min(packed, coo_size);
        packed = std::min(packed + required[s], coo_size);
      } else {
        coo_begin = chained;
      }
      const int64_t coo_end = coo_size;
      const ScGroups& sg = scs[s];
      const int64_t b0 = sg.offsets[m], b1 = sg.offsets[m + 1];
      const int64_t K = b1 - b0;
      int rp_index = rp_begin;
      const int rp_end = rp_begin + rp_per_bucket;
      int64_t coo = coo_begin;
      int cur_p = 0;
      int64_t processed = 0;
      auto valid = [&]() {
        if (processed == K && coo == coo_end) return true;
        if (rp_index >= rp_end || coo >= coo_end) return false;
        return true;
      };
      auto advance = [&](int target) {
        while (cur_p < target) {
          if (!valid()) return;
          rp[rp_index++] = static_cast<int32_t>(coo);
          while (coo % kAlign != 0 && coo < coo_end) {
            eid[coo] = INT_MAX;
            sid[coo] = INT_MAX;
            gains[coo] = kNan;
            ++coo;
          }
          ++cur_p;
        }
      };
      for (int64_t i = b0; i < b1; ++i) {
        const Coo& x = sg.coos[i];
        advance(x.col % NS);
        if (!valid()) {
          dropped += K - processed;
          break;
        }
        eid[coo] = x.col / NS;
        sid[coo] = x.row % bps;
        gains[coo] = x.gain;
        ++coo;
        ++processed;
      }
      advance(NS);
      while (rp_index < rp_end) rp[rp_index++] = static_cast<int32_t>(coo);
      // PadCooBuffer(kAlignOnly) after each minibatch segment.
      while (coo % kAlign != 0 && coo < coo_size) {
        eid[coo] = INT_MAX;
        sid[coo] = INT_MAX;
        gains[coo] = kNan;
        ++coo;
      }
      chained = coo;
      rp_begin += rp_per_bucket;
    }
  }
  return dropped;
}

}  // namespace

extern "C" {

// Bucket of a column id (CooFormat::GetBucketId with the reference's
// HighwayHash, coo_format.h:140-145).
uint32_t ref_minibatching_bucket(int32_t col_id) { return BucketOf(col_id); }

// HighwayHash-64 of `size` bytes under `key`.
uint64_t ref_highway_hash64(const uint8_t* data, int64_t size,
                            const uint64_t* key) {
  return HighwayHash64(data, static_cast<size_t>(size), key);
}

// ComputeMinibatchingSplit<n> (n a power of two); `values` is modified as in
// the reference.
uint64_t ref_compute_minibatching_split(int32_t* values, int n,
                                        int max_value) {
  return ComputeSplit(values, n, max_value);
}

// MergeBuckets<n>: writes the merged (left, right) pairs to `pairs` (2 per
// merge, at most n - 1 merges) and returns their number.
int ref_merge_buckets(uint64_t split, int n, int32_t* pairs) {
  int k = 0;
  ForEachMerge(split, n, [&](int l, int r) {
    pairs[2 * k] = l;
    pairs[2 * k + 1] = r;
    ++k;
  });
  return k;
}

// PartitionedCooTensors::Merge<buckets> (buckets a power of two up to 64,
// `split` of buckets - 1 bits): bucket b holds the next sizes[b] entries of
// (rows, cols, gains). Writes the merged entries back and the minibatch
// offsets (minibatches + 1) to `offsets`; returns the number of
// minibatches.
int ref_merge_partitioned(int buckets, const int32_t* sizes, int32_t* rows,
                          int32_t* cols, float* gains, int num_scs,
                          uint64_t split, int32_t* offsets) {
  ScGroups sg;
  sg.offsets.assign(1, 0);
  int64_t total = 0;
  for (int b = 0; b < buckets; ++b) {
    total += sizes[b];
    sg.offsets.push_back(static_cast<int>(total));
  }
  for (int64_t i = 0; i < total; ++i) {
    sg.coos.push_back({rows[i], cols[i], gains[i]});
  }
  MergeSc(split, num_scs, &sg, buckets);
  for (int64_t i = 0; i < total; ++i) {
    rows[i] = sg.coos[i].row;
    cols[i] = sg.coos[i].col;
    gains[i] = sg.coos[i].gain;
  }
  const int nmb = static_cast<int>(sg.offsets.size()) - 1;
  for (int m = 0; m <= nmb; ++m) offsets[m] = sg.offsets[m];
  return nmb;
}

// One pass of minibatching preprocessing of one stacked table for all local
// devices (features in row_offset order, enable_minibatching true).
//   stage 0: first pass: group without buckets or drops, write the stats and
//            the one-minibatch CSR; *flag_or_split = 1 if some partition of
//            some SC exceeds a limit (minibatching required).
//   stage 1: bucket pass: *flag_or_split = the split, OR over SCs and
//            devices.
//   stage 2: bucket pass, merge by `split`, write the CSR of
//            popcount(split) + 1 minibatches.
// rp holds L * S * 64 * max(NS, 8) entries, of which the first
// S * minibatches * max(NS, 8) per device are written. *dropped: ids
// dropped by the pass (grouping and the static buffer). Returns 0, 1
// (invalid batch split) or 2 (stage 1/2: a bucket exceeds a limit and
// dropping is off; LOG(FATAL) in the reference).
int ref_preprocess_stack_minibatching(
    const RefFeature* features, int n_features, int local_device_count,
    int global_device_count, int num_sc_per_device, int combiner,
    int has_variable_weights, int max_ids_per_partition,
    int max_unique_ids_per_partition, int allow_id_dropping,
    int64_t coo_size_per_device, int stage, uint64_t split, int32_t* rp,
    int32_t* eid, int32_t* sid, float* gains, int32_t* max_ids,
    int32_t* max_unique, int32_t* required, int64_t* dropped,
    uint64_t* flag_or_split) {
  const int L = local_device_count;
  const int S = num_sc_per_device;
  const int NS = S * global_device_count;
  const int rpb = std::max(NS, kAlign);
  const bool buckets = stage != 0;
  int64_t total_ids = 0;
  for (int f = 0; f < n_features; ++f) {
    total_ids += features[f].row_splits[features[f].num_rows];
  }
  std::vector<int32_t> rows(total_ids), cols(total_ids);
  std::vector<float> gn(total_ids);
  std::vector<int64_t> sizes(S);
  int64_t all_dropped = 0;
  uint64_t acc = 0;
  int status = 0;
  for (int d = 0; d < L; ++d) {
    int32_t bfd = 0;
    if (ref_extract_device(features, n_features, d, L, global_device_count, S,
                           combiner, rows.data(), cols.data(), gn.data(),
                           sizes.data(), &bfd) != 0) {
      return 1;
    }
    std::vector<ScGroups> scs(S);
    std::vector<int32_t> req(S, 0);
    int64_t base = 0;
    for (int s = 0; s < S; ++s) {
      GroupOut go;
      GroupSc(rows.data() + base, cols.data() + base, gn.data() + base,
              sizes[s], has_variable_weights != 0, NS, buckets, true,
              max_ids_per_partition, max_unique_ids_per_partition,
              allow_id_dropping != 0, &scs[s], &go);
      base += sizes[s];
      all_dropped += go.dropped;
      const int B = buckets ? kMaxBuckets : 1;
      int32_t obs_max_ids = 0, obs_max_unique = 0;
      int64_t rq = 0;
      for (int p = 0; p < NS; ++p) {
        int32_t sum_ids = 0, sum_unique = 0;
        for (int b = 0; b < B; ++b) {
          const int32_t oi = go.obs_ids[static_cast<size_t>(p) * B + b];
          const int32_t ou = go.obs_unique[static_cast<size_t>(p) * B + b];
          sum_ids += oi;
          sum_unique += ou;
          obs_max_ids = std::max(obs_max_ids, oi);
          obs_max_unique = std::max(obs_max_unique, ou);
        }
        rq += RoundUp(sum_ids, kAlign);
        if (!buckets) {
          max_ids[d * NS + p] = std::max(s == 0 ? 0 : max_ids[d * NS + p], sum_ids);
          max_unique[d * NS + p] =
              std::max(s == 0 ? 0 : max_unique[d * NS + p], sum_unique);
        }
        if (buckets) {
          // UpdateMinibatchingSplit (sort_and_group_coo_tensors_impl.h:
          // 116-151) with the split type.
          acc |= ComputeSplit(go.obs_ids.data() + static_cast<size_t>(p) * B,
                              B, max_ids_per_partition);
          acc |= ComputeSplit(go.obs_unique.data() + static_cast<size_t>(p) * B,
                              B, max_unique_ids_per_partition);
        } else if (sum_ids > max_ids_per_partition ||
                   sum_unique > max_unique_ids_per_partition) {
          acc = 1;  // ... with the bool type
        }
      }
      req[s] = static_cast<int32_t>(rq);
      if (!buckets) required[d * S + s] = static_cast<int32_t>(rq);
      if (buckets && !allow_id_dropping &&
          (obs_max_ids > max_ids_per_partition ||
           obs_max_unique > max_unique_ids_per_partition)) {
        status = 2;  // ValidateMaxIdsOrDie
      }
    }
    if (stage == 1) continue;
    if (stage == 2) {
      for (auto& sg : scs) MergeSc(split, NS, &sg);
    }
    const int bps = (bfd + S - 1) / S;
    // The first pass's sizes place the SCs of the one-minibatch layout; the
    // second pass never uses them (its minibatches are chained).
    std::vector<int32_t> place(S);
    for (int s = 0; s < S; ++s) place[s] = stage == 0 ? req[s] : 0;
    all_dropped += FillMinibatchingDevice(
        scs, NS, bps, coo_size_per_device, rpb, place.data(),
        rp + static_cast<int64_t>(d) * S * kMaxBuckets * rpb,
        eid + d * coo_size_per_device, sid + d * coo_size_per_device,
        gains + d * coo_size_per_device);
  }
  *dropped = all_dropped;
  *flag_or_split = acc;
  return status;
}

// ComputeTheoreticalMaxCooBufferSize (input_preprocessing_util.cc:244-255):
// with minibatching every SC packs all its minibatches into one buffer, so
// the bound is 64 times larger.
int64_t ref_theoretical_max_coo_buffer_size_ex(int max_ids_per_partition,
                                               int global_device_count,
                                               int num_sc_per_device,
                                               int enable_minibatching) {
  const int64_t num_scs = int64_t{global_device_count} * num_sc_per_device;
  return RoundUp(max_ids_per_partition, kAlign) * num_sc_per_device * num_scs *
         (enable_minibatching ? kMaxBuckets : 1);
}

int64_t ref_theoretical_max_coo_buffer_size(int max_ids_per_partition,
                                            int global_device_count,
                                            int num_sc_per_device) {
  return ref_theoretical_max_coo_buffer_size_ex(
      max_ids_per_partition, global_device_count, num_sc_per_device, 0);
}

// ComputeCooBufferSizePerDevice (input_preprocessing_util.cc:256-312):
// returns -1 when the suggestion exceeds the theoretical maximum (CHECK).
int64_t ref_coo_buffer_size_per_device_ex(int max_ids_per_partition,
                                          int64_t suggested,
                                          int global_device_count,
                                          int num_sc_per_device,
                                          int enable_minibatching) {
  const int64_t theoretical = ref_theoretical_max_coo_buffer_size_ex(
      max_ids_per_partition, global_device_count, num_sc_per_device,
      enable_minibatching);
  if (suggested <= 0) return theoretical;
  const int64_t v = RoundUp(suggested, int64_t{kAlign} * num_sc_per_device);
  if (v > theoretical) return -1;
  return v;
}

int64_t ref_coo_buffer_size_per_device(int max_ids_per_partition,
                                       int64_t suggested, int global_device_count,
                                       int num_sc_per_device) {
  return ref_coo_buffer_size_per_device_ex(max_ids_per_partition, suggested,
                                           global_device_count,
                                           num_sc_per_device, 0);
}

// ---------------------------------------------------------------------------
// Lookup and update: the semantics the reference's tests hold the TPU ops to.
// For local SparseCore s and partition p, entries j in
// [roundup8(rp[p-1]) (0 for p = 0), rp[p]) of segment s contribute
//   act[s*bps + sid[j]] += gains[j] * T[p*(V/NS) + eid[j]].
// The gradient of a table row is the sum over all its entries of
// gains[j] * act_grad[s*bps + sid[j]]; the optimizer runs once per touched
// row. Work is split over threads by embedding column, so each thread sums in
// the same (CSR) order as a serial loop: results are deterministic and do not
// depend on the thread count.
// ---------------------------------------------------------------------------

}  // extern "C"

namespace {

struct CsrEntry {
  int64_t act_row;
  int64_t table_row;
  float gain;
};

// num_minibatches > 0: the minibatching layout (input_preprocessing_util.cc:
// 135-143, :331-473; input_preprocessing.py:243-284): segment s holds
// num_minibatches blocks of rp_per_segment row pointers, row pointers are
// positions in the whole buffer, and each partition starts at the aligned
// end of the one before it in buffer order (the first at 0).
std::vector<CsrEntry> CollectEntries(const int32_t* rp, const int32_t* eid,
                                     const int32_t* sid, const float* gains,
                                     int64_t coo_size, int num_segments,
                                     int num_partitions, int rp_per_segment,
                                     int num_minibatches, int64_t table_rows,
                                     int64_t batch) {
  std::vector<CsrEntry> out;
  const int64_t per_seg = coo_size / num_segments;
  const int64_t bps = batch / num_segments;
  const int64_t rows_per_partition = table_rows / num_partitions;
  if (num_minibatches > 0) {
    int64_t prev_end = 0;
    for (int s = 0; s < num_segments; ++s) {
      for (int m = 0; m < num_minibatches; ++m) {
        const int32_t* r =
            rp + (static_cast<int64_t>(s) * num_minibatches + m) *
                     rp_per_segment;
        for (int p = 0; p < num_partitions; ++p) {
          const int64_t start = RoundUp(prev_end, kAlign);
          const int64_t end = std::min<int64_t>(r[p], coo_size);
          for (int64_t j = start; j < end; ++j) {
            out.push_back({s * bps + sid[j], p * rows_per_partition + eid[j],
                           gains[j]});
          }
          prev_end = std::max(end, start);
        }
      }
    }
    return out;
  }
  for (int s = 0; s < num_segments; ++s) {
    const int32_t* r = rp + static_cast<int64_t>(s) * rp_per_segment;
    const int64_t base = s * per_seg;
    int64_t start = 0;
    for (int p = 0; p < num_partitions; ++p) {
      const int64_t end = r[p];
      for (int64_t j = start; j < end; ++j) {
        out.push_back({s * bps + sid[base + j],
                       p * rows_per_partition + eid[base + j],
                       gains[base + j]});
      }
      start = RoundUp(end, kAlign);
    }
  }
  return out;
}

template <typename Fn>
void ParallelColumns(int dim, int threads, Fn fn) {
  threads = std::max(1, std::min(threads, dim));
  if (threads == 1) {
    fn(0, dim);
    return;
  }
  std::vector<std::thread> pool;
  const int chunk = (dim + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const int lo = t * chunk;
    const int hi = std::min(dim, lo + chunk);
    if (lo >= hi) break;
    pool.emplace_back(fn, lo, hi);
  }
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

int ref_sparse_dense_matmul(const int32_t* rp, const int32_t* eid,
                            const int32_t* sid, const float* gains,
                            int64_t coo_size, int num_segments,
                            int num_partitions, int rp_per_segment,
                            int num_minibatches, const float* table,
                            int64_t table_rows, int dim, float* act,
                            int64_t batch, int threads) {
  const std::vector<CsrEntry> e = CollectEntries(
      rp, eid, sid, gains, coo_size, num_segments, num_partitions,
      rp_per_segment, num_minibatches, table_rows, batch);
  std::memset(act, 0, sizeof(float) * batch * dim);
  ParallelColumns(dim, threads, [&](int lo, int hi) {
    for (const CsrEntry& x : e) {
      const float* t = table + x.table_row * dim;
      float* a = act + x.act_row * dim;
      for (int d = lo; d < hi; ++d) a[d] += x.gain * t[d];
    }
  });
  return 0;
}

// Optimizer kinds (as SCEMB_OPTIMIZER_* of include/scemb.h).
enum {
  kSgd = 0,
  kAdagrad = 1,
  kAdam = 2,
  kAdagradMomentum = 3,
  kFtrl = 4,
  kLaprop = 5,
  kF2a = 6,
};

}  // extern "C"

namespace {

// One table value t with its summed gradient g and slot values s0, s1, for
// the hyperparameters h in the order of the reference primitive's operands;
// then clipping (primitives/utils.py:24-59). Each branch restates the
// reference's row-wise update body, operation by operation.
float ApplyUpdate(int kind, const float* h, int flags, float t, float* s0,
                  float* s1, float g, int clip_mask, float min_value,
                  float max_value) {
  float v;
  switch (kind) {
    case kSgd:  // optimizers_computation.py:22-69
      v = t - g * h[0];
      break;
    case kAdagrad: {  // sparse_dense_matmul_grad_with_adagrad.py:205-233
      const float acc = *s0 + g * g;
      *s0 = acc;
      v = t - (h[0] * g) / std::sqrt(acc);
      break;
    }
    case kAdam: {  // sparse_dense_matmul_grad_with_adam.py:283-338
      // h: alpha_t, beta_1, beta_2, epsilon_hat; slots momentum, velocity.
      const float grad_square = g * g;
      const float m = *s0 + (1.0f - h[1]) * (g - *s0);
      const float vel = *s1 + (1.0f - h[2]) * (grad_square - *s1);
      const float update = (h[0] * m) / (std::sqrt(vel) + h[3]);
      *s0 = m;
      *s1 = vel;
      v = t - update;
      break;
    }
    case kAdagradMomentum: {
      // sparse_dense_matmul_grad_with_adagrad_momentum.py:256-311
      // h: lr, momentum, beta2, epsilon, exponent, use_nesterov; slots
      // accumulator, momentum.
      const float grad_sq = g * g;
      const float accum_plus = *s0 + grad_sq;
      const float scaled_accum = h[2] * *s0 + (1.0f - h[2]) * grad_sq;
      const float a = h[2] == 1.0f ? accum_plus : scaled_accum;
      const float neg_inv_exp = -1.0f / h[4];
      const float p = std::pow(a + h[3], neg_inv_exp);
      const float scaled_grad = p * g;
      const float m = h[1] * *s1 + scaled_grad;
      const float nesterov_update = h[1] * m + scaled_grad;
      const float update = h[5] != 0.0f ? nesterov_update : m;
      *s0 = a;
      *s1 = m;
      v = t - h[0] * update;
      break;
    }
    case kFtrl: {  // sparse_dense_matmul_grad_with_ftrl.py:260-335
      // h: lr, lr_power, l1, l2, beta; slots accumulator, linear.
      const bool by_lr = (flags & 1) != 0;
      const float a = *s0 + g * g;
      const float neg_lr_pow = -h[1];
      const float p_old = std::pow(*s0, neg_lr_pow);
      const float p_new = std::pow(a, neg_lr_pow);
      const float delta_p = p_new - p_old;
      const float linear =
          by_lr ? (*s1 + h[0] * g) - delta_p * t
                : (*s1 + g) - (delta_p / h[0]) * t;
      const float scale = by_lr ? h[0] : 1.0f;
      const float l1_scaled = h[2] * scale;
      // stablehlo.clamp(min, x, max) = min(max(x, min), max)
      const float clamped = std::min(std::max(linear, -l1_scaled), l1_scaled);
      const float numerator = h[2] == 0.0f ? -linear : clamped - linear;
      const float denominator =
          by_lr ? (p_new + 2.0f * (h[0] * h[3])) + h[4]
                : (p_new + h[4]) / h[0] + 2.0f * h[3];
      *s0 = a;
      *s1 = linear;
      v = numerator / denominator;
      break;
    }
    case kLaprop: {  // sparse_dense_matmul_grad_with_laprop.py:282-340
      // h: lr, b1, decay_rate, eps; slots mu, nu.
      const float grad_square = g * g + h[3];
      const float nu = *s1 * h[2] + (1.0f - h[2]) * grad_square;
      const float update = g / std::sqrt(nu);
      const float term_2 = std::pow(1.0f - std::pow(h[1], 2.0f), 0.5f);
      const float u = h[1] * *s0 + term_2 * update;
      *s0 = u;
      *s1 = nu;
      v = t - h[0] * u;
      break;
    }
    default: {  // kF2a: sparse_dense_matmul_grad_with_f2a.py:244-290
      // h: lr, rho, l1, l2, max_lr_multiplier, global_step; slots
      // accumulator, local_step.
      const float local_step = *s1 + 1.0f;
      const float safe_global_step = std::max(h[5], 1.0f);
      const float frequency_ratio = safe_global_step / local_step;
      const float fa =
          std::min(std::pow(frequency_ratio, h[1]), h[4]);
      const float a = *s0 + g * g;
      const float denominator = std::sqrt(a);
      // stablehlo.sign: -1, +1, or the value itself for +-0 and NaN.
      const float sign = t > 0.0f ? 1.0f : (t < 0.0f ? -1.0f : t);
      const float l1_decay = h[2] * sign;
      const float l2_shrinkage = h[3] * t;
      const float grad_scaled = (g * fa) / denominator;
      const float update_sum = grad_scaled + (l1_decay + l2_shrinkage);
      *s0 = a;
      *s1 = local_step;
      v = t - h[0] * update_sum;
      break;
    }
  }
  if (clip_mask & 1) v = std::max(min_value, v);
  if (clip_mask & 2) v = std::min(max_value, v);
  return v;
}

}  // namespace

extern "C" {

// Backward + optimizer `kind` (kSgd ...). slot0 / slot1: the optimizer's
// slot variables (null when it has fewer), hp: its hyperparameters. flags
// bit 0: FTRL's multiply_linear_by_learning_rate. clip_mask bit 0: min,
// bit 1: max.
int ref_sparse_dense_matmul_grad_optimizer(
    const int32_t* rp, const int32_t* eid, const int32_t* sid,
    const float* gains, int64_t coo_size, int num_segments,
    int num_partitions, int rp_per_segment, int num_minibatches,
    const float* act_grad, int64_t batch, float* table, float* slot0,
    float* slot1, int64_t table_rows, int dim, int kind, const float* hp,
    int flags, int clip_mask, float min_value, float max_value, int threads) {
  const std::vector<CsrEntry> e = CollectEntries(
      rp, eid, sid, gains, coo_size, num_segments, num_partitions,
      rp_per_segment, num_minibatches, table_rows, batch);
  // Dense slot per touched row, assigned in first-touch order.
  std::vector<int64_t> touched;
  std::vector<int64_t> slot_of(e.size());
  {
    std::vector<std::pair<int64_t, int64_t>> order(e.size());
    for (size_t i = 0; i < e.size(); ++i) order[i] = {e[i].table_row, (int64_t)i};
    std::sort(order.begin(), order.end());
    for (size_t i = 0; i < order.size(); ++i) {
      if (i == 0 || order[i].first != order[i - 1].first) {
        touched.push_back(order[i].first);
      }
      slot_of[order[i].second] = static_cast<int64_t>(touched.size()) - 1;
    }
  }
  std::vector<float> grad(touched.size() * static_cast<size_t>(dim), 0.0f);
  ParallelColumns(dim, threads, [&](int lo, int hi) {
    for (size_t i = 0; i < e.size(); ++i) {
      const float* gr = act_grad + e[i].act_row * dim;
      float* gs = grad.data() + slot_of[i] * dim;
      for (int d = lo; d < hi; ++d) gs[d] += e[i].gain * gr[d];
    }
    float unused0 = 0.0f, unused1 = 0.0f;
    for (size_t u = 0; u < touched.size(); ++u) {
      const int64_t off = touched[u] * dim;
      const float* g = grad.data() + u * dim;
      for (int d = lo; d < hi; ++d) {
        float* a = slot0 ? slot0 + off + d : &unused0;
        float* b = slot1 ? slot1 + off + d : &unused1;
        table[off + d] = ApplyUpdate(kind, hp, flags, table[off + d], a, b,
                                     g[d], clip_mask, min_value, max_value);
      }
    }
  });
  return 0;
}

// optimizer: 0 = SGD, 1 = Adagrad (accumulator). clip_mask bit0: min,
// bit1: max.
int ref_sparse_dense_matmul_grad(const int32_t* rp, const int32_t* eid,
                                 const int32_t* sid, const float* gains,
                                 int64_t coo_size, int num_segments,
                                 int num_partitions, int rp_per_segment,
                                 int num_minibatches, const float* act_grad,
                                 int64_t batch, float* table,
                                 float* accumulator, int64_t table_rows,
                                 int dim, int optimizer, float learning_rate,
                                 int clip_mask, float min_value,
                                 float max_value, int threads) {
  const float hp[1] = {learning_rate};
  return ref_sparse_dense_matmul_grad_optimizer(
      rp, eid, sid, gains, coo_size, num_segments, num_partitions,
      rp_per_segment, num_minibatches, act_grad, batch, table,
      optimizer == kSgd ? nullptr : accumulator, nullptr, table_rows, dim,
      optimizer == kSgd ? kSgd : kAdagrad, hp, 0, clip_mask, min_value,
      max_value, threads);
}

}  // extern "C"
