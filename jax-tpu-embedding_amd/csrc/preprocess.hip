// GPU preprocessing of one stacked table: the reference's
// PreprocessSparseDenseMatmulInput (jax_tpu_embedding/sparsecore/lib/core/
// input_preprocessing.cc:800-959), bit-exact, including single-host
// minibatching as one call per pass:
//   pass 0   the first pass (no buckets, nothing dropped): stats, the CSR of
//            one minibatch, and whether a partition exceeds a limit
//   pass 1   the bucket pass: keys carry the column's HighwayHash bucket
//            (coo_format.h:140-185); per (SC, partition) the bucket counts
//            give the split of the 64-bucket tree
//            (sort_and_group_coo_tensors_impl.h:116-151)
//   pass 2   the bucket pass again, written as the minibatches of the
//            split that every stack's pass 1 OR-ed together
//            (partitioned_coo_tensors.h:157-215,
//            input_preprocessing_util.cc:331-473)
//
// Stages (segment g = local_device * S + local_sc):
//   plan      (host)  split-then-stack slices, input_preprocessing.cc:312-436
//   extract           per weighted row its combiner divisor (one thread per
//                     row, sequential float sums); then one thread per id:
//                     sample id, column id (coo_format.h:120-135), combiner
//                     gain (process_coo_tensors_impl.h:39-136), sort key
//                     (segment, partition, local id) = rotr32(col, log2 NS)
//   sort              stable LSD radix sort of (key, extraction index). The
//                     reference sorts 64-bit keys whose low field is the row
//                     id (unity weights) or the extraction index (weighted);
//                     a stable sort on the column field alone gives the same
//                     order whenever rows are non-decreasing in extraction
//                     order, which the planner checks; otherwise row digits
//                     are sorted first.
//   group             the sequential grouping loop of
//                     sort_and_group_coo_tensors_impl.h:196-311 restated as
//                     scans: run starts (new (col,row)), column starts,
//                     per-partition ordinals -> keep/drop, merged gains
//                     summed in sorted order.
//   fill              FillBufferSegment (input_preprocessing_util.cc:167-208)
//                     replayed per segment over partition counts (row
//                     pointers, alignment padding, static-buffer drops), then
//                     a scatter of the kept runs.
#include <algorithm>
#include <cstring>
#include <memory>
#include <vector>

#include "../../include/scemb.h"
#include "common.h"
#include "radix.h"
#include "scan.h"

namespace scemb {

// The longest row (returned) and the shortest (*least, at most 0) of host
// row splits [num_rows + 1]; the second also copies them to dst
// (rowsplits.cc).
int64_t RowLengthRange(const int64_t* sp, int64_t num_rows, int64_t* least);
int64_t CopyRowLengthRange(const int64_t* sp, int64_t num_rows, int64_t* dst,
                           int64_t* least);

namespace {

constexpr uint32_t kDataMask26 = (1u << 26) - 1;
// Sample-view slot of an extraction position that starts no written run.
constexpr uint64_t kNoEntry = ~0ull;  // table rows stay below 2^32 - 1
// int64 counters after the stats: dropped ids, limit exceeded, bad ids,
// grouped entries, minibatching required (pass 0), minibatching split
// (pass 1).
constexpr int kNumCounters = 6;

struct SliceDesc {
  int64_t id_begin;
  int64_t out_begin;
  int64_t row_start;
  int64_t row_prefix;
  int32_t num_rows;
  int32_t sample_base;
  int32_t feature;
  int32_t segment;
};

struct FeatureDev {
  const int32_t* ids;
  const float* weights;
  const int64_t* splits;
  int64_t valency;
  int32_t col_offset;
  int32_t col_shift;
};
static_assert(sizeof(SliceDesc) % 4 == 0 && sizeof(FeatureDev) % 4 == 0,
              "descriptors are uploaded as 32-bit words");

struct KeyLayout {
  int log2ns;
  int32_t ns_mask;
  bool compact;     // (p, local) packed in local_bits + log2ns bits
  int local_bits;   // compact: bits of the local id
  int col_bits;     // bits of the column part of the key
  int seg_bits;
  int mb_bits;      // bucket bits between segment and column (0 or 6)
  int64_t col_bound;
};

// ---------------------------------------------------------------------------
// Minibatching bucket of a column id: HighwayHash-64 of the id's 4 bytes
// under the reference's fixed key, modulo 64 (coo_format.h:31-49, :140-145).
// HighwayHash (google/highwayhash): four 64-bit lanes each of v0, v1, mul0,
// mul1; a 4-byte input is one remainder packet (length folded into v0, the
// 32-bit halves of v1 rotated by the length, the bytes at the packet's
// start), then four permute-and-update rounds.
// ---------------------------------------------------------------------------

struct HhLanes {
  uint64_t v0[4], v1[4], mul0[4], mul1[4];
};

__device__ __forceinline__ void HhZipperAdd(uint64_t v1, uint64_t v0,
                                            uint64_t& add1, uint64_t& add0) {
  add0 += (((v0 & 0xff000000ull) | (v1 & 0xff00000000ull)) >> 24) |
          (((v0 & 0xff0000000000ull) | (v1 & 0xff000000000000ull)) >> 16) |
          (v0 & 0xff0000ull) | ((v0 & 0xff00ull) << 32) |
          ((v1 & 0xff00000000000000ull) >> 8) | (v0 << 56);
  add1 += (((v1 & 0xff000000ull) | (v0 & 0xff00000000ull)) >> 24) |
          (v1 & 0xff0000ull) | ((v1 & 0xff0000000000ull) >> 16) |
          ((v1 & 0xff00ull) << 24) | ((v0 & 0xff000000000000ull) >> 8) |
          ((v1 & 0xffull) << 48) | (v0 & 0xff00000000000000ull);
}

__device__ __forceinline__ void HhRound(HhLanes& h, const uint64_t (&in)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h.v1[i] += h.mul0[i] + in[i];
    h.mul0[i] ^= (h.v1[i] & 0xffffffffull) * (h.v0[i] >> 32);
    h.v0[i] += h.mul1[i];
    h.mul1[i] ^= (h.v0[i] & 0xffffffffull) * (h.v1[i] >> 32);
  }
  HhZipperAdd(h.v1[1], h.v1[0], h.v0[1], h.v0[0]);
  HhZipperAdd(h.v1[3], h.v1[2], h.v0[3], h.v0[2]);
  HhZipperAdd(h.v0[1], h.v0[0], h.v1[1], h.v1[0]);
  HhZipperAdd(h.v0[3], h.v0[2], h.v1[3], h.v1[2]);
}

__device__ __forceinline__ uint32_t MinibatchingBucket(uint32_t col) {
  constexpr uint64_t kKey[4] = {0x4451e30f87db9609ull, 0xca7358a1fd2737f8ull,
                                0x4b2c991fcee4fdeaull, 0x0b2658e18326f6baull};
  constexpr uint64_t kInit0[4] = {0xdbe6d5d5fe4cce2full, 0xa4093822299f31d0ull,
                                  0x13198a2e03707344ull, 0x243f6a8885a308d3ull};
  constexpr uint64_t kInit1[4] = {0x3bd39e10cb0ef593ull, 0xc0acf169b5f18a8cull,
                                  0xbe5466cf34e90c6cull, 0x452821e638d01377ull};
  HhLanes h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h.mul0[i] = kInit0[i];
    h.mul1[i] = kInit1[i];
    h.v0[i] = kInit0[i] ^ kKey[i];
    h.v1[i] = kInit1[i] ^ ((kKey[i] >> 32) | (kKey[i] << 32));
    // Remainder of 4 bytes.
    h.v0[i] += (uint64_t{4} << 32) + 4;
    const uint32_t lo = static_cast<uint32_t>(h.v1[i]);
    const uint32_t hi = static_cast<uint32_t>(h.v1[i] >> 32);
    h.v1[i] = static_cast<uint64_t>((lo << 4) | (lo >> 28)) |
              (static_cast<uint64_t>((hi << 4) | (hi >> 28)) << 32);
  }
  uint64_t packet[4] = {static_cast<uint64_t>(col), 0, 0, 0};
  HhRound(h, packet);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t perm[4] = {(h.v0[2] >> 32) | (h.v0[2] << 32),
                              (h.v0[3] >> 32) | (h.v0[3] << 32),
                              (h.v0[0] >> 32) | (h.v0[0] << 32),
                              (h.v0[1] >> 32) | (h.v0[1] << 32)};
    HhRound(h, perm);
  }
  return static_cast<uint32_t>((h.v0[0] + h.v1[0] + h.mul0[0] + h.mul1[0]) &
                               (kMaxMinibatches - 1));
}

__device__ __forceinline__ uint32_t Rotr32(uint32_t x, int s) {
  return s == 0 ? x : ((x >> s) | (x << (32 - s)));
}
__device__ __forceinline__ uint32_t Rotl32(uint32_t x, int s) {
  return s == 0 ? x : ((x << s) | (x >> (32 - s)));
}

template <typename K>
__device__ __forceinline__ K ColKey(uint32_t col, const KeyLayout& kl) {
  if (kl.compact) {
    const uint32_t p = col & static_cast<uint32_t>(kl.ns_mask);
    const uint32_t local = col >> kl.log2ns;
    return (static_cast<K>(p) << kl.local_bits) | static_cast<K>(local);
  }
  return static_cast<K>(Rotr32(col, kl.log2ns));
}

// Partition and local id from the column part of a key.
template <typename K>
__device__ __forceinline__ void DecodeCol(K ck, const KeyLayout& kl,
                                          uint32_t* p, uint32_t* local) {
  if (kl.compact) {
    *p = static_cast<uint32_t>(ck >> kl.local_bits);
    *local = static_cast<uint32_t>(ck) &
             ((kl.local_bits >= 32) ? 0xffffffffu : ((1u << kl.local_bits) - 1u));
  } else {
    const uint32_t col = Rotl32(static_cast<uint32_t>(ck), kl.log2ns);
    *p = col & static_cast<uint32_t>(kl.ns_mask);
    *local = col >> kl.log2ns;
  }
}

template <typename K>
__device__ __forceinline__ K SentinelKey() {
  return ~K(0);
}

// Index of the last slice whose outputs (or rows, with by_rows) start at or
// before `pos`; slices are in output order and both offsets are
// non-decreasing.
__device__ __forceinline__ int FindSlice(const SliceDesc* slices,
                                         int num_slices, int64_t pos,
                                         bool by_rows) {
  int lo = 0, hi = num_slices - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    const int64_t start =
        by_rows ? slices[mid].row_prefix : slices[mid].out_begin;
    if (start <= pos) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Combiner divisor of every input row with weights (ComputeWeightDivisor,
// process_coo_tensors_impl.h:60-74): the weights summed in id order in
// float (mean), or the square root of the float sum of double squares
// (sqrtn). One thread per row: the sums are sequential, as in the reference.
// (One wavefront per row, with the weights loaded 64 at a time and added
// from lane broadcasts, measured 2.3x slower at c3: it serialises what 64
// rows per wavefront do side by side.)
__global__ __launch_bounds__(256) void RowDivisors(
    const SliceDesc* slices, int num_slices, const FeatureDev* feats,
    int64_t total_rows, int combiner, float* divisor) {
  const int64_t gr = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gr >= total_rows) return;
  const SliceDesc sl = slices[FindSlice(slices, num_slices, gr, true)];
  const FeatureDev f = feats[sl.feature];
  const int64_t r = sl.row_start + (gr - sl.row_prefix);
  const int64_t b = f.splits != nullptr ? f.splits[r] : r * f.valency;
  const int64_t e = f.splits != nullptr ? f.splits[r + 1] : b + f.valency;
  float s = 0.0f;
  if (combiner == 1) {
    for (int64_t k = b; k < e; ++k) s = s + f.weights[k];
    divisor[gr] = s;
  } else {
    for (int64_t k = b; k < e; ++k) {
      const double w = static_cast<double>(f.weights[k]);
      s = static_cast<float>(static_cast<double>(s) + w * w);
    }
    divisor[gr] = sqrtf(s);
  }
}

// Last row r in [lo, hi] with splits[r] <= target (splits[lo] <= target).
// With empty rows several rows share a start; the last of them is the
// non-empty row holding position `target`.
__device__ __forceinline__ int64_t LastRowAtOrBefore(const int64_t* splits,
                                                     int64_t lo, int64_t hi,
                                                     int64_t target) {
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (splits[mid] <= target) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The same over 32-bit staged offsets (rows [0, hi]).
__device__ __forceinline__ int LastRowAtOrBefore32(const int32_t* splits,
                                                   int hi, int32_t target) {
  int lo = 0;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (splits[mid] <= target) lo = mid; else hi = mid - 1;
  }
  return lo;
}

constexpr int kExtractBlock = 256;
constexpr int kExtractStagedSplits = 2 * kExtractBlock + 2;

// Where an ExtractIds block reads from: the slice holding both its first and
// last output positions (-1 when they lie in different slices) and, for a
// ragged feature, the input rows of those two positions.
struct BlockRows {
  int32_t slice;
  int32_t pad;
  int64_t lo;
  int64_t hi;
};

// Where an extraction block reads from, found for all blocks at once before
// the extraction (so that an extraction thread only searches the few rows
// its block spans), without any search over the row splits:
//   - the thread of block b writes its slice, or -1 when its first and last
//     output positions lie in different slices (BlockSliceOf);
//   - the thread of input row r of a ragged slice writes r as `lo` of every
//     block whose first position the row covers and as `hi` of every block
//     whose last position it covers (RowBlockBounds).
// Each output position of a ragged slice lies in exactly one non-empty row,
// so every single-slice block of a ragged slice gets both rows from the
// rows' own two splits. The extraction clamps them into the slice's rows
// (ClampBlockRows), so that rows written for other input keep its reads in
// range.
__device__ __forceinline__ void BlockSliceOf(const SliceDesc* slices,
                                             int num_slices,
                                             int64_t total_ids, int64_t blk,
                                             BlockRows* out) {
  const int64_t first = blk * kExtractBlock;
  const int64_t last = min(first + kExtractBlock, total_ids) - 1;
  const int sf = FindSlice(slices, num_slices, first, false);
  out[blk].slice = sf == FindSlice(slices, num_slices, last, false) ? sf : -1;
}

__device__ __forceinline__ void RowBlockBounds(const SliceDesc* slices,
                                               int num_slices,
                                               const FeatureDev* feats,
                                               int64_t total_ids, int64_t gr,
                                               BlockRows* out) {
  const int s = FindSlice(slices, num_slices, gr, true);
  const SliceDesc sl = slices[s];
  const int64_t* splits = feats[sl.feature].splits;
  if (splits == nullptr) return;
  const int64_t r = sl.row_start + (gr - sl.row_prefix);
  const int64_t out_end =
      s + 1 < num_slices ? slices[s + 1].out_begin : total_ids;
  const int64_t a = max(sl.out_begin + (splits[r] - sl.id_begin),
                        sl.out_begin);
  const int64_t e = min(sl.out_begin + (splits[r + 1] - sl.id_begin),
                        out_end);
  for (int64_t blk = a / kExtractBlock; blk * kExtractBlock < e; ++blk) {
    const int64_t first = blk * kExtractBlock;
    const int64_t last = min(first + kExtractBlock, total_ids) - 1;
    if (first >= a) out[blk].lo = r;
    if (last >= a && last < e) out[blk].hi = r;
  }
}

// The rows [*lo, *hi] of a single-slice block, clamped into its slice.
__device__ __forceinline__ void ClampBlockRows(const BlockRows& br,
                                               const SliceDesc& sl,
                                               int64_t* lo, int64_t* hi) {
  const int64_t top = sl.row_start + sl.num_rows - 1;
  *lo = min(max(br.lo, sl.row_start), top);
  *hi = min(max(br.hi, *lo), top);
}

// BlockSliceOf for blocks [0, num_blocks), RowBlockBounds for rows
// [0, total_rows).
__global__ __launch_bounds__(256) void BlockBounds(const SliceDesc* slices,
                                                   int num_slices,
                                                   const FeatureDev* feats,
                                                   int64_t total_ids,
                                                   int64_t num_blocks,
                                                   int64_t total_rows,
                                                   BlockRows* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < num_blocks) BlockSliceOf(slices, num_slices, total_ids, i, out);
  if (i < total_rows) {
    RowBlockBounds(slices, num_slices, feats, total_ids, i, out);
  }
}

// One thread per extracted id (output position o, in slice order): finds its
// slice and input row, then writes the sort key (segment, column) -- or the
// sentinel for an id outside the table --, the extraction index, the sample
// id and gain packed into one word (sample in the low half), and, for the
// optional row pass, the row key. Consecutive threads write consecutive
// positions. Gains: unit weights give 1, 1/n or 1/sqrt(n) for a row of n
// ids (process_coo_tensors_impl.h:39-56); weights are divided by the row's
// divisor (RowDivisors; 1 for sum).
template <typename K>
__global__ __launch_bounds__(kExtractBlock) void ExtractIds(
    const SliceDesc* slices, int num_slices, const FeatureDev* feats,
    const BlockRows* block_rows, int64_t total_ids, int combiner,
    int has_weights, const float* divisor, KeyLayout kl, K* keys,
    uint32_t* vals, uint64_t* row_gain, uint32_t* row_keys,
    int row_key_bits_seg_shift, int64_t* counters) {
  // The row splits a block spans ([lo, hi + 1] of one ragged feature),
  // staged in LDS when they fit, so that each id finds its row there.
  __shared__ int64_t s_splits[kExtractStagedSplits];
  const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const BlockRows br = block_rows[blockIdx.x];
  const int block_slice = br.slice;
  int64_t row_lo = 0, row_hi = -1;
  bool staged = false;
  if (block_slice >= 0) {  // uniform over the block
    ClampBlockRows(br, slices[block_slice], &row_lo, &row_hi);
    const int64_t* sp = feats[slices[block_slice].feature].splits;
    const int64_t cnt = row_hi - row_lo + 2;
    if (sp != nullptr && cnt <= kExtractStagedSplits) {
      for (int64_t i = threadIdx.x; i < cnt; i += blockDim.x) {
        s_splits[i] = sp[row_lo + i];
      }
      staged = true;
    }
  }
  __syncthreads();
  bool bad = false;
  if (o < total_ids) {
    const int si = block_slice >= 0 ? block_slice
                                    : FindSlice(slices, num_slices, o, false);
    const SliceDesc sl = slices[si];
    const FeatureDev f = feats[sl.feature];
    const int64_t p = sl.id_begin + (o - sl.out_begin);  // input position
    int64_t r, b, e;
    if (staged) {
      const int64_t k = LastRowAtOrBefore(s_splits, 0, row_hi - row_lo, p);
      r = row_lo + k;
      b = s_splits[k];
      e = s_splits[k + 1];
    } else if (f.splits != nullptr) {
      // Last row of the slice starting at or before p.
      int64_t lo = sl.row_start, hi = sl.row_start + sl.num_rows - 1;
      if (block_slice >= 0) {
        lo = row_lo;
        hi = row_hi;
      }
      r = LastRowAtOrBefore(f.splits, lo, hi, p);
      b = f.splits[r];
      e = f.splits[r + 1];
    } else {
      r = p / f.valency;
      b = r * f.valency;
      e = b + f.valency;
    }
    const int64_t local_row = r - sl.row_start;
    const uint32_t sample = static_cast<uint32_t>(sl.sample_base + local_row);
    float gain = 1.0f;
    if (has_weights) {
      gain = f.weights[p] /
             (combiner == 0 ? 1.0f : divisor[sl.row_prefix + local_row]);
    } else if (combiner == 1) {
      gain = 1.0f / static_cast<float>(static_cast<int>(e - b));
    } else if (combiner == 2) {
      gain = 1.0f / sqrtf(static_cast<float>(static_cast<int>(e - b)));
    }
    const int32_t id = f.ids[p];
    // GetColId: ((id + shift) & mask) + (id & ~mask) + offset.
    const int32_t col = ((id + f.col_shift) & kl.ns_mask) + (id & ~kl.ns_mask) +
                        f.col_offset;
    const bool ok = id >= 0 && col >= 0 &&
                    (kl.col_bound <= 0 || static_cast<int64_t>(col) < kl.col_bound);
    K vseg = static_cast<K>(sl.segment);
    if (kl.mb_bits > 0) {
      vseg = (vseg << kl.mb_bits) |
             static_cast<K>(MinibatchingBucket(static_cast<uint32_t>(col)));
    }
    const K seg_part = vseg << kl.col_bits;
    keys[o] = ok ? (seg_part | ColKey<K>(static_cast<uint32_t>(col), kl))
                 : SentinelKey<K>();
    vals[o] = static_cast<uint32_t>(o);
    row_gain[o] = static_cast<uint64_t>(sample) |
                  (static_cast<uint64_t>(__float_as_uint(gain)) << 32);
    if (row_keys != nullptr) {
      row_keys[o] = (static_cast<uint32_t>(sl.segment) << row_key_bits_seg_shift) |
                    sample;
    }
    bad = !ok;
  }
  const uint64_t m = __ballot(bad);
  if (m != 0 && (threadIdx.x % kWave) == 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(&counters[2]),
              static_cast<unsigned long long>(__popcll(m)));
  }
}

template <typename K>
__global__ void GatherKeys(const K* keys, const uint32_t* idx, int64_t n,
                           K* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = keys[idx[i]];
}

__global__ void FillI32(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Flags and partition boundaries over the sorted sequence. Each element's
// row and gain are gathered once, as one packed word (sidx); the previous
// element's row comes from the neighbouring thread through LDS (from memory
// at block starts).
template <typename K>
__global__ __launch_bounds__(256) void GroupFlags(
    const K* skeys, const uint32_t* sidx, const uint64_t* row_gain, int64_t n,
    KeyLayout kl, int num_partitions, uint32_t* srows, float* sgains,
    uint64_t* flags, int32_t* part_first, int32_t* part_last,
    uint64_t* view_entry) {
  __shared__ uint32_t s_row[256];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  // The sample view's slots (when built) start empty; ScatterRuns fills the
  // ones where a written run starts.
  if (view_entry != nullptr && i < n) view_entry[i] = kNoEntry;
  const K key = i < n ? skeys[i] : SentinelKey<K>();
  const bool valid = key != SentinelKey<K>();
  uint32_t row = 0;
  if (valid) {
    const uint64_t rg = row_gain[sidx[i]];
    row = static_cast<uint32_t>(rg);
    srows[i] = row;
    sgains[i] = __uint_as_float(static_cast<uint32_t>(rg >> 32));
  }
  s_row[threadIdx.x] = row;
  __syncthreads();
  if (i >= n) return;
  uint64_t f = 0;
  if (valid) {
    const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
    uint32_t p, local;
    DecodeCol<K>(key & col_mask, kl, &p, &local);
    const int64_t seg = static_cast<int64_t>(key >> kl.col_bits);
    const int64_t bucket = seg * num_partitions + p;
    bool new_col = true, new_run = true, new_bucket = true;
    if (i > 0) {
      const K pk = skeys[i - 1];
      if (pk == key) {
        new_col = false;
        new_bucket = false;
        // Same key, so element i - 1 is valid and its row was loaded.
        const uint32_t prev_row =
            threadIdx.x > 0 ? s_row[threadIdx.x - 1]
                            : static_cast<uint32_t>(row_gain[sidx[i - 1]]);
        new_run = prev_row != row;
      } else {
        uint32_t pp, pl;
        DecodeCol<K>(pk & col_mask, kl, &pp, &pl);
        new_bucket = static_cast<int64_t>(pk >> kl.col_bits) != seg || pp != p;
      }
    }
    f = (new_run ? 1ull : 0ull) | ((new_col ? 1ull : 0ull) << 32);
    if (new_bucket) part_first[bucket] = static_cast<int32_t>(i);
    bool last = i + 1 == n;
    if (!last) {
      const K nk = skeys[i + 1];
      if (nk == SentinelKey<K>()) {
        last = true;
      } else if (nk != key) {
        uint32_t np, nl;
        DecodeCol<K>(nk & col_mask, kl, &np, &nl);
        last = static_cast<int64_t>(nk >> kl.col_bits) != seg || np != p;
      }
    }
    if (last) part_last[bucket] = static_cast<int32_t>(i);
  }
  flags[i] = f;
}

// run_pos[r] = sorted position where run r starts; run_pos[R] = end.
template <typename K>
__global__ __launch_bounds__(256) void RunPositions(const K* skeys,
                                                    const uint64_t* flags,
                                                    const uint64_t* scan,
                                                    int64_t n,
                                                    uint32_t* run_pos) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t f = flags[i];
  const uint32_t r = static_cast<uint32_t>(scan[i]);
  if (f & 1ull) run_pos[r] = static_cast<uint32_t>(i);
  if (skeys[i] != SentinelKey<K>()) {
    const bool last = i + 1 == n || skeys[i + 1] == SentinelKey<K>();
    if (last) run_pos[r + static_cast<uint32_t>(f & 1ull)] =
        static_cast<uint32_t>(i + 1);
  }
}

struct Limits {
  int32_t max_ids;
  int32_t max_unique;
  int32_t allow_dropping;
};

template <typename K>
__global__ __launch_bounds__(256) void RunReduce(
    const K* skeys, const float* sgains, const uint64_t* flags,
    const uint64_t* scan, const uint32_t* run_pos, const uint64_t* totals,
    int64_t n_upper, KeyLayout kl, int num_partitions,
    const int32_t* part_first, Limits lim, float* run_gain,
    uint32_t* keep, int64_t* counters) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r > n_upper) return;
  const int64_t runs = static_cast<int64_t>(static_cast<uint32_t>(totals[0]));
  if (r >= runs) {
    keep[r] = 0;
    return;
  }
  const int64_t i0 = run_pos[r];
  const int64_t i1 = run_pos[r + 1];
  float g = sgains[i0];
  for (int64_t k = i0 + 1; k < i1; ++k) g = g + sgains[k];
  run_gain[r] = g;
  uint32_t k_ok = 1;
  if (lim.allow_dropping) {
    const K key = skeys[i0];
    const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
    uint32_t p, local;
    DecodeCol<K>(key & col_mask, kl, &p, &local);
    const int64_t bucket =
        static_cast<int64_t>(key >> kl.col_bits) * num_partitions + p;
    const int64_t first = part_first[bucket];
    const uint64_t fs = scan[first];
    const uint64_t si = scan[i0];
    const int64_t u = r - static_cast<int64_t>(static_cast<uint32_t>(fs)) + 1;
    const int64_t c = static_cast<int64_t>(si >> 32) +
                      static_cast<int64_t>(flags[i0] >> 32) -
                      static_cast<int64_t>(fs >> 32);
    if (u > lim.max_ids || c > lim.max_unique) {
      k_ok = 0;
      atomicAdd(reinterpret_cast<unsigned long long*>(&counters[0]),
                static_cast<unsigned long long>(i1 - i0));
    }
  }
  keep[r] = k_ok;
}

struct BucketStats {
  int32_t obs_ids;
  int32_t obs_unique;
  int32_t kept;
  int32_t kept_first;
};

__device__ __forceinline__ BucketStats ReduceBucket(
    const int32_t* part_first, const int32_t* part_last,
    const uint64_t* flags, const uint64_t* scan, const uint32_t* keep_scan,
    int64_t bkt) {
  BucketStats s{0, 0, 0, 0};
  const int32_t f = part_first[bkt];
  if (f >= 0) {
    const int32_t l = part_last[bkt];
    const uint64_t fs = scan[f];
    const uint64_t ls = scan[l];
    const uint64_t lf = flags[l];
    const uint32_t rf = static_cast<uint32_t>(fs);
    const uint32_t rend = static_cast<uint32_t>(ls) + static_cast<uint32_t>(lf & 1ull);
    s.obs_ids = static_cast<int32_t>(rend - rf);
    s.obs_unique = static_cast<int32_t>(
        static_cast<uint32_t>(ls >> 32) + static_cast<uint32_t>(lf >> 32) -
        static_cast<uint32_t>(fs >> 32));
    s.kept_first = static_cast<int32_t>(keep_scan[rf]);
    s.kept = static_cast<int32_t>(keep_scan[rend] - keep_scan[rf]);
  }
  return s;
}

__global__ __launch_bounds__(256) void BucketReduce(
    const int32_t* part_first, const int32_t* part_last,
    const uint64_t* flags, const uint64_t* scan, const uint32_t* keep_scan,
    int64_t num_buckets, BucketStats* stats) {
  const int64_t bkt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (bkt >= num_buckets) return;
  stats[bkt] = ReduceBucket(part_first, part_last, flags, scan, keep_scan, bkt);
}

// BucketReduce's inputs, for the kernels that fold it in.
struct BucketReduceArgs {
  const int32_t* part_first;
  const int32_t* part_last;
  const uint64_t* flags;
  const uint64_t* scan;
  const uint32_t* keep_scan;
  int64_t num_buckets;  // 0: the stats were reduced beforehand
  BucketStats* out;
  // Not null: every sorted entry is its own run (grouped at extraction) and
  // col_heads[b] counts bucket b's distinct columns; flags, scan and
  // keep_scan are unused.
  const int32_t* col_heads;
};

// Stats of one bucket whose entries are all distinct (row, column) pairs
// and all kept: part_first..part_last of the sorted entries.
__device__ __forceinline__ BucketStats UniqueBucket(const int32_t* part_first,
                                                    const int32_t* part_last,
                                                    const int32_t* col_heads,
                                                    int64_t bkt) {
  BucketStats s{0, 0, 0, 0};
  const int32_t f = part_first[bkt];
  if (f >= 0) {
    s.obs_ids = part_last[bkt] - f + 1;
    s.obs_unique = col_heads[bkt];
    s.kept = s.obs_ids;
    s.kept_first = f;
  }
  return s;
}

struct FillPlan {
  int64_t start;      // absolute position of the first kept entry
  int32_t fit;        // kept entries that fit the static buffer
  int32_t pad_begin;  // alignment padding written after this partition
  int32_t pad_end;
  int32_t pad_seg;    // padding positions are relative to this segment
};

struct FillParams {
  int32_t local_devices;
  int32_t segs_per_device;  // S
  int32_t num_partitions;   // NS
  int32_t rp_per_segment;
  int64_t coo_size;         // per device
  int32_t max_ids;
  int32_t max_unique;
  int32_t allow_dropping;
  int32_t mb_bits;          // bucket bits of the key (0 or 6)
  int32_t absolute;         // padding positions are device positions
  int32_t num_minibatches;  // minibatching layout: minibatches per SC
  uint8_t minibatch_of[kMaxMinibatches];  // bucket -> minibatch
};

// One thread per segment replays FillBufferSegment over partition counts; a
// second loop reduces device stats (max over local SCs). With
// br.num_buckets > 0 the block first reduces the bucket stats itself
// (BucketReduce folded in; bstats is then br.out).
__device__ __forceinline__ void FillPlanBody(
    const BucketStats* bstats, const FillParams& fp, int32_t* rp_out,
    FillPlan* plans, int32_t* stat_max_ids, int32_t* stat_max_unique,
    int32_t* stat_required, int64_t* counters, const BucketReduceArgs& br) {
  if (br.num_buckets > 0) {
    for (int64_t bkt = threadIdx.x; bkt < br.num_buckets; bkt += blockDim.x) {
      br.out[bkt] = br.col_heads != nullptr
                        ? UniqueBucket(br.part_first, br.part_last,
                                       br.col_heads, bkt)
                        : ReduceBucket(br.part_first, br.part_last, br.flags,
                                       br.scan, br.keep_scan, bkt);
    }
    __syncthreads();
  }
  const int S = fp.segs_per_device;
  const int NS = fp.num_partitions;
  const int num_segments = fp.local_devices * S;
  const int64_t per_sc = fp.coo_size / S;
  for (int g = threadIdx.x; g < num_segments; g += blockDim.x) {
    const int s = g % S;
    const BucketStats* bs = bstats + static_cast<int64_t>(g) * NS;
    FillPlan* pl = plans + static_cast<int64_t>(g) * NS;
    int32_t* rp = rp_out + static_cast<int64_t>(g) * fp.rp_per_segment;
    int64_t total = 0, req = 0;
    bool over = false;
    for (int p = 0; p < NS; ++p) {
      total += bs[p].kept;
      req += (static_cast<int64_t>(bs[p].obs_ids) + kAlign - 1) / kAlign * kAlign;
      pl[p].start = 0;
      pl[p].fit = 0;
      pl[p].pad_begin = 0;
      pl[p].pad_end = 0;
      pl[p].pad_seg = g;
      if (bs[p].obs_ids > fp.max_ids || bs[p].obs_unique > fp.max_unique) {
        over = true;
      }
    }
    stat_required[g] = static_cast<int32_t>(req);
    if (over && !fp.allow_dropping) {
      atomicMax(reinterpret_cast<unsigned long long*>(&counters[1]), 1ull);
    }
    const int64_t coo_begin = min(static_cast<int64_t>(s) * per_sc, fp.coo_size);
    const int64_t coo_end = coo_begin + per_sc;
    int64_t coo = coo_begin;
    int64_t processed = 0;
    int rpi = 0;
    int cur = 0;
    auto valid = [&]() {
      if (processed == total && coo == coo_end) return true;
      if (rpi >= fp.rp_per_segment || coo >= coo_end) return false;
      return true;
    };
    auto advance = [&](int target) {
      while (cur < target) {
        if (!valid()) return;
        rp[rpi++] = static_cast<int32_t>(coo - coo_begin);
        int64_t nc = (coo + kAlign - 1) / kAlign * kAlign;
        if (nc > coo_end) nc = coo_end;
        pl[cur].pad_begin = static_cast<int32_t>(coo - coo_begin);
        pl[cur].pad_end = static_cast<int32_t>(nc - coo_begin);
        coo = nc;
        ++cur;
      }
    };
    bool dropped_rest = false;
    for (int p = 0; p < NS && !dropped_rest; ++p) {
      const int64_t kp = bs[p].kept;
      if (kp == 0) continue;
      advance(p);
      if (!valid()) {
        dropped_rest = true;
        break;
      }
      const int64_t room = coo_end - coo;
      const int64_t take = kp < room ? kp : room;
      pl[p].start = coo;
      pl[p].fit = static_cast<int32_t>(take);
      coo += take;
      processed += take;
      if (take < kp) {
        dropped_rest = true;
        break;
      }
    }
    advance(NS);
    while (rpi < fp.rp_per_segment) {
      rp[rpi++] = static_cast<int32_t>(coo - coo_begin);
    }
    if (total > processed) {
      atomicAdd(reinterpret_cast<unsigned long long*>(&counters[0]),
                static_cast<unsigned long long>(total - processed));
    }
  }
  for (int dp = threadIdx.x; dp < fp.local_devices * NS; dp += blockDim.x) {
    const int d = dp / NS, p = dp % NS;
    int32_t mi = 0, mu = 0;
    for (int s = 0; s < S; ++s) {
      const BucketStats& b = bstats[static_cast<int64_t>(d * S + s) * NS + p];
      mi = max(mi, b.obs_ids);
      mu = max(mu, b.obs_unique);
    }
    stat_max_ids[dp] = mi;
    stat_max_unique[dp] = mu;
  }
}

__global__ __launch_bounds__(256) void FillPlanKernel(
    const BucketStats* bstats, FillParams fp, int32_t* rp_out,
    FillPlan* plans, int32_t* stat_max_ids, int32_t* stat_max_unique,
    int32_t* stat_required, int64_t* counters, BucketReduceArgs br) {
  FillPlanBody(bstats, fp, rp_out, plans, stat_max_ids, stat_max_unique,
               stat_required, counters, br);
}

// FillPlanKernel's arguments for a grouped launch (one block per problem).
struct FillPlanArgs {
  static constexpr int kBlock = 256;
  const BucketStats* bstats;
  FillParams fp;
  int32_t* rp_out;
  FillPlan* plans;
  int32_t* stat_max_ids;
  int32_t* stat_max_unique;
  int32_t* stat_required;
  int64_t* counters;
  BucketReduceArgs br;
  __device__ static void Run(const FillPlanArgs& a, uint32_t, uint32_t) {
    FillPlanBody(a.bstats, a.fp, a.rp_out, a.plans, a.stat_max_ids,
                 a.stat_max_unique, a.stat_required, a.counters, a.br);
  }
};

// The minibatching layout (input_preprocessing_util.cc:135-143, :331-473):
// one thread per device replays FillBufferSegment over the (SC, minibatch)
// segments in order. A segment's partition p takes the kept entries of
// every bucket of the minibatch in bucket order (the partition-stable merge
// of partitioned_coo_tensors.h:162-181); row pointers are device positions;
// with one minibatch SC s starts at the summed required sizes of the SCs
// before it, with several each segment starts where the previous ended.
// Pass 0 (one bucket) also writes the stats and flags a partition over a
// limit (minibatching required); pass 2 flags a bucket over a limit when
// dropping is off (ValidateMaxIdsOrDie).
__global__ __launch_bounds__(64) void FillPlanMinibatch(
    const BucketStats* bstats, FillParams fp, int pass, int32_t* rp_out,
    FillPlan* plans, int32_t* stat_max_ids, int32_t* stat_max_unique,
    int32_t* stat_required, int64_t* counters) {
  const int S = fp.segs_per_device;
  const int NS = fp.num_partitions;
  const int B = 1 << fp.mb_bits;
  const int nmb = fp.num_minibatches;
  const int RPB = fp.rp_per_segment;
  const int64_t coo_size = fp.coo_size;
  for (int d = threadIdx.x; d < fp.local_devices; d += blockDim.x) {
    int32_t* rp = rp_out + static_cast<int64_t>(d) * S * kMaxMinibatches * RPB;
    int64_t packed = 0, chained = 0, dropped = 0;
    int rp_begin = 0;
    bool required = false, over = false;
    for (int s = 0; s < S; ++s) {
      const int64_t g = static_cast<int64_t>(d) * S + s;
      const BucketStats* bs = bstats + g * B * NS;  // [b][p]
      FillPlan* pl = plans + g * B * NS;
      int64_t req = 0;
      for (int p = 0; p < NS; ++p) {
        int64_t ids = 0;
        for (int b = 0; b < B; ++b) {
          const BucketStats& x = bs[b * NS + p];
          ids += x.obs_ids;
          if (x.obs_ids > fp.max_ids || x.obs_unique > fp.max_unique) {
            over = true;
          }
          FillPlan& q = pl[b * NS + p];
          q.start = 0;
          q.fit = 0;
          q.pad_begin = 0;
          q.pad_end = 0;
          q.pad_seg = static_cast<int32_t>(g);
        }
        req += (ids + kAlign - 1) / kAlign * kAlign;
      }
      if (pass == 0) {
        stat_required[g] = static_cast<int32_t>(req);
        required = required || over;
      }
      for (int m = 0; m < nmb; ++m) {
        int64_t coo_begin;
        if (nmb == 1) {
          coo_begin = min(packed, coo_size);
          packed = min(packed + req, coo_size);
        } else {
          coo_begin = chained;
        }
        const int64_t coo_end = coo_size;
        int64_t total = 0;
        for (int b = 0; b < B; ++b) {
          if (fp.minibatch_of[b] != m) continue;
          for (int p = 0; p < NS; ++p) total += bs[b * NS + p].kept;
        }
        int64_t coo = coo_begin, processed = 0;
        int rpi = rp_begin;
        const int rp_end = rp_begin + RPB;
        int cur = 0;
        auto valid = [&]() {
          if (processed == total && coo == coo_end) return true;
          if (rpi >= rp_end || coo >= coo_end) return false;
          return true;
        };
        // The partition's padding is recorded with the minibatch's first
        // bucket.
        int first_b = 0;
        while (first_b < B - 1 && fp.minibatch_of[first_b] != m) ++first_b;
        auto advance = [&](int target) {
          while (cur < target) {
            if (!valid()) return;
            rp[rpi++] = static_cast<int32_t>(coo);
            int64_t nc = (coo + kAlign - 1) / kAlign * kAlign;
            if (nc > coo_end) nc = coo_end;
            FillPlan& q = pl[first_b * NS + cur];
            q.pad_begin = static_cast<int32_t>(coo);
            q.pad_end = static_cast<int32_t>(nc);
            coo = nc;
            ++cur;
          }
        };
        for (int p = 0; p < NS; ++p) {
          int64_t kp = 0;
          for (int b = 0; b < B; ++b) {
            if (fp.minibatch_of[b] == m) kp += bs[b * NS + p].kept;
          }
          if (kp == 0) continue;
          advance(p);
          if (!valid()) break;
          const int64_t room = coo_end - coo;
          const int64_t take = kp < room ? kp : room;
          int64_t off = 0;
          for (int b = 0; b < B; ++b) {
            if (fp.minibatch_of[b] != m) continue;
            const int64_t kb = bs[b * NS + p].kept;
            FillPlan& q = pl[b * NS + p];
            q.start = coo + off;
            int64_t fit = take - off;
            fit = fit < 0 ? 0 : (fit > kb ? kb : fit);
            q.fit = static_cast<int32_t>(fit);
            off += kb;
          }
          coo += take;
          processed += take;
          if (take < kp) break;
        }
        advance(NS);
        while (rpi < rp_end) rp[rpi++] = static_cast<int32_t>(coo);
        dropped += total - processed;
        chained = coo;
        rp_begin += RPB;
      }
    }
    if (pass == 0 && required) {
      atomicMax(reinterpret_cast<unsigned long long*>(&counters[4]), 1ull);
    }
    if (pass != 0 && over && !fp.allow_dropping) {
      atomicMax(reinterpret_cast<unsigned long long*>(&counters[1]), 1ull);
    }
    if (dropped > 0) {
      atomicAdd(reinterpret_cast<unsigned long long*>(&counters[0]),
                static_cast<unsigned long long>(dropped));
    }
  }
  if (pass != 0) return;
  for (int dp = threadIdx.x; dp < fp.local_devices * NS; dp += blockDim.x) {
    const int d = dp / NS, p = dp % NS;
    int32_t mi = 0, mu = 0;
    for (int s = 0; s < S; ++s) {
      const BucketStats& b = bstats[static_cast<int64_t>(d * S + s) * NS + p];
      mi = max(mi, b.obs_ids);
      mu = max(mu, b.obs_unique);
    }
    stat_max_ids[dp] = mi;
    stat_max_unique[dp] = mu;
  }
}

// FillPlanMinibatch for one device per block, with the device's bucket counts
// in LDS: slot totals ((SC, minibatch, partition): the kept entries of the
// minibatch's buckets) and the per-bucket plans are computed in parallel;
// one thread replays FillBufferSegment over the slots, as FillPlanMinibatch
// does. Needs S * 64 * NS <= kLdsPlanCells (bucket counts) slots and cells.
constexpr int kLdsPlanCells = 2048;

__global__ __launch_bounds__(256) void FillPlanMinibatchLds(
    const BucketStats* bstats, FillParams fp, int pass, int32_t* rp_out,
    FillPlan* plans, int32_t* stat_max_ids, int32_t* stat_max_unique,
    int32_t* stat_required, int64_t* counters) {
  __shared__ int32_t s_kept[kLdsPlanCells];    // [s][b][p]
  __shared__ int32_t s_total[kLdsPlanCells];   // [s][m][p], then slot take
  __shared__ int32_t s_start[kLdsPlanCells];   // [s][m][p]
  __shared__ int32_t s_pad0[kLdsPlanCells];
  __shared__ int32_t s_pad1[kLdsPlanCells];
  __shared__ int32_t s_req[kMaxMinibatches];   // per SC (S <= 64 here)
  __shared__ int32_t s_first[kMaxMinibatches + 1];
  const int d = blockIdx.x;
  const int tid = threadIdx.x;
  const int S = fp.segs_per_device;
  const int NS = fp.num_partitions;
  const int B = 1 << fp.mb_bits;
  const int nmb = fp.num_minibatches;
  const int RPB = fp.rp_per_segment;
  const int64_t coo_size = fp.coo_size;
  const int cells = S * B * NS;
  const int slots = S * nmb * NS;
  const BucketStats* bs = bstats + static_cast<int64_t>(d) * cells;
  FillPlan* pl = plans + static_cast<int64_t>(d) * cells;
  int32_t* rp = rp_out + static_cast<int64_t>(d) * S * kMaxMinibatches * RPB;
  // Bucket counts to LDS; a cell over a limit.
  bool over = false;
  for (int c = tid; c < cells; c += blockDim.x) {
    const BucketStats x = bs[c];
    s_kept[c] = x.kept;
    over = over || x.obs_ids > fp.max_ids || x.obs_unique > fp.max_unique;
  }
  // First bucket of each minibatch (buckets of one minibatch are a range).
  for (int b = tid; b < B; b += blockDim.x) {
    const int m = fp.minibatch_of[b];
    if (b == 0 || fp.minibatch_of[b - 1] != m) s_first[m] = b;
  }
  if (tid == 0) s_first[nmb] = B;
  // Required sizes: per partition the observed ids of all buckets, aligned.
  for (int sc = tid; sc < S; sc += blockDim.x) {
    int64_t req = 0;
    for (int p = 0; p < NS; ++p) {
      int64_t ids = 0;
      for (int b = 0; b < B; ++b) ids += bs[(sc * B + b) * NS + p].obs_ids;
      req += (ids + kAlign - 1) / kAlign * kAlign;
    }
    s_req[sc] = static_cast<int32_t>(req);
    if (pass == 0) {
      stat_required[static_cast<int64_t>(d) * S + sc] =
          static_cast<int32_t>(req);
    }
  }
  const bool any_over = __syncthreads_or(over);
  // Slot totals and cleared plans.
  for (int t = tid; t < slots; t += blockDim.x) {
    const int p = t % NS;
    const int m = (t / NS) % nmb;
    const int sc = t / NS / nmb;
    int32_t k = 0;
    for (int b = s_first[m]; b < s_first[m + 1]; ++b) {
      k += s_kept[(sc * B + b) * NS + p];
    }
    s_total[t] = k;
    s_start[t] = 0;
    s_pad0[t] = 0;
    s_pad1[t] = 0;
  }
  __syncthreads();
  if (tid == 0) {
    // FillBufferSegment over the (SC, minibatch) segments; s_total becomes
    // the slot's take.
    int64_t packed = 0, chained = 0, dropped = 0;
    int rp_begin = 0;
    for (int sc = 0; sc < S; ++sc) {
      for (int m = 0; m < nmb; ++m) {
        int64_t coo_begin;
        if (nmb == 1) {
          coo_begin = min(packed, coo_size);
          packed = min(packed + static_cast<int64_t>(s_req[sc]), coo_size);
        } else {
          coo_begin = chained;
        }
        const int base = (sc * nmb + m) * NS;
        int64_t total = 0;
        for (int p = 0; p < NS; ++p) total += s_total[base + p];
        const int64_t coo_end = coo_size;
        int64_t coo = coo_begin, processed = 0;
        int rpi = rp_begin;
        const int rp_end = rp_begin + RPB;
        int cur = 0;
        auto valid = [&]() {
          if (processed == total && coo == coo_end) return true;
          if (rpi >= rp_end || coo >= coo_end) return false;
          return true;
        };
        auto advance = [&](int target) {
          while (cur < target) {
            if (!valid()) return;
            rp[rpi++] = static_cast<int32_t>(coo);
            int64_t nc = (coo + kAlign - 1) / kAlign * kAlign;
            if (nc > coo_end) nc = coo_end;
            s_pad0[base + cur] = static_cast<int32_t>(coo);
            s_pad1[base + cur] = static_cast<int32_t>(nc);
            coo = nc;
            ++cur;
          }
        };
        bool stop = false;
        for (int p = 0; p < NS; ++p) {
          const int64_t kp = s_total[base + p];
          s_total[base + p] = 0;
          if (stop || kp == 0) continue;
          advance(p);
          if (!valid()) {
            stop = true;
            continue;
          }
          const int64_t room = coo_end - coo;
          const int64_t take = kp < room ? kp : room;
          s_start[base + p] = static_cast<int32_t>(coo);
          s_total[base + p] = static_cast<int32_t>(take);
          coo += take;
          processed += take;
          if (take < kp) stop = true;
        }
        advance(NS);
        while (rpi < rp_end) rp[rpi++] = static_cast<int32_t>(coo);
        dropped += total - processed;
        chained = coo;
        rp_begin += RPB;
      }
    }
    if (pass == 0 && any_over) {
      atomicMax(reinterpret_cast<unsigned long long*>(&counters[4]), 1ull);
    }
    if (pass != 0 && any_over && !fp.allow_dropping) {
      atomicMax(reinterpret_cast<unsigned long long*>(&counters[1]), 1ull);
    }
    if (dropped > 0) {
      atomicAdd(reinterpret_cast<unsigned long long*>(&counters[0]),
                static_cast<unsigned long long>(dropped));
    }
  }
  __syncthreads();
  // Per-bucket plans: the bucket's entries follow those of the minibatch's
  // earlier buckets in the slot; the slot's padding goes with its first
  // bucket.
  for (int c = tid; c < cells; c += blockDim.x) {
    const int p = c % NS;
    const int b = (c / NS) % B;
    const int sc = c / NS / B;
    const int m = fp.minibatch_of[b];
    const int slot = (sc * nmb + m) * NS + p;
    int32_t off = 0;
    for (int b2 = s_first[m]; b2 < b; ++b2) off += s_kept[(sc * B + b2) * NS + p];
    const int32_t kb = s_kept[c];
    int32_t fit = s_total[slot] - off;
    fit = fit < 0 ? 0 : (fit > kb ? kb : fit);
    FillPlan q;
    q.start = static_cast<int64_t>(s_start[slot]) + off;
    q.fit = fit;
    const bool first = b == s_first[m];
    q.pad_begin = first ? s_pad0[slot] : 0;
    q.pad_end = first ? s_pad1[slot] : 0;
    q.pad_seg = d * S + sc;
    pl[c] = q;
  }
  if (pass != 0) return;
  for (int p = tid; p < NS; p += blockDim.x) {
    int32_t mi = 0, mu = 0;
    for (int sc = 0; sc < S; ++sc) {
      const BucketStats& x = bs[sc * NS + p];
      mi = max(mi, x.obs_ids);
      mu = max(mu, x.obs_unique);
    }
    stat_max_ids[static_cast<int64_t>(d) * NS + p] = mi;
    stat_max_unique[static_cast<int64_t>(d) * NS + p] = mu;
  }
}

// ComputeMinibatchingSplit (minibatching_splits_impl.h:58-81) over the 64
// bucket values of v: bottom-up, a node whose children sum past the limit is
// split and keeps the larger child, otherwise it keeps the sum.
__device__ uint64_t SplitOf(int32_t* v, int32_t limit) {
  uint64_t split = 0;
  int index = 0;
  for (int size = 2; size <= kMaxMinibatches; size *= 2) {
    for (int i = 0; i < kMaxMinibatches; i += size, ++index) {
      const int32_t l = v[i], r = v[i + size / 2];
      if (l + r > limit) {
        split |= uint64_t{1} << index;
        v[i] = l > r ? l : r;
      } else {
        v[i] = l + r;
      }
    }
  }
  return split;
}

// Pass 0, only when a limit was exceeded (counters[4], set by the fill
// plan): the bucket pass's observed counts straight from this pass's runs.
// A run is a distinct (column, row) of one SC, and the bucket pass counts
// exactly those (merged duplicates and repeats of dropped ones are not
// observed, sort_and_group_coo_tensors_impl.h:245-274); its distinct
// columns are the unique ids. So per (SC, bucket, partition): runs, and runs
// that start a column. Block-local counts in LDS when they fit.
constexpr int kLdsCountCells = 2048;

template <typename K>
__global__ __launch_bounds__(256) void BucketCountsOfRuns(
    const K* skeys, const uint32_t* run_pos, const uint64_t* flags,
    const uint64_t* totals, KeyLayout kl, int num_partitions, int64_t cells,
    const int64_t* counters, BucketStats* counts) {
  __shared__ int32_t s_ids[kLdsCountCells];
  __shared__ int32_t s_uniq[kLdsCountCells];
  if (counters[4] == 0) return;
  const bool lds = cells <= kLdsCountCells;
  if (lds) {
    for (int64_t c = threadIdx.x; c < cells; c += blockDim.x) {
      s_ids[c] = 0;
      s_uniq[c] = 0;
    }
    __syncthreads();
  }
  const int64_t runs = static_cast<int64_t>(static_cast<uint32_t>(totals[0]));
  const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       r < runs; r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i0 = run_pos[r];
    const K key = skeys[i0];
    uint32_t p, local;
    DecodeCol<K>(key & col_mask, kl, &p, &local);
    const int64_t seg = static_cast<int64_t>(key >> kl.col_bits);
    const uint32_t col = (local << kl.log2ns) | p;
    const int64_t cell =
        (seg * kMaxMinibatches + MinibatchingBucket(col)) * num_partitions + p;
    const bool new_col = ((flags[i0] >> 32) & 1ull) != 0;
    if (lds) {
      atomicAdd(&s_ids[cell], 1);
      if (new_col) atomicAdd(&s_uniq[cell], 1);
    } else {
      atomicAdd(&counts[cell].obs_ids, 1);
      if (new_col) atomicAdd(&counts[cell].obs_unique, 1);
    }
  }
  if (!lds) return;
  __syncthreads();
  for (int64_t c = threadIdx.x; c < cells; c += blockDim.x) {
    if (s_ids[c] != 0) atomicAdd(&counts[c].obs_ids, s_ids[c]);
    if (s_uniq[c] != 0) atomicAdd(&counts[c].obs_unique, s_uniq[c]);
  }
}

// Per (SC, partition) the split of its bucket counts, ids and unique ids,
// OR-ed into counters[5] (UpdateMinibatchingSplit,
// sort_and_group_coo_tensors_impl.h:116-151); a bucket over a limit with
// dropping off sets counters[1]. Pass 1 runs it on its own counts; pass 0
// on BucketCountsOfRuns's, and only when a limit was exceeded.
__global__ __launch_bounds__(64) void MinibatchSplit(const BucketStats* bstats,
                                                     FillParams fp,
                                                     int only_if_required,
                                                     int64_t* counters) {
  if (only_if_required && counters[4] == 0) return;
  const int NS = fp.num_partitions;
  const int64_t n = static_cast<int64_t>(fp.local_devices) *
                    fp.segs_per_device * NS;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int64_t g = t / NS;
  const int p = static_cast<int>(t % NS);
  int32_t ids[kMaxMinibatches], uniq[kMaxMinibatches];
  bool over = false;
  for (int b = 0; b < kMaxMinibatches; ++b) {
    const BucketStats& x = bstats[(g * kMaxMinibatches + b) * NS + p];
    ids[b] = x.obs_ids;
    uniq[b] = x.obs_unique;
    over = over || x.obs_ids > fp.max_ids || x.obs_unique > fp.max_unique;
  }
  const uint64_t split = SplitOf(ids, fp.max_ids) | SplitOf(uniq, fp.max_unique);
  if (split != 0) {
    atomicOr(reinterpret_cast<unsigned long long*>(&counters[5]),
             static_cast<unsigned long long>(split));
  }
  if (over && !fp.allow_dropping) {
    atomicMax(reinterpret_cast<unsigned long long*>(&counters[1]), 1ull);
  }
}

// What the sample view needs of every run written to the CSR, indexed by
// the extraction position of the run's first id (null: no view).
struct ViewParts {
  const uint32_t* sidx;  // sorted position -> extraction position
  uint64_t* entry;       // [M] table row | gain bits << 32, or kNoEntry
  uint32_t* pos;         // [M + 1] view positions (scan of entry != kNoEntry)
  int64_t rows_per_partition;
};
template <typename K>
__global__ __launch_bounds__(256) void ScatterRuns(
    const K* skeys, const uint32_t* srows, const uint32_t* run_pos,
    const float* run_gain, const uint32_t* keep, const uint32_t* keep_scan,
    const uint64_t* totals, int64_t n_upper, KeyLayout kl, FillParams fp,
    int32_t bps, const BucketStats* bstats, const FillPlan* plans,
    int32_t* eid, int32_t* sid, float* gains, ViewParts view) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n_upper) return;
  const int64_t runs = static_cast<int64_t>(static_cast<uint32_t>(totals[0]));
  if (r >= runs || !keep[r]) return;
  const int64_t i0 = run_pos[r];
  const K key = skeys[i0];
  const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
  uint32_t p, local;
  DecodeCol<K>(key & col_mask, kl, &p, &local);
  const int64_t seg = static_cast<int64_t>(key >> kl.col_bits);
  const int64_t bucket = seg * fp.num_partitions + p;
  const int64_t k = static_cast<int64_t>(keep_scan[r]) - bstats[bucket].kept_first;
  const FillPlan pl = plans[bucket];
  if (k >= pl.fit) return;
  const int64_t d = (seg >> kl.mb_bits) / fp.segs_per_device;
  const int64_t pos = d * fp.coo_size + pl.start + k;
  eid[pos] = static_cast<int32_t>(local);
  sid[pos] = static_cast<int32_t>(srows[i0] % static_cast<uint32_t>(bps));
  gains[pos] = run_gain[r];
  if (view.entry != nullptr && local < view.rows_per_partition) {
    // One 8-byte store per run, at the run's first input position; the
    // activation row (one device: the stacked sample id) is read back from
    // the extraction-order rows when the view is compacted.
    view.entry[view.sidx[i0]] =
        static_cast<uint64_t>(p * view.rows_per_partition + local) |
        (static_cast<uint64_t>(__float_as_uint(run_gain[r])) << 32);
  }
}

// 1 where a written run starts (input order), 0 elsewhere and at m.
__global__ __launch_bounds__(256) void MarkEntries(const uint64_t* entry,
                                                   int64_t m, uint32_t* mark) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i <= m) mark[i] = i < m && entry[i] != kNoEntry ? 1u : 0u;
}

// The sample view in extraction order, which is activation-row order: the
// run starting at extraction position e goes to view position pos[e]
// (exclusive scan of the marks) with key row_gain[e]'s row; positions from
// pos[m] to n get the unused key.
__global__ __launch_bounds__(256) void ViewCompact(
    const uint32_t* pos, const uint64_t* row_gain, const uint64_t* ventry,
    int64_t m, int64_t n, uint32_t unused_key, uint32_t* keys,
    uint64_t* entries) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < m && pos[i + 1] > pos[i]) {
    keys[pos[i]] = static_cast<uint32_t>(row_gain[i]);
    entries[pos[i]] = ventry[i];
  }
  if (i < n && i >= static_cast<int64_t>(pos[m])) {
    keys[i] = unused_key;
    entries[i] = 0;
  }
}

// Also copies the grouped-entry total into the counters when `totals` (low
// half of a 64-bit scan total) or `total32` is not null (after the scatter,
// which reads it).
__device__ __forceinline__ void WritePaddingBody(
    uint32_t blk, const FillPlan* plans, int64_t num_buckets,
    const FillParams& fp, int32_t* eid, int32_t* sid, float* gains,
    const uint64_t* totals, const uint32_t* total32, int64_t* counters) {
  const int64_t t = static_cast<int64_t>(blk) * blockDim.x + threadIdx.x;
  if (t == 0 && totals != nullptr) {
    counters[3] = static_cast<int64_t>(static_cast<uint32_t>(totals[0]));
  }
  if (t == 0 && total32 != nullptr) {
    counters[3] = static_cast<int64_t>(total32[0]);
  }
  const int64_t bkt = t / kAlign;
  const int k = static_cast<int>(t % kAlign);
  if (bkt >= num_buckets) return;
  const FillPlan pl = plans[bkt];
  const int32_t pos_rel = pl.pad_begin + k;
  if (pos_rel >= pl.pad_end) return;
  const int64_t seg = pl.pad_seg;
  const int64_t d = seg / fp.segs_per_device;
  const int64_t s = seg % fp.segs_per_device;
  const int64_t per_sc = fp.coo_size / fp.segs_per_device;
  const int64_t coo_begin =
      fp.absolute ? 0 : (s * per_sc < fp.coo_size ? s * per_sc : fp.coo_size);
  const int64_t pos = d * fp.coo_size + coo_begin + pos_rel;
  eid[pos] = kPadInt;
  sid[pos] = kPadInt;
  gains[pos] = __uint_as_float(kNanBits);
}

__global__ __launch_bounds__(256) void WritePadding(const FillPlan* plans,
                                                    int64_t num_buckets,
                                                    FillParams fp, int32_t* eid,
                                                    int32_t* sid, float* gains,
                                                    const uint64_t* totals,
                                                    const uint32_t* total32,
                                                    int64_t* counters) {
  WritePaddingBody(blockIdx.x, plans, num_buckets, fp, eid, sid, gains, totals,
                   total32, counters);
}

// WritePadding's arguments for a grouped launch.
struct WritePaddingArgs {
  static constexpr int kBlock = 256;
  const FillPlan* plans;
  int64_t num_buckets;
  FillParams fp;
  int32_t* eid;
  int32_t* sid;
  float* gains;
  const uint64_t* totals;
  const uint32_t* total32;
  int64_t* counters;
  __device__ static void Run(const WritePaddingArgs& a, uint32_t blk,
                             uint32_t) {
    WritePaddingBody(blk, a.plans, a.num_buckets, a.fp, a.eid, a.sid, a.gains,
                     a.totals, a.total32, a.counters);
  }
};

__global__ void ZeroI64(int64_t* p, int n) {
  if (threadIdx.x < n) p[threadIdx.x] = 0;
}

__global__ void StoreTotal(const uint64_t* totals, int64_t* counters) {
  counters[3] = static_cast<int64_t>(static_cast<uint32_t>(totals[0]));
}

// ---------------------------------------------------------------------------
// Grouping at extraction. Where the sample rows of a stack's features are
// disjoint, two ids share (row, column) only if one input row holds the same
// id twice; the grouping of sort_and_group_coo_tensors_impl.h:196-311 then
// merges exactly the copies of an id within one input row, summing their
// gains in input order. ExtractUnique does that while it extracts, so that
// the sort sees one entry per (row, column) and every sorted entry is its
// own run. The sample view is the extraction-order compaction of those
// entries (ViewWrite); the CSR is the sorted entries (GroupUnique,
// ScatterUnique).
// ---------------------------------------------------------------------------

// Input positions of one ExtractUnique block's rows staged in LDS, and the
// longest row the route is taken for: a block of kExtractBlock consecutive
// ids then spans at most kExtractBlock + 2 * (kDedupMaxRow - 1) positions,
// which fit the staging.
constexpr int kDedupStage = 2048;
constexpr int64_t kDedupMaxRow = 896;
// Rows of one ExtractUnique block whose splits (as 32-bit offsets from the
// block's first row) and divisors are staged; blocks spanning more rows (only
// with many empty rows) read the splits from memory. Sized so that a
// weighted block stays under 20 KB of LDS: eight blocks per CU.
constexpr int kUniqueStagedSplits = 448;
static_assert(kExtractBlock + 2 * (kDedupMaxRow - 1) <= kDedupStage,
              "a block's rows must fit the staging");

// Combiner divisor of one row (ComputeWeightDivisor,
// process_coo_tensors_impl.h:60-74): the weights summed in order in float
// (mean, combiner 1), or the square root of the float sum of double squares
// (sqrtn, combiner 2). Weights are loaded eight at a time ahead of the
// sequential sum.
template <typename W>
__device__ __forceinline__ float RowDivisor(const W* w, int n, int combiner) {
  float s = 0.0f;
  int k = 0;
  if (combiner == 1) {
    for (; k + 8 <= n; k += 8) {
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = w[k + j];
#pragma unroll
      for (int j = 0; j < 8; ++j) s = s + x[j];
    }
    for (; k < n; ++k) s = s + w[k];
    return s;
  }
  for (; k + 8 <= n; k += 8) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = w[k + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double d = static_cast<double>(x[j]);
      s = static_cast<float>(static_cast<double>(s) + d * d);
    }
  }
  for (; k < n; ++k) {
    const double d = static_cast<double>(w[k]);
    s = static_cast<float>(static_cast<double>(s) + d * d);
  }
  return sqrtf(s);
}

// The id at position q of a row of n ids (ids, weights w): whether it is the
// row's first copy of that id, and its gain summed with the gains of the
// later copies in input order. Weighted gains are w / div, with div the
// row's divisor (computed here unless `have_div`); unit weights give the
// combiner's 1, 1/n or 1/sqrt(n). One pass, eight ids at a time, counts the
// copies before and after q; only a first copy with later copies walks the
// row again to add their gains.
template <typename T, typename W>
__device__ __forceinline__ bool ScanRow(const T* ids, const W* w, int n, int q,
                                        bool has_weights, int combiner,
                                        bool have_div, float* div,
                                        int32_t* id_out, float* gain_out) {
  const int32_t id = ids[q];
  *id_out = id;
  if (has_weights && !have_div) *div = RowDivisor(w, n, combiner);
  float unit = 1.0f;
  if (!has_weights && combiner == 1) {
    unit = 1.0f / static_cast<float>(n);
  } else if (!has_weights && combiner == 2) {
    unit = 1.0f / sqrtf(static_cast<float>(n));
  }
  int before = 0, after = 0;
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    int32_t a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = ids[k + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool eq = a[j] == id;
      before += eq && k + j < q;
      after += eq && k + j > q;
    }
  }
  for (; k < n; ++k) {
    const bool eq = ids[k] == id;
    before += eq && k < q;
    after += eq && k > q;
  }
  float gain = has_weights ? w[q] / *div : unit;
  if (before == 0 && after > 0) {
    for (k = q + 1; k < n; ++k) {
      if (ids[k] == id) gain = gain + (has_weights ? w[k] / *div : unit);
    }
  }
  *gain_out = gain;
  return before == 0;
}

// LDS hash set of a block's staged rows: slot = (row start << 11) | position
// of the first copy of an id in that row (both relative to the staged span,
// so below 2^11), or kSlotEmpty; a slot's key (row start, id) never changes
// once claimed, only its position can drop (atomicMin). A 16-bit count per
// slot tracks the copies.
constexpr int kDedupSlots = kDedupStage;
constexpr uint32_t kSlotEmpty = 0xffffffffu;
static_assert(kDedupStage <= 2048, "positions must fit 11 bits");

__device__ __forceinline__ uint32_t DedupHash(int32_t id, uint32_t row_start) {
  const uint32_t h = static_cast<uint32_t>(id) * 0x9e3779b1u ^
                     (row_start + 0x7f4a7c15u) * 0x85ebca77u;
  return (h ^ (h >> 15)) & (kDedupSlots - 1);
}

// Inserts position x (row start rs, id) and counts the copy.
__device__ __forceinline__ void DedupInsert(uint32_t* table, uint32_t* counts,
                                            const int32_t* s_ids, uint32_t rs,
                                            uint32_t x, int32_t id) {
  const uint32_t mine = (rs << 11) | x;
  uint32_t h = DedupHash(id, rs);
  for (;;) {
    uint32_t cur = table[h];
    if (cur == kSlotEmpty) {
      cur = atomicCAS(&table[h], kSlotEmpty, mine);
      if (cur == kSlotEmpty) break;
    }
    if ((cur >> 11) == rs && s_ids[cur & 2047u] == id) {
      atomicMin(&table[h], mine);
      break;
    }
    h = (h + 1) & (kDedupSlots - 1);
  }
  atomicAdd(&counts[h >> 1], 1u << ((h & 1u) * 16));
}

// The slot of (row start rs, id), which is in the set.
__device__ __forceinline__ uint32_t DedupFind(const uint32_t* table,
                                              const int32_t* s_ids,
                                              uint32_t rs, int32_t id) {
  uint32_t h = DedupHash(id, rs);
  for (;;) {
    const uint32_t cur = table[h];
    if ((cur >> 11) == rs && s_ids[cur & 2047u] == id) return h;
    h = (h + 1) & (kDedupSlots - 1);
  }
}

// One thread per extracted id, laid out as ExtractIds. The block stages the
// ids of the rows it spans in LDS. With unit weights (kHashed) every staged
// position enters an LDS hash set keyed by (row, id), which keeps the first
// position of each key and counts its copies: an id is its row's first copy
// when the set holds its position, and the first copy's gain is the
// combiner's unit summed once per copy, in order. With weights (not kHashed)
// the block also stages the weights and, for a weighted mean or sqrtn, each
// row's divisor (one thread per row, the sequential sums of RowDivisors);
// each id scans its row for copies (ScanRow) and a first copy adds the later
// copies' w / divisor in input order. Blocks whose rows do not fit the
// staging scan each row from memory. The first copy of an id writes its key
// and (sample, summed gain); later copies and ids outside the table write
// the sentinel key. With `view_counts`, each block also counts its entries
// that enter the sample view (a first copy whose local row is below
// `view_rows`).
template <typename K, bool kHashed>
__device__ __forceinline__ void ExtractUniqueBody(
    uint32_t blk, const SliceDesc* slices, int num_slices,
    const FeatureDev* feats, const BlockRows* block_rows, int64_t total_ids,
    int combiner, int rows_of_one, const KeyLayout& kl, int64_t view_rows,
    K* keys, uint64_t* pay, uint32_t* view_counts, int64_t* counters) {
  constexpr bool kWeighted = !kHashed;
  __shared__ int32_t s_splits[kUniqueStagedSplits];  // splits - span_b
  __shared__ int32_t s_ids[kDedupStage];
  __shared__ float s_w[kWeighted ? kDedupStage : 1];
  __shared__ float s_div[kWeighted ? kUniqueStagedSplits : 1];
  __shared__ uint32_t s_table[kHashed ? kDedupSlots : 1];
  __shared__ uint32_t s_counts[kHashed ? kDedupSlots / 2 : 1];
  const int64_t blk_first = static_cast<int64_t>(blk) * blockDim.x;
  const int64_t o = blk_first + threadIdx.x;
  const BlockRows br = block_rows[blk];
  const int block_slice = br.slice;
  int64_t row_lo = 0, row_hi = -1;
  if (block_slice >= 0) ClampBlockRows(br, slices[block_slice], &row_lo, &row_hi);
  const bool need_div = kWeighted && combiner != 0;
  bool staged = false;       // row splits [row_lo, row_hi + 1] in s_splits
                             // (relative to span_b)
  bool ids_staged = false;   // ids (and weights) [span_b, span_e) in LDS
  int64_t span_b = 0, span_e = 0;
  int64_t div_row0 = 0;      // row of s_div[0]
  int div_rows = 0;          // rows with a divisor in s_div
  int64_t valency = 0;       // dense feature of the block
  // With unit weights and no row of two ids there is nothing to merge: no
  // staging, no hash set.
  const bool stage = !(kHashed && rows_of_one);
  if (block_slice >= 0) {  // uniform over the block
    const SliceDesc bsl = slices[block_slice];
    const FeatureDev bf = feats[bsl.feature];
    if (bf.splits != nullptr) {
      span_b = bf.splits[row_lo];
      span_e = bf.splits[row_hi + 1];
      const int64_t cnt = row_hi - row_lo + 2;
      if (cnt <= kUniqueStagedSplits) {
        // A stack holds fewer than 2^31 ids: the offsets fit 32 bits.
        for (int64_t i = threadIdx.x; i < cnt; i += blockDim.x) {
          s_splits[i] = static_cast<int32_t>(bf.splits[row_lo + i] - span_b);
        }
        staged = true;
      }
    } else if (bf.valency > 0) {
      valency = bf.valency;
      const int64_t o_last = min(blk_first + kExtractBlock, total_ids) - 1;
      const int64_t p_first = bsl.id_begin + (blk_first - bsl.out_begin);
      const int64_t p_last = bsl.id_begin + (o_last - bsl.out_begin);
      span_b = p_first / valency * valency;
      span_e = (p_last / valency + 1) * valency;
    }
    if (stage && span_e > span_b && span_e - span_b <= kDedupStage) {
      const int n = static_cast<int>(span_e - span_b);
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        s_ids[i] = bf.ids[span_b + i];
        if constexpr (kWeighted) s_w[i] = bf.weights[span_b + i];
      }
      ids_staged = true;
      if (need_div) {
        const int64_t rows =
            valency > 0 ? (span_e - span_b) / valency
                        : (staged ? row_hi - row_lo + 1 : 0);
        if (rows <= kUniqueStagedSplits) {
          div_rows = static_cast<int>(rows);
          div_row0 = valency > 0 ? span_b / valency : row_lo;
        }
      }
    }
  }
  // The hash set needs every staged position's row start: dense rows, or
  // staged splits.
  const bool hashed = kHashed && ids_staged && (valency > 0 || staged);
  if constexpr (kHashed) {
    if (hashed) {
      for (int i = threadIdx.x; i < kDedupSlots; i += blockDim.x) {
        s_table[i] = kSlotEmpty;
      }
      for (int i = threadIdx.x; i < kDedupSlots / 2; i += blockDim.x) {
        s_counts[i] = 0;
      }
    }
  }
  __syncthreads();
  if constexpr (kWeighted) {
    for (int t = threadIdx.x; t < div_rows; t += blockDim.x) {
      const int64_t b = valency > 0 ? t * valency : s_splits[t];
      const int64_t e = valency > 0 ? b + valency : s_splits[t + 1];
      s_div[t] = RowDivisor(s_w + b, static_cast<int>(e - b), combiner);
    }
  }
  // Each id's slice and row.
  int si = 0;
  int64_t p = 0, r = 0, b = 0, e = 0;
  if (o < total_ids) {
    si = block_slice >= 0 ? block_slice
                          : FindSlice(slices, num_slices, o, false);
    const SliceDesc sl = slices[si];
    const FeatureDev f = feats[sl.feature];
    p = sl.id_begin + (o - sl.out_begin);  // input position
    if (staged) {
      const int k = LastRowAtOrBefore32(
          s_splits, static_cast<int>(row_hi - row_lo),
          static_cast<int32_t>(p - span_b));
      r = row_lo + k;
      b = span_b + s_splits[k];
      e = span_b + s_splits[k + 1];
    } else if (f.splits != nullptr) {
      int64_t lo = sl.row_start, hi = sl.row_start + sl.num_rows - 1;
      if (block_slice >= 0) {
        lo = row_lo;
        hi = row_hi;
      }
      r = LastRowAtOrBefore(f.splits, lo, hi, p);
      b = f.splits[r];
      e = f.splits[r + 1];
    } else {
      r = p / f.valency;
      b = r * f.valency;
      e = b + f.valency;
    }
  }
  if constexpr (kHashed) {
    if (hashed) {
      // The block's own ids, then the rest of its first row before them (row
      // start 0) and of its last row after them.
      if (o < total_ids) {
        DedupInsert(s_table, s_counts, s_ids,
                    static_cast<uint32_t>(b - span_b),
                    static_cast<uint32_t>(p - span_b), s_ids[p - span_b]);
      }
      const SliceDesc bsl = slices[block_slice];
      const int64_t o_last = min(blk_first + kExtractBlock, total_ids) - 1;
      const int head = static_cast<int>(bsl.id_begin +
                                        (blk_first - bsl.out_begin) - span_b);
      const int tail = static_cast<int>(bsl.id_begin +
                                        (o_last - bsl.out_begin) - span_b) + 1;
      const int span = static_cast<int>(span_e - span_b);
      const uint32_t last_start =
          valency > 0
              ? static_cast<uint32_t>((tail - 1) / valency * valency)
              : static_cast<uint32_t>(s_splits[row_hi - row_lo]);
      for (int x = threadIdx.x; x < head; x += blockDim.x) {
        DedupInsert(s_table, s_counts, s_ids, 0u, static_cast<uint32_t>(x),
                    s_ids[x]);
      }
      for (int x = tail + threadIdx.x; x < span; x += blockDim.x) {
        DedupInsert(s_table, s_counts, s_ids, last_start,
                    static_cast<uint32_t>(x), s_ids[x]);
      }
    }
  }
  __syncthreads();
  bool bad = false;
  bool view_entry = false;
  if (o < total_ids) {
    const SliceDesc sl = slices[si];
    const FeatureDev f = feats[sl.feature];
    const int n = static_cast<int>(e - b);
    const int q = static_cast<int>(p - b);  // position in the row
    int32_t id;
    float gain;
    bool first;
    if constexpr (kHashed) {
      float unit = 1.0f;
      if (combiner == 1) {
        unit = 1.0f / static_cast<float>(n);
      } else if (combiner == 2) {
        unit = 1.0f / sqrtf(static_cast<float>(n));
      }
      float div = 1.0f;
      if (hashed) {
        id = s_ids[p - span_b];
        const uint32_t h = DedupFind(s_table, s_ids,
                                     static_cast<uint32_t>(b - span_b), id);
        first = (s_table[h] & 2047u) == static_cast<uint32_t>(p - span_b);
        const uint32_t copies =
            (s_counts[h >> 1] >> ((h & 1u) * 16)) & 0xffffu;
        gain = unit;
        if (first) {
          for (uint32_t c = 1; c < copies; ++c) gain = gain + unit;
        }
      } else if (!stage) {
        id = f.ids[p];
        first = true;
        gain = unit;
      } else if (ids_staged) {
        const int64_t off = b - span_b;
        first = ScanRow(s_ids + off, s_ids + off, n, q, false, combiner, true,
                        &div, &id, &gain);
      } else {
        first = ScanRow(f.ids + b, f.ids + b, n, q, false, combiner, true,
                        &div, &id, &gain);
      }
    } else {
      float div = 1.0f;
      if (need_div && r - div_row0 >= 0 && r - div_row0 < div_rows) {
        div = s_div[r - div_row0];
      }
      const bool table_div = !need_div || (r - div_row0 >= 0 &&
                                           r - div_row0 < div_rows);
      if (ids_staged) {
        const int64_t off = b - span_b;
        first = ScanRow(s_ids + off, s_w + off, n, q, true, combiner,
                        table_div, &div, &id, &gain);
      } else {
        first = ScanRow(f.ids + b, f.weights + b, n, q, true, combiner,
                        table_div, &div, &id, &gain);
      }
    }
    const int32_t col = ((id + f.col_shift) & kl.ns_mask) + (id & ~kl.ns_mask) +
                        f.col_offset;
    const bool ok = id >= 0 && col >= 0 &&
                    (kl.col_bound <= 0 || static_cast<int64_t>(col) < kl.col_bound);
    const bool take = ok && first;
    const K seg_part = static_cast<K>(sl.segment) << kl.col_bits;
    keys[o] = take ? (seg_part | ColKey<K>(static_cast<uint32_t>(col), kl))
                   : SentinelKey<K>();
    if (take) {
      const uint32_t sample =
          static_cast<uint32_t>(sl.sample_base + (r - sl.row_start));
      pay[o] = static_cast<uint64_t>(sample) |
               (static_cast<uint64_t>(__float_as_uint(gain)) << 32);
    }
    view_entry = take && (static_cast<int64_t>(static_cast<uint32_t>(col) >>
                                               kl.log2ns) < view_rows);
    bad = !ok;
  }
  const uint64_t m = __ballot(bad);
  if (m != 0 && (threadIdx.x % kWave) == 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(&counters[2]),
              static_cast<unsigned long long>(__popcll(m)));
  }
  if (view_counts != nullptr) {
    const int c = __syncthreads_count(view_entry);
    if (threadIdx.x == 0) view_counts[blk] = static_cast<uint32_t>(c);
  }
}

// ExtractUnique's arguments for a grouped launch: one block per
// kExtractBlock extracted ids.
template <typename K, bool kHashed>
struct ExtractUniqueArgs {
  static constexpr int kBlock = kExtractBlock;
  const SliceDesc* slices;
  int num_slices;
  const FeatureDev* feats;
  const BlockRows* block_rows;
  int64_t total_ids;
  int combiner;
  int rows_of_one;
  KeyLayout kl;
  int64_t view_rows;
  K* keys;
  uint64_t* pay;
  uint32_t* view_counts;
  int64_t* counters;
  __device__ static void Run(const ExtractUniqueArgs& a, uint32_t blk,
                             uint32_t) {
    ExtractUniqueBody<K, kHashed>(blk, a.slices, a.num_slices, a.feats,
                                  a.block_rows, a.total_ids, a.combiner,
                                  a.rows_of_one, a.kl, a.view_rows, a.keys,
                                  a.pay, a.view_counts, a.counters);
  }
};

// The sample view from ExtractUnique's arrays: the entries a block counted
// go, in extraction order, to view_off[block] onwards (positions at or past
// n are not written); positions from *view_total to n get the unused key.
// The grid covers max(extraction blocks, n / 256).
template <typename K>
__device__ __forceinline__ void ViewWriteBody(
    uint32_t blk, const K* keys, const uint64_t* pay, const uint32_t* view_off,
    const uint32_t* view_total, int64_t m, int64_t n, const KeyLayout& kl,
    int64_t view_rows, uint32_t unused_key, uint32_t* vkeys,
    uint64_t* ventries) {
  __shared__ uint32_t smem[kExtractBlock / kWave + 1];
  const int64_t o = static_cast<int64_t>(blk) * blockDim.x + threadIdx.x;
  if (static_cast<int64_t>(blk) * blockDim.x < m) {  // uniform
    bool in_view = false;
    uint32_t p = 0, local = 0;
    if (o < m) {
      const K key = keys[o];
      if (key != SentinelKey<K>()) {
        const K col_mask =
            kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
        DecodeCol<K>(key & col_mask, kl, &p, &local);
        in_view = static_cast<int64_t>(local) < view_rows;
      }
    }
    uint32_t count;
    const uint32_t rank =
        BlockExclusiveScan<uint32_t, kExtractBlock>(in_view ? 1u : 0u, smem,
                                                    &count);
    if (in_view) {
      const int64_t q = static_cast<int64_t>(view_off[blk]) + rank;
      if (q < n) {
        const uint64_t v = pay[o];
        vkeys[q] = static_cast<uint32_t>(v);
        ventries[q] = static_cast<uint64_t>(
                          static_cast<int64_t>(p) * view_rows + local) |
                      (v & 0xffffffff00000000ull);
      }
    }
  }
  if (o < n && o >= static_cast<int64_t>(view_total[0])) {
    vkeys[o] = unused_key;
    ventries[o] = 0;
  }
}

template <typename K>
struct ViewWriteArgs {
  static constexpr int kBlock = kExtractBlock;
  const K* keys;
  const uint64_t* pay;
  const uint32_t* view_off;
  const uint32_t* view_total;
  int64_t m;
  int64_t n;
  KeyLayout kl;
  int64_t view_rows;
  uint32_t unused_key;
  uint32_t* vkeys;
  uint64_t* ventries;
  __device__ static void Run(const ViewWriteArgs& a, uint32_t blk, uint32_t) {
    ViewWriteBody<K>(blk, a.keys, a.pay, a.view_off, a.view_total, a.m, a.n,
                     a.kl, a.view_rows, a.unused_key, a.vkeys, a.ventries);
  }
};

// First pass source of the sort: the extraction arrays, sentinel keys left
// out (duplicates and ids outside the table), so that the later passes and
// the CSR see only the *total entries the first pass took.
template <typename K>
struct UniqueSource {
  const K* keys;
  const uint64_t* pay;
  __device__ bool LoadKey(int64_t i, K* k) const {
    *k = keys[i];
    return *k != SentinelKey<K>();
  }
  __device__ bool Load(int64_t i, K* k, uint64_t* v) const {
    *k = keys[i];
    if (*k == SentinelKey<K>()) return false;
    *v = pay[i];
    return true;
  }
  __device__ void Rejected(int64_t) const {}
};

constexpr int kGroupItems = 8;  // sorted entries per GroupUnique thread

// Over the *total sorted entries: each bucket's first and last position, and
// its distinct columns, counted per block in LDS (one add per wave while
// the wave lies in one bucket, the usual case) and then added with one
// atomic per bucket and block (integer sums: the order does not matter).
// col_heads starts at zero.
template <typename K>
__device__ __forceinline__ void GroupUniqueBody(
    uint32_t blk, const K* skeys, const uint32_t* total, const KeyLayout& kl,
    int num_partitions, int32_t* part_first, int32_t* part_last,
    int32_t* col_heads) {
  __shared__ int32_t s_cnt[256];
  const int64_t n = static_cast<int64_t>(total[0]);
  const int64_t base = static_cast<int64_t>(blk) * 256 * kGroupItems;
  if (base >= n) return;  // uniform
  const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
  auto bucket_of = [&](K key) -> int64_t {
    uint32_t p, local;
    DecodeCol<K>(key & col_mask, kl, &p, &local);
    return static_cast<int64_t>(key >> kl.col_bits) * num_partitions + p;
  };
  s_cnt[threadIdx.x] = 0;
  const int64_t b0 = bucket_of(skeys[base]);
  // Every key this thread needs, loaded before any store (the stores could
  // alias them as far as the compiler knows).
  K cur[kGroupItems], prev[kGroupItems], next[kGroupItems];
#pragma unroll
  for (int it = 0; it < kGroupItems; ++it) {
    const int64_t i = base + static_cast<int64_t>(it) * 256 + threadIdx.x;
    cur[it] = i < n ? skeys[i] : K(0);
    prev[it] = i > 0 && i < n ? skeys[i - 1] : K(0);
    next[it] = i + 1 < n ? skeys[i + 1] : K(0);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kGroupItems; ++it) {
    const int64_t i = base + static_cast<int64_t>(it) * 256 + threadIdx.x;
    const bool active = i < n;
    int64_t bkt = -1;
    bool new_col = false;
    if (active) {
      const K key = cur[it];
      bkt = bucket_of(key);
      bool new_bucket = true;
      new_col = true;
      if (i > 0) {
        new_col = prev[it] != key;
        new_bucket = new_col && bucket_of(prev[it]) != bkt;
      }
      if (new_bucket) part_first[bkt] = static_cast<int32_t>(i);
      bool last = i + 1 == n;
      if (!last) last = next[it] != key && bucket_of(next[it]) != bkt;
      if (last) part_last[bkt] = static_cast<int32_t>(i);
    }
    // The wave's first active lane is lane 0 (positions ascend with lanes).
    const int64_t wave_bkt = __shfl(bkt, 0, kWave);
    const uint64_t heads = __ballot(new_col);
    const uint64_t other = __ballot(active && bkt != wave_bkt);
    if (other == 0) {
      if (__lane_id() == 0 && heads != 0) {
        const int64_t rel = wave_bkt - b0;
        const int c = __popcll(heads);
        if (rel < 256) {
          atomicAdd(&s_cnt[rel], c);
        } else {
          atomicAdd(&col_heads[wave_bkt], c);
        }
      }
    } else if (new_col) {
      const int64_t rel = bkt - b0;  // >= 0: buckets ascend with the key
      if (rel < 256) {
        atomicAdd(&s_cnt[rel], 1);
      } else {
        atomicAdd(&col_heads[bkt], 1);
      }
    }
  }
  __syncthreads();
  if (s_cnt[threadIdx.x] != 0) {
    atomicAdd(&col_heads[b0 + threadIdx.x], s_cnt[threadIdx.x]);
  }
}

template <typename K>
struct GroupUniqueArgs {
  static constexpr int kBlock = 256;
  const K* skeys;
  const uint32_t* total;
  KeyLayout kl;
  int num_partitions;
  int32_t* part_first;
  int32_t* part_last;
  int32_t* col_heads;
  __device__ static void Run(const GroupUniqueArgs& a, uint32_t blk,
                             uint32_t) {
    GroupUniqueBody<K>(blk, a.skeys, a.total, a.kl, a.num_partitions,
                       a.part_first, a.part_last, a.col_heads);
  }
};

// One thread per sorted entry: the CSR position is the bucket's planned
// start plus the entry's rank in its bucket (every entry is kept; those
// past the bucket's room in the static buffer are not written).
template <typename K>
__device__ __forceinline__ void ScatterUniqueBody(
    uint32_t blk, const K* skeys, const uint64_t* spay, const uint32_t* total,
    const KeyLayout& kl, const FillParams& fp, int32_t bps,
    const int32_t* part_first, const FillPlan* plans, int32_t* eid,
    int32_t* sid, float* gains) {
  const int64_t i = static_cast<int64_t>(blk) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(total[0])) return;
  const K key = skeys[i];
  const K col_mask = kl.col_bits >= 64 ? ~K(0) : ((K(1) << kl.col_bits) - 1);
  uint32_t p, local;
  DecodeCol<K>(key & col_mask, kl, &p, &local);
  const int64_t seg = static_cast<int64_t>(key >> kl.col_bits);
  const int64_t bucket = seg * fp.num_partitions + p;
  const int64_t k = i - part_first[bucket];
  const FillPlan pl = plans[bucket];
  if (k >= pl.fit) return;
  const int64_t d = seg / fp.segs_per_device;
  const int64_t pos = d * fp.coo_size + pl.start + k;
  const uint64_t v = spay[i];
  eid[pos] = static_cast<int32_t>(local);
  sid[pos] = static_cast<int32_t>(static_cast<uint32_t>(v) %
                                  static_cast<uint32_t>(bps));
  gains[pos] = __uint_as_float(static_cast<uint32_t>(v >> 32));
}

template <typename K>
struct ScatterUniqueArgs {
  static constexpr int kBlock = 256;
  const K* skeys;
  const uint64_t* spay;
  const uint32_t* total;
  KeyLayout kl;
  FillParams fp;
  int32_t bps;
  const int32_t* part_first;
  const FillPlan* plans;
  int32_t* eid;
  int32_t* sid;
  float* gains;
  __device__ static void Run(const ScatterUniqueArgs& a, uint32_t blk,
                             uint32_t) {
    ScatterUniqueBody<K>(blk, a.skeys, a.spay, a.total, a.kl, a.fp, a.bps,
                         a.part_first, a.plans, a.eid, a.sid, a.gains);
  }
};

// ---------------------------------------------------------------------------
// Host planning.
// ---------------------------------------------------------------------------

struct Plan {
  int L, G, S, NS, log2ns, rp_per_seg;
  int64_t coo_size, bps, batch_for_device;
  int64_t total_ids, total_rows;
  std::vector<SliceDesc> slices;
  bool rows_monotone;  // features' sample rows non-decreasing per segment
  bool rows_disjoint;  // and no sample row shared by two features
  KeyLayout kl;
  bool wide_keys;
  int row_key_seg_shift;
  int row_bits;
};

int MakePlan(const scemb_feature_t* feats, int nf,
             const scemb_preprocess_options_t* o, Plan* pl,
             std::vector<std::vector<int64_t>>* splits_cache) {
  if (o == nullptr || (nf > 0 && feats == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null arguments");
  }
  // PreprocessSparseDenseMatmulInputOptions::Validate
  // (input_preprocessing_util.cc:490-522) and the empty-input check of
  // input_preprocessing.cc:815-817, in their order and with their messages.
  const int L = o->local_device_count, G = o->global_device_count,
            S = o->num_sc_per_device;
  if (L <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "local_device_count must be greater than 0, but got " +
                    std::to_string(L));
  }
  if (G <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "global_device_count must be greater than 0, but got " +
                    std::to_string(G));
  }
  if (G < L) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "global_device_count must be greater than or equal to "
                "local_device_count, but got " +
                    std::to_string(G) + " vs " + std::to_string(L));
  }
  if (S <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "num_sc_per_device must be greater than 0, but got " +
                    std::to_string(S));
  }
  const int64_t ns = static_cast<int64_t>(S) * G;
  if (ns > (1 << 20) || (ns & (ns - 1)) != 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "Total number of SparseCores (" + std::to_string(ns) +
                    ") must be a power of 2.");
  }
  if (nf <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "input_batches cannot be empty.");
  }
  if (o->combiner < 0 || o->combiner > 2) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unknown combiner");
  }
  if (o->coo_buffer_size_per_device <= 0 ||
      o->coo_buffer_size_per_device >= 0x7fffffff) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "coo buffer size is out of the valid range (0, INT_MAX)");
  }
  if (o->max_ids_per_partition <= 0 || o->max_unique_ids_per_partition <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "id limits must be positive");
  }
  if (o->enable_minibatching) {
    if (o->minibatching_pass < 0 || o->minibatching_pass > 2) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "minibatching_pass must be 0, 1 or 2");
    }
  }
  pl->L = L;
  pl->G = G;
  pl->S = S;
  pl->NS = static_cast<int>(ns);
  pl->log2ns = BitWidth(static_cast<uint64_t>(ns)) - 1;
  pl->rp_per_seg = std::max(pl->NS, kAlign);
  pl->coo_size = o->coo_buffer_size_per_device;
  int64_t bfd = 0;
  for (int f = 0; f < nf; ++f) {
    if (feats[f].num_rows < 0 || feats[f].nnz < 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "negative feature size");
    }
    if (feats[f].row_splits == nullptr && feats[f].valency < 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "negative valency");
    }
    bfd += feats[f].num_rows / L;
  }
  if (bfd > kDataMask26) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "The total local batch size for device (including stacked "
                "tables) exceeds the maximum limit supported by the "
                "SparseCore CooFormat sorting key (67108863).");
  }
  if (bfd % S != 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "batch_size_for_device must be divisible by num_sc_per_device");
  }
  if (bfd < static_cast<int64_t>(S) * nf) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "Batch size must be greater or equal to the number of features "
                "stacked together (per feature slice).");
  }
  pl->batch_for_device = bfd;
  pl->bps = bfd / S;
  // Host row splits for planning.
  splits_cache->assign(nf, {});
  for (int f = 0; f < nf; ++f) {
    const scemb_feature_t& ft = feats[f];
    if (ft.row_splits != nullptr && ft.row_splits_host == nullptr) {
      auto& v = (*splits_cache)[f];
      v.resize(ft.num_rows + 1);
      SCEMB_HIP(hipMemcpy(v.data(), ft.row_splits,
                          sizeof(int64_t) * (ft.num_rows + 1),
                          hipMemcpyDeviceToHost));
    }
  }
  auto split_at = [&](int f, int64_t r) -> int64_t {
    const scemb_feature_t& ft = feats[f];
    if (ft.row_splits == nullptr) return r * ft.valency;
    if (ft.row_splits_host != nullptr) return ft.row_splits_host[r];
    return (*splits_cache)[f][r];
  };
  pl->slices.clear();
  int64_t out = 0, rows = 0;
  pl->rows_monotone = true;
  pl->rows_disjoint = true;
  for (int d = 0; d < L; ++d) {
    for (int s = 0; s < S; ++s) {
      int64_t prev_last = -1;
      for (int f = 0; f < nf; ++f) {
        const scemb_feature_t& ft = feats[f];
        const int64_t per_split = ft.num_rows / (static_cast<int64_t>(L) * S);
        const int64_t start = (static_cast<int64_t>(d) * S + s) * per_split;
        const int64_t end = std::min(ft.num_rows, start + per_split);
        SliceDesc sd;
        sd.id_begin = split_at(f, start);
        const int64_t id_end = split_at(f, end);
        if (id_end < sd.id_begin || id_end > ft.nnz) {
          return Fail(SCEMB_ERR_INVALID_ARGUMENT, "row splits out of range");
        }
        sd.out_begin = out;
        sd.row_start = start;
        sd.row_prefix = rows;
        sd.num_rows = static_cast<int32_t>(end - start);
        sd.sample_base = static_cast<int32_t>(
            s * pl->bps + ft.row_offset / (static_cast<int64_t>(G) * S));
        sd.feature = f;
        sd.segment = d * S + s;
        if (sd.num_rows > 0) {
          if (sd.sample_base < prev_last) pl->rows_monotone = false;
          if (sd.sample_base <= prev_last) pl->rows_disjoint = false;
          prev_last = sd.sample_base + sd.num_rows - 1;
          pl->slices.push_back(sd);
        }
        out += id_end - sd.id_begin;
        rows += sd.num_rows;
      }
    }
  }
  pl->total_ids = out;
  pl->total_rows = rows;
  // With weights the sort key carries the extraction position, not the
  // sample row, so duplicates of one (row, column) are adjacent after the
  // sort only when rows ascend in extraction order. The reference merges a
  // duplicate into the last kept entry even across a dropped one
  // (sort_and_group_coo_tensors_impl.h:251-259); the grouping here merges
  // adjacent duplicates, which is the same whenever rows ascend. Features in
  // row_offset order (as GetStackedTableMetadata gives them) always do.
  if (o->has_variable_weights && o->allow_id_dropping && !pl->rows_monotone) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "weighted features with id dropping must come in row_offset "
                "order (sample rows ascending across the stack's features)");
  }
  if (out >= (int64_t{1} << 31) - 1) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "too many ids in one stack");
  }
  KeyLayout& kl = pl->kl;
  kl.log2ns = pl->log2ns;
  kl.ns_mask = pl->NS - 1;
  kl.col_bound = o->col_id_bound;
  if (o->col_id_bound > 0) {
    kl.compact = true;
    kl.local_bits = BitWidth(static_cast<uint64_t>(o->col_id_bound - 1) >> pl->log2ns);
    kl.col_bits = kl.local_bits + pl->log2ns;
  } else {
    kl.compact = false;
    kl.local_bits = 32 - pl->log2ns;
    kl.col_bits = 32;
  }
  kl.seg_bits = BitWidth(static_cast<uint64_t>(L) * S - 1);
  kl.mb_bits = o->enable_minibatching && o->minibatching_pass > 0
                   ? BitWidth(kMaxMinibatches - 1)
                   : 0;
  pl->wide_keys = kl.col_bits + kl.mb_bits + kl.seg_bits > 31;
  const int sample_bits = BitWidth(static_cast<uint64_t>(std::max<int64_t>(bfd - 1, 0)));
  pl->row_key_seg_shift = sample_bits;
  pl->row_bits = sample_bits + kl.seg_bits;
  if (pl->row_bits > 32) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "too many segments");
  }
  return 0;
}

struct Buffers {
  void* keys;
  void* keys_alt;
  uint32_t* vals;
  uint32_t* vals_alt;
  uint64_t* row_gain;
  BlockRows* block_rows;
  uint32_t* row_keys;
  uint32_t* row_keys_alt;
  uint32_t* srows;
  float* sgains;
  uint64_t* flags;
  uint64_t* scan;
  uint64_t* totals;
  uint32_t* run_pos;
  float* run_gain;
  uint32_t* keep;
  uint32_t* keep_scan;
  int32_t* part_first;
  int32_t* part_last;
  BucketStats* bstats;
  FillPlan* plans;
  SliceDesc* slices;
  FeatureDev* feats;
};

// Copies of small host arrays into device memory through kernel arguments
// (up to kUploadWords words per launch), ordered on `stream` like any
// kernel: nothing waits on the host side and the source may be released as
// soon as the launch call returns.
constexpr int kUploadWords = 768;
struct UploadChunk {
  uint32_t words[kUploadWords];
};

__global__ __launch_bounds__(256) void UploadKernel(UploadChunk c, int n,
                                                    uint32_t* dst) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = c.words[i];
}

// The set-up of one call in one launch, when both descriptor arrays fit in
// one chunk: zeroed counters, partition bounds at -1, zeroed split counts,
// and the slice and feature descriptors copied from the kernel arguments.
struct SetupArgs {
  int32_t* stats;  // the stats slots before the counters
  int64_t stats_words;
  int64_t* counters;
  int32_t* part_first;
  int32_t* part_last;
  int64_t num_buckets;
  int32_t* split_words;  // may be null
  int64_t num_split_words;
  uint32_t* slices;
  uint32_t* feats;
  int32_t slice_words;
  int32_t feat_words;
  // BlockBounds of the extraction, read from the descriptors in the chunk.
  int32_t num_slices;
  int64_t total_ids;
  int64_t extract_blocks;
  int64_t total_rows;
  BlockRows* block_rows;
};

__global__ __launch_bounds__(256) void SetupKernel(UploadChunk c,
                                                   SetupArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < a.stats_words) a.stats[i] = 0;
  if (i < kNumCounters) a.counters[i] = 0;
  if (i < a.num_buckets) {
    a.part_first[i] = -1;
    a.part_last[i] = -1;
  }
  if (a.split_words != nullptr && i < a.num_split_words) a.split_words[i] = 0;
  if (i < a.slice_words) {
    a.slices[i] = c.words[i];
  } else if (i < a.slice_words + a.feat_words) {
    a.feats[i - a.slice_words] = c.words[i];
  }
  if (a.extract_blocks > 0) {
    const SliceDesc* sl = reinterpret_cast<const SliceDesc*>(c.words);
    if (i < a.extract_blocks) {
      BlockSliceOf(sl, a.num_slices, a.total_ids, i, a.block_rows);
    }
    if (i < a.total_rows) {
      RowBlockBounds(
          sl, a.num_slices,
          reinterpret_cast<const FeatureDev*>(c.words + a.slice_words),
          a.total_ids, i, a.block_rows);
    }
  }
}

int UploadBytes(const void* src, size_t bytes, void* dst,
                hipStream_t stream) {
  if (bytes == 0) return 0;
  if (bytes % 4 != 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "upload size not word aligned");
  }
  const uint32_t* w = static_cast<const uint32_t*>(src);
  uint32_t* d = static_cast<uint32_t*>(dst);
  const size_t total = bytes / 4;
  for (size_t off = 0; off < total; off += kUploadWords) {
    const int n = static_cast<int>(
        total - off < static_cast<size_t>(kUploadWords) ? total - off
                                                         : kUploadWords);
    UploadChunk c;
    std::memcpy(c.words, w + off, sizeof(uint32_t) * n);
    hipLaunchKernelGGL(UploadKernel, dim3(1), dim3(256), 0, stream, c, n,
                       d + off);
    SCEMB_LAUNCH_CHECK();
  }
  return 0;
}

// What the set-up of one call prepares besides the stats and counters.
struct SetupTargets {
  int32_t* part_first;  // [num_buckets] set to -1
  int32_t* part_last;
  int64_t num_buckets;
  int32_t* zero_words;  // [num_zero_words] cleared (may be null)
  int64_t num_zero_words;
  SliceDesc* slices;    // descriptor copies
  FeatureDev* feats;
  BlockRows* block_rows;  // row bounds of the extraction blocks
  int64_t extract_blocks;  // 0: nothing to extract
};

// Checks the feature pointers, then enqueues the set-up: the stats slots
// before the counters and the counters cleared, partition bounds at -1, the
// zero words cleared, the slice and feature descriptors copied and the
// extraction blocks' row bounds computed. One launch when the descriptors
// fit one chunk of kernel arguments (no pageable host copy, no host
// synchronisation); otherwise one launch per part.
int EnqueueSetup(const scemb_feature_t* feats, int nf,
                 const scemb_preprocess_options_t* o, const Plan& pl,
                 int64_t counters_off, int32_t* stats, int64_t* counters,
                 const SetupTargets& t, hipStream_t stream) {
  std::vector<FeatureDev> fd(nf);
  for (int f = 0; f < nf; ++f) {
    fd[f].ids = feats[f].ids;
    fd[f].weights = o->has_variable_weights ? feats[f].weights : nullptr;
    fd[f].splits = feats[f].row_splits;
    fd[f].valency = feats[f].valency;
    fd[f].col_offset = feats[f].col_offset;
    fd[f].col_shift = feats[f].col_shift;
    if (feats[f].nnz > 0 && feats[f].ids == nullptr) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null ids");
    }
    if (o->has_variable_weights && feats[f].nnz > 0 &&
        feats[f].weights == nullptr) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "weights required for every feature of a weighted stack");
    }
  }
  const size_t slice_bytes = sizeof(SliceDesc) * pl.slices.size();
  const size_t feat_bytes = sizeof(FeatureDev) * nf;
  const int num_slices = static_cast<int>(pl.slices.size());
  // Rows of dense features bound no block: the row-side pass runs only when
  // some feature is ragged.
  bool any_ragged = false;
  for (int f = 0; f < nf; ++f) any_ragged |= feats[f].row_splits != nullptr;
  const int64_t bound_rows =
      t.extract_blocks > 0 && any_ragged ? pl.total_rows : 0;
  if (slice_bytes + feat_bytes <= sizeof(UploadChunk)) {
    UploadChunk c;
    std::memcpy(c.words, pl.slices.data(), slice_bytes);
    std::memcpy(reinterpret_cast<char*>(c.words) + slice_bytes, fd.data(),
                feat_bytes);
    SetupArgs a;
    a.stats = stats;
    a.stats_words = counters_off;
    a.counters = counters;
    a.part_first = t.part_first;
    a.part_last = t.part_last;
    a.num_buckets = t.num_buckets;
    a.split_words = t.zero_words;
    a.num_split_words = t.zero_words != nullptr ? t.num_zero_words : 0;
    a.slices = reinterpret_cast<uint32_t*>(t.slices);
    a.feats = reinterpret_cast<uint32_t*>(t.feats);
    a.slice_words = static_cast<int32_t>(slice_bytes / 4);
    a.feat_words = static_cast<int32_t>(feat_bytes / 4);
    a.num_slices = num_slices;
    a.total_ids = pl.total_ids;
    a.extract_blocks = t.extract_blocks;
    a.total_rows = bound_rows;
    a.block_rows = t.block_rows;
    const int64_t work = std::max<int64_t>(
        {int64_t{kNumCounters}, counters_off, t.num_buckets,
         a.num_split_words,
         static_cast<int64_t>((slice_bytes + feat_bytes) / 4),
         a.extract_blocks, a.total_rows});
    hipLaunchKernelGGL(SetupKernel, dim3(CeilDiv(work, 256)), dim3(256), 0,
                       stream, c, a);
    SCEMB_LAUNCH_CHECK();
    return 0;
  }
  hipLaunchKernelGGL(FillI32, dim3(CeilDiv(counters_off, 256)), dim3(256), 0,
                     stream, stats, counters_off, 0);
  SCEMB_LAUNCH_CHECK();
  hipLaunchKernelGGL(ZeroI64, dim3(1), dim3(64), 0, stream, counters,
                     kNumCounters);
  SCEMB_LAUNCH_CHECK();
  int st = UploadBytes(pl.slices.data(), slice_bytes, t.slices, stream);
  if (st != 0) return st;
  st = UploadBytes(fd.data(), feat_bytes, t.feats, stream);
  if (st != 0) return st;
  hipLaunchKernelGGL(FillI32, dim3(CeilDiv(t.num_buckets, 256)), dim3(256), 0,
                     stream, t.part_first, t.num_buckets, -1);
  SCEMB_LAUNCH_CHECK();
  hipLaunchKernelGGL(FillI32, dim3(CeilDiv(t.num_buckets, 256)), dim3(256), 0,
                     stream, t.part_last, t.num_buckets, -1);
  SCEMB_LAUNCH_CHECK();
  if (t.zero_words != nullptr && t.num_zero_words > 0) {
    hipLaunchKernelGGL(FillI32, dim3(CeilDiv(t.num_zero_words, 256)),
                       dim3(256), 0, stream, t.zero_words, t.num_zero_words,
                       0);
    SCEMB_LAUNCH_CHECK();
  }
  if (t.extract_blocks > 0) {
    hipLaunchKernelGGL(BlockBounds,
                       dim3(CeilDiv(std::max(t.extract_blocks, bound_rows),
                                    256)),
                       dim3(256), 0, stream, t.slices, num_slices, t.feats,
                       pl.total_ids, t.extract_blocks, bound_rows,
                       t.block_rows);
    SCEMB_LAUNCH_CHECK();
  }
  return 0;
}

template <typename K>
int RunPipeline(const scemb_feature_t* feats, int nf,
                const scemb_preprocess_options_t* o,
                const scemb_preprocess_output_t* out, const Plan& pl,
                Arena& ws, hipStream_t stream) {
  const int64_t M = pl.total_ids;
  const bool minibatching = o->enable_minibatching != 0;
  const int pass = minibatching ? o->minibatching_pass : 0;
  const int64_t num_buckets = static_cast<int64_t>(pl.L) * pl.S *
                              (int64_t{1} << pl.kl.mb_bits) * pl.NS;
  const bool need_row_pass = !o->has_variable_weights && !pl.rows_monotone;
  Buffers b;
  b.keys = ws.Take<K>(M);
  b.keys_alt = ws.Take<K>(M);
  b.vals = ws.Take<uint32_t>(M);
  b.vals_alt = ws.Take<uint32_t>(M);
  b.row_gain = ws.Take<uint64_t>(M);
  const int64_t extract_blocks = CeilDiv(M, kExtractBlock);
  b.block_rows = ws.Take<BlockRows>(extract_blocks);
  b.row_keys = need_row_pass ? ws.Take<uint32_t>(M) : nullptr;
  b.row_keys_alt = need_row_pass ? ws.Take<uint32_t>(M) : nullptr;
  b.srows = ws.Take<uint32_t>(M);
  b.sgains = ws.Take<float>(M);
  b.flags = ws.Take<uint64_t>(M);
  b.scan = ws.Take<uint64_t>(M);
  b.totals = ws.Take<uint64_t>(2);
  b.run_pos = ws.Take<uint32_t>(M + 1);
  b.run_gain = ws.Take<float>(M);
  b.keep = ws.Take<uint32_t>(M + 1);
  b.keep_scan = ws.Take<uint32_t>(M + 1);
  b.part_first = ws.Take<int32_t>(num_buckets);
  b.part_last = ws.Take<int32_t>(num_buckets);
  b.bstats = ws.Take<BucketStats>(num_buckets);
  b.plans = ws.Take<FillPlan>(num_buckets);
  b.slices = ws.Take<SliceDesc>(static_cast<int64_t>(pl.slices.size()));
  b.feats = ws.Take<FeatureDev>(nf);
  // Pass 0 of minibatching: the bucket counts its runs give (used only when
  // a limit is exceeded).
  const int64_t split_cells =
      static_cast<int64_t>(pl.L) * pl.S * kMaxMinibatches * pl.NS;
  BucketStats* split_counts =
      minibatching && pass == 0 ? ws.Take<BucketStats>(split_cells) : nullptr;
  // Per-row divisors of weighted mean / sqrtn.
  float* divisors = o->has_variable_weights && o->combiner != 0
                        ? ws.Take<float>(pl.total_rows)
                        : nullptr;
  ViewParts view{};
  // The bucket pass writes no CSR, so no view either. (Measuring, the view's
  // buffers are null: `has_view` says whether there is one.)
  const bool has_view = o->build_sample_view && !(minibatching && pass == 1);
  if (has_view) {
    if (pl.L != 1 || pl.G != 1) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "the sample view needs one local and one global device");
    }
    if (!pl.rows_monotone) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "the sample view needs features whose sample rows do not "
                  "overlap (row_offset order)");
    }
    if (o->table_rows <= 0 || o->table_rows % pl.NS != 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "table_rows must be a positive multiple of the partitions");
    }
    view.entry = ws.Take<uint64_t>(M);
    view.pos = ws.Take<uint32_t>(M + 1);
    view.rows_per_partition = o->table_rows / pl.NS;
  }
  const bool measuring = ws.measuring();
  const int64_t counters_off = RoundUp(2 * static_cast<int64_t>(pl.L) * pl.NS +
                                       static_cast<int64_t>(pl.L) * pl.S, 2);
  uint64_t split = 0;
  int num_minibatches = 1;
  if (minibatching && pass == 2) {
    split = o->minibatching_split;
    if ((split >> (kMaxMinibatches - 1)) != 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "minibatching_split has at most 63 bits");
    }
    num_minibatches = __builtin_popcountll(split) + 1;
  }
  int64_t* counters = nullptr;
  if (!measuring) {
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    if (out == nullptr || out->row_pointers == nullptr || out->stats == nullptr ||
        out->embedding_ids == nullptr || out->sample_ids == nullptr ||
        out->gains == nullptr) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null output buffer");
    }
    if (view.entry != nullptr &&
        (out->view_keys == nullptr || out->view_entries == nullptr)) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null sample view buffer");
    }
    counters = reinterpret_cast<int64_t*>(out->stats + counters_off);
    if ((reinterpret_cast<uintptr_t>(counters) & 7u) != 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "stats buffer must be 8-byte aligned");
    }
    const SetupTargets tg{b.part_first, b.part_last, num_buckets,
                          reinterpret_cast<int32_t*>(split_counts),
                          split_counts != nullptr
                              ? split_cells * static_cast<int64_t>(
                                                  sizeof(BucketStats) / 4)
                              : 0,
                          b.slices, b.feats, b.block_rows,
                          M > 0 ? extract_blocks : 0};
    const int su = EnqueueSetup(feats, nf, o, pl, counters_off, out->stats,
                                counters, tg, stream);
    if (su != 0) return su;
    if (divisors != nullptr && pl.total_rows > 0) {
      hipLaunchKernelGGL(RowDivisors, dim3(CeilDiv(pl.total_rows, 256)),
                         dim3(256), 0, stream, b.slices,
                         static_cast<int>(pl.slices.size()), b.feats,
                         pl.total_rows, o->combiner, divisors);
      SCEMB_LAUNCH_CHECK();
    }
    if (M > 0) {
      const int num_slices = static_cast<int>(pl.slices.size());
      hipLaunchKernelGGL((ExtractIds<K>), dim3(extract_blocks),
                         dim3(kExtractBlock), 0, stream, b.slices, num_slices,
                         b.feats, b.block_rows, M, o->combiner,
                         o->has_variable_weights ? 1 : 0, divisors, pl.kl,
                         static_cast<K*>(b.keys), b.vals, b.row_gain,
                         b.row_keys, pl.row_key_seg_shift, counters);
      SCEMB_LAUNCH_CHECK();
    }
  }
  // Sort: optional row pass, then the column key. One extra key bit keeps the
  // all-ones sentinel of rejected ids strictly above every valid key.
  const int sort_bits = pl.kl.col_bits + pl.kl.mb_bits + pl.kl.seg_bits + 1;
  K* skeys = static_cast<K*>(b.keys);
  uint32_t* sidx = b.vals;
  int st = 0;
  if (need_row_pass) {
    bool alt = false;
    st = RadixSortPairs<uint32_t, uint32_t>(b.row_keys, b.vals, b.row_keys_alt,
                                            b.vals_alt, M, 0, pl.row_bits, ws,
                                            stream, &alt);
    if (st != 0) return st;
    uint32_t* idx = alt ? b.vals_alt : b.vals;
    if (!measuring && M > 0) {
      hipLaunchKernelGGL((GatherKeys<K>), dim3(CeilDiv(M, 256)), dim3(256), 0,
                         stream, static_cast<K*>(b.keys), idx, M,
                         static_cast<K*>(b.keys_alt));
      SCEMB_LAUNCH_CHECK();
    }
    // Keys now in keys_alt (row order), indices in idx.
    uint32_t* idx_other = alt ? b.vals : b.vals_alt;
    bool alt2 = false;
    st = RadixSortPairs<K, uint32_t>(static_cast<K*>(b.keys_alt), idx,
                                     static_cast<K*>(b.keys), idx_other, M, 0,
                                     sort_bits, ws, stream, &alt2);
    if (st != 0) return st;
    skeys = alt2 ? static_cast<K*>(b.keys) : static_cast<K*>(b.keys_alt);
    sidx = alt2 ? idx_other : idx;
  } else {
    bool alt = false;
    st = RadixSortPairs<K, uint32_t>(static_cast<K*>(b.keys), b.vals,
                                     static_cast<K*>(b.keys_alt), b.vals_alt,
                                     M, 0, sort_bits, ws, stream, &alt);
    if (st != 0) return st;
    skeys = alt ? static_cast<K*>(b.keys_alt) : static_cast<K*>(b.keys);
    sidx = alt ? b.vals_alt : b.vals;
  }
  if (!measuring && M > 0) {
    hipLaunchKernelGGL((GroupFlags<K>), dim3(CeilDiv(M, 256)), dim3(256), 0,
                       stream, skeys, sidx, b.row_gain, M, pl.kl, pl.NS,
                       b.srows, b.sgains, b.flags, b.part_first, b.part_last,
                       view.entry);
    SCEMB_LAUNCH_CHECK();
  }
  st = ExclusiveScan<uint64_t>(b.flags, b.scan, M, b.totals, ws, stream);
  if (st != 0) return st;
  if (!measuring && M > 0) {
    hipLaunchKernelGGL((RunPositions<K>), dim3(CeilDiv(M, 256)), dim3(256), 0,
                       stream, skeys, b.flags, b.scan, M, b.run_pos);
    SCEMB_LAUNCH_CHECK();
  }
  // The first minibatching pass never drops (it only decides whether
  // minibatching is needed, sort_and_group_coo_tensors_impl.h:222-226).
  const Limits lim{o->max_ids_per_partition, o->max_unique_ids_per_partition,
                   minibatching && pass == 0 ? 0 : o->allow_id_dropping};
  if (!measuring) {
    if (M > 0) {
      hipLaunchKernelGGL((RunReduce<K>), dim3(CeilDiv(M + 1, 256)), dim3(256),
                         0, stream, skeys, b.sgains, b.flags, b.scan,
                         b.run_pos, b.totals, M, pl.kl, pl.NS, b.part_first,
                         lim, b.run_gain, b.keep, counters);
      SCEMB_LAUNCH_CHECK();
    } else {
      hipLaunchKernelGGL(FillI32, dim3(1), dim3(256), 0, stream,
                         reinterpret_cast<int32_t*>(b.keep), int64_t{1}, 0);
      SCEMB_LAUNCH_CHECK();
    }
  }
  st = ExclusiveScan<uint32_t>(b.keep, b.keep_scan, M + 1, nullptr, ws,
                               stream);
  if (st != 0) return st;
  if (measuring) {
    // The view's scan runs last; size its temporaries at the same point.
    return has_view ? ExclusiveScan<uint32_t>(nullptr, nullptr, M + 1,
                                              nullptr, ws, stream)
                    : 0;
  }
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  // Without minibatching the fill plan's single block reduces the bucket
  // stats first (one launch less).
  BucketReduceArgs bra{b.part_first, b.part_last, b.flags, b.scan,
                       b.keep_scan, minibatching ? 0 : num_buckets, b.bstats,
                       nullptr};
  if (minibatching) {
    hipLaunchKernelGGL(BucketReduce, dim3(CeilDiv(num_buckets, 256)),
                       dim3(256), 0, stream, b.part_first, b.part_last,
                       b.flags, b.scan, b.keep_scan, num_buckets, b.bstats);
    SCEMB_LAUNCH_CHECK();
  }
  FillParams fp;
  fp.local_devices = pl.L;
  fp.segs_per_device = pl.S;
  fp.num_partitions = pl.NS;
  fp.rp_per_segment = pl.rp_per_seg;
  fp.coo_size = pl.coo_size;
  fp.max_ids = o->max_ids_per_partition;
  fp.max_unique = o->max_unique_ids_per_partition;
  fp.allow_dropping = o->allow_id_dropping;
  fp.mb_bits = pl.kl.mb_bits;
  fp.absolute = minibatching ? 1 : 0;
  fp.num_minibatches = num_minibatches;
  // Minibatch of each bucket: the boundary between buckets b - 1 and b is
  // where the two halves of one node of the merge tree meet (level t =
  // trailing zeros of b plus one, node b >> t); the buckets on either side
  // fall into different minibatches iff that node is split
  // (minibatching_splits_impl.h:84-131).
  {
    int mb = 0;
    fp.minibatch_of[0] = 0;
    for (int bkt = 1; bkt < kMaxMinibatches; ++bkt) {
      const int t = __builtin_ctz(static_cast<unsigned>(bkt)) + 1;
      int index = 0;
      for (int l = 1; l < t; ++l) index += kMaxMinibatches >> l;
      index += bkt >> t;
      mb += static_cast<int>((split >> index) & 1u);
      fp.minibatch_of[bkt] = static_cast<uint8_t>(mb);
    }
  }
  int32_t* stat_max_ids = out->stats;
  int32_t* stat_max_unique = out->stats + static_cast<int64_t>(pl.L) * pl.NS;
  int32_t* stat_required = out->stats + 2 * static_cast<int64_t>(pl.L) * pl.NS;
  if (minibatching && pass == 1) {
    const int64_t cells = static_cast<int64_t>(pl.L) * pl.S * pl.NS;
    hipLaunchKernelGGL(MinibatchSplit, dim3(CeilDiv(cells, 64)), dim3(64), 0,
                       stream, b.bstats, fp, 0, counters);
    SCEMB_LAUNCH_CHECK();
    if (M > 0) {
      hipLaunchKernelGGL(StoreTotal, dim3(1), dim3(1), 0, stream, b.totals,
                         counters);
      SCEMB_LAUNCH_CHECK();
    }
    return 0;
  }
  if (minibatching) {
    const int64_t cells = static_cast<int64_t>(pl.S) *
                          (int64_t{1} << pl.kl.mb_bits) * pl.NS;
    if (cells <= kLdsPlanCells && pl.S <= kMaxMinibatches) {
      hipLaunchKernelGGL(FillPlanMinibatchLds, dim3(pl.L), dim3(256), 0,
                         stream, b.bstats, fp, pass, out->row_pointers,
                         b.plans, stat_max_ids, stat_max_unique,
                         stat_required, counters);
    } else {
      hipLaunchKernelGGL(FillPlanMinibatch, dim3(1), dim3(64), 0, stream,
                         b.bstats, fp, pass, out->row_pointers, b.plans,
                         stat_max_ids, stat_max_unique, stat_required,
                         counters);
    }
  } else {
    hipLaunchKernelGGL(FillPlanKernel, dim3(1), dim3(256), 0, stream, b.bstats,
                       fp, out->row_pointers, b.plans, stat_max_ids,
                       stat_max_unique, stat_required, counters, bra);
  }
  SCEMB_LAUNCH_CHECK();
  if (split_counts != nullptr && M > 0) {
    // Both kernels return at once unless the fill plan flagged a limit.
    const int64_t grid = std::min<int64_t>(CeilDiv(M, 4096), 1024);
    hipLaunchKernelGGL((BucketCountsOfRuns<K>), dim3(grid), dim3(256), 0,
                       stream, skeys, b.run_pos, b.flags, b.totals, pl.kl,
                       pl.NS, split_cells, counters, split_counts);
    SCEMB_LAUNCH_CHECK();
    FillParams sp = fp;
    sp.mb_bits = BitWidth(kMaxMinibatches - 1);
    const int64_t cells = static_cast<int64_t>(pl.L) * pl.S * pl.NS;
    hipLaunchKernelGGL(MinibatchSplit, dim3(CeilDiv(cells, 64)), dim3(64), 0,
                       stream, split_counts, sp, 1, counters);
    SCEMB_LAUNCH_CHECK();
  }
  // GroupFlags cleared the view's slots.
  if (view.entry != nullptr) view.sidx = sidx;
  if (M > 0) {
    hipLaunchKernelGGL((ScatterRuns<K>), dim3(CeilDiv(M, 256)), dim3(256), 0,
                       stream, skeys, b.srows, b.run_pos, b.run_gain, b.keep,
                       b.keep_scan, b.totals, M, pl.kl, fp,
                       static_cast<int32_t>(pl.bps), b.bstats, b.plans,
                       out->embedding_ids, out->sample_ids, out->gains, view);
    SCEMB_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(WritePadding, dim3(CeilDiv(num_buckets * kAlign, 256)),
                     dim3(256), 0, stream, b.plans, num_buckets, fp,
                     out->embedding_ids, out->sample_ids, out->gains,
                     M > 0 ? b.totals : nullptr, nullptr, counters);
  SCEMB_LAUNCH_CHECK();
  if (view.entry != nullptr) {
    hipLaunchKernelGGL(MarkEntries, dim3(CeilDiv(M + 1, 256)), dim3(256), 0,
                       stream, view.entry, M, view.pos);
    SCEMB_LAUNCH_CHECK();
    st = ExclusiveScan<uint32_t>(view.pos, view.pos, M + 1, nullptr, ws,
                                 stream);
    if (st != 0) return st;
    const int64_t n = pl.coo_size;
    const int64_t grid = M > n ? M : n;
    if (grid > 0) {
      hipLaunchKernelGGL(ViewCompact, dim3(CeilDiv(grid, 256)), dim3(256), 0,
                         stream, view.pos, b.row_gain, view.entry, M, n,
                         static_cast<uint32_t>(pl.batch_for_device),
                         out->view_keys, out->view_entries);
      SCEMB_LAUNCH_CHECK();
    }
  }
  return 0;
}

// The route of grouping at extraction: set-up, ExtractUnique, the sample
// view (a scan of the blocks' counts, then ViewWrite), a stable LSD radix
// sort of the distinct (row, column) entries on the key, whose first pass
// leaves out the sentinel keys, then GroupUnique, the fill plan,
// ScatterUnique and the padding. Same outputs as RunPipeline for the calls
// Preprocess routes here.
// One stack of the route that groups at extraction, between PrepareUnique
// (buffers carved from the stack's workspace, checks, the set-up launch and
// every later stage's arguments) and EnqueueUnique (the stages of several
// stacks together, one grouped launch per stage, common.h).
template <typename K>
struct UniqueStack {
  Arena* ws = nullptr;
  bool measuring = true;
  bool weighted = false;
  int64_t M = 0;
  int64_t extract_blocks = 0;
  radix::DigitPlan dp{};
  int key_bits = 0;
  int64_t tiles = 0;
  K* keys = nullptr;
  K* keys_alt = nullptr;
  uint64_t* pay = nullptr;
  uint64_t* pay_alt = nullptr;
  bool view = false;
  uint32_t* view_off = nullptr;
  uint32_t* view_total = nullptr;
  bool view_grouped = false;  // the view's scan is a grouped scan
  uint32_t* view_partial = nullptr;
  uint32_t* hist = nullptr;
  bool hist_grouped = false;  // so are the sort's scans
  uint32_t* hist_partial = nullptr;
  uint32_t* totals = nullptr;        // [passes], cleared by the set-up
  ExtractUniqueArgs<K, true> ex;     // fields shared by both variants
  int64_t view_grid = 0;
  ViewWriteArgs<K> vw;
  GroupUniqueArgs<K> gu;
  FillPlanArgs fill;
  ScatterUniqueArgs<K> sc;
  WritePaddingArgs pad;
  int64_t pad_blocks = 0;
};

template <typename K>
int PrepareUnique(const scemb_feature_t* feats, int nf,
                  const scemb_preprocess_options_t* o,
                  const scemb_preprocess_output_t* out, const Plan& pl,
                  Arena& ws, hipStream_t stream, UniqueStack<K>* u) {
  const int64_t M = pl.total_ids;
  const int64_t num_buckets = static_cast<int64_t>(pl.L) * pl.S * pl.NS;
  const int64_t extract_blocks = CeilDiv(M, kExtractBlock);
  const bool view = o->build_sample_view != 0;
  u->ws = &ws;
  u->measuring = ws.measuring();
  u->weighted = o->has_variable_weights != 0;
  u->M = M;
  u->extract_blocks = extract_blocks;
  u->view = view;
  u->keys = ws.Take<K>(M);
  u->keys_alt = ws.Take<K>(M);
  u->pay = ws.Take<uint64_t>(M);
  u->pay_alt = ws.Take<uint64_t>(M);
  BlockRows* block_rows = ws.Take<BlockRows>(extract_blocks);
  u->view_off = view ? ws.Take<uint32_t>(extract_blocks) : nullptr;
  int32_t* part_first = ws.Take<int32_t>(num_buckets);
  int32_t* part_last = ws.Take<int32_t>(num_buckets);
  u->key_bits = std::max(1, pl.kl.col_bits + pl.kl.seg_bits);
  u->dp = radix::PlanDigits(u->key_bits);
  // Cleared by the set-up launch: the buckets' distinct-column counts, the
  // sort's per-pass totals and the view's total, so that a stack of no ids
  // (whose scans are not launched) reads zeros.
  const int64_t head_words = RoundUp(num_buckets, 64);
  const int64_t cleared = head_words + RoundUp(u->dp.passes + 1, 64);
  int32_t* col_heads = ws.Take<int32_t>(cleared);
  u->totals = col_heads == nullptr
                  ? nullptr
                  : reinterpret_cast<uint32_t*>(col_heads + head_words);
  u->view_total = view && u->totals != nullptr ? u->totals + u->dp.passes
                                               : nullptr;
  BucketStats* bstats = ws.Take<BucketStats>(num_buckets);
  FillPlan* plans = ws.Take<FillPlan>(num_buckets);
  SliceDesc* slices =
      ws.Take<SliceDesc>(static_cast<int64_t>(pl.slices.size()));
  FeatureDev* fdev = ws.Take<FeatureDev>(nf);
  u->tiles = CeilDiv(M, radix::kSortTile);
  const int64_t cells = u->tiles * (int64_t{1} << u->dp.digit);
  u->hist = ws.Take<uint32_t>(cells);
  // The scans' tile sums for grouped scans; a scan too long for one is left
  // to ExclusiveScan, whose temporaries EnqueueUnique takes from ws.
  const int64_t view_words = view ? GroupedScanPartialWords(extract_blocks) : 0;
  const int64_t hist_words = GroupedScanPartialWords(cells);
  u->view_grouped = view_words > 0;
  u->hist_grouped = hist_words > 0;
  u->view_partial = view_words > 0 ? ws.Take<uint32_t>(view_words) : nullptr;
  u->hist_partial = hist_words > 0 ? ws.Take<uint32_t>(hist_words) : nullptr;
  if (view) {
    if (pl.L != 1 || pl.G != 1) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "the sample view needs one local and one global device");
    }
    if (o->table_rows <= 0 || o->table_rows % pl.NS != 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "table_rows must be a positive multiple of the partitions");
    }
  }
  const int64_t view_rows = view ? o->table_rows / pl.NS : 0;
  const int64_t counters_off = RoundUp(2 * static_cast<int64_t>(pl.L) * pl.NS +
                                       static_cast<int64_t>(pl.L) * pl.S, 2);
  const int num_slices = static_cast<int>(pl.slices.size());
  int64_t* counters = nullptr;
  if (!u->measuring) {
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    if (out == nullptr || out->row_pointers == nullptr || out->stats == nullptr ||
        out->embedding_ids == nullptr || out->sample_ids == nullptr ||
        out->gains == nullptr) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null output buffer");
    }
    if (view && (out->view_keys == nullptr || out->view_entries == nullptr)) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null sample view buffer");
    }
    counters = reinterpret_cast<int64_t*>(out->stats + counters_off);
    if ((reinterpret_cast<uintptr_t>(counters) & 7u) != 0) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "stats buffer must be 8-byte aligned");
    }
    const SetupTargets tg{part_first, part_last, num_buckets, col_heads,
                          cleared,    slices,    fdev,        block_rows,
                          M > 0 ? extract_blocks : 0};
    const int su = EnqueueSetup(feats, nf, o, pl, counters_off, out->stats,
                                counters, tg, stream);
    if (su != 0) return su;
  }
  // Only dense features of one id per row are known to need no merging
  // (max_row_length is a hint and may understate).
  int rows_of_one = 1;
  for (int f = 0; f < nf; ++f) {
    if (feats[f].row_splits != nullptr || feats[f].valency > 1) {
      rows_of_one = 0;
    }
  }
  u->ex = ExtractUniqueArgs<K, true>{
      slices,      num_slices,  fdev, block_rows, M,           o->combiner,
      rows_of_one, pl.kl,       view_rows,        u->keys,     u->pay,
      u->view_off, counters};
  if (view) {
    const int64_t n = pl.coo_size;
    u->view_grid = std::max(extract_blocks, CeilDiv(n, kExtractBlock));
    u->vw = ViewWriteArgs<K>{u->keys,  u->pay, u->view_off,
                             u->view_total, M,  n,
                             pl.kl,    view_rows,
                             static_cast<uint32_t>(pl.batch_for_device),
                             out != nullptr ? out->view_keys : nullptr,
                             out != nullptr ? out->view_entries : nullptr};
  }
  const bool odd = u->dp.passes % 2 == 1;
  const K* skeys = odd ? u->keys_alt : u->keys;
  const uint64_t* spay = odd ? u->pay_alt : u->pay;
  u->gu = GroupUniqueArgs<K>{skeys,      u->totals, pl.kl,    pl.NS,
                             part_first, part_last, col_heads};
  FillParams fp;
  fp.local_devices = pl.L;
  fp.segs_per_device = pl.S;
  fp.num_partitions = pl.NS;
  fp.rp_per_segment = pl.rp_per_seg;
  fp.coo_size = pl.coo_size;
  fp.max_ids = o->max_ids_per_partition;
  fp.max_unique = o->max_unique_ids_per_partition;
  fp.allow_dropping = 0;
  fp.mb_bits = 0;
  fp.absolute = 0;
  fp.num_minibatches = 1;
  for (int bkt = 0; bkt < kMaxMinibatches; ++bkt) fp.minibatch_of[bkt] = 0;
  const BucketReduceArgs bra{part_first, part_last, nullptr,   nullptr,
                             nullptr,    num_buckets, bstats, col_heads};
  int32_t* stats = out != nullptr ? out->stats : nullptr;
  u->fill = FillPlanArgs{
      bstats,
      fp,
      out != nullptr ? out->row_pointers : nullptr,
      plans,
      stats,
      stats == nullptr ? nullptr : stats + static_cast<int64_t>(pl.L) * pl.NS,
      stats == nullptr ? nullptr
                       : stats + 2 * static_cast<int64_t>(pl.L) * pl.NS,
      counters,
      bra};
  u->sc = ScatterUniqueArgs<K>{
      skeys,
      spay,
      u->totals,
      pl.kl,
      fp,
      static_cast<int32_t>(pl.bps),
      part_first,
      plans,
      out != nullptr ? out->embedding_ids : nullptr,
      out != nullptr ? out->sample_ids : nullptr,
      out != nullptr ? out->gains : nullptr};
  u->pad = WritePaddingArgs{plans,
                            num_buckets,
                            fp,
                            out != nullptr ? out->embedding_ids : nullptr,
                            out != nullptr ? out->sample_ids : nullptr,
                            out != nullptr ? out->gains : nullptr,
                            nullptr,
                            u->totals,
                            counters};
  u->pad_blocks = CeilDiv(num_buckets * kAlign, 256);
  return 0;
}

// The stages of every stack in `st` (all prepared for the same workspace
// mode), in order, each one grouped launch over the stacks that have work in
// it: extraction, the view's scan and write, the radix passes (histogram,
// scan, scatter), grouping, the fill plan, the scatter into the CSR and the
// padding. Measuring, only the temporaries of scans left to ExclusiveScan are
// taken.
template <typename K, bool kHashed>
int EnqueueUnique(UniqueStack<K>* const* st, int n, hipStream_t stream) {
  const bool measuring = n > 0 && st[0]->measuring;
  std::vector<int64_t> blocks(n);
  int rc = 0;
  // Extraction.
  if (!measuring) {
    std::vector<ExtractUniqueArgs<K, kHashed>> ex(n);
    for (int i = 0; i < n; ++i) {
      const ExtractUniqueArgs<K, true>& e = st[i]->ex;
      ex[i] = ExtractUniqueArgs<K, kHashed>{
          e.slices,      e.num_slices, e.feats,     e.block_rows, e.total_ids,
          e.combiner,    e.rows_of_one, e.kl,       e.view_rows,  e.keys,
          e.pay,         e.view_counts, e.counters};
      blocks[i] = st[i]->extract_blocks;
    }
    rc = LaunchGrouped(ex.data(), blocks.data(), n, stream);
    if (rc != 0) return rc;
  }
  // The sample view: scan of the blocks' counts, then the write.
  {
    std::vector<ScanJob<uint32_t>> jobs;
    for (int i = 0; i < n; ++i) {
      UniqueStack<K>& u = *st[i];
      if (!u.view || u.extract_blocks == 0) continue;
      if (u.view_grouped) {
        jobs.push_back(ScanJob<uint32_t>{u.view_off, u.view_off,
                                         u.extract_blocks, u.view_total,
                                         u.view_partial});
      } else {
        rc = ExclusiveScan<uint32_t>(u.view_off, u.view_off, u.extract_blocks,
                                     u.view_total, *u.ws, stream);
        if (rc != 0) return rc;
      }
    }
    if (!measuring && !jobs.empty()) {
      rc = GroupedExclusiveScan(jobs.data(), static_cast<int>(jobs.size()),
                                stream);
      if (rc != 0) return rc;
    }
    if (!measuring) {
      std::vector<ViewWriteArgs<K>> vw(n);
      for (int i = 0; i < n; ++i) {
        vw[i] = st[i]->vw;
        blocks[i] = st[i]->view ? st[i]->view_grid : 0;
      }
      rc = LaunchGrouped(vw.data(), blocks.data(), n, stream);
      if (rc != 0) return rc;
    }
  }
  // The sort. Pass p writes (keys_alt, pay_alt) when p is even; pass 0 reads
  // the extraction arrays without the merged copies.
  using Arr = radix::ArraySource<K, uint64_t>;
  using Sink = radix::ArraySink<K, uint64_t>;
  int max_passes = 0;
  for (int i = 0; i < n; ++i) max_passes = std::max(max_passes, st[i]->dp.passes);
  for (int pass = 0; pass < max_passes; ++pass) {
    std::vector<radix::RadixHistogramArgs<K, UniqueSource<K>>> h0(n);
    std::vector<radix::RadixHistogramArgs<K, Arr>> hn(n);
    std::vector<radix::RadixScatterArgs<K, uint64_t, UniqueSource<K>, Sink>>
        s0(n);
    std::vector<radix::RadixScatterArgs<K, uint64_t, Arr, Sink>> sn(n);
    std::vector<ScanJob<uint32_t>> jobs;
    for (int i = 0; i < n; ++i) {
      UniqueStack<K>& u = *st[i];
      blocks[i] = 0;
      if (pass >= u.dp.passes || u.M == 0) continue;
      blocks[i] = u.tiles;
      const int shift = pass * u.dp.digit;
      const int pbits =
          u.key_bits - shift < u.dp.digit ? u.key_bits - shift : u.dp.digit;
      const uint32_t mask = (1u << pbits) - 1u;
      const int64_t cells = u.tiles * (int64_t{1} << pbits);
      const bool even = pass % 2 == 0;
      const Arr arr{even ? u.keys : u.keys_alt, even ? u.pay : u.pay_alt};
      const Sink sink{even ? u.keys_alt : u.keys, even ? u.pay_alt : u.pay};
      const UniqueSource<K> first{u.keys, u.pay};
      h0[i] = {first, u.M, nullptr, 0, shift, mask, u.tiles, u.hist};
      hn[i] = {arr, u.M, u.totals, 1, shift, mask, u.tiles, u.hist};
      s0[i] = {first, sink,  u.M,   nullptr,  0,
               shift, mask,  pbits, u.tiles,  u.hist,
               u.totals + pass, false};
      sn[i] = {arr,   sink,  u.M,   u.totals, 1,
               shift, mask,  pbits, u.tiles,  u.hist,
               u.totals + pass, false};
      if (u.hist_grouped) {
        jobs.push_back(ScanJob<uint32_t>{u.hist, u.hist, cells,
                                         u.totals + pass, u.hist_partial});
      }
    }
    if (!measuring) {
      rc = pass == 0 ? LaunchGrouped(h0.data(), blocks.data(), n, stream)
                     : LaunchGrouped(hn.data(), blocks.data(), n, stream);
      if (rc != 0) return rc;
      if (!jobs.empty()) {
        rc = GroupedExclusiveScan(jobs.data(), static_cast<int>(jobs.size()),
                                  stream);
        if (rc != 0) return rc;
      }
    }
    for (int i = 0; i < n; ++i) {
      UniqueStack<K>& u = *st[i];
      if (pass >= u.dp.passes || u.M == 0 || u.hist_grouped) continue;
      const int shift = pass * u.dp.digit;
      const int pbits =
          u.key_bits - shift < u.dp.digit ? u.key_bits - shift : u.dp.digit;
      rc = ExclusiveScan<uint32_t>(u.hist, u.hist,
                                   u.tiles * (int64_t{1} << pbits),
                                   u.totals + pass, *u.ws, stream);
      if (rc != 0) return rc;
    }
    if (!measuring) {
      rc = pass == 0 ? LaunchGrouped(s0.data(), blocks.data(), n, stream)
                     : LaunchGrouped(sn.data(), blocks.data(), n, stream);
      if (rc != 0) return rc;
    }
  }
  if (measuring) return 0;
  for (int i = 0; i < n; ++i) {
    if (st[i]->ws->overflow()) {
      return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    }
  }
  // Grouping, the fill plan, the CSR scatter and the padding.
  {
    std::vector<GroupUniqueArgs<K>> gu(n);
    for (int i = 0; i < n; ++i) {
      gu[i] = st[i]->gu;
      blocks[i] = CeilDiv(st[i]->M, int64_t{256} * kGroupItems);
    }
    rc = LaunchGrouped(gu.data(), blocks.data(), n, stream);
    if (rc != 0) return rc;
  }
  {
    std::vector<FillPlanArgs> fill(n);
    for (int i = 0; i < n; ++i) {
      fill[i] = st[i]->fill;
      blocks[i] = 1;
    }
    rc = LaunchGrouped(fill.data(), blocks.data(), n, stream);
    if (rc != 0) return rc;
  }
  {
    std::vector<ScatterUniqueArgs<K>> sc(n);
    for (int i = 0; i < n; ++i) {
      sc[i] = st[i]->sc;
      blocks[i] = CeilDiv(st[i]->M, 256);
    }
    rc = LaunchGrouped(sc.data(), blocks.data(), n, stream);
    if (rc != 0) return rc;
  }
  std::vector<WritePaddingArgs> pad(n);
  for (int i = 0; i < n; ++i) {
    pad[i] = st[i]->pad;
    blocks[i] = st[i]->pad_blocks;
  }
  return LaunchGrouped(pad.data(), blocks.data(), n, stream);
}

template <typename K>
int RunUniquePipeline(const scemb_feature_t* feats, int nf,
                      const scemb_preprocess_options_t* o,
                      const scemb_preprocess_output_t* out, const Plan& pl,
                      Arena& ws, hipStream_t stream) {
  UniqueStack<K> u;
  int rc = PrepareUnique<K>(feats, nf, o, out, pl, ws, stream, &u);
  if (rc != 0) return rc;
  UniqueStack<K>* one = &u;
  return u.weighted ? EnqueueUnique<K, false>(&one, 1, stream)
                    : EnqueueUnique<K, true>(&one, 1, stream);
}

// The most ids of one row over the stack's features: a dense feature's
// valency, else the caller's hint, else a pass over the host row splits (the
// caller's, or the copy MakePlan made of device-only ones).
int64_t MaxRowLength(const scemb_feature_t* feats, int nf,
                     const std::vector<std::vector<int64_t>>& cache) {
  int64_t most = 0;
  for (int f = 0; f < nf; ++f) {
    const scemb_feature_t& ft = feats[f];
    if (ft.row_splits == nullptr) {
      most = std::max<int64_t>(most, ft.valency);
    } else if (ft.max_row_length > 0) {
      most = std::max<int64_t>(most, ft.max_row_length);
    } else {
      const int64_t* sp = ft.row_splits_host != nullptr ? ft.row_splits_host
                                                        : cache[f].data();
      int64_t least = 0;
      most = std::max<int64_t>(most, RowLengthRange(sp, ft.num_rows, &least));
    }
  }
  return most;
}

// Grouping at extraction needs every (row, column) pair to come from one
// input row (disjoint sample rows) and keeps every entry (no id dropping, no
// minibatching). With the sample view it also needs a static buffer that
// holds any input within the limits: the view is written before the fill
// plan and so cannot leave out entries the buffer has no room for. Its
// duplicate scan costs the square of the row length, so rows longer than the
// LDS staging go the other way.
bool GroupsAtExtraction(const scemb_feature_t* feats, int nf,
                        const scemb_preprocess_options_t* o, const Plan& pl,
                        const std::vector<std::vector<int64_t>>& cache) {
  return (o->flags & SCEMB_PREPROCESS_GROUP_AFTER_SORT) == 0 &&
         !o->enable_minibatching && !o->allow_id_dropping &&
         pl.rows_disjoint &&
         (!o->build_sample_view ||
          pl.coo_size >= RoundUp(o->max_ids_per_partition, kAlign) *
                             static_cast<int64_t>(pl.S) * pl.NS) &&
         MaxRowLength(feats, nf, cache) <= kDedupMaxRow;
}

int Preprocess(const scemb_feature_t* feats, int nf,
               const scemb_preprocess_options_t* o,
               const scemb_preprocess_output_t* out, Arena& ws,
               hipStream_t stream) {
  Plan pl;
  std::vector<std::vector<int64_t>> cache;
  int st = MakePlan(feats, nf, o, &pl, &cache);
  if (st != 0) return st;
  if (GroupsAtExtraction(feats, nf, o, pl, cache)) {
    return pl.wide_keys
               ? RunUniquePipeline<uint64_t>(feats, nf, o, out, pl, ws, stream)
               : RunUniquePipeline<uint32_t>(feats, nf, o, out, pl, ws, stream);
  }
  if (pl.wide_keys) {
    return RunPipeline<uint64_t>(feats, nf, o, out, pl, ws, stream);
  }
  return RunPipeline<uint32_t>(feats, nf, o, out, pl, ws, stream);
}

// The stacks of one call: those grouping at extraction are prepared in job
// order (each one's set-up launch), then their stages are enqueued together,
// one grouped launch per stage for the stacks of one key width and weighting;
// the other stacks run whole, first.
template <typename K>
struct UniqueClasses {
  std::vector<std::unique_ptr<UniqueStack<K>>> weighted, unit;
  int Add(const scemb_preprocess_job_t& j, const Plan& pl, Arena& ws,
          hipStream_t stream) {
    auto u = std::make_unique<UniqueStack<K>>();
    const int rc = PrepareUnique<K>(j.features, j.num_features, j.options,
                                    j.outputs, pl, ws, stream, u.get());
    if (rc != 0) return rc;
    (u->weighted ? weighted : unit).push_back(std::move(u));
    return 0;
  }
  int Enqueue(hipStream_t stream) {
    std::vector<UniqueStack<K>*> w, h;
    for (auto& u : weighted) w.push_back(u.get());
    for (auto& u : unit) h.push_back(u.get());
    int rc = w.empty() ? 0
                       : EnqueueUnique<K, false>(w.data(),
                                                 static_cast<int>(w.size()),
                                                 stream);
    if (rc != 0 || h.empty()) return rc;
    return EnqueueUnique<K, true>(h.data(), static_cast<int>(h.size()), stream);
  }
};

int PreprocessJobs(const scemb_preprocess_job_t* jobs, int n,
                   hipStream_t stream) {
  if (n < 0 || (n > 0 && jobs == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null jobs");
  }
  std::vector<Arena> arenas;
  arenas.reserve(n);  // the prepared stacks keep pointers to their arenas
  UniqueClasses<uint32_t> narrow;
  UniqueClasses<uint64_t> wide;
  for (int i = 0; i < n; ++i) {
    const scemb_preprocess_job_t& j = jobs[i];
    if (j.workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
    arenas.emplace_back(j.workspace, j.workspace_bytes);
    Arena& ws = arenas.back();
    Plan pl;
    std::vector<std::vector<int64_t>> cache;
    int rc = MakePlan(j.features, j.num_features, j.options, &pl, &cache);
    if (rc != 0) return rc;
    if (GroupsAtExtraction(j.features, j.num_features, j.options, pl, cache)) {
      rc = pl.wide_keys ? wide.Add(j, pl, ws, stream)
                        : narrow.Add(j, pl, ws, stream);
    } else if (pl.wide_keys) {
      rc = RunPipeline<uint64_t>(j.features, j.num_features, j.options,
                                 j.outputs, pl, ws, stream);
    } else {
      rc = RunPipeline<uint32_t>(j.features, j.num_features, j.options,
                                 j.outputs, pl, ws, stream);
    }
    if (rc != 0) return rc;
  }
  const int rc = narrow.Enqueue(stream);
  return rc != 0 ? rc : wide.Enqueue(stream);
}

}  // namespace
}  // namespace scemb

using namespace scemb;

extern "C" {

int64_t scemb_preprocess_stats_counters_offset(
    const scemb_preprocess_options_t* o) {
  if (o == nullptr) return -1;
  const int64_t L = o->local_device_count;
  const int64_t NS = static_cast<int64_t>(o->num_sc_per_device) *
                     o->global_device_count;
  return RoundUp(2 * L * NS + L * o->num_sc_per_device, 2);
}

int64_t scemb_preprocess_stats_size(const scemb_preprocess_options_t* o) {
  const int64_t off = scemb_preprocess_stats_counters_offset(o);
  return off < 0 ? -1 : off + 2 * kNumCounters;
}

size_t scemb_preprocess_workspace_size(const scemb_feature_t* features,
                                       int32_t num_features,
                                       const scemb_preprocess_options_t* o) {
  Arena ws(nullptr, 0);
  if (Preprocess(features, num_features, o, nullptr, ws, nullptr) != 0) {
    return 0;
  }
  return ws.used() + 256;
}

int scemb_preprocess_stacked_tables(const scemb_preprocess_job_t* jobs,
                                    int32_t num_jobs, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("preprocess_call", s);
  const int rc = PreprocessJobs(jobs, num_jobs, s);
  ProfileEnd(prof, s);
  return rc;
}

int scemb_preprocess_stacked_table(const scemb_feature_t* features,
                                   int32_t num_features,
                                   const scemb_preprocess_options_t* o,
                                   const scemb_preprocess_output_t* out,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  Arena ws(workspace, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("preprocess_call", s);
  const int rc = Preprocess(features, num_features, o, out, ws, s);
  ProfileEnd(prof, s);
  return rc;
}

int scemb_check_row_splits(const int64_t* row_splits, int64_t num_rows,
                           int64_t nnz, int64_t* max_row_length) {
  if (row_splits == nullptr || num_rows < 0 || max_row_length == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null row splits");
  }
  int64_t least = 0;
  const int64_t most = RowLengthRange(row_splits, num_rows, &least);
  if (row_splits[0] != 0 || row_splits[num_rows] != nnz || least < 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "row_splits must start at 0, be non-decreasing and end at the "
                "number of values.");
  }
  *max_row_length = most;
  return 0;
}

int scemb_stage_row_splits(const int64_t* row_splits, int64_t num_rows,
                           int64_t nnz, int64_t* dst,
                           int64_t* max_row_length) {
  if (row_splits == nullptr || dst == nullptr || num_rows < 0 ||
      max_row_length == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null row splits");
  }
  int64_t least = 0;
  const int64_t most = CopyRowLengthRange(row_splits, num_rows, dst, &least);
  if (row_splits[0] != 0 || row_splits[num_rows] != nnz || least < 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "row_splits must start at 0, be non-decreasing and end at the "
                "number of values.");
  }
  *max_row_length = most;
  return 0;
}

int64_t scemb_compute_theoretical_max_coo_buffer_size(
    int32_t max_ids_per_partition, int32_t global_device_count,
    int32_t num_sc_per_device, int32_t enable_minibatching) {
  const int64_t num_scs = static_cast<int64_t>(global_device_count) * num_sc_per_device;
  return RoundUp(max_ids_per_partition, kAlign) * num_sc_per_device * num_scs *
         (enable_minibatching ? kMaxMinibatches : 1);
}

int64_t scemb_compute_coo_buffer_size_per_device(
    int32_t max_ids_per_partition, int64_t suggested, int32_t global_device_count,
    int32_t num_sc_per_device, int32_t enable_minibatching) {
  const int64_t theoretical = scemb_compute_theoretical_max_coo_buffer_size(
      max_ids_per_partition, global_device_count, num_sc_per_device,
      enable_minibatching);
  if (suggested <= 0) return theoretical;
  const int64_t v = RoundUp(suggested, static_cast<int64_t>(kAlign) * num_sc_per_device);
  return v > theoretical ? -1 : v;
}

int32_t scemb_compute_row_pointers_size_per_device(int32_t global_device_count,
                                                   int32_t num_sc_per_device,
                                                   int32_t enable_minibatching) {
  const int32_t ns = global_device_count * num_sc_per_device;
  return std::max(ns, kAlign) * num_sc_per_device *
         (enable_minibatching ? kMaxMinibatches : 1);
}

}  // extern "C"
