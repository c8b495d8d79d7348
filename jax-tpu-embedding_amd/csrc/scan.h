// Device-wide exclusive prefix sum and stable LSD radix sort (gfx950).
#pragma once

#include "common.h"

namespace scemb {

// Exclusive scan of n values (in and out may alias). When `total` is not
// null, the sum of all n values is written to total[0]. Temporaries come from
// `ws`; call with ws.base == nullptr to size them.
template <typename T>
int ExclusiveScan(const T* in, T* out, int64_t n, T* total, Arena& ws,
                  hipStream_t stream);

// One scan of a grouped launch: the exclusive scan of in[0, n) into out (may
// alias in), the sum into *total when total is set, with `partial` holding
// GroupedScanPartialWords(n) words.
template <typename T>
struct ScanJob {
  const T* in;
  T* out;
  int64_t n;
  T* total;
  T* partial;
};

// Words of ScanJob::partial for n values; 0 when n values take more tiles
// than a grouped scan handles (ExclusiveScan then).
int64_t GroupedScanPartialWords(int64_t n);

// The scans of jobs[0, n) in two grouped launches (common.h). Every job must
// have GroupedScanPartialWords(job.n) > 0; a job of no values with a total
// writes a zero total.
template <typename T>
int GroupedExclusiveScan(const ScanJob<T>* jobs, int n, hipStream_t stream);

// Stable LSD radix sort of (key, value) pairs on key bits [begin_bit,
// end_bit), in the fewest passes of at most 8 bits (digit widths balanced),
// ping-ponging between (keys, vals) and (keys_alt, vals_alt). *in_alt tells
// where the result ended up.
template <typename K, typename V>
int RadixSortPairs(K* keys, V* vals, K* keys_alt, V* vals_alt, int64_t n,
                   int begin_bit, int end_bit, Arena& ws, hipStream_t stream,
                   bool* in_alt);

}  // namespace scemb
