// Device-wide scan and stable LSD radix sort.
//
// Scan: reduce-then-scan over 2048-element tiles (256 threads x 8 items).
// Up to 8192 tiles the scanning blocks add up the tile sums before them
// themselves (two launches); beyond, the tile sums are scanned recursively.
//
// Radix sort: per digit pass (up to 8 bits, passes balanced over the key
// span), (1) per-tile digit histograms, (2) an exclusive scan of the
// digit-major histogram matrix, (3) a stable scatter, staged through LDS so
// that the writes of a tile come out bucket by bucket (radix.h).
#include "scan.h"

#include <vector>

#include "radix.h"

#include "../../include/scemb.h"

namespace scemb {
namespace {

constexpr int kScanBlock = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanBlock * kScanItems;

template <typename T>
__device__ __forceinline__ void ScanReduceTilesBody(uint32_t blk, const T* in,
                                                    int64_t n, T* partial) {
  __shared__ T smem[kScanBlock / kWave + 1];
  const int64_t base = static_cast<int64_t>(blk) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) s += in[i];
  }
  T total;
  BlockExclusiveScan<T, kScanBlock>(s, smem, &total);
  if (threadIdx.x == 0) partial[blk] = total;
}

template <typename T>
__global__ __launch_bounds__(kScanBlock) void ScanReduceTiles(const T* in,
                                                               int64_t n,
                                                               T* partial) {
  ScanReduceTilesBody<T>(blockIdx.x, in, n, partial);
}

template <typename T>
__global__ __launch_bounds__(kScanBlock) void ScanTiles(const T* in, T* out,
                                                         int64_t n,
                                                         const T* offsets,
                                                         T* total_out) {
  __shared__ T smem[kScanBlock / kWave + 1];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  T v[kScanItems];
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    v[k] = i < n ? in[i] : T(0);
    s += v[k];
  }
  T total;
  T run = BlockExclusiveScan<T, kScanBlock>(s, smem, &total);
  const T off = offsets ? offsets[blockIdx.x] : T(0);
  run += off;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) out[i] = run;
    run += v[k];
  }
  if (total_out != nullptr && threadIdx.x == 0 &&
      blockIdx.x == gridDim.x - 1) {
    total_out[0] = off + total;
  }
}

// ScanTiles whose tile offset is the sum of the partial sums of the tiles
// before it, added up by the block itself (integer sums: any order gives the
// same value), so that no separate scan of the partial sums is launched.
template <typename T>
__device__ __forceinline__ void ScanTilesPrefixBody(uint32_t blk,
                                                    uint32_t nblk, const T* in,
                                                    T* out, int64_t n,
                                                    const T* partial,
                                                    T* total_out) {
  __shared__ T smem[kScanBlock / kWave + 1];
  T pre = 0;
  for (int64_t j = threadIdx.x; j < static_cast<int64_t>(blk);
       j += kScanBlock) {
    pre += partial[j];
  }
  T off;
  BlockExclusiveScan<T, kScanBlock>(pre, smem, &off);
  const int64_t base = static_cast<int64_t>(blk) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  T v[kScanItems];
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    v[k] = i < n ? in[i] : T(0);
    s += v[k];
  }
  T total;
  T run = BlockExclusiveScan<T, kScanBlock>(s, smem, &total) + off;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) out[i] = run;
    run += v[k];
  }
  if (total_out != nullptr && threadIdx.x == 0 && blk == nblk - 1) {
    total_out[0] = off + total;
  }
}

template <typename T>
__global__ __launch_bounds__(kScanBlock) void ScanTilesPrefix(
    const T* in, T* out, int64_t n, const T* partial, T* total_out) {
  ScanTilesPrefixBody<T>(blockIdx.x, gridDim.x, in, out, n, partial,
                         total_out);
}

// The two launches of a scan as grouped arguments (common.h).
template <typename T>
struct ScanReduceArgs {
  static constexpr int kBlock = kScanBlock;
  const T* in;
  int64_t n;
  T* partial;
  __device__ static void Run(const ScanReduceArgs& a, uint32_t blk, uint32_t) {
    ScanReduceTilesBody<T>(blk, a.in, a.n, a.partial);
  }
};

template <typename T>
struct ScanPrefixArgs {
  static constexpr int kBlock = kScanBlock;
  const T* in;
  T* out;
  int64_t n;
  const T* partial;
  T* total;
  __device__ static void Run(const ScanPrefixArgs& a, uint32_t blk,
                             uint32_t nblk) {
    ScanTilesPrefixBody<T>(blk, nblk, a.in, a.out, a.n, a.partial, a.total);
  }
};

// Up to this many tiles, each block of the second launch adds up the
// partial sums before it (at most this many loads spread over 256 threads).
constexpr int64_t kPrefixTilesMax = 8192;

}  // namespace

template <typename T>
int ExclusiveScan(const T* in, T* out, int64_t n, T* total, Arena& ws,
                  hipStream_t stream) {
  if (n <= 0) {
    if (total != nullptr && !ws.measuring()) {
      // Nothing to scan: the total is zero.
      T* t = total;
      hipLaunchKernelGGL(ScanTiles<T>, dim3(1), dim3(kScanBlock), 0, stream,
                         t, t, int64_t{0}, nullptr, t);
      SCEMB_LAUNCH_CHECK();
    }
    return 0;
  }
  const int64_t tiles = CeilDiv(n, kScanTile);
  if (tiles == 1) {
    if (ws.measuring()) return 0;
    hipLaunchKernelGGL(ScanTiles<T>, dim3(1), dim3(kScanBlock), 0, stream, in,
                       out, n, nullptr, total);
    SCEMB_LAUNCH_CHECK();
    return 0;
  }
  T* partial = ws.Take<T>(tiles);
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  if (!measuring) {
    hipLaunchKernelGGL(ScanReduceTiles<T>, dim3(tiles), dim3(kScanBlock), 0,
                       stream, in, n, partial);
    SCEMB_LAUNCH_CHECK();
  }
  if (tiles <= kPrefixTilesMax) {
    if (!measuring) {
      hipLaunchKernelGGL(ScanTilesPrefix<T>, dim3(tiles), dim3(kScanBlock), 0,
                         stream, in, out, n, partial, total);
      SCEMB_LAUNCH_CHECK();
    }
    return 0;
  }
  int st = ExclusiveScan<T>(partial, partial, tiles, nullptr, ws, stream);
  if (st != 0) return st;
  if (!measuring) {
    hipLaunchKernelGGL(ScanTiles<T>, dim3(tiles), dim3(kScanBlock), 0, stream,
                       in, out, n, partial, total);
    SCEMB_LAUNCH_CHECK();
  }
  return 0;
}

int64_t GroupedScanPartialWords(int64_t n) {
  const int64_t tiles = std::max<int64_t>(1, CeilDiv(n, kScanTile));
  return tiles <= kPrefixTilesMax ? tiles : 0;
}

template <typename T>
int GroupedExclusiveScan(const ScanJob<T>* jobs, int n, hipStream_t stream) {
  std::vector<ScanReduceArgs<T>> red(n);
  std::vector<ScanPrefixArgs<T>> pre(n);
  std::vector<int64_t> blocks(n);
  for (int i = 0; i < n; ++i) {
    const ScanJob<T>& j = jobs[i];
    // Nothing to scan writes a zero total (one block of no elements).
    blocks[i] = j.n > 0 ? CeilDiv(j.n, kScanTile) : (j.total != nullptr);
    if (blocks[i] > kPrefixTilesMax) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "grouped scan: too many tiles");
    }
    red[i] = ScanReduceArgs<T>{j.in, std::max<int64_t>(j.n, 0), j.partial};
    pre[i] = ScanPrefixArgs<T>{j.in, j.out, std::max<int64_t>(j.n, 0),
                               j.partial, j.total};
  }
  int st = LaunchGrouped(red.data(), blocks.data(), n, stream);
  if (st != 0) return st;
  return LaunchGrouped(pre.data(), blocks.data(), n, stream);
}

template int GroupedExclusiveScan<uint32_t>(const ScanJob<uint32_t>*, int,
                                            hipStream_t);

template int ExclusiveScan<uint32_t>(const uint32_t*, uint32_t*, int64_t,
                                     uint32_t*, Arena&, hipStream_t);
template int ExclusiveScan<uint64_t>(const uint64_t*, uint64_t*, int64_t,
                                     uint64_t*, Arena&, hipStream_t);
template int ExclusiveScan<int64_t>(const int64_t*, int64_t*, int64_t,
                                    int64_t*, Arena&, hipStream_t);

// ---------------------------------------------------------------------------
// Radix sort (kernels in radix.h).
// ---------------------------------------------------------------------------

template <typename K, typename V>
int RadixSortPairs(K* keys, V* vals, K* keys_alt, V* vals_alt, int64_t n,
                   int begin_bit, int end_bit, Arena& ws, hipStream_t stream,
                   bool* in_alt) {
  using radix::kSortBlock;
  using radix::kSortTile;
  *in_alt = false;
  if (n <= 1 || end_bit <= begin_bit) return 0;
  if (n > (int64_t{1} << 32) - 1) {
    return Fail(1, "radix sort: more than 2^32-1 elements");
  }
  const radix::DigitPlan plan = radix::PlanDigits(end_bit - begin_bit);
  const int64_t tiles = CeilDiv(n, kSortTile);
  uint32_t* hist = ws.Take<uint32_t>(tiles * (int64_t{1} << plan.digit));
  uint32_t* total = ws.Take<uint32_t>(1);
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  K* src_k = keys;
  V* src_v = vals;
  K* dst_k = keys_alt;
  V* dst_v = vals_alt;
  for (int shift = begin_bit; shift < end_bit; shift += plan.digit) {
    const int bits = end_bit - shift < plan.digit ? end_bit - shift
                                                  : plan.digit;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t cells = tiles * (int64_t{1} << bits);
    const radix::ArraySource<K, V> src{src_k, src_v};
    if (!measuring) {
      hipLaunchKernelGGL((radix::RadixHistogramK<K, radix::ArraySource<K, V>>),
                         dim3(tiles), dim3(kSortBlock), 0, stream, src, n,
                         nullptr, 0, shift, mask, tiles, hist);
      SCEMB_LAUNCH_CHECK();
    }
    const int st = ExclusiveScan<uint32_t>(hist, hist, cells, total, ws,
                                           stream);
    if (st != 0) return st;
    if (!measuring) {
      const radix::ArraySink<K, V> sink{dst_k, dst_v};
      hipLaunchKernelGGL(
          (radix::RadixScatterK<K, V, radix::ArraySource<K, V>,
                                radix::ArraySink<K, V>>),
          dim3(tiles), dim3(kSortBlock), 0, stream, src, sink, n, nullptr, 0,
          shift, mask, bits, tiles, hist, total, false);
      SCEMB_LAUNCH_CHECK();
    }
    K* tk = src_k;
    src_k = dst_k;
    dst_k = tk;
    V* tv = src_v;
    src_v = dst_v;
    dst_v = tv;
    *in_alt = !*in_alt;
  }
  return 0;
}

template int RadixSortPairs<uint32_t, uint32_t>(uint32_t*, uint32_t*,
                                                uint32_t*, uint32_t*, int64_t,
                                                int, int, Arena&, hipStream_t,
                                                bool*);
template int RadixSortPairs<uint32_t, uint64_t>(uint32_t*, uint64_t*,
                                                uint32_t*, uint64_t*, int64_t,
                                                int, int, Arena&, hipStream_t,
                                                bool*);
template int RadixSortPairs<uint64_t, uint32_t>(uint64_t*, uint32_t*,
                                                uint64_t*, uint32_t*, int64_t,
                                                int, int, Arena&, hipStream_t,
                                                bool*);

}  // namespace scemb
