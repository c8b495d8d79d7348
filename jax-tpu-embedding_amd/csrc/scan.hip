// Device-wide scan and stable LSD radix sort.
//
// Scan: reduce-then-scan over 2048-element tiles (256 threads x 8 items),
// recursing on the tile sums.
//
// Radix sort: per 8-bit digit pass, (1) per-tile digit histograms, (2) an
// exclusive scan of the digit-major histogram matrix, (3) a stable scatter.
// Stability inside a tile comes from processing it in 256-element chunks in
// position order and ranking equal digits within each wave with 8 ballots
// (wave-level multisplit), then across waves and chunks through LDS counters.
#include "scan.h"

#include "../../include/scemb.h"

namespace scemb {
namespace {

constexpr int kScanBlock = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanBlock * kScanItems;

template <typename T>
__global__ __launch_bounds__(kScanBlock) void ScanReduceTiles(const T* in,
                                                               int64_t n,
                                                               T* partial) {
  __shared__ T smem[kScanBlock / kWave + 1];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) s += in[i];
  }
  T total;
  BlockExclusiveScan<T, kScanBlock>(s, smem, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
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
  int st = ExclusiveScan<T>(partial, partial, tiles, nullptr, ws, stream);
  if (st != 0) return st;
  if (!measuring) {
    hipLaunchKernelGGL(ScanTiles<T>, dim3(tiles), dim3(kScanBlock), 0, stream,
                       in, out, n, partial, total);
    SCEMB_LAUNCH_CHECK();
  }
  return 0;
}

template int ExclusiveScan<uint32_t>(const uint32_t*, uint32_t*, int64_t,
                                     uint32_t*, Arena&, hipStream_t);
template int ExclusiveScan<uint64_t>(const uint64_t*, uint64_t*, int64_t,
                                     uint64_t*, Arena&, hipStream_t);
template int ExclusiveScan<int64_t>(const int64_t*, int64_t*, int64_t,
                                    int64_t*, Arena&, hipStream_t);

// ---------------------------------------------------------------------------
// Radix sort.
// ---------------------------------------------------------------------------

namespace {

constexpr int kSortBlock = 256;
constexpr int kSortChunks = 8;
constexpr int kSortTile = kSortBlock * kSortChunks;
constexpr int kRadix = 256;
constexpr int kSortWaves = kSortBlock / kWave;

template <typename K>
__device__ __forceinline__ uint32_t Digit(K key, int shift, uint32_t mask) {
  return static_cast<uint32_t>(key >> shift) & mask;
}

template <typename K>
__global__ __launch_bounds__(kSortBlock) void RadixHistogram(
    const K* keys, int64_t n, int shift, uint32_t mask, int64_t tiles,
    uint32_t* hist) {
  __shared__ uint32_t h[kRadix];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    const int64_t i = base + c * kSortBlock + threadIdx.x;
    if (i < n) atomicAdd(&h[Digit(keys[i], shift, mask)], 1u);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * tiles + blockIdx.x] = h[threadIdx.x];
}

template <typename K, typename V>
__global__ __launch_bounds__(kSortBlock) void RadixScatter(
    const K* keys, const V* vals, K* keys_out, V* vals_out, int64_t n,
    int shift, uint32_t mask, int digit_bits, int64_t tiles,
    const uint32_t* offsets) {
  __shared__ uint32_t run_base[kRadix];
  __shared__ uint32_t wave_cnt[kSortWaves][kRadix];
  __shared__ uint32_t global_off[kRadix];
  const int t = threadIdx.x;
  const int wave = t / kWave;
  run_base[t] = 0;
  global_off[t] = offsets[static_cast<int64_t>(t) * tiles + blockIdx.x];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
  const uint64_t lt = LaneMaskLt();
  for (int c = 0; c < kSortChunks; ++c) {
    const int64_t i = base + c * kSortBlock + t;
    const bool active = i < n;
    K key = 0;
    V val = 0;
    uint32_t d = 0;
    if (active) {
      key = keys[i];
      val = vals[i];
      d = Digit(key, shift, mask);
    }
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) wave_cnt[w][t] = 0;
    __syncthreads();
    uint64_t match = __ballot(active);
    for (int b = 0; b < digit_bits; ++b) {
      const uint64_t bits = __ballot((d >> b) & 1u);
      match &= ((d >> b) & 1u) ? bits : ~bits;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(match & lt));
    if (active && (match & lt) == 0) {
      wave_cnt[wave][d] = static_cast<uint32_t>(__popcll(match));
    }
    __syncthreads();
    {
      uint32_t r = run_base[t];
#pragma unroll
      for (int w = 0; w < kSortWaves; ++w) {
        const uint32_t cnt = wave_cnt[w][t];
        wave_cnt[w][t] = r;
        r += cnt;
      }
      run_base[t] = r;
    }
    __syncthreads();
    if (active) {
      const uint32_t pos = global_off[d] + wave_cnt[wave][d] + rank;
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
  }
}

}  // namespace

template <typename K, typename V>
int RadixSortPairs(K* keys, V* vals, K* keys_alt, V* vals_alt, int64_t n,
                   int begin_bit, int end_bit, Arena& ws, hipStream_t stream,
                   bool* in_alt) {
  *in_alt = false;
  if (n <= 1 || end_bit <= begin_bit) return 0;
  if (n > (int64_t{1} << 32) - 1) {
    return Fail(1, "radix sort: more than 2^32-1 elements");
  }
  const int64_t tiles = CeilDiv(n, kSortTile);
  uint32_t* hist = ws.Take<uint32_t>(tiles * kRadix);
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  K* src_k = keys;
  V* src_v = vals;
  K* dst_k = keys_alt;
  V* dst_v = vals_alt;
  for (int shift = begin_bit; shift < end_bit; shift += 8) {
    const int bits = end_bit - shift < 8 ? end_bit - shift : 8;
    const uint32_t mask = (1u << bits) - 1u;
    if (!measuring) {
      hipLaunchKernelGGL(RadixHistogram<K>, dim3(tiles), dim3(kSortBlock), 0,
                         stream, src_k, n, shift, mask, tiles, hist);
      SCEMB_LAUNCH_CHECK();
    }
    const int st = ExclusiveScan<uint32_t>(hist, hist, tiles * kRadix, nullptr,
                                           ws, stream);
    if (st != 0) return st;
    if (!measuring) {
      hipLaunchKernelGGL((RadixScatter<K, V>), dim3(tiles), dim3(kSortBlock),
                         0, stream, src_k, src_v, dst_k, dst_v, n, shift, mask,
                         bits, tiles, hist);
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
