// Device-wide scan and stable LSD radix sort.
//
// Scan: reduce-then-scan over 2048-element tiles (256 threads x 8 items).
// Up to 8192 tiles the scanning blocks add up the tile sums before them
// themselves (two launches); beyond, the tile sums are scanned recursively.
//
// Radix sort: per digit pass (up to 8 bits, passes balanced over the key
// span), (1) per-tile digit histograms, (2) an exclusive scan of the
// digit-major histogram matrix, (3) a stable scatter, staged through LDS so
// that the writes of a tile come out bucket by bucket.
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

// ScanTiles whose tile offset is the sum of the partial sums of the tiles
// before it, added up by the block itself (integer sums: any order gives the
// same value), so that no separate scan of the partial sums is launched.
template <typename T>
__global__ __launch_bounds__(kScanBlock) void ScanTilesPrefix(
    const T* in, T* out, int64_t n, const T* partial, T* total_out) {
  __shared__ T smem[kScanBlock / kWave + 1];
  T pre = 0;
  for (int64_t j = threadIdx.x; j < static_cast<int64_t>(blockIdx.x);
       j += kScanBlock) {
    pre += partial[j];
  }
  T off;
  BlockExclusiveScan<T, kScanBlock>(pre, smem, &off);
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
  T run = BlockExclusiveScan<T, kScanBlock>(s, smem, &total) + off;
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
constexpr int kMaxDigitBits = 8;
constexpr int kMaxRadix = 1 << kMaxDigitBits;
constexpr int kSortWaves = kSortBlock / kWave;

template <typename K>
__device__ __forceinline__ uint32_t Digit(K key, int shift, uint32_t mask) {
  return static_cast<uint32_t>(key >> shift) & mask;
}

// hist[d * tiles + tile] = keys of digit d in the tile.
template <typename K>
__global__ __launch_bounds__(kSortBlock) void RadixHistogram(
    const K* keys, int64_t n, int shift, uint32_t mask, int64_t tiles,
    uint32_t* hist) {
  __shared__ uint32_t h[kMaxRadix];
  const int radix = static_cast<int>(mask) + 1;
  for (int d = threadIdx.x; d < radix; d += kSortBlock) h[d] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    const int64_t i = base + c * kSortBlock + threadIdx.x;
    if (i < n) atomicAdd(&h[Digit(keys[i], shift, mask)], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < radix; d += kSortBlock) {
    hist[static_cast<int64_t>(d) * tiles + blockIdx.x] = h[d];
  }
}

// Stable scatter of one tile (kSortTile consecutive elements) into the
// digit buckets. Each element's rank inside its bucket comes from the chunks
// (256 elements, in position order) before it, the waves before it in its
// chunk and the lanes before it in its wave with the same digit (ballots).
// The tile is first reordered by digit in LDS, then written out in that
// order: consecutive threads then write consecutive positions of a bucket,
// instead of one element per bucket and store.
template <typename K, typename V>
__global__ __launch_bounds__(kSortBlock) void RadixScatter(
    const K* keys, const V* vals, K* keys_out, V* vals_out, int64_t n,
    int shift, uint32_t mask, int digit_bits, int64_t tiles,
    const uint32_t* offsets) {
  __shared__ uint32_t run_base[kMaxRadix];    // bucket fill so far (tile)
  __shared__ uint32_t wave_cnt[kSortWaves][kMaxRadix];
  __shared__ uint32_t global_off[kMaxRadix];  // bucket start (output)
  __shared__ uint32_t tile_off[kMaxRadix];    // bucket start (tile)
  __shared__ uint32_t scan_tmp[kSortBlock / kWave + 1];
  __shared__ K s_keys[kSortTile];
  __shared__ V s_vals[kSortTile];
  const int t = threadIdx.x;
  const int wave = t / kWave;
  const int radix = static_cast<int>(mask) + 1;
  const int64_t blk = blockIdx.x;
  const int64_t base = blk * kSortTile;
  const int tile_n =
      static_cast<int>(n - base < kSortTile ? n - base : kSortTile);
  // Bucket sizes of this tile from the scanned histogram: the next cell's
  // offset minus this one's (the last cell: n minus it).
  uint32_t cnt_local[kMaxRadix / kSortBlock];
#pragma unroll
  for (int k = 0; k < kMaxRadix / kSortBlock; ++k) {
    const int d = t + k * kSortBlock;
    cnt_local[k] = 0;
    if (d < radix) {
      const int64_t cell = static_cast<int64_t>(d) * tiles + blk;
      const uint32_t off = offsets[cell];
      const uint32_t next = cell + 1 < static_cast<int64_t>(radix) * tiles
                                ? offsets[cell + 1]
                                : static_cast<uint32_t>(n);
      global_off[d] = off;
      run_base[d] = 0;
      cnt_local[k] = next - off;
    }
  }
  // Tile offsets of the buckets: exclusive scan over digits, thread t holding
  // digits t, t + 256, ... (one round per 256 digits).
#pragma unroll
  for (int k = 0; k < kMaxRadix / kSortBlock; ++k) {
    uint32_t total;
    const uint32_t ex =
        BlockExclusiveScan<uint32_t, kSortBlock>(cnt_local[k], scan_tmp,
                                                 &total);
    const int d = t + k * kSortBlock;
    // Digits of round k follow all digits of earlier rounds.
    __shared__ uint32_t round_base;
    if (k == 0 && t == 0) round_base = 0;
    __syncthreads();
    if (d < radix) tile_off[d] = round_base + ex;
    __syncthreads();
    if (t == 0) round_base += total;
    __syncthreads();
  }
  const uint64_t lt = LaneMaskLt();
  for (int c = 0; c < kSortChunks; ++c) {
    const int li = c * kSortBlock + t;  // position inside the tile
    const bool active = li < tile_n;
    K key = 0;
    V val = 0;
    uint32_t d = 0;
    if (active) {
      key = keys[base + li];
      val = vals[base + li];
      d = Digit(key, shift, mask);
    }
    for (int b = t; b < radix; b += kSortBlock) {
#pragma unroll
      for (int w = 0; w < kSortWaves; ++w) wave_cnt[w][b] = 0;
    }
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
    for (int b = t; b < radix; b += kSortBlock) {
      uint32_t r = run_base[b];
#pragma unroll
      for (int w = 0; w < kSortWaves; ++w) {
        const uint32_t cnt = wave_cnt[w][b];
        wave_cnt[w][b] = r;
        r += cnt;
      }
      run_base[b] = r;
    }
    __syncthreads();
    if (active) {
      const uint32_t pos = tile_off[d] + wave_cnt[wave][d] + rank;
      s_keys[pos] = key;
      s_vals[pos] = val;
    }
    __syncthreads();
  }
  // Write out in tile-sorted order: element j of digit d goes to
  // global_off[d] + (j - tile_off[d]).
  for (int j = t; j < tile_n; j += kSortBlock) {
    const K key = s_keys[j];
    const uint32_t d = Digit(key, shift, mask);
    const uint32_t pos = global_off[d] + (static_cast<uint32_t>(j) - tile_off[d]);
    keys_out[pos] = key;
    vals_out[pos] = s_vals[j];
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
  // Fewest passes of at most kMaxDigitBits bits, balanced (27 bits: four
  // passes of 7; 21: three of 7; 16: two of 8).
  const int span = end_bit - begin_bit;
  const int passes = (span + kMaxDigitBits - 1) / kMaxDigitBits;
  const int digit = (span + passes - 1) / passes;
  const int64_t tiles = CeilDiv(n, kSortTile);
  uint32_t* hist = ws.Take<uint32_t>(tiles * (int64_t{1} << digit));
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  K* src_k = keys;
  V* src_v = vals;
  K* dst_k = keys_alt;
  V* dst_v = vals_alt;
  for (int shift = begin_bit; shift < end_bit; shift += digit) {
    const int bits = end_bit - shift < digit ? end_bit - shift : digit;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t cells = tiles * (int64_t{1} << bits);
    if (!measuring) {
      hipLaunchKernelGGL(RadixHistogram<K>, dim3(tiles), dim3(kSortBlock), 0,
                         stream, src_k, n, shift, mask, tiles, hist);
      SCEMB_LAUNCH_CHECK();
    }
    const int st = ExclusiveScan<uint32_t>(hist, hist, cells, nullptr, ws,
                                           stream);
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
