// Stable LSD radix sort passes over a source and into a sink (gfx950).
//
// One pass sorts by one digit of at most kMaxDigitBits bits:
//   RadixHistogramK  per-tile digit histograms (LDS atomics, one per digit
//                    and wave), digit-major
//   ExclusiveScan    of the histogram matrix (scan.h), with the total
//   RadixScatterK    stable scatter of each tile into the digit buckets
// The source decides which input positions take part (a position it
// declines is dropped: it is neither counted nor written), so a pass can
// read a CSR directly and compact it; the sink decides how an element is
// written, so the last pass can emit a derived payload. ArraySource and
// ArraySink are the plain (keys, values) arrays.
//
// Stability inside a tile comes from ranking each wave's share of the tile
// in position order (one ballot per digit bit, wave-level multisplit) and
// ordering the waves' shares by wave (RadixScatterK).
#pragma once

#include "common.h"

namespace scemb {
namespace radix {

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

template <typename K, typename V>
struct ArraySource {
  const K* keys;
  const V* vals;
  __device__ bool LoadKey(int64_t i, K* k) const {
    *k = keys[i];
    return true;
  }
  __device__ bool Load(int64_t i, K* k, V* v) const {
    *k = keys[i];
    *v = vals[i];
    return true;
  }
};

template <typename K, typename V>
struct ArraySink {
  K* keys;
  V* vals;
  __device__ void Store(uint32_t pos, K k, V v) const {
    keys[pos] = k;
    vals[pos] = v;
  }
  __device__ void Fill(int64_t) const {}
};

// Positions [0, n) of the source, or [0, min(n, *n_dev)) when n_dev is set.
__device__ __forceinline__ int64_t ActiveCount(int64_t n,
                                               const uint32_t* n_dev) {
  if (n_dev == nullptr) return n;
  const int64_t m = static_cast<int64_t>(*n_dev);
  return m < n ? m : n;
}

// hist[d * tiles + tile] = elements of digit d in the tile.
template <typename K, typename Src>
__global__ __launch_bounds__(kSortBlock) void RadixHistogramK(
    Src src, int64_t n, const uint32_t* n_dev, int shift, uint32_t mask,
    int64_t tiles, uint32_t* hist) {
  __shared__ uint32_t h[kMaxRadix];
  const int radix = static_cast<int>(mask) + 1;
  for (int d = threadIdx.x; d < radix; d += kSortBlock) h[d] = 0;
  __syncthreads();
  const int64_t m = ActiveCount(n, n_dev);
  const int64_t tile = blockIdx.x;
  const int64_t base = tile * kSortTile;
  const int digit_bits = __popc(mask);
  const uint64_t lt = LaneMaskLt();
  // All of the thread's keys first: the source reads through pointers that
  // the compiler cannot tell apart from the LDS counters, so loads issued
  // between the atomics would each wait for the one before.
  K keys[kSortChunks];
  bool act[kSortChunks];
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    const int64_t i = base + c * kSortBlock + threadIdx.x;
    act[c] = i < m && src.LoadKey(i, &keys[c]);
  }
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    const bool active = act[c];
    const uint32_t d = active ? Digit(keys[c], shift, mask) : 0u;
    // Lanes of one digit add their count through one atomic (runs of equal
    // keys would otherwise serialise on one LDS address).
    uint64_t match = __ballot(active);
    for (int b = 0; b < digit_bits; ++b) {
      const uint64_t bits = __ballot((d >> b) & 1u);
      match &= ((d >> b) & 1u) ? bits : ~bits;
    }
    if (active && (match & lt) == 0) {
      atomicAdd(&h[d], static_cast<uint32_t>(__popcll(match)));
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < radix; d += kSortBlock) {
    hist[static_cast<int64_t>(d) * tiles + tile] = h[d];
  }
}

// Stable scatter of one tile (kSortTile consecutive source positions) into
// the digit buckets; `offsets` is the scanned histogram matrix. With
// `fill_tail`, the block also hands the output positions of its tile range
// at or past *total (the number of elements taken) to sink.Fill.
//
// Wave w ranks positions [w * kWaveSpan, (w + 1) * kWaveSpan) of the tile, 64
// at a time in position order: the lanes holding one digit find each other
// with one ballot per digit bit, and the lowest of them adds their count to
// the wave's own LDS counter for that digit (no block barrier per chunk).
// One scan over (wave, digit) then gives every element its place in the
// tile, which is staged in LDS bucket by bucket and written out so that
// consecutive threads write consecutive output positions.
constexpr int kWaveSpan = kSortTile / kSortWaves;   // 512 positions
constexpr int kWaveChunks = kWaveSpan / kWave;      // 8 chunks of 64

template <typename K, typename V, typename Src, typename Sink>
__global__ __launch_bounds__(kSortBlock) void RadixScatterK(
    Src src, Sink sink, int64_t n, const uint32_t* n_dev, int shift,
    uint32_t mask, int digit_bits, int64_t tiles, const uint32_t* offsets,
    const uint32_t* total, bool fill_tail) {
  __shared__ uint32_t wave_cnt[kSortWaves][kMaxRadix];
  __shared__ uint32_t global_off[kMaxRadix];  // bucket start (output)
  __shared__ uint32_t tile_off[kMaxRadix];    // bucket start (tile)
  __shared__ uint32_t scan_tmp[kSortBlock / kWave + 1];
  __shared__ K s_keys[kSortTile];
  __shared__ V s_vals[kSortTile];
  const int t = threadIdx.x;
  const int wave = t / kWave;
  const int lane = t % kWave;
  const int radix = static_cast<int>(mask) + 1;
  const int64_t blk = blockIdx.x;
  const int64_t base = blk * kSortTile;
  if (fill_tail) {
    const int64_t taken = static_cast<int64_t>(*total);
    for (int64_t i = base + t; i < base + kSortTile && i < n;
         i += kSortBlock) {
      if (i >= taken) sink.Fill(i);
    }
  }
  const int64_t m = ActiveCount(n, n_dev);
  if (base >= m) return;  // uniform: the whole block
  const int tile_n =
      static_cast<int>(m - base < kSortTile ? m - base : kSortTile);
  for (int b = t; b < radix; b += kSortBlock) {
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) wave_cnt[w][b] = 0;
    global_off[b] = offsets[static_cast<int64_t>(b) * tiles + blk];
  }
  __syncthreads();
  const uint64_t lt = LaneMaskLt();
  K key[kWaveChunks];
  V val[kWaveChunks];
  uint32_t dig[kWaveChunks];
  uint32_t rank[kWaveChunks];  // among the wave's elements of the digit
  bool act[kWaveChunks];
  // Loads first (see RadixHistogramK), then the ranking.
#pragma unroll
  for (int c = 0; c < kWaveChunks; ++c) {
    const int li = wave * kWaveSpan + c * kWave + lane;
    key[c] = 0;
    val[c] = 0;
    act[c] = li < tile_n && src.Load(base + li, &key[c], &val[c]);
  }
#pragma unroll
  for (int c = 0; c < kWaveChunks; ++c) {
    const bool active = act[c];
    const uint32_t d = active ? Digit(key[c], shift, mask) : 0u;
    uint64_t match = __ballot(active);
    for (int b = 0; b < digit_bits; ++b) {
      const uint64_t bits = __ballot((d >> b) & 1u);
      match &= ((d >> b) & 1u) ? bits : ~bits;
    }
    // The lowest lane of each digit group bumps the wave's counter; the
    // group reads the count before the bump from it.
    const bool leader = active && (match & lt) == 0;
    uint32_t before = 0;
    if (leader) {
      before = wave_cnt[wave][d];
      wave_cnt[wave][d] = before + static_cast<uint32_t>(__popcll(match));
    }
    const int src_lane = active ? __ffsll(static_cast<long long>(match)) - 1
                                : lane;
    before = static_cast<uint32_t>(
        __shfl(static_cast<int>(before), src_lane, kWave));
    dig[c] = active ? d : 0xffffffffu;
    rank[c] = before + static_cast<uint32_t>(__popcll(match & lt));
  }
  __syncthreads();
  // Per digit: the waves' counts become exclusive wave bases, their sum the
  // tile's bucket size, scanned over digits into the tile offsets.
  constexpr int kRounds = kMaxRadix / kSortBlock;
  uint32_t cnt[kRounds];
#pragma unroll
  for (int k = 0; k < kRounds; ++k) {
    const int d = t + k * kSortBlock;
    uint32_t r = 0;
    if (d < radix) {
#pragma unroll
      for (int w = 0; w < kSortWaves; ++w) {
        const uint32_t c = wave_cnt[w][d];
        wave_cnt[w][d] = r;
        r += c;
      }
    }
    cnt[k] = r;
  }
  uint32_t round_base = 0;
#pragma unroll
  for (int k = 0; k < kRounds; ++k) {
    uint32_t round_total;
    const uint32_t ex = BlockExclusiveScan<uint32_t, kSortBlock>(
        cnt[k], scan_tmp, &round_total);
    const int d = t + k * kSortBlock;
    if (d < radix) tile_off[d] = round_base + ex;
    round_base += round_total;
    __syncthreads();
  }
  const int tile_taken = static_cast<int>(round_base);
#pragma unroll
  for (int c = 0; c < kWaveChunks; ++c) {
    if (dig[c] != 0xffffffffu) {
      const uint32_t pos = tile_off[dig[c]] + wave_cnt[wave][dig[c]] + rank[c];
      s_keys[pos] = key[c];
      s_vals[pos] = val[c];
    }
  }
  __syncthreads();
  // Element j of digit d goes to global_off[d] + (j - tile_off[d]).
  for (int j = t; j < tile_taken; j += kSortBlock) {
    const K k = s_keys[j];
    const uint32_t d = Digit(k, shift, mask);
    sink.Store(global_off[d] + (static_cast<uint32_t>(j) - tile_off[d]), k,
               s_vals[j]);
  }
}

// Digit plan: the fewest passes of at most kMaxDigitBits bits over `span`
// key bits, widths balanced (17 bits: three of 6; 21: three of 7; 26: four
// of 7).
struct DigitPlan {
  int passes;
  int digit;
};
inline DigitPlan PlanDigits(int span) {
  DigitPlan p;
  p.passes = span <= 0 ? 0 : (span + kMaxDigitBits - 1) / kMaxDigitBits;
  p.digit = p.passes == 0 ? 0 : (span + p.passes - 1) / p.passes;
  return p;
}

}  // namespace radix
}  // namespace scemb
