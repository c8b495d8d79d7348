// Stable LSD radix sort passes over a source and into a sink (gfx950).
//
// One pass sorts by one digit of at most kMaxDigitBits bits:
//   RadixHistogramK  per-tile digit histograms (LDS atomics: one per wave
//                    whose lanes share a digit, else one per lane),
//                    digit-major
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
  __device__ void Rejected(int64_t) const {}
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

// Positions [0, n) of the source, or [0, min(n, max(n_dev[0, words)))) when
// n_dev is set: one device count (words = 1), or a segment's row pointers,
// whose largest value bounds the positions any partition covers whatever
// their order.
__device__ __forceinline__ int64_t ActiveCount(int64_t n,
                                               const uint32_t* n_dev,
                                               int words) {
  if (n_dev == nullptr) return n;
  int64_t m = 0;
  for (int w = 0; w < words; ++w) {
    const int64_t v = static_cast<int64_t>(n_dev[w]);
    m = v > m ? v : m;
  }
  return m < n ? m : n;
}

// hist[d * tiles + tile] = elements of digit d in the tile. The positions
// the source declines go to src.Rejected after all loads are issued.
// The body of work-group `tile` (RadixHistogramK and grouped launches).
template <typename K, typename Src>
__device__ __forceinline__ void RadixHistogramBody(
    uint32_t tile_index, Src src, int64_t n, const uint32_t* n_dev,
    int n_dev_words, int shift, uint32_t mask, int64_t tiles, uint32_t* hist) {
  __shared__ uint32_t h[kMaxRadix];
  const int radix = static_cast<int>(mask) + 1;
  for (int d = threadIdx.x; d < radix; d += kSortBlock) h[d] = 0;
  __syncthreads();
  const int64_t m = ActiveCount(n, n_dev, n_dev_words);
  const int64_t tile = tile_index;
  const int64_t base = tile * kSortTile;
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
    // A wave whose active lanes share one digit (a run of equal keys, as the
    // later passes see them) adds its count with one atomic; otherwise each
    // lane adds one, which costs less than finding the lanes of each digit.
    const uint64_t live = __ballot(active);
    if (live == 0) continue;  // uniform
    const int first = __ffsll(static_cast<long long>(live)) - 1;
    const uint32_t d0 = static_cast<uint32_t>(
        __shfl(static_cast<int>(d), first, kWave));
    if (__ballot(active && d == d0) == live) {
      if (LaneId() == first) {
        atomicAdd(&h[d0], static_cast<uint32_t>(__popcll(live)));
      }
    } else if (active) {
      atomicAdd(&h[d], 1u);
    }
  }
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    const int64_t i = base + c * kSortBlock + threadIdx.x;
    if (i < m && !act[c]) src.Rejected(i);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < radix; d += kSortBlock) {
    hist[static_cast<int64_t>(d) * tiles + tile] = h[d];
  }
}

template <typename K, typename Src>
__global__ __launch_bounds__(kSortBlock) void RadixHistogramK(
    Src src, int64_t n, const uint32_t* n_dev, int n_dev_words, int shift,
    uint32_t mask, int64_t tiles, uint32_t* hist) {
  RadixHistogramBody<K, Src>(blockIdx.x, src, n, n_dev, n_dev_words, shift,
                             mask, tiles, hist);
}

// RadixHistogramK's arguments for a grouped launch (common.h).
template <typename K, typename Src>
struct RadixHistogramArgs {
  static constexpr int kBlock = kSortBlock;
  Src src;
  int64_t n;
  const uint32_t* n_dev;
  int n_dev_words;
  int shift;
  uint32_t mask;
  int64_t tiles;
  uint32_t* hist;
  __device__ static void Run(const RadixHistogramArgs& a, uint32_t blk,
                             uint32_t) {
    RadixHistogramBody<K, Src>(blk, a.src, a.n, a.n_dev, a.n_dev_words,
                               a.shift, a.mask, a.tiles, a.hist);
  }
};

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
__device__ __forceinline__ void RadixScatterBody(
    uint32_t tile_index, Src src, Sink sink, int64_t n, const uint32_t* n_dev,
    int n_dev_words, int shift, uint32_t mask, int digit_bits, int64_t tiles,
    const uint32_t* offsets, const uint32_t* total, bool fill_tail) {
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
  const int64_t blk = tile_index;
  const int64_t base = blk * kSortTile;
  if (fill_tail) {
    const int64_t taken = static_cast<int64_t>(*total);
    for (int64_t i = base + t; i < base + kSortTile && i < n;
         i += kSortBlock) {
      if (i >= taken) sink.Fill(i);
    }
  }
  const int64_t m = ActiveCount(n, n_dev, n_dev_words);
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

template <typename K, typename V, typename Src, typename Sink>
__global__ __launch_bounds__(kSortBlock) void RadixScatterK(
    Src src, Sink sink, int64_t n, const uint32_t* n_dev, int n_dev_words,
    int shift, uint32_t mask, int digit_bits, int64_t tiles, const uint32_t* offsets,
    const uint32_t* total, bool fill_tail) {
  RadixScatterBody<K, V, Src, Sink>(blockIdx.x, src, sink, n, n_dev,
                                    n_dev_words, shift, mask, digit_bits,
                                    tiles, offsets, total, fill_tail);
}

// RadixScatterK's arguments for a grouped launch (common.h).
template <typename K, typename V, typename Src, typename Sink>
struct RadixScatterArgs {
  static constexpr int kBlock = kSortBlock;
  Src src;
  Sink sink;
  int64_t n;
  const uint32_t* n_dev;
  int n_dev_words;
  int shift;
  uint32_t mask;
  int digit_bits;
  int64_t tiles;
  const uint32_t* offsets;
  const uint32_t* total;
  bool fill_tail;
  __device__ static void Run(const RadixScatterArgs& a, uint32_t blk,
                             uint32_t) {
    RadixScatterBody<K, V, Src, Sink>(blk, a.src, a.sink, a.n, a.n_dev,
                                      a.n_dev_words, a.shift, a.mask,
                                      a.digit_bits, a.tiles, a.offsets,
                                      a.total, a.fill_tail);
  }
};

// --- Two-stage sort: one pass on the high digit, then a sort per bucket ----
//
// After one RadixScatterK pass on the digit above the low `lb` key bits,
// bucket d (the keys whose high digit is d) occupies
// [offsets[d * tiles], offsets[(d + 1) * tiles]) of that pass's output, in
// input order. RadixBucketSortK gives each bucket one block of 16 waves,
// which sorts it stably by the low lb bits:
//   - a chunk of at most kBucketChunk elements is read into LDS with
//     coalesced loads, as (low key bits, position in the chunk) pairs;
//   - one or two LDS passes of at most kBucketDigitMax bits sort the pairs
//     stably: each wave ranks its own contiguous span of the chunk in order
//     (one ballot per digit bit finds the lanes of one digit; the lowest of
//     them bumps the wave's counter), a block scan over (digit, wave) gives
//     the bases, and a second walk places every pair;
//   - the sorted chunk is written out coalesced: the full key is the bucket
//     digit over the low bits, and the value is read at its position.
// A bucket of one chunk is then done. A larger bucket is first counted per
// low-key value (LDS atomics and a scan give each value's start); each
// sorted chunk then places a value's elements after the ones that earlier
// chunks placed.
constexpr int kBucketWaves = 16;
constexpr int kBucketBlock = kBucketWaves * kWave;
constexpr int kBucketChunk = 8192;
constexpr int kBucketDigitMax = 7;
constexpr int kBucketMaxBits = 13;  // two LDS passes; 2^13 value starts

// One stable LDS pass over pairs [0, m) of (sk, si)[from] into [1 - from],
// by bits [shift, shift + bits) of the key. Each wave ranks its span once
// (ballots) and keeps every element's digit and rank in registers across
// the scan, so the placement walk only adds the (digit, wave) base.
constexpr int kBucketWaveChunks = kBucketChunk / kBucketWaves / kWave;

__device__ __forceinline__ void BucketLdsPass(
    uint16_t (*sk)[kBucketChunk], uint16_t (*si)[kBucketChunk],
    uint16_t (*wcnt)[1 << kBucketDigitMax], uint32_t* scan_tmp, int from,
    int m, int shift, int bits) {
  const int t = threadIdx.x;
  const int wave = t / kWave;
  const int lane = t % kWave;
  const uint32_t mask = (1u << bits) - 1u;
  const int digits = 1 << bits;
  const int span = ((m + kBucketWaves - 1) / kBucketWaves + kWave - 1) /
                   kWave * kWave;
  const int w0 = wave * span;
  const int w1 = w0 + span < m ? w0 + span : m;
  const uint64_t lt = LaneMaskLt();
  for (int v = lane; v < digits; v += kWave) wcnt[wave][v] = 0;
  uint16_t key[kBucketWaveChunks];
  uint16_t idx[kBucketWaveChunks];
  uint16_t dig[kBucketWaveChunks];
  uint16_t rank[kBucketWaveChunks];
#pragma unroll
  for (int c = 0; c < kBucketWaveChunks; ++c) {
    const int i = w0 + c * kWave + lane;
    const bool active = i < w1;
    key[c] = active ? sk[from][i] : 0;
    idx[c] = active ? si[from][i] : 0;
  }
#pragma unroll
  for (int c = 0; c < kBucketWaveChunks; ++c) {
    if (w0 + c * kWave >= w1) break;  // uniform: the wave's span ended
    const bool active = w0 + c * kWave + lane < w1;
    const uint32_t v = (static_cast<uint32_t>(key[c]) >> shift) & mask;
    uint64_t match = __ballot(active);
    for (int b = 0; b < bits; ++b) {
      const uint64_t bb = __ballot((v >> b) & 1u);
      match &= ((v >> b) & 1u) ? bb : ~bb;
    }
    const bool leader = active && (match & lt) == 0;
    uint32_t before = 0;
    if (leader) {
      before = wcnt[wave][v];
      wcnt[wave][v] = static_cast<uint16_t>(before + __popcll(match));
    }
    const int src_lane =
        active ? __ffsll(static_cast<long long>(match)) - 1 : lane;
    before = static_cast<uint32_t>(
        __shfl(static_cast<int>(before), src_lane, kWave));
    dig[c] = static_cast<uint16_t>(v);
    rank[c] = static_cast<uint16_t>(before + __popcll(match & lt));
  }
  __syncthreads();
  // Exclusive scan over cells (digit, wave), digit-major: cells 2t, 2t + 1.
  {
    const int c0 = 2 * t;
    const int cells = digits * kBucketWaves;
    uint32_t a = 0, b2 = 0;
    if (c0 < cells) a = wcnt[c0 % kBucketWaves][c0 / kBucketWaves];
    if (c0 + 1 < cells) b2 = wcnt[(c0 + 1) % kBucketWaves][(c0 + 1) / kBucketWaves];
    uint32_t all;
    const uint32_t ex =
        BlockExclusiveScan<uint32_t, kBucketBlock>(a + b2, scan_tmp, &all);
    if (c0 < cells) {
      wcnt[c0 % kBucketWaves][c0 / kBucketWaves] = static_cast<uint16_t>(ex);
    }
    if (c0 + 1 < cells) {
      wcnt[(c0 + 1) % kBucketWaves][(c0 + 1) / kBucketWaves] =
          static_cast<uint16_t>(ex + a);
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kBucketWaveChunks; ++c) {
    const int i = w0 + c * kWave + lane;
    if (i < w1) {
      const uint32_t pos = static_cast<uint32_t>(wcnt[wave][dig[c]]) + rank[c];
      if (pos < static_cast<uint32_t>(m)) {
        sk[1 - from][pos] = key[c];
        si[1 - from][pos] = idx[c];
      }
    }
  }
  __syncthreads();
}

// One bucket [lo, hi) of digit d, by the whole block.
template <typename K, typename V, typename Sink>
__device__ __forceinline__ void BucketSort(
    const K* keys, const V* vals, const Sink& sink, int64_t lo, int64_t hi,
    int d, int lb, uint16_t (*sk)[kBucketChunk], uint16_t (*si)[kBucketChunk],
    uint16_t (*wcnt)[1 << kBucketDigitMax], uint32_t* next, uint16_t* head,
    uint32_t* scan_tmp, bool try_unique) {
  constexpr int kPer = kBucketChunk / kBucketBlock;  // elements per thread
  const int t = threadIdx.x;
  const int64_t size = hi - lo;
  const uint32_t lmask = (1u << lb) - 1u;
  const K high = static_cast<K>(static_cast<uint64_t>(d) << lb);
  const int values = 1 << lb;
  const bool chunked = size > kBucketChunk;
  if (chunked) {
    for (int v = t; v < values; v += kBucketBlock) next[v] = 0;
    __syncthreads();
    for (int64_t i0 = lo; i0 < hi; i0 += kBucketBlock * kPer) {
      K k[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = i0 + u * kBucketBlock + t;
        k[u] = i < hi ? keys[i] : K{0};
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        if (i0 + u * kBucketBlock + t < hi) {
          atomicAdd(&next[static_cast<uint32_t>(k[u]) & lmask], 1u);
        }
      }
    }
    __syncthreads();
    // Thread t scans values [t * per, (t + 1) * per).
    const int per = (values + kBucketBlock - 1) / kBucketBlock;
    const int v0 = t * per;
    uint32_t sum = 0;
    for (int v = v0; v < v0 + per && v < values; ++v) sum += next[v];
    uint32_t all;
    uint32_t run =
        BlockExclusiveScan<uint32_t, kBucketBlock>(sum, scan_tmp, &all);
    for (int v = v0; v < v0 + per && v < values; ++v) {
      const uint32_t c = next[v];
      next[v] = run;
      run += c;
    }
  }
  const int b0 = lb <= kBucketDigitMax ? lb : lb / 2;
  const int b1 = lb - b0;
  for (int64_t c0 = lo; c0 < hi; c0 += kBucketChunk) {
    const int m = static_cast<int>(hi - c0 < kBucketChunk ? hi - c0
                                                          : kBucketChunk);
    __syncthreads();  // the previous chunk is out of LDS
    {
      K k[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int i = u * kBucketBlock + t;
        k[u] = i < m ? keys[c0 + i] : K{0};
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int i = u * kBucketBlock + t;
        if (i < m) {
          sk[0][i] = static_cast<uint16_t>(static_cast<uint32_t>(k[u]) & lmask);
          si[0][i] = static_cast<uint16_t>(i);
        }
      }
    }
    __syncthreads();
    // A bucket of one chunk whose low keys never repeat (at most one entry
    // per activation row) needs no ranking: a count per low key, then each
    // present key's place is the number of present keys below it. Any
    // repeat falls back to the ranked passes, with the same result.
    bool placed = false;
    if (try_unique && !chunked) {
      for (int v = t; v < values; v += kBucketBlock) next[v] = 0;
      __syncthreads();
      bool dup = false;
      for (int i = t; i < m; i += kBucketBlock) {
        const uint32_t v = sk[0][i] & lmask;
        dup = dup || atomicAdd(&next[v], 1u) != 0;
        head[v] = static_cast<uint16_t>(i);
      }
      if (!__syncthreads_or(dup)) {
        const int per = (values + kBucketBlock - 1) / kBucketBlock;
        const int v0 = t * per;
        uint32_t sum = 0;
        for (int v = v0; v < v0 + per && v < values; ++v) sum += next[v];
        uint32_t all;
        uint32_t pos =
            BlockExclusiveScan<uint32_t, kBucketBlock>(sum, scan_tmp, &all);
        for (int v = v0; v < v0 + per && v < values; ++v) {
          if (next[v] != 0 && pos < static_cast<uint32_t>(m)) {
            sk[1][pos] = static_cast<uint16_t>(v);
            si[1][pos] = head[v];
            ++pos;
          }
        }
        __syncthreads();
        placed = true;
      }
    }
    int cur = 1;
    if (!placed) {
      BucketLdsPass(sk, si, wcnt, scan_tmp, 0, m, 0, b0);
      if (b1 > 0) {
        BucketLdsPass(sk, si, wcnt, scan_tmp, 1, m, b0, b1);
        cur = 0;
      }
    }
    // Every pair of [0, m) was placed; the masks below only keep LDS and
    // value reads in range whatever the keys hold.
    if (chunked) {
      for (int i = t; i < m; i += kBucketBlock) {
        const uint32_t v = sk[cur][i] & lmask;
        if (i == 0 || (sk[cur][i - 1] & lmask) != v) {
          head[v] = static_cast<uint16_t>(i);
        }
      }
      __syncthreads();
    }
    V x[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = u * kBucketBlock + t;
      const int j = i < m ? si[cur][i] : m;
      x[u] = j < m ? vals[c0 + j] : V{0};
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = u * kBucketBlock + t;
      if (i < m) {
        const uint32_t v = sk[cur][i] & lmask;
        const int64_t rel =
            chunked ? static_cast<int64_t>(next[v]) + (i - head[v])
                    : (c0 - lo) + i;
        // rel < size by construction; the test keeps every store inside the
        // bucket whatever the keys hold.
        if (rel < size) {
          sink.Store(static_cast<uint32_t>(lo + rel), high | static_cast<K>(v),
                     x[u]);
        }
      }
    }
    if (chunked) {
      __syncthreads();
      for (int i = t; i < m; i += kBucketBlock) {
        const uint32_t v = sk[cur][i] & lmask;
        if (i == m - 1 || (sk[cur][i + 1] & lmask) != v) {
          next[v] += i - head[v] + 1;
        }
      }
    }
  }
}

template <typename K, typename V, typename Sink>
__global__ __launch_bounds__(kBucketBlock) void RadixBucketSortK(
    const K* keys, const V* vals, Sink sink, const uint32_t* offsets,
    int64_t tiles, int buckets, const uint32_t* total, int lb, int64_t n,
    bool fill_tail, bool try_unique) {
  __shared__ uint16_t sk[2][kBucketChunk];
  __shared__ uint16_t si[2][kBucketChunk];
  __shared__ uint16_t wcnt[kBucketWaves][1 << kBucketDigitMax];
  __shared__ uint32_t next[1 << kBucketMaxBits];  // buckets of several chunks
  __shared__ uint16_t head[1 << kBucketMaxBits];
  __shared__ uint32_t scan_tmp[kBucketWaves + 1];
  const int t = threadIdx.x;
  // The three bounds load together (no store before them).
  const int d = blockIdx.x;
  const int64_t taken = static_cast<int64_t>(*total);
  const int64_t lo = offsets[static_cast<int64_t>(d) * tiles];
  const int64_t hi =
      d + 1 < buckets ? offsets[static_cast<int64_t>(d + 1) * tiles] : taken;
  if (hi > lo) {  // uniform: the whole block
    BucketSort<K, V, Sink>(keys, vals, sink, lo, hi, d, lb, sk, si, wcnt,
                           next, head, scan_tmp, try_unique);
  }
  if (fill_tail) {
    for (int64_t i = taken + static_cast<int64_t>(blockIdx.x) * kBucketBlock +
                     t;
         i < n; i += static_cast<int64_t>(gridDim.x) * kBucketBlock) {
      sink.Fill(i);
    }
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
