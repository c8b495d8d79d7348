// Forward gather-reduce and backward segmented reduce fused with the SGD /
// Adagrad row update (the SparseDenseMatmulOp and
// SparseDenseMatmulGradOpWithOptimizerUpdate custom calls of
// jax_tpu_embedding/sparsecore/lib/core/primitives/).
//
// Both directions are one segmented reduction over a stream of entries
// (key, row, gain) sorted by key:
//   forward   key = activation row, gathered row = table row
//             epilogue: store the activation row (rows without entries are
//             zero-filled)
//   backward  key = table row, gathered row = activation-gradient row
//             epilogue: optimizer update of the table row (and accumulator)
// The stream comes from one of three places:
//   * the CSR itself when it is already sorted by table row (backward; one
//     segment, as the preprocessing emits it: partitions in order, embedding
//     ids ascending inside each partition);
//   * a sample view built once per preprocessed batch (forward);
//   * otherwise ExpandCsr + a stable radix sort inside the call.
//
// SegReduce gives every 256-thread block a fixed slice of 256 stream entries
// (perfect load balance however skewed the keys are). A block is split into
// P = 256 / G sub-groups of G lanes; sub-group s owns entries [s*G, s*G + G)
// of the slice and its lanes cover G * VEC columns of a row (16-byte loads).
// A sub-group walks its entries kUnroll at a time, issuing all row loads of a
// batch (and, for runs that end inside the batch, the table / accumulator
// loads of the update) before accumulating. A run that is complete inside
// one sub-group is finished there; pieces of runs that cross sub-groups are
// combined through LDS in sub-group order; pieces of runs that cross blocks
// leave one partial row per block and SegFinish adds them in block order.
// Every row is reduced and written exactly once, in a fixed order: no float
// atomics and run-to-run identical results.
#include "../../include/scemb.h"
#include "common.h"
#include "scan.h"

namespace scemb {
namespace {

constexpr int kBlock = 256;  // threads per block = stream entries per block
// Entries whose rows a sub-group loads together (memory-level parallelism;
// the backward also holds the table / accumulator rows of the runs that end
// in the batch). Batches of about one entry per activation row ("one-hot")
// gain from the wide setting; multi-hot batches, whose gathers mostly hit
// cache, from the higher occupancy of the narrow one (fewer registers).
constexpr int kFwdUnrollWide = 8;
constexpr int kFwdUnrollNarrow = 4;
constexpr int kBwdUnrollWide = 4;
constexpr int kBwdUnrollNarrow = 2;
// Entries per activation row up to which a batch counts as one-hot.
constexpr int64_t kOneHotMaxEntriesPerRow = 2;
// Streaming (nontemporal) access for data touched once per call, so the
// last-level cache keeps table rows: activations written by the forward
// always; activation gradients read by the backward for one-hot batches
// only (a multi-hot batch re-reads every gradient row from cache many
// times). Table and accumulator rows stay cacheable: the next forward reads
// the rows the backward has just written.
constexpr bool kNtAct = true;
constexpr bool kNtTable = false;
constexpr uint32_t kSkip = 0xffffffffu;  // key of an entry outside any run

// Per-block flags left by SegReduce for SegFinish.
constexpr uint32_t kFlagHeadEnd = 1;  // a run from earlier blocks ends here
constexpr uint32_t kFlagOwner = 2;    // a run starts here, continues past
constexpr uint32_t kFlagMiddle = 4;   // the whole block lies inside one run

// Per-sub-group piece flags (LDS).
constexpr uint32_t kHasHead = 1;   // first entry continues the previous run
constexpr uint32_t kHeadEnds = 2;  // ... and that run ends in this range
constexpr uint32_t kHasTail = 4;   // a run starts here and continues past

enum { kSrcSorted = 0, kSrcCsr = 1 };
enum { kEpiFwd = 0, kEpiSgd = 1, kEpiAdagrad = 2 };

struct Csr {
  const int32_t* rp;
  const int32_t* eid;
  const int32_t* sid;
  const float* gains;
  int64_t per_segment;  // coo_size / num_segments
  int32_t num_segments;
  int32_t num_partitions;
  int32_t rp_per_segment;
};

__device__ __forceinline__ uint64_t Pack(uint32_t lo, float g) {
  return static_cast<uint64_t>(lo) |
         (static_cast<uint64_t>(__float_as_uint(g)) << 32);
}
__device__ __forceinline__ uint32_t PackedIndex(uint64_t p) {
  return static_cast<uint32_t>(p);
}
__device__ __forceinline__ float PackedGain(uint64_t p) {
  return __uint_as_float(static_cast<uint32_t>(p >> 32));
}

// Partition of position `off` of a segment whose row pointers are `rp`
// (partitions start at 8-aligned offsets), or -1 for padding.
__device__ __forceinline__ int PartitionOf(const int32_t* rp, int nparts,
                                           int64_t per_segment, int64_t off) {
  int64_t start = 0;
  for (int q = 0; q < nparts; ++q) {
    int64_t end = rp[q];
    if (end > per_segment) end = per_segment;
    if (off < end) return off >= start ? q : -1;
    start = (end + kAlign - 1) / kAlign * kAlign;
  }
  return -1;
}

// One (key, payload) pair per COO position; padding and invalid entries get
// the sentinel key, which sorts last.
template <bool kBySample>
__global__ __launch_bounds__(256) void ExpandCsr(Csr csr, int64_t bps,
                                                 int64_t rows_per_partition,
                                                 uint32_t sentinel,
                                                 uint32_t* keys,
                                                 uint64_t* payload,
                                                 uint32_t* status) {
  const int64_t n = csr.per_segment * csr.num_segments;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int s = static_cast<int>(j / csr.per_segment);
  const int64_t off = j - static_cast<int64_t>(s) * csr.per_segment;
  const int p = PartitionOf(csr.rp + static_cast<int64_t>(s) * csr.rp_per_segment,
                            csr.num_partitions, csr.per_segment, off);
  uint32_t key = sentinel;
  uint64_t pay = 0;
  if (p >= 0) {
    const int32_t e = csr.eid[j];
    const int32_t sm = csr.sid[j];
    if (e >= 0 && e < rows_per_partition && sm >= 0 && sm < bps) {
      const uint32_t trow =
          static_cast<uint32_t>(p * rows_per_partition + e);
      const uint32_t arow = static_cast<uint32_t>(s * bps + sm);
      const float g = csr.gains[j];
      if (kBySample) {
        key = arow;
        pay = Pack(trow, g);
      } else {
        key = trow;
        pay = Pack(arow, g);
      }
    } else if (status != nullptr) {
      atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
    }
  }
  keys[j] = key;
  payload[j] = pay;
}

template <int VEC>
struct Vec;
typedef float NativeF4 __attribute__((ext_vector_type(4)));
template <>
struct Vec<4> {
  using T = float4;
  __device__ static T Zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ static T Load(const float* p) {
    return *reinterpret_cast<const float4*>(p);
  }
  __device__ static void Store(float* p, T v) {
    *reinterpret_cast<float4*>(p) = v;
  }
  __device__ static T LoadNT(const float* p) {
    const NativeF4 v =
        __builtin_nontemporal_load(reinterpret_cast<const NativeF4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  __device__ static void StoreNT(float* p, T v) {
    const NativeF4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<NativeF4*>(p));
  }
  __device__ static T Fma(T acc, float g, T v) {
    acc.x = acc.x + g * v.x;
    acc.y = acc.y + g * v.y;
    acc.z = acc.z + g * v.z;
    acc.w = acc.w + g * v.w;
    return acc;
  }
  __device__ static T Add(T a, T b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
  __device__ static float Get(const T& v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
  }
  __device__ static void Set(T& v, int k, float x) {
    if (k == 0) v.x = x;
    else if (k == 1) v.y = x;
    else if (k == 2) v.z = x;
    else v.w = x;
  }
};
template <>
struct Vec<1> {
  using T = float;
  __device__ static T Zero() { return 0.f; }
  __device__ static T Load(const float* p) { return *p; }
  __device__ static void Store(float* p, T v) { *p = v; }
  __device__ static T LoadNT(const float* p) {
    return __builtin_nontemporal_load(p);
  }
  __device__ static void StoreNT(float* p, T v) {
    __builtin_nontemporal_store(v, p);
  }
  __device__ static T Fma(T acc, float g, T v) { return acc + g * v; }
  __device__ static T Add(T a, T b) { return a + b; }
  __device__ static float Get(const T& v, int) { return v; }
  __device__ static void Set(T& v, int, float x) { v = x; }
};

template <int VEC, bool NT>
__device__ __forceinline__ typename Vec<VEC>::T LoadRow(const float* p) {
  return NT ? Vec<VEC>::LoadNT(p) : Vec<VEC>::Load(p);
}
template <int VEC, bool NT>
__device__ __forceinline__ void StoreRow(float* p, typename Vec<VEC>::T v) {
  if (NT) {
    Vec<VEC>::StoreNT(p, v);
  } else {
    Vec<VEC>::Store(p, v);
  }
}

struct OptParams {
  const float* lr_ptr;
  float lr_value;
  int32_t clip_mask;
  float min_value;
  float max_value;
};

// Where the stream comes from.
struct StreamArgs {
  const uint32_t* keys;     // kSrcSorted
  const uint64_t* entries;  // kSrcSorted: row | gain bits << 32
  uint32_t sentinel;        // kSrcSorted: keys >= sentinel are unused
  int64_t src_rows;         // kSrcSorted: rows of the gathered matrix
  Csr csr;                  // kSrcCsr (one segment)
  int64_t rows_per_partition;
  int64_t bps;
  int64_t n;
};

constexpr int kMaxRowBlocks = SCEMB_MAX_ROW_BLOCKS;

// The activation matrix (forward output, backward input) as per-feature row
// blocks: stacked rows [first, end) of block b live at data[b] with
// stride[b] floats between rows and width[b] leading columns (the rest of
// the dim columns are padding: not written, read as zero). n == 0: one
// dense [batch, dim] matrix.
struct RowMap {
  int32_t n;
  int64_t first[kMaxRowBlocks];
  int64_t end[kMaxRowBlocks];
  int64_t stride[kMaxRowBlocks];
  int32_t width[kMaxRowBlocks];
  float* data[kMaxRowBlocks];
};

// What the reduction reads and writes.
struct RowArgs {
  const float* src;  // gathered rows
  float* dst;        // activations (forward) or table (backward)
  float* accum;      // Adagrad accumulator
  int64_t dim;
  int64_t batch;     // forward: rows of dst
  bool stream_src;   // gathered rows are read about once: nontemporal loads
  RowMap act;        // activation layout (dst forward, src backward)
  OptParams opt;
  float* partials;   // [2 * num_blocks, dim]
  uint32_t* block_flags;
  uint32_t* block_keys;
  uint32_t* status;
};

template <int SRC>
__device__ __forceinline__ uint32_t FetchEntry(const StreamArgs& s, int64_t e,
                                               uint64_t* ent,
                                               uint32_t* status) {
  if (SRC == kSrcSorted) {
    const uint32_t k = s.keys[e];
    *ent = s.entries[e];
    if (k >= s.sentinel) return kSkip;
    if (PackedIndex(*ent) >= s.src_rows) {
      // Keeps the key (and so the run structure) but contributes nothing.
      if (status != nullptr) atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
      *ent = Pack(0, 0.0f);
    }
    return k;
  } else {
    *ent = 0;
    const int p = PartitionOf(s.csr.rp, s.csr.num_partitions,
                              s.csr.per_segment, e);
    if (p < 0) return kSkip;
    const int32_t id = s.csr.eid[e];
    const int32_t sm = s.csr.sid[e];
    if (id < 0 || id >= s.rows_per_partition || sm < 0 || sm >= s.bps) {
      if (status != nullptr) atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
      return kSkip;
    }
    *ent = Pack(static_cast<uint32_t>(sm), s.csr.gains[e]);
    return static_cast<uint32_t>(p * s.rows_per_partition + id);
  }
}

template <int OPT>
__device__ __forceinline__ float UpdateOne(float t, float* a, float g,
                                           float lr, const OptParams& o) {
  float v;
  if (OPT == kEpiSgd) {
    v = t - g * lr;
  } else {
    const float acc = *a + g * g;
    *a = acc;
    v = t - (lr * g) / sqrtf(acc);
  }
  if (o.clip_mask & 1) v = fmaxf(o.min_value, v);
  if (o.clip_mask & 2) v = fminf(o.max_value, v);
  return v;
}

// The row map staged in LDS by every block that reads or writes
// activations through it.
struct RowMapLds {
  int32_t n;
  int64_t first[kMaxRowBlocks];
  int64_t end[kMaxRowBlocks];
  int64_t stride[kMaxRowBlocks];
  int32_t width[kMaxRowBlocks];
  float* data[kMaxRowBlocks];
};

// Copies the row map into LDS; the caller synchronises the block after.
__device__ __forceinline__ void StageRowMap(const RowMap& m, RowMapLds* s) {
  const int t = threadIdx.x;
  if (t == 0) s->n = m.n;
  if (t < m.n) {
    s->first[t] = m.first[t];
    s->end[t] = m.end[t];
    s->stride[t] = m.stride[t];
    s->width[t] = m.width[t];
    s->data[t] = m.data[t];
  }
}

// Address of columns [col, col + VEC) of activation row `row`, or null when
// the row lies in no block or the columns in its padding. Without a map
// (kMapped false) the activations are one dense matrix.
template <bool kMapped>
__device__ __forceinline__ float* ActAddr(const RowMapLds& m, float* dense,
                                          int64_t dim, int64_t row,
                                          int64_t col) {
  if (!kMapped) return dense + row * dim + col;
  if (m.n == 0) return nullptr;
  int lo = 0, hi = m.n;  // last block whose first row is <= row
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (m.first[mid] <= row) lo = mid; else hi = mid;
  }
  if (row < m.first[lo] || row >= m.end[lo] || col >= m.width[lo]) {
    return nullptr;
  }
  return m.data[lo] + (row - m.first[lo]) * m.stride[lo] + col;
}

// Epilogue for the finished row `key` at column `col`, given the table and
// accumulator values already loaded (backward) -- or the store (forward).
template <int VEC, int EPI, bool kMapped>
__device__ __forceinline__ void Epilogue(const RowArgs& r,
                                         const RowMapLds& m, uint32_t key,
                                         int64_t col, typename Vec<VEC>::T g,
                                         typename Vec<VEC>::T t,
                                         typename Vec<VEC>::T a, float lr) {
  using V = Vec<VEC>;
  const int64_t off = static_cast<int64_t>(key) * r.dim + col;
  if (EPI == kEpiFwd) {
    float* p = ActAddr<kMapped>(m, r.dst, r.dim, key, col);
    if (p != nullptr) StoreRow<VEC, kNtAct>(p, g);
    return;
  }
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float ak = V::Get(a, k);
    V::Set(t, k, UpdateOne<EPI>(V::Get(t, k), &ak, V::Get(g, k), lr, r.opt));
    V::Set(a, k, ak);
  }
  StoreRow<VEC, kNtTable>(r.dst + off, t);
  if (EPI == kEpiAdagrad) StoreRow<VEC, kNtTable>(r.accum + off, a);
}

template <int VEC, int EPI, bool kMapped>
__device__ __forceinline__ void EpilogueLoad(const RowArgs& r,
                                             const RowMapLds& m, uint32_t key,
                                             int64_t col,
                                             typename Vec<VEC>::T g,
                                             float lr) {
  using V = Vec<VEC>;
  typename V::T t = V::Zero(), a = V::Zero();
  const int64_t off = static_cast<int64_t>(key) * r.dim + col;
  if (EPI != kEpiFwd) t = V::Load(r.dst + off);
  if (EPI == kEpiAdagrad) a = V::Load(r.accum + off);
  Epilogue<VEC, EPI, kMapped>(r, m, key, col, g, t, a, lr);
}

__device__ __forceinline__ uint64_t LowBits(int k) {
  return k >= 64 ? ~0ull : ((1ull << k) - 1);
}

template <int G, int VEC, bool kMapped>
__device__ __forceinline__ void ZeroRows(const RowMapLds& m, float* dst,
                                         int64_t dim, int64_t lo, int64_t hi,
                                         int cl) {
  using V = Vec<VEC>;
  for (int64_t row = lo; row < hi; ++row) {
    for (int64_t col = static_cast<int64_t>(cl) * VEC; col < dim;
         col += static_cast<int64_t>(G) * VEC) {
      float* p = ActAddr<kMapped>(m, dst, dim, row, col);
      if (p != nullptr) StoreRow<VEC, kNtAct>(p, V::Zero());
    }
  }
}

template <int G, int VEC, int SRC, int EPI, int kUnroll, bool kMapped>
__global__ __launch_bounds__(kBlock) void SegReduce(StreamArgs st, RowArgs r) {
  using V = Vec<VEC>;
  using T = typename V::T;
  constexpr int P = kBlock / G;
  __shared__ uint32_t s_key[kBlock + 2];  // [0]: entry before, [257]: after
  __shared__ uint64_t s_ent[kBlock];
  __shared__ T s_part[2 * P][G];
  __shared__ uint32_t s_info[P];
  __shared__ RowMapLds s_map;

  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t cb = blk * kBlock;
  const int64_t n = st.n;
  // Blocks that lie wholly in the padding after the last entry (CSR buffers
  // are sized for the worst case) only clear their flag: with the CSR, past
  // the end of the last partition; with a sorted stream, after an unused key
  // (unused keys sort last, and the first one still has gaps to fill).
  {
    bool tail;
    if (SRC == kSrcCsr) {
      int64_t end = 0;
      for (int q = 0; q < st.csr.num_partitions; ++q) {
        end = st.csr.rp[q] > end ? st.csr.rp[q] : end;
      }
      tail = cb >= end;
    } else {
      tail = cb > 0 && st.keys[cb - 1] >= st.sentinel;
    }
    if (tail) {
      if (tid == 0) r.block_flags[blk] = 0;
      return;
    }
  }
  if (kMapped) StageRowMap(r.act, &s_map);
  {
    uint64_t en = 0;
    uint32_t k = kSkip;
    if (cb + tid < n) k = FetchEntry<SRC>(st, cb + tid, &en, r.status);
    s_key[tid + 1] = k;
    s_ent[tid] = en;
    if (tid == 0) {
      uint64_t d;
      s_key[0] = cb > 0 ? FetchEntry<SRC>(st, cb - 1, &d, nullptr) : kSkip;
    }
    if (tid == kBlock - 1) {
      uint64_t d;
      s_key[kBlock + 1] =
          cb + kBlock < n ? FetchEntry<SRC>(st, cb + kBlock, &d, nullptr)
                          : kSkip;
    }
  }
  __syncthreads();

  const int sub = tid / G;
  const int cl = tid % G;
  const int base = sub * G;  // first entry of the sub-group in the block
  const int64_t left = n - (cb + base);
  const int cnt = left <= 0 ? 0 : (left < G ? static_cast<int>(left) : G);
  const uint32_t my_key = s_key[tid + 1];
  const uint32_t prev_key = s_key[tid];
  const bool mine = cl < cnt;
  const bool valid = mine && my_key != kSkip;

  if (r.status != nullptr && mine) {
    const bool bad = SRC == kSrcCsr
                         ? (valid && prev_key != kSkip && prev_key > my_key)
                         : (cb + tid > 0 && prev_key > my_key);
    if (bad) atomicOr(r.status, SCEMB_STATUS_UNSORTED);
  }

  const int wshift = (tid % kWave) / G * G;
  const uint64_t gmask = LowBits(G);
  const uint64_t valid_m = (__ballot(valid) >> wshift) & gmask;
  const uint64_t start_m =
      (__ballot(valid && my_key != prev_key) >> wshift) & gmask;
  const uint64_t end_m =
      (__ballot(valid && (cl == cnt - 1 || my_key != s_key[tid + 2])) >>
       wshift) & gmask;

  if (EPI == kEpiFwd) {
    // Activation rows without entries: rows strictly between the clamped
    // keys of consecutive entries, before the first and after the last.
    const int64_t e = cb + tid;
    const int64_t ck = my_key == kSkip ? r.batch : my_key;
    const int64_t cp = e == 0 ? -1 : (prev_key == kSkip ? r.batch : prev_key);
    const bool gap = mine && ck > cp + 1;
    uint64_t m = (__ballot(gap) >> wshift) & gmask;
    while (m) {
      const int l = __ffsll(static_cast<long long>(m)) - 1;
      m &= m - 1;
      const int64_t lo = __shfl(static_cast<int>(cp + 1), wshift + l);
      const int64_t hi = __shfl(static_cast<int>(ck), wshift + l);
      ZeroRows<G, VEC, kMapped>(s_map, r.dst, r.dim, lo, hi, cl);
    }
    const bool tail_gap = mine && e == n - 1 && ck + 1 < r.batch;
    m = (__ballot(tail_gap) >> wshift) & gmask;
    if (m) {
      const int l = __ffsll(static_cast<long long>(m)) - 1;
      const int64_t lo = __shfl(static_cast<int>(ck + 1), wshift + l);
      ZeroRows<G, VEC, kMapped>(s_map, r.dst, r.dim, lo, r.batch, cl);
    }
  }

  // Pieces of this sub-group's range that are not whole runs.
  const bool head_cont = (valid_m & 1) && !(start_m & 1);
  bool tail_cont = false;
  if (cnt > 0) {
    const uint32_t kl = s_key[base + cnt];
    tail_cont = kl != kSkip && kl == s_key[base + cnt + 1];
  }
  const bool whole = head_cont && tail_cont &&
                     (start_m & ~1ull & LowBits(cnt)) == 0;
  const uint32_t info = (head_cont ? kHasHead : 0) |
                        (head_cont && !whole ? kHeadEnds : 0) |
                        (tail_cont && !whole ? kHasTail : 0);
  if (cl == 0) s_info[sub] = info;
  if (tid == 0) {
    const int last = n - cb < kBlock ? static_cast<int>(n - cb) : kBlock;
    const uint32_t kf = s_key[1], kl = s_key[last];
    const bool from_prev = kf != kSkip && kf == s_key[0];
    const bool to_next = kl != kSkip && kl == s_key[last + 1];
    uint32_t f;
    if (from_prev && to_next && kf == kl) {
      f = kFlagMiddle;
    } else {
      f = (from_prev ? kFlagHeadEnd : 0) | (to_next ? kFlagOwner : 0);
    }
    r.block_flags[blk] = f;
    if (f & kFlagOwner) r.block_keys[blk] = kl;
  }

  const float lr = EPI == kEpiFwd
                       ? 0.f
                       : (r.opt.lr_ptr != nullptr ? *r.opt.lr_ptr
                                                  : r.opt.lr_value);
  const int64_t dim = r.dim;
  for (int64_t col0 = 0; col0 < dim; col0 += static_cast<int64_t>(G) * VEC) {
    const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
    const bool col_ok = col < dim;
    T acc = V::Zero();
    for (int q = 0; q < cnt; q += kUnroll) {
      T v[kUnroll];
      T tv[kUnroll];
      T av[kUnroll];
      float gn[kUnroll];
      uint32_t kk[kUnroll];
      bool fin[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = q + u;
        const bool val = idx < cnt && ((valid_m >> idx) & 1);
        uint64_t en = 0;
        kk[u] = kSkip;
        if (val) {
          en = s_ent[base + idx];
          kk[u] = s_key[base + idx + 1];
        }
        gn[u] = PackedGain(en);
        v[u] = V::Zero();
        if (val && col_ok) {
          // Forward: table rows (dense); backward: activation-gradient rows
          // through the row map.
          const float* p =
              EPI == kEpiFwd
                  ? r.src + static_cast<int64_t>(PackedIndex(en)) * dim + col
                  : ActAddr<kMapped>(s_map, const_cast<float*>(r.src), dim,
                                     PackedIndex(en), col);
          if (p != nullptr) v[u] = r.stream_src ? V::LoadNT(p) : V::Load(p);
        }
        const bool is_end = val && ((end_m >> idx) & 1);
        const bool first = (start_m & ~1ull & LowBits(idx + 1)) == 0;
        const bool head_piece = head_cont && first;
        const bool tail_piece = idx == cnt - 1 && tail_cont;
        fin[u] = is_end && !head_piece && !tail_piece;
        tv[u] = V::Zero();
        av[u] = V::Zero();
        if (EPI != kEpiFwd && fin[u] && col_ok) {
          const int64_t off = static_cast<int64_t>(kk[u]) * dim + col;
          tv[u] = V::Load(r.dst + off);
          if (EPI == kEpiAdagrad) av[u] = V::Load(r.accum + off);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = q + u;
        if (idx < cnt && ((valid_m >> idx) & 1)) {
          acc = V::Fma(acc, gn[u], v[u]);
          if ((end_m >> idx) & 1) {
            if (fin[u]) {
              if (col_ok) {
                Epilogue<VEC, EPI, kMapped>(r, s_map, kk[u], col, acc, tv[u],
                                            av[u], lr);
              }
            } else {
              const bool first = (start_m & ~1ull & LowBits(idx + 1)) == 0;
              s_part[head_cont && first ? 2 * sub : 2 * sub + 1][cl] = acc;
            }
            acc = V::Zero();
          }
        }
      }
    }
    __syncthreads();
    // Runs crossing sub-group boundaries: the sub-group holding a run's first
    // piece in this block adds the following sub-groups' head pieces.
    for (int job = 0; job < 2; ++job) {
      const bool active =
          job == 0 ? (sub == 0 && (info & kHasHead)) : (info & kHasTail) != 0;
      if (!active) continue;
      T g = s_part[job == 0 ? 0 : 2 * sub + 1][cl];
      bool ended = job == 0 && (info & kHeadEnds);
      for (int tt = sub + 1; !ended && tt < P; ++tt) {
        const uint32_t inf = s_info[tt];
        if (!(inf & kHasHead)) break;
        g = V::Add(g, s_part[2 * tt][cl]);
        ended = (inf & kHeadEnds) != 0;
      }
      const uint32_t key = job == 0 ? s_key[1] : s_key[base + cnt];
      if (job == 1 && ended) {
        if (col_ok) EpilogueLoad<VEC, EPI, kMapped>(r, s_map, key, col, g, lr);
      } else if (col_ok) {
        const int64_t slot = job == 1 ? 2 * blk + 1 : 2 * blk;
        V::Store(r.partials + slot * dim + col, g);
      }
    }
    __syncthreads();
  }
}

// Runs that cross blocks: the block where such a run starts (kFlagOwner)
// finds the block where it ends (the next kFlagHeadEnd; every block between
// is kFlagMiddle), adds the partial rows in block order and applies the
// epilogue once.
template <int G, int VEC, int EPI, bool kMapped>
__global__ __launch_bounds__(kBlock) void SegFinish(int64_t num_blocks,
                                                    RowArgs r) {
  using V = Vec<VEC>;
  using T = typename V::T;
  constexpr int P = kBlock / G;
  constexpr int kWaves = kBlock / kWave;
  __shared__ T s_part[P][G];
  __shared__ int64_t s_end[kWaves];
  __shared__ RowMapLds s_map;
  const int64_t blk = blockIdx.x;
  if (!(r.block_flags[blk] & kFlagOwner)) return;
  const int tid = threadIdx.x;
  if (kMapped) {
    StageRowMap(r.act, &s_map);
    __syncthreads();
  }
  const int sub = tid / G;
  const int cl = tid % G;
  const uint32_t key = r.block_keys[blk];
  int64_t c1 = -1;
  for (int64_t b0 = blk + 1; b0 < num_blocks && c1 < 0; b0 += kBlock) {
    const int64_t c = b0 + tid;
    const bool is_end = c < num_blocks && (r.block_flags[c] & kFlagHeadEnd);
    const uint64_t m = __ballot(is_end);
    if (tid % kWave == 0) {
      s_end[tid / kWave] =
          m ? b0 + (tid / kWave) * kWave +
                  (__ffsll(static_cast<long long>(m)) - 1)
            : -1;
    }
    __syncthreads();
    for (int w = 0; w < kWaves; ++w) {
      if (s_end[w] >= 0) {
        c1 = s_end[w];
        break;
      }
    }
    __syncthreads();
  }
  if (c1 < 0) {
    if (tid == 0 && r.status != nullptr) {
      atomicOr(r.status, SCEMB_STATUS_BAD_ENTRY);
    }
    return;
  }
  const int64_t m = c1 - blk + 1;  // partial rows: 2*blk+1, then 2*(blk+q)
  const float lr = EPI == kEpiFwd
                       ? 0.f
                       : (r.opt.lr_ptr != nullptr ? *r.opt.lr_ptr
                                                  : r.opt.lr_value);
  const int64_t dim = r.dim;
  for (int64_t col0 = 0; col0 < dim; col0 += static_cast<int64_t>(G) * VEC) {
    const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
    const bool col_ok = col < dim;
    T acc = V::Zero();
    if (col_ok) {
      int64_t q = sub;
      for (; q + 3 * P < m; q += 4 * P) {
        const T p0 = V::Load(r.partials +
                             (q == 0 ? 2 * blk + 1 : 2 * (blk + q)) * dim + col);
        const T p1 = V::Load(r.partials + 2 * (blk + q + P) * dim + col);
        const T p2 = V::Load(r.partials + 2 * (blk + q + 2 * P) * dim + col);
        const T p3 = V::Load(r.partials + 2 * (blk + q + 3 * P) * dim + col);
        acc = V::Add(acc, p0);
        acc = V::Add(acc, p1);
        acc = V::Add(acc, p2);
        acc = V::Add(acc, p3);
      }
      for (; q < m; q += P) {
        acc = V::Add(acc, V::Load(r.partials +
                                  (q == 0 ? 2 * blk + 1 : 2 * (blk + q)) * dim +
                                  col));
      }
    }
    s_part[sub][cl] = acc;
    __syncthreads();
    if (sub == 0) {
      T g = s_part[0][cl];
      for (int s = 1; s < P; ++s) g = V::Add(g, s_part[s][cl]);
      if (col_ok) EpilogueLoad<VEC, EPI, kMapped>(r, s_map, key, col, g, lr);
    }
    __syncthreads();
  }
}

__global__ void FillF32(float* p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

struct Geometry {
  int64_t n;  // COO positions
  int64_t bps;
  int64_t rows_per_partition;
};

int CheckCsr(const scemb_csr_t* csr, int64_t batch, int64_t table_rows,
             int32_t dim, Geometry* geo) {
  if (csr == nullptr) return Fail(SCEMB_ERR_INVALID_ARGUMENT, "csr is null");
  if (csr->num_segments <= 0 || csr->num_partitions <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "num_segments and num_partitions must be positive");
  }
  if (csr->row_pointers_per_segment < csr->num_partitions) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "row_pointers_per_segment must be >= num_partitions");
  }
  if (csr->coo_size < 0 || dim <= 0 || batch < 0 || table_rows < 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "negative size");
  }
  if (batch % csr->num_segments != 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "device_batch_size must be divisible by num_segments");
  }
  if (table_rows % csr->num_partitions != 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "table rows must be divisible by num_partitions");
  }
  if (table_rows >= (int64_t{1} << 32) - 1 || batch >= (int64_t{1} << 31) - 1) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "table or batch too large");
  }
  const int64_t per_seg = csr->coo_size / csr->num_segments;
  geo->n = per_seg * csr->num_segments;
  if (geo->n >= (int64_t{1} << 31) - 1) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "coo buffer too large");
  }
  geo->bps = batch / csr->num_segments;
  geo->rows_per_partition = table_rows / csr->num_partitions;
  if (geo->n > 0 && (csr->row_pointers == nullptr ||
                     csr->embedding_ids == nullptr ||
                     csr->sample_ids == nullptr || csr->gains == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null CSR buffer");
  }
  return 0;
}

Csr MakeCsr(const scemb_csr_t* csr) {
  Csr c;
  c.rp = csr->row_pointers;
  c.eid = csr->embedding_ids;
  c.sid = csr->sample_ids;
  c.gains = csr->gains;
  c.per_segment = csr->coo_size / csr->num_segments;
  c.num_segments = csr->num_segments;
  c.num_partitions = csr->num_partitions;
  c.rp_per_segment = csr->row_pointers_per_segment;
  return c;
}

// Lanes per row (>= 4) and vector width for a row of `dim` floats.
void PickLayout(int64_t dim, bool vec4_ok, int* g, int* vec) {
  *vec = vec4_ok && dim % 4 == 0 ? 4 : 1;
  const int64_t lanes = CeilDiv(dim, *vec);
  int gg = 4;
  while (gg < lanes && gg < kWave) gg <<= 1;
  *g = gg;
}

bool Aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

struct SortBuffers {
  uint32_t* keys;
  uint64_t* pay;
  uint32_t* keys_alt;
  uint64_t* pay_alt;
};

SortBuffers TakeSortBuffers(Arena& ws, int64_t n) {
  SortBuffers b;
  b.keys = ws.Take<uint32_t>(n);
  b.pay = ws.Take<uint64_t>(n);
  b.keys_alt = ws.Take<uint32_t>(n);
  b.pay_alt = ws.Take<uint64_t>(n);
  return b;
}

struct SegBuffers {
  int64_t num_blocks;
  float* partials;
  uint32_t* flags;
  uint32_t* keys;
};

SegBuffers TakeSegBuffers(Arena& ws, int64_t n, int64_t dim) {
  SegBuffers b;
  b.num_blocks = CeilDiv(n, kBlock);
  b.partials = ws.Take<float>(2 * b.num_blocks * dim);
  b.flags = ws.Take<uint32_t>(b.num_blocks);
  b.keys = ws.Take<uint32_t>(b.num_blocks);
  return b;
}

template <int SRC, int EPI, bool kMapped>
int LaunchSegMapped(const StreamArgs& st, RowArgs r, const SegBuffers& sb,
                    int g, int vec, bool one_hot, const char* reduce_span,
                    const char* finish_span, hipStream_t stream) {
  constexpr int kWide = EPI == kEpiFwd ? kFwdUnrollWide : kBwdUnrollWide;
  constexpr int kNarrow = EPI == kEpiFwd ? kFwdUnrollNarrow : kBwdUnrollNarrow;
  r.partials = sb.partials;
  r.block_flags = sb.flags;
  r.block_keys = sb.keys;
  const dim3 grid(static_cast<uint32_t>(sb.num_blocks));
#define SCEMB_SEG_CASE(GG, VV)                                                \
  if (g == GG && vec == VV) {                                                \
    int prof = ProfileBegin(reduce_span, stream);                            \
    if (one_hot) {                                                           \
      hipLaunchKernelGGL((SegReduce<GG, VV, SRC, EPI, kWide, kMapped>), grid, \
                         dim3(kBlock), 0, stream, st, r);                     \
    } else {                                                                 \
      hipLaunchKernelGGL((SegReduce<GG, VV, SRC, EPI, kNarrow, kMapped>),     \
                         grid, dim3(kBlock), 0, stream, st, r);               \
    }                                                                        \
    ProfileEnd(prof, stream);                                                 \
    SCEMB_LAUNCH_CHECK();                                                     \
    prof = ProfileBegin(finish_span, stream);                                 \
    hipLaunchKernelGGL((SegFinish<GG, VV, EPI, kMapped>), grid, dim3(kBlock), \
                       0, stream, sb.num_blocks, r);                          \
    ProfileEnd(prof, stream);                                                 \
    SCEMB_LAUNCH_CHECK();                                                     \
    return 0;                                                                 \
  }
  SCEMB_SEG_CASE(4, 1) SCEMB_SEG_CASE(8, 1) SCEMB_SEG_CASE(16, 1)
  SCEMB_SEG_CASE(32, 1) SCEMB_SEG_CASE(64, 1) SCEMB_SEG_CASE(4, 4)
  SCEMB_SEG_CASE(8, 4) SCEMB_SEG_CASE(16, 4) SCEMB_SEG_CASE(32, 4)
  SCEMB_SEG_CASE(64, 4)
#undef SCEMB_SEG_CASE
  return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unsupported layout");
}

// Launches SegReduce + SegFinish for the layout picked for `dim`; `one_hot`
// selects the wide unroll, `mapped` the kernels that address activations
// through the row map in `r.act` (which may hold no block at all).
template <int SRC, int EPI>
int LaunchSeg(const StreamArgs& st, const RowArgs& r, const SegBuffers& sb,
              int g, int vec, bool one_hot, bool mapped,
              const char* reduce_span, const char* finish_span,
              hipStream_t stream) {
  if (mapped) {
    return LaunchSegMapped<SRC, EPI, true>(st, r, sb, g, vec, one_hot,
                                           reduce_span, finish_span, stream);
  }
  return LaunchSegMapped<SRC, EPI, false>(st, r, sb, g, vec, one_hot,
                                          reduce_span, finish_span, stream);
}

// Sample-major stream of a CSR into (keys, entries): expand + stable sort.
// The result lands in (b.keys, b.pay) or the alt pair (*in_alt).
int BuildSampleStream(const scemb_csr_t* csr, const Geometry& geo,
                      int64_t batch, const SortBuffers& b, Arena& ws,
                      uint32_t* status, hipStream_t stream, bool* in_alt) {
  const int64_t n = geo.n;
  if (!ws.measuring() && n > 0) {
    hipLaunchKernelGGL(ExpandCsr<true>, dim3(CeilDiv(n, 256)), dim3(256), 0,
                       stream, MakeCsr(csr), geo.bps, geo.rows_per_partition,
                       static_cast<uint32_t>(batch), b.keys, b.pay, status);
    SCEMB_LAUNCH_CHECK();
  }
  const int key_bits = BitWidth(static_cast<uint64_t>(batch));
  return RadixSortPairs<uint32_t, uint64_t>(b.keys, b.pay, b.keys_alt,
                                            b.pay_alt, n, 0, key_bits, ws,
                                            stream, in_alt);
}

// Checks per-feature row blocks against a [batch, dim] activation matrix and
// packs them for the kernels; *vec4_ok tells whether every block allows
// 16-byte row accesses.
int MakeRowMap(const scemb_row_block_t* blocks, int32_t num_blocks,
               int64_t batch, int32_t dim, RowMap* m, bool* vec4_ok) {
  if (num_blocks < 0 || num_blocks > kMaxRowBlocks ||
      (num_blocks > 0 && blocks == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "between 0 and SCEMB_MAX_ROW_BLOCKS row blocks required");
  }
  *m = RowMap{};
  m->n = num_blocks;
  *vec4_ok = true;
  int64_t prev_end = 0;
  for (int32_t b = 0; b < num_blocks; ++b) {
    const scemb_row_block_t& k = blocks[b];
    if (k.first_row < prev_end || k.num_rows < 0 ||
        k.first_row + k.num_rows > batch) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "row blocks must be ascending, disjoint and inside the "
                  "batch");
    }
    if (k.width <= 0 || k.width > dim || k.row_stride < k.width ||
        (k.num_rows > 0 && k.data == nullptr)) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "row block needs data, 0 < width <= dim and "
                  "row_stride >= width");
    }
    m->first[b] = k.first_row;
    m->end[b] = k.first_row + k.num_rows;
    m->stride[b] = k.row_stride;
    m->width[b] = k.width;
    m->data[b] = k.data;
    *vec4_ok = *vec4_ok && k.width % 4 == 0 && k.row_stride % 4 == 0 &&
               Aligned16(k.data);
    prev_end = m->end[b];
  }
  return 0;
}

__global__ void FillStrided(float* p, int64_t rows, int64_t width,
                            int64_t stride, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < rows * width) p[(i / width) * stride + i % width] = v;
}

// `map` (may be null): the activations as per-feature row blocks instead of
// the dense `act`.
int ForwardImpl(const scemb_csr_t* csr, const scemb_sample_view_t* view,
                const float* table, int64_t table_rows, int32_t dim,
                float* act, const RowMap* map, bool map_vec4,
                int64_t batch, Arena& ws, uint32_t* status,
                hipStream_t stream) {
  StreamArgs st{};
  st.sentinel = static_cast<uint32_t>(batch);
  st.src_rows = table_rows;
  if (view != nullptr) {
    if (view->size < 0 || (view->size > 0 && (view->keys == nullptr ||
                                              view->entries == nullptr))) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "bad sample view");
    }
    if (view->device_batch_size != batch || view->table_rows != table_rows) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "sample view was built for another batch size or table");
    }
    if (dim <= 0 || batch < 0 || batch >= (int64_t{1} << 31) - 1 ||
        view->size >= (int64_t{1} << 31) - 1) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "bad size");
    }
    st.n = view->size;
    st.keys = view->keys;
    st.entries = view->entries;
  } else {
    Geometry geo;
    const int rc = CheckCsr(csr, batch, table_rows, dim, &geo);
    if (rc != 0) return rc;
    st.n = geo.n;
    SortBuffers b = TakeSortBuffers(ws, geo.n);
    bool in_alt = false;
    if (!ws.measuring() && ws.overflow()) {
      return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    }
    if (ws.measuring() || (geo.n > 0 && batch > 0)) {
      const int rc2 = BuildSampleStream(csr, geo, batch, b, ws, status,
                                        stream, &in_alt);
      if (rc2 != 0) return rc2;
    }
    st.keys = in_alt ? b.keys_alt : b.keys;
    st.entries = in_alt ? b.pay_alt : b.pay;
  }
  const SegBuffers sb = TakeSegBuffers(ws, st.n, dim);
  if (ws.measuring()) return 0;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  if (batch == 0) return 0;
  if (st.n == 0 || table_rows == 0) {
    if (map == nullptr) {
      hipLaunchKernelGGL(FillF32, dim3(CeilDiv(batch * dim, 256)), dim3(256),
                         0, stream, act, batch * dim, 0.0f);
      SCEMB_LAUNCH_CHECK();
    }
    for (int32_t b = 0; map != nullptr && b < map->n; ++b) {
      const int64_t rows = map->end[b] - map->first[b];
      if (rows == 0) continue;
      hipLaunchKernelGGL(FillStrided,
                         dim3(CeilDiv(rows * map->width[b], 256)), dim3(256),
                         0, stream, map->data[b], rows,
                         static_cast<int64_t>(map->width[b]), map->stride[b],
                         0.0f);
      SCEMB_LAUNCH_CHECK();
    }
    return 0;
  }
  RowArgs r{};
  r.src = table;
  r.dst = act;
  r.dim = dim;
  r.batch = batch;
  r.status = status;
  if (map != nullptr) r.act = *map;
  int g, vec;
  PickLayout(dim, Aligned16(table) && (map != nullptr ? map_vec4
                                                      : Aligned16(act)),
             &g, &vec);
  const int64_t hint = view != nullptr ? view->num_entries
                                        : csr->num_entries;
  const int64_t entries = hint > 0 && hint < st.n ? hint : st.n;
  const bool one_hot = entries <= kOneHotMaxEntriesPerRow * batch;
  return LaunchSeg<kSrcSorted, kEpiFwd>(st, r, sb, g, vec, one_hot,
                                        map != nullptr, "fwd_reduce",
                                        "fwd_finish", stream);
}

// `map` (may be null): the activation gradients as per-feature row blocks
// instead of the dense `act_grad`.
template <int EPI>
int GradImpl(const scemb_csr_t* csr, const float* act_grad, const RowMap* map,
             bool map_vec4, int64_t batch, float* table, float* accum,
             int64_t table_rows, int32_t dim, const OptParams& opt, Arena& ws,
             uint32_t* status, hipStream_t stream) {
  Geometry geo;
  int rc = CheckCsr(csr, batch, table_rows, dim, &geo);
  if (rc != 0) return rc;
  const int64_t n = geo.n;
  const bool direct =
      (csr->flags & SCEMB_CSR_SORTED_BY_ROW) != 0 && csr->num_segments == 1;
  StreamArgs st{};
  st.n = n;
  if (direct) {
    st.csr = MakeCsr(csr);
    st.rows_per_partition = geo.rows_per_partition;
    st.bps = geo.bps;
  } else {
    SortBuffers b = TakeSortBuffers(ws, n);
    bool in_alt = false;
    if (!ws.measuring()) {
      if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
      if (n > 0 && batch > 0) {
        hipLaunchKernelGGL(ExpandCsr<false>, dim3(CeilDiv(n, 256)), dim3(256),
                           0, stream, MakeCsr(csr), geo.bps,
                           geo.rows_per_partition,
                           static_cast<uint32_t>(table_rows), b.keys, b.pay,
                           status);
        SCEMB_LAUNCH_CHECK();
      }
    }
    if (n > 0 && batch > 0) {
      rc = RadixSortPairs<uint32_t, uint64_t>(
          b.keys, b.pay, b.keys_alt, b.pay_alt, n, 0,
          BitWidth(static_cast<uint64_t>(table_rows)), ws, stream, &in_alt);
      if (rc != 0) return rc;
    }
    st.keys = in_alt ? b.keys_alt : b.keys;
    st.entries = in_alt ? b.pay_alt : b.pay;
    st.sentinel = static_cast<uint32_t>(table_rows);
    st.src_rows = batch;
  }
  const SegBuffers sb = TakeSegBuffers(ws, n, dim);
  if (ws.measuring()) return 0;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  if (n == 0 || batch == 0) return 0;
  RowArgs r{};
  r.src = act_grad;
  r.dst = table;
  r.accum = accum;
  r.dim = dim;
  r.batch = batch;
  r.opt = opt;
  r.status = status;
  if (map != nullptr) r.act = *map;
  // Entries per activation row: how often each gradient row is gathered.
  const int64_t entries =
      csr->num_entries > 0 && csr->num_entries < n ? csr->num_entries : n;
  const bool one_hot = entries <= kOneHotMaxEntriesPerRow * batch;
  r.stream_src = one_hot;
  int g, vec;
  PickLayout(dim, Aligned16(table) &&
                      (map != nullptr ? map_vec4 : Aligned16(act_grad)) &&
                      (EPI != kEpiAdagrad || Aligned16(accum)), &g, &vec);
  if (direct) {
    return LaunchSeg<kSrcCsr, EPI>(st, r, sb, g, vec, one_hot, map != nullptr,
                                   "bwd_reduce", "bwd_finish", stream);
  }
  return LaunchSeg<kSrcSorted, EPI>(st, r, sb, g, vec, one_hot,
                                    map != nullptr, "bwd_reduce",
                                    "bwd_finish", stream);
}

int BuildViewImpl(const scemb_csr_t* csr, int64_t batch, int64_t table_rows,
                  uint32_t* keys, uint64_t* entries, Arena& ws,
                  uint32_t* status, hipStream_t stream) {
  Geometry geo;
  const int rc = CheckCsr(csr, batch, table_rows, 1, &geo);
  if (rc != 0) return rc;
  SortBuffers b;
  b.keys = keys;
  b.pay = entries;
  b.keys_alt = ws.Take<uint32_t>(geo.n);
  b.pay_alt = ws.Take<uint64_t>(geo.n);
  if (!ws.measuring()) {
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    if (geo.n > 0 && (keys == nullptr || entries == nullptr)) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null view buffer");
    }
  }
  bool in_alt = false;
  const int rc2 = BuildSampleStream(csr, geo, batch, b, ws, status, stream,
                                    &in_alt);
  if (rc2 != 0 || ws.measuring()) return rc2;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  if (in_alt && geo.n > 0) {
    SCEMB_HIP(hipMemcpyAsync(keys, b.keys_alt, geo.n * sizeof(uint32_t),
                             hipMemcpyDeviceToDevice, stream));
    SCEMB_HIP(hipMemcpyAsync(entries, b.pay_alt, geo.n * sizeof(uint64_t),
                             hipMemcpyDeviceToDevice, stream));
  }
  return 0;
}

}  // namespace
}  // namespace scemb

namespace scemb {
namespace {

int ForwardEntry(const scemb_csr_t* csr, const scemb_sample_view_t* view,
                 const float* table, int64_t table_rows, int32_t dim,
                 float* activations, const scemb_row_block_t* blocks,
                 int32_t num_blocks, bool mapped, int64_t batch,
                 void* workspace, size_t workspace_bytes,
                 uint32_t* device_status, void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (table == nullptr || (!mapped && activations == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null table or activations");
  }
  RowMap map;
  bool vec4 = false;
  if (mapped) {
    const int rc = MakeRowMap(blocks, num_blocks, batch, dim, &map, &vec4);
    if (rc != 0) return rc;
  }
  Arena ws(workspace, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("fwd_call", s);
  const int rc = ForwardImpl(csr, view, table, table_rows, dim, activations,
                             mapped ? &map : nullptr, vec4, batch, ws,
                             device_status, s);
  ProfileEnd(prof, s);
  return rc;
}

template <int EPI>
int GradEntry(const scemb_csr_t* csr, const float* activations_grad,
              const scemb_row_block_t* blocks, int32_t num_blocks,
              bool mapped, int64_t batch, float* table, float* accumulator,
              int64_t table_rows, int32_t dim, const float* learning_rate,
              float learning_rate_value, int32_t clip_mask, float min_value,
              float max_value, void* workspace, size_t workspace_bytes,
              uint32_t* device_status, void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (table == nullptr || (EPI == kEpiAdagrad && accumulator == nullptr) ||
      (!mapped && activations_grad == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "null table, accumulator or gradient");
  }
  if ((clip_mask & 3) == 3 && min_value > max_value) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "min_value must be less than or equal to max_value");
  }
  RowMap map;
  bool vec4 = false;
  if (mapped) {
    const int rc = MakeRowMap(blocks, num_blocks, batch, dim, &map, &vec4);
    if (rc != 0) return rc;
  }
  Arena ws(workspace, workspace_bytes);
  OptParams o{learning_rate, learning_rate_value, clip_mask, min_value,
              max_value};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("bwd_call", s);
  const int rc = GradImpl<EPI>(csr, activations_grad, mapped ? &map : nullptr,
                               vec4, batch, table, accumulator, table_rows,
                               dim, o, ws, device_status, s);
  ProfileEnd(prof, s);
  return rc;
}

}  // namespace
}  // namespace scemb

using namespace scemb;

extern "C" {

size_t scemb_sparse_dense_matmul_workspace_size(
    const scemb_csr_t* csr, const scemb_sample_view_t* view,
    int64_t device_batch_size, int64_t table_rows, int32_t dim) {
  Arena ws(nullptr, 0);
  if (ForwardImpl(csr, view, nullptr, table_rows, dim, nullptr, nullptr,
                  false, device_batch_size, ws, nullptr, nullptr) != 0) {
    return 0;
  }
  return ws.used() + 256;
}

int scemb_sparse_dense_matmul(const scemb_csr_t* csr,
                              const scemb_sample_view_t* view,
                              const float* table, int64_t table_rows,
                              int32_t dim, float* activations,
                              int64_t device_batch_size, void* workspace,
                              size_t workspace_bytes, uint32_t* device_status,
                              void* stream) {
  return ForwardEntry(csr, view, table, table_rows, dim, activations, nullptr,
                      0, false, device_batch_size, workspace, workspace_bytes,
                      device_status, stream);
}

int scemb_sparse_dense_matmul_to_blocks(
    const scemb_csr_t* csr, const scemb_sample_view_t* view,
    const float* table, int64_t table_rows, int32_t dim,
    const scemb_row_block_t* outputs, int32_t num_outputs,
    int64_t device_batch_size, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  return ForwardEntry(csr, view, table, table_rows, dim, nullptr, outputs,
                      num_outputs, true, device_batch_size, workspace,
                      workspace_bytes, device_status, stream);
}

size_t scemb_build_sample_view_workspace_size(const scemb_csr_t* csr,
                                              int64_t device_batch_size,
                                              int64_t table_rows) {
  Arena ws(nullptr, 0);
  if (BuildViewImpl(csr, device_batch_size, table_rows, nullptr, nullptr, ws,
                    nullptr, nullptr) != 0) {
    return 0;
  }
  return ws.used() + 256;
}

int scemb_build_sample_view(const scemb_csr_t* csr, int64_t device_batch_size,
                            int64_t table_rows, uint32_t* keys,
                            uint64_t* entries, void* workspace,
                            size_t workspace_bytes, uint32_t* device_status,
                            void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  Arena ws(workspace, workspace_bytes);
  return BuildViewImpl(csr, device_batch_size, table_rows, keys, entries, ws,
                       device_status, static_cast<hipStream_t>(stream));
}

size_t scemb_sparse_dense_matmul_grad_workspace_size(const scemb_csr_t* csr,
                                                     int64_t device_batch_size,
                                                     int64_t table_rows,
                                                     int32_t dim) {
  Arena ws(nullptr, 0);
  OptParams o{nullptr, 0.f, 0, 0.f, 0.f};
  if (GradImpl<kEpiSgd>(csr, nullptr, nullptr, false, device_batch_size,
                        nullptr, nullptr, table_rows, dim, o, ws, nullptr,
                        nullptr) != 0) {
    return 0;
  }
  return ws.used() + 256;
}

int scemb_sparse_dense_matmul_grad_with_sgd(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  return GradEntry<kEpiSgd>(csr, activations_grad, nullptr, 0, false,
                            device_batch_size, table, nullptr, table_rows,
                            dim, learning_rate, learning_rate_value,
                            clip_mask, min_value, max_value, workspace,
                            workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_sgd_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  return GradEntry<kEpiSgd>(csr, nullptr, activation_grads, num_blocks, true,
                            device_batch_size, table, nullptr, table_rows,
                            dim, learning_rate, learning_rate_value,
                            clip_mask, min_value, max_value, workspace,
                            workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_adagrad(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, float* accumulator,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  return GradEntry<kEpiAdagrad>(csr, activations_grad, nullptr, 0, false,
                                device_batch_size, table, accumulator,
                                table_rows, dim, learning_rate,
                                learning_rate_value, clip_mask, min_value,
                                max_value, workspace, workspace_bytes,
                                device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    float* accumulator, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  return GradEntry<kEpiAdagrad>(csr, nullptr, activation_grads, num_blocks,
                                true, device_batch_size, table, accumulator,
                                table_rows, dim, learning_rate,
                                learning_rate_value, clip_mask, min_value,
                                max_value, workspace, workspace_bytes,
                                device_status, stream);
}

}  // extern "C"
