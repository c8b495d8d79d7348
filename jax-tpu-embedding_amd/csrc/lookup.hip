// Forward gather-reduce and backward segmented reduce fused with the SGD /
// Adagrad row update (the SparseDenseMatmulOp and
// SparseDenseMatmulGradOpWithOptimizerUpdate custom calls of
// jax_tpu_embedding/sparsecore/lib/core/primitives/).
//
// Both directions start from the reference's CSR-wrapped COO buffers:
//   1. ExpandCsr resolves every position of the COO buffer to its partition
//      (row pointers), validates ids, and emits one (key, payload) pair:
//      forward  key = activation row,  payload = (table row, gain)
//      backward key = table row,       payload = (activation row, gain)
//      Padding and invalid slots get a sentinel key that sorts last.
//   2. A stable LSD radix sort groups the pairs by key (CSR order is kept
//      inside each group, so sums run in CSR order).
//   3. Forward: one sub-wave (G lanes, 16-byte loads) per activation row sums
//      gain * table row over its group and writes the row once.
//      Backward: one wavefront per fixed chunk of the sorted pairs walks the
//      runs of equal table rows; a run inside the chunk is reduced and the
//      optimizer applied directly; a run crossing chunk boundaries leaves one
//      partial per chunk, and the wave that completes the run (integer
//      counter, no float atomics) adds the partials in chunk order and
//      applies the optimizer once.
#include "../../include/scemb.h"
#include "common.h"
#include "scan.h"

namespace scemb {
namespace {

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
  const int32_t* rp = csr.rp + static_cast<int64_t>(s) * csr.rp_per_segment;
  int p = -1;
  int64_t start = 0;
  for (int q = 0; q < csr.num_partitions; ++q) {
    int64_t end = rp[q];
    if (end > csr.per_segment) end = csr.per_segment;
    if (off < end) {
      if (off >= start) p = q;
      break;
    }
    start = (end + kAlign - 1) / kAlign * kAlign;
  }
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

// sp[b] = first sorted position whose key is >= b, for b in [0, batch].
__global__ __launch_bounds__(256) void GroupStarts(const uint32_t* keys,
                                                   int64_t n, int64_t batch,
                                                   int32_t* sp) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b > batch) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(keys[mid]) < b) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  sp[b] = static_cast<int32_t>(lo);
}

template <int VEC>
struct Vec;
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
  __device__ static T ShflXor(T v, int m) {
    return make_float4(__shfl_xor(v.x, m), __shfl_xor(v.y, m),
                       __shfl_xor(v.z, m), __shfl_xor(v.w, m));
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
  __device__ static T Fma(T acc, float g, T v) { return acc + g * v; }
  __device__ static T Add(T a, T b) { return a + b; }
  __device__ static T ShflXor(T v, int m) { return __shfl_xor(v, m); }
  __device__ static float Get(const T& v, int) { return v; }
  __device__ static void Set(T& v, int, float x) { v = x; }
};

// Forward: sub-wave of G lanes per activation row.
template <int G, int VEC>
__global__ __launch_bounds__(256) void FwdGather(const int32_t* sp,
                                                 const uint64_t* payload,
                                                 const float* table,
                                                 int64_t dim, float* act,
                                                 int64_t batch) {
  using V = Vec<VEC>;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / G;
  const int lane = static_cast<int>(gtid % G);
  if (row >= batch) return;
  const int32_t lo = sp[row];
  const int32_t hi = sp[row + 1];
  for (int64_t c = static_cast<int64_t>(lane) * VEC; c < dim;
       c += static_cast<int64_t>(G) * VEC) {
    typename V::T acc = V::Zero();
    int32_t i = lo;
    for (; i + 4 <= hi; i += 4) {
      const uint64_t p0 = payload[i], p1 = payload[i + 1],
                     p2 = payload[i + 2], p3 = payload[i + 3];
      const typename V::T v0 =
          V::Load(table + static_cast<int64_t>(PackedIndex(p0)) * dim + c);
      const typename V::T v1 =
          V::Load(table + static_cast<int64_t>(PackedIndex(p1)) * dim + c);
      const typename V::T v2 =
          V::Load(table + static_cast<int64_t>(PackedIndex(p2)) * dim + c);
      const typename V::T v3 =
          V::Load(table + static_cast<int64_t>(PackedIndex(p3)) * dim + c);
      acc = V::Fma(acc, PackedGain(p0), v0);
      acc = V::Fma(acc, PackedGain(p1), v1);
      acc = V::Fma(acc, PackedGain(p2), v2);
      acc = V::Fma(acc, PackedGain(p3), v3);
    }
    for (; i < hi; ++i) {
      const uint64_t p0 = payload[i];
      acc = V::Fma(acc, PackedGain(p0),
                   V::Load(table + static_cast<int64_t>(PackedIndex(p0)) * dim + c));
    }
    V::Store(act + row * dim + c, acc);
  }
}

struct OptParams {
  const float* lr_ptr;
  float lr_value;
  int32_t clip_mask;
  float min_value;
  float max_value;
};

template <int OPT>
__device__ __forceinline__ float UpdateOne(float t, float* a, float g,
                                           float lr, const OptParams& o) {
  float v;
  if (OPT == 0) {
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

template <int VEC, int OPT>
__device__ __forceinline__ void ApplyUpdate(float* table, float* accum,
                                            int64_t row, int64_t dim,
                                            int64_t c, typename Vec<VEC>::T g,
                                            float lr, const OptParams& o) {
  using V = Vec<VEC>;
  float* tp = table + row * dim + c;
  typename V::T t = V::Load(tp);
  typename V::T a = V::Zero();
  float* ap = nullptr;
  if (OPT == 1) {
    ap = accum + row * dim + c;
    a = V::Load(ap);
  }
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float ak = V::Get(a, k);
    const float nv = UpdateOne<OPT>(V::Get(t, k), &ak, V::Get(g, k), lr, o);
    V::Set(t, k, nv);
    V::Set(a, k, ak);
  }
  V::Store(tp, t);
  if (OPT == 1) V::Store(ap, a);
}

// Sum of gain * act_grad rows over sorted positions [a, b) for the column
// tile starting at `c`, reduced over the P = 64 / G sub-waves of the wave so
// that every sub-wave holds the total.
template <int G, int VEC>
__device__ __forceinline__ typename Vec<VEC>::T RunSum(
    const uint64_t* payload, int64_t a, int64_t b, const float* act_grad,
    int64_t dim, int64_t c, int sub) {
  using V = Vec<VEC>;
  constexpr int P = kWave / G;
  typename V::T acc = V::Zero();
  const bool col_ok = c < dim;
  int64_t i = a + sub;
  if (col_ok) {
    for (; i + 3 * P < b; i += 4 * P) {
      const uint64_t p0 = payload[i], p1 = payload[i + P],
                     p2 = payload[i + 2 * P], p3 = payload[i + 3 * P];
      const typename V::T v0 =
          V::Load(act_grad + static_cast<int64_t>(PackedIndex(p0)) * dim + c);
      const typename V::T v1 =
          V::Load(act_grad + static_cast<int64_t>(PackedIndex(p1)) * dim + c);
      const typename V::T v2 =
          V::Load(act_grad + static_cast<int64_t>(PackedIndex(p2)) * dim + c);
      const typename V::T v3 =
          V::Load(act_grad + static_cast<int64_t>(PackedIndex(p3)) * dim + c);
      acc = V::Fma(acc, PackedGain(p0), v0);
      acc = V::Fma(acc, PackedGain(p1), v1);
      acc = V::Fma(acc, PackedGain(p2), v2);
      acc = V::Fma(acc, PackedGain(p3), v3);
    }
    for (; i < b; i += P) {
      const uint64_t p0 = payload[i];
      acc = V::Fma(acc, PackedGain(p0),
                   V::Load(act_grad + static_cast<int64_t>(PackedIndex(p0)) * dim + c));
    }
  }
#pragma unroll
  for (int m = G; m < kWave; m <<= 1) acc = V::Add(acc, V::ShflXor(acc, m));
  return acc;
}

// First index in [lo, hi) whose key differs from `key` (keys sorted), or hi.
__device__ __forceinline__ int64_t RunEnd(const uint32_t* keys, int64_t lo,
                                          int64_t hi, uint32_t key) {
  for (int64_t base = lo; base < hi; base += kWave) {
    const int64_t idx = base + __lane_id();
    const uint32_t k = idx < hi ? keys[idx] : key;
    const uint64_t diff = __ballot(k != key);
    if (diff) return base + (__ffsll(static_cast<long long>(diff)) - 1);
  }
  return hi;
}

__device__ __forceinline__ int64_t LowerBound(const uint32_t* keys, int64_t lo,
                                              int64_t hi, uint32_t key) {
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < key) lo = mid + 1; else hi = mid;
  }
  return lo;
}
__device__ __forceinline__ int64_t UpperBound(const uint32_t* keys, int64_t lo,
                                              int64_t hi, uint32_t key) {
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] <= key) lo = mid + 1; else hi = mid;
  }
  return lo;
}

template <int G, int VEC, int OPT>
__global__ __launch_bounds__(256) void BwdFused(
    const uint32_t* keys, const uint64_t* payload, int64_t n, int64_t chunk,
    int64_t num_chunks, const float* act_grad, int64_t dim, float* table,
    float* accum, uint32_t sentinel, OptParams opt, float* partials,
    uint32_t* counters) {
  using V = Vec<VEC>;
  const int64_t c =
      (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (c >= num_chunks) return;
  const int lane = __lane_id();
  const int sub = lane / G;
  const int col_lane = lane % G;
  const float lr = opt.lr_ptr != nullptr ? *opt.lr_ptr : opt.lr_value;
  const int64_t cb = c * chunk;
  const int64_t ce = cb + chunk < n ? cb + chunk : n;
  int64_t i = cb;
  while (i < ce) {
    const uint32_t key = keys[i];
    if (key >= sentinel) break;
    const int64_t j = RunEnd(keys, i + 1, ce, key);
    const bool head_cont = i == cb && c > 0 && keys[cb - 1] == key;
    const bool tail_cont = j == ce && ce < n && keys[ce] == key;
    const int64_t row = key;
    if (!head_cont && !tail_cont) {
      for (int64_t col = static_cast<int64_t>(col_lane) * VEC; col < dim;
           col += static_cast<int64_t>(G) * VEC) {
        const typename V::T g = RunSum<G, VEC>(payload, i, j, act_grad, dim, col, sub);
        if (sub == 0) ApplyUpdate<VEC, OPT>(table, accum, row, dim, col, g, lr, opt);
      }
    } else {
      const int64_t rs = head_cont ? LowerBound(keys, 0, cb, key) : i;
      const int64_t re = tail_cont ? UpperBound(keys, ce, n, key) : j;
      const int64_t c0 = rs / chunk;
      const int64_t c1 = (re - 1) / chunk;
      const int64_t slot = c == c0 ? 2 * c0 + 1 : 2 * c;
      for (int64_t col = static_cast<int64_t>(col_lane) * VEC; col < dim;
           col += static_cast<int64_t>(G) * VEC) {
        const typename V::T g = RunSum<G, VEC>(payload, i, j, act_grad, dim, col, sub);
        if (sub == 0) V::Store(partials + slot * dim + col, g);
      }
      ReleaseFence();
      uint32_t old = 0;
      if (lane == 0) old = atomicAdd(&counters[c0], 1u);
      old = __shfl(old, 0);
      if (static_cast<int64_t>(old) == c1 - c0) {
        AcquireFence();
        if (sub == 0) {
          for (int64_t col = static_cast<int64_t>(col_lane) * VEC; col < dim;
               col += static_cast<int64_t>(G) * VEC) {
            typename V::T g = V::Load(partials + (2 * c0 + 1) * dim + col);
            for (int64_t cc = c0 + 1; cc <= c1; ++cc) {
              g = V::Add(g, V::Load(partials + (2 * cc) * dim + col));
            }
            ApplyUpdate<VEC, OPT>(table, accum, row, dim, col, g, lr, opt);
          }
        }
      }
    }
    i = j;
  }
}

__global__ void FillU32(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void FillF32(float* p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

struct Geometry {
  int64_t n;          // expanded positions
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

// Lanes per row and vector width for a row of `dim` floats.
void PickLayout(int64_t dim, bool vec4_ok, int* g, int* vec) {
  *vec = vec4_ok && dim % 4 == 0 ? 4 : 1;
  const int64_t lanes = CeilDiv(dim, *vec);
  int gg = 1;
  while (gg < lanes && gg < kWave) gg <<= 1;
  *g = gg;
}

bool Aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Carves the sort buffers; returns the sort arena usage through `ws`.
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

int ForwardImpl(const scemb_csr_t* csr, const float* table, int64_t table_rows,
                int32_t dim, float* act, int64_t batch, Arena& ws,
                uint32_t* status, hipStream_t stream) {
  Geometry geo;
  int st = CheckCsr(csr, batch, table_rows, dim, &geo);
  if (st != 0) return st;
  const int64_t n = geo.n;
  SortBuffers b = TakeSortBuffers(ws, n);
  int32_t* sp = ws.Take<int32_t>(batch + 1);
  const int key_bits = BitWidth(static_cast<uint64_t>(batch));
  bool in_alt = false;
  const bool measuring = ws.measuring();
  if (!measuring) {
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    if (batch == 0) return 0;
    if (n == 0) {
      hipLaunchKernelGGL(FillF32, dim3(CeilDiv(batch * dim, 256)), dim3(256),
                         0, stream, act, batch * dim, 0.0f);
      SCEMB_LAUNCH_CHECK();
      return 0;
    }
    hipLaunchKernelGGL(ExpandCsr<true>, dim3(CeilDiv(n, 256)), dim3(256), 0,
                       stream, MakeCsr(csr), geo.bps, geo.rows_per_partition,
                       static_cast<uint32_t>(batch), b.keys, b.pay, status);
    SCEMB_LAUNCH_CHECK();
  }
  st = RadixSortPairs<uint32_t, uint64_t>(b.keys, b.pay, b.keys_alt, b.pay_alt,
                                          n, 0, key_bits, ws, stream, &in_alt);
  if (st != 0) return st;
  if (measuring) return 0;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  const uint32_t* keys = in_alt ? b.keys_alt : b.keys;
  const uint64_t* pay = in_alt ? b.pay_alt : b.pay;
  hipLaunchKernelGGL(GroupStarts, dim3(CeilDiv(batch + 1, 256)), dim3(256), 0,
                     stream, keys, n, batch, sp);
  SCEMB_LAUNCH_CHECK();
  int g, vec;
  PickLayout(dim, Aligned16(table) && Aligned16(act), &g, &vec);
  const int64_t threads = batch * g;
  const dim3 grid(static_cast<uint32_t>(CeilDiv(threads, 256)));
#define SCEMB_FWD_CASE(GG, VV)                                                 \
  if (g == GG && vec == VV) {                                                 \
    const int prof = ProfileBegin("fwd_gather", stream);                      \
    hipLaunchKernelGGL((FwdGather<GG, VV>), grid, dim3(256), 0, stream, sp,    \
                       pay, table, static_cast<int64_t>(dim), act, batch);     \
    ProfileEnd(prof, stream);                                                  \
    SCEMB_LAUNCH_CHECK();                                                      \
    return 0;                                                                  \
  }
  SCEMB_FWD_CASE(1, 1) SCEMB_FWD_CASE(2, 1) SCEMB_FWD_CASE(4, 1)
  SCEMB_FWD_CASE(8, 1) SCEMB_FWD_CASE(16, 1) SCEMB_FWD_CASE(32, 1)
  SCEMB_FWD_CASE(64, 1) SCEMB_FWD_CASE(1, 4) SCEMB_FWD_CASE(2, 4)
  SCEMB_FWD_CASE(4, 4) SCEMB_FWD_CASE(8, 4) SCEMB_FWD_CASE(16, 4)
  SCEMB_FWD_CASE(32, 4) SCEMB_FWD_CASE(64, 4)
#undef SCEMB_FWD_CASE
  return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unsupported layout");
}

int64_t BwdChunk(int64_t n) {
  // Enough waves to fill 256 CUs several times over, pieces of >= 32.
  int64_t chunk = 64;
  while (chunk > 32 && CeilDiv(n, chunk) < 256 * 16) chunk >>= 1;
  return chunk;
}

template <int OPT>
int GradImpl(const scemb_csr_t* csr, const float* act_grad, int64_t batch,
             float* table, float* accum, int64_t table_rows, int32_t dim,
             const OptParams& opt, Arena& ws, uint32_t* status,
             hipStream_t stream) {
  Geometry geo;
  int st = CheckCsr(csr, batch, table_rows, dim, &geo);
  if (st != 0) return st;
  const int64_t n = geo.n;
  SortBuffers b = TakeSortBuffers(ws, n);
  const int64_t chunk = BwdChunk(n);
  const int64_t num_chunks = CeilDiv(n, chunk);
  uint32_t* counters = ws.Take<uint32_t>(num_chunks);
  float* partials = ws.Take<float>(2 * num_chunks * static_cast<int64_t>(dim));
  const int key_bits = BitWidth(static_cast<uint64_t>(table_rows));
  bool in_alt = false;
  const bool measuring = ws.measuring();
  if (!measuring) {
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    if (n == 0 || batch == 0) return 0;
    hipLaunchKernelGGL(ExpandCsr<false>, dim3(CeilDiv(n, 256)), dim3(256), 0,
                       stream, MakeCsr(csr), geo.bps, geo.rows_per_partition,
                       static_cast<uint32_t>(table_rows), b.keys, b.pay,
                       status);
    SCEMB_LAUNCH_CHECK();
  }
  st = RadixSortPairs<uint32_t, uint64_t>(b.keys, b.pay, b.keys_alt, b.pay_alt,
                                          n, 0, key_bits, ws, stream, &in_alt);
  if (st != 0) return st;
  if (measuring) return 0;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  const uint32_t* keys = in_alt ? b.keys_alt : b.keys;
  const uint64_t* pay = in_alt ? b.pay_alt : b.pay;
  hipLaunchKernelGGL(FillU32, dim3(CeilDiv(num_chunks, 256)), dim3(256), 0,
                     stream, counters, num_chunks, 0u);
  SCEMB_LAUNCH_CHECK();
  int g, vec;
  PickLayout(dim, Aligned16(table) && Aligned16(act_grad) &&
                      (OPT == 0 || Aligned16(accum)), &g, &vec);
  const dim3 grid(static_cast<uint32_t>(CeilDiv(num_chunks * kWave, 256)));
#define SCEMB_BWD_CASE(GG, VV)                                                \
  if (g == GG && vec == VV) {                                                \
    const int prof = ProfileBegin("bwd_update", stream);                     \
    hipLaunchKernelGGL((BwdFused<GG, VV, OPT>), grid, dim3(256), 0, stream,  \
                       keys, pay, n, chunk, num_chunks, act_grad,             \
                       static_cast<int64_t>(dim), table, accum,               \
                       static_cast<uint32_t>(table_rows), opt, partials,      \
                       counters);                                             \
    ProfileEnd(prof, stream);                                                 \
    SCEMB_LAUNCH_CHECK();                                                     \
    return 0;                                                                 \
  }
  SCEMB_BWD_CASE(1, 1) SCEMB_BWD_CASE(2, 1) SCEMB_BWD_CASE(4, 1)
  SCEMB_BWD_CASE(8, 1) SCEMB_BWD_CASE(16, 1) SCEMB_BWD_CASE(32, 1)
  SCEMB_BWD_CASE(64, 1) SCEMB_BWD_CASE(1, 4) SCEMB_BWD_CASE(2, 4)
  SCEMB_BWD_CASE(4, 4) SCEMB_BWD_CASE(8, 4) SCEMB_BWD_CASE(16, 4)
  SCEMB_BWD_CASE(32, 4) SCEMB_BWD_CASE(64, 4)
#undef SCEMB_BWD_CASE
  return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unsupported layout");
}

}  // namespace
}  // namespace scemb

using namespace scemb;

extern "C" {

size_t scemb_sparse_dense_matmul_workspace_size(const scemb_csr_t* csr,
                                                int64_t device_batch_size,
                                                int64_t table_rows,
                                                int32_t dim) {
  Arena ws(nullptr, 0);
  if (ForwardImpl(csr, nullptr, table_rows, dim, nullptr, device_batch_size,
                  ws, nullptr, nullptr) != 0) {
    return 0;
  }
  return ws.used() + 256;
}

int scemb_sparse_dense_matmul(const scemb_csr_t* csr, const float* table,
                              int64_t table_rows, int32_t dim,
                              float* activations, int64_t device_batch_size,
                              void* workspace, size_t workspace_bytes,
                              uint32_t* device_status, void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (table == nullptr || activations == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null table or activations");
  }
  Arena ws(workspace, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("fwd_call", s);
  const int rc = ForwardImpl(csr, table, table_rows, dim, activations,
                             device_batch_size, ws, device_status, s);
  ProfileEnd(prof, s);
  return rc;
}

size_t scemb_sparse_dense_matmul_grad_workspace_size(const scemb_csr_t* csr,
                                                     int64_t device_batch_size,
                                                     int64_t table_rows,
                                                     int32_t dim) {
  Arena ws(nullptr, 0);
  OptParams o{nullptr, 0.f, 0, 0.f, 0.f};
  if (GradImpl<0>(csr, nullptr, device_batch_size, nullptr, nullptr,
                  table_rows, dim, o, ws, nullptr, nullptr) != 0) {
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
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (table == nullptr || activations_grad == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "null table or gradient");
  }
  if ((clip_mask & 3) == 3 && min_value > max_value) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "min_value must be less than or equal to max_value");
  }
  Arena ws(workspace, workspace_bytes);
  OptParams o{learning_rate, learning_rate_value, clip_mask, min_value,
              max_value};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("bwd_call", s);
  const int rc = GradImpl<0>(csr, activations_grad, device_batch_size, table,
                             nullptr, table_rows, dim, o, ws, device_status, s);
  ProfileEnd(prof, s);
  return rc;
}

int scemb_sparse_dense_matmul_grad_with_adagrad(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, float* accumulator,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (table == nullptr || accumulator == nullptr ||
      activations_grad == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "null table, accumulator or gradient");
  }
  if ((clip_mask & 3) == 3 && min_value > max_value) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "min_value must be less than or equal to max_value");
  }
  Arena ws(workspace, workspace_bytes);
  OptParams o{learning_rate, learning_rate_value, clip_mask, min_value,
              max_value};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("bwd_call", s);
  const int rc = GradImpl<1>(csr, activations_grad, device_batch_size, table,
                             accumulator, table_rows, dim, o, ws,
                             device_status, s);
  ProfileEnd(prof, s);
  return rc;
}

}  // extern "C"
