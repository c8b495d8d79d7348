// C ABI of the lookup (SparseDenseMatmulOp) and of the backward + optimizer
// update (SparseDenseMatmulGradOpWithOptimizerUpdate) custom calls of
// jax_tpu_embedding/sparsecore/lib/core/primitives/: the forward, the sample
// view, SGD and Adagrad here; the optimizers with two slot variables in
// optimizer_*.hip.
#include "segreduce.h"
#include "radix.h"

namespace scemb {
namespace {

__global__ void FillF32(float* p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// One-entry-per-row CSRs: each valid entry claims its activation row's slot
// (count 1, packed entry). A second claim is flagged.
__global__ __launch_bounds__(256) void SlotByRow(Csr csr, int64_t bps,
                                                 int64_t rows_per_partition,
                                                 uint32_t* count,
                                                 uint64_t* slot,
                                                 uint32_t* status) {
  const int64_t n = CsrPositions(csr);
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n) return;
  int s = 0;
  const int p = LocateEntry(csr, j, &s);
  if (p < 0) return;
  const int32_t e = csr.eid[j];
  const int32_t sm = csr.sid[j];
  if (e < 0 || e >= rows_per_partition || sm < 0 || sm >= bps) {
    if (status != nullptr) atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
    return;
  }
  const int64_t arow = s * bps + sm;
  if (atomicAdd(&count[arow], 1u) != 0 && status != nullptr) {
    atomicOr(status, SCEMB_STATUS_SHARED_ROW);
  }
  slot[arow] = Pack(static_cast<uint32_t>(p * rows_per_partition + e),
                    csr.gains[j]);
}

// pos = exclusive scan of the slot counts (pos[batch] = entries): row r's
// entry goes to pos[r]; positions from pos[batch] on get the unused key.
__global__ __launch_bounds__(256) void CompactSlots(const uint32_t* pos,
                                                    const uint64_t* slot,
                                                    int64_t batch, int64_t n,
                                                    uint32_t* keys,
                                                    uint64_t* entries) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < batch && pos[i + 1] > pos[i]) {
    keys[pos[i]] = static_cast<uint32_t>(i);
    entries[pos[i]] = slot[i];
  }
  if (i < n && i >= static_cast<int64_t>(pos[batch])) {
    keys[i] = static_cast<uint32_t>(batch);
    entries[i] = 0;
  }
}

__global__ void FillU32(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// --- Grouping a CSR by activation row --------------------------------------
//
// A stable LSD radix sort by activation row whose first pass reads the CSR
// itself (padding and invalid entries dropped, the packed (table row, gain)
// as payload), so no expanded copy is written first; each row's entries
// keep their CSR order. Keys span BitWidth(batch - 1) bits (no sentinel
// value to make room for); the last pass fills the positions past the
// entries with the unused key.

// The loads do not report entries outside the table: an atomic between them
// would keep the compiler from issuing one position's loads before the
// previous position's atomic, so RadixHistogramK hands the positions it did
// not take to Rejected once all of its loads are out.
struct CsrRowSource {
  Csr csr;
  int64_t bps;
  int64_t rows_per_partition;
  uint32_t* status;
  __device__ bool Entry(int s, int p, int32_t e, int32_t sm,
                        uint32_t* k) const {
    if (p < 0 || e < 0 || e >= rows_per_partition || sm < 0 || sm >= bps) {
      return false;
    }
    *k = static_cast<uint32_t>(s * bps + sm);
    return true;
  }
  // Every position below the geometry's n lies inside the CSR arrays, so
  // the loads need not wait for the partition test.
  __device__ bool LoadKey(int64_t j, uint32_t* k) const {
    int s = 0;
    const int p = LocateEntry(csr, j, &s);
    return Entry(s, p, csr.eid[j], csr.sid[j], k);
  }
  __device__ bool Load(int64_t j, uint32_t* k, uint64_t* v) const {
    int s = 0;
    const int p = LocateEntry(csr, j, &s);
    const int32_t e = csr.eid[j];
    const float g = csr.gains[j];
    if (!Entry(s, p, e, csr.sid[j], k)) return false;
    *v = Pack(static_cast<uint32_t>(p * rows_per_partition + e), g);
    return true;
  }
  // A position LoadKey declined: an entry (not padding) outside the table
  // or the batch sets SCEMB_STATUS_BAD_ENTRY.
  __device__ void Rejected(int64_t j) const {
    if (status == nullptr) return;
    int s = 0;
    if (LocateEntry(csr, j, &s) < 0) return;
    const int32_t e = csr.eid[j];
    const int32_t sm = csr.sid[j];
    if (e < 0 || e >= rows_per_partition || sm < 0 || sm >= bps) {
      atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
    }
  }
};

// The stream arrays; positions past the entries get the unused key.
struct StreamSink {
  uint32_t* keys;
  uint64_t* entries;
  uint32_t sentinel;
  __device__ void Store(uint32_t pos, uint32_t k, uint64_t v) const {
    keys[pos] = k;
    entries[pos] = v;
  }
  __device__ void Fill(int64_t pos) const {
    keys[pos] = sentinel;
    entries[pos] = 0;
  }
};

// Keys of 9 to 8 + radix::kBucketMaxBits bits: one pass on the top 8 bits
// into (b.keys_alt, b.pay_alt), then RadixBucketSortK into (b.keys, b.pay),
// which also fills the positions past the entries. Same result as the LSD
// passes: each bucket's elements arrive in CSR order and keep it.
int GroupByRowInBuckets(const CsrRowSource& src, int64_t n,
                        const uint32_t* n_dev, int n_dev_words, int bits,
                        int64_t batch, bool try_unique,
                        const SortBuffers& b, Arena& ws, hipStream_t stream) {
  using radix::kSortBlock;
  using radix::kSortTile;
  constexpr int hb = radix::kMaxDigitBits;
  const int lb = bits - hb;
  const int buckets = 1 << hb;
  const int64_t tiles = CeilDiv(n, kSortTile);
  uint32_t* hist = ws.Take<uint32_t>(tiles * buckets);
  uint32_t* total = ws.Take<uint32_t>(1);
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  const uint32_t mask = static_cast<uint32_t>(buckets - 1);
  if (!measuring) {
    hipLaunchKernelGGL((radix::RadixHistogramK<uint32_t, CsrRowSource>),
                       dim3(tiles), dim3(kSortBlock), 0, stream, src, n,
                       n_dev, n_dev_words, lb, mask, tiles, hist);
    SCEMB_LAUNCH_CHECK();
  }
  const int st = ExclusiveScan<uint32_t>(hist, hist, tiles * buckets, total,
                                         ws, stream);
  if (st != 0 || measuring) return st;
  const radix::ArraySink<uint32_t, uint64_t> mid{b.keys_alt, b.pay_alt};
  hipLaunchKernelGGL(
      (radix::RadixScatterK<uint32_t, uint64_t, CsrRowSource,
                            radix::ArraySink<uint32_t, uint64_t>>),
      dim3(tiles), dim3(kSortBlock), 0, stream, src, mid, n, n_dev,
      n_dev_words, lb, mask, hb, tiles, hist, total, false);
  SCEMB_LAUNCH_CHECK();
  const StreamSink sink{b.keys, b.pay, static_cast<uint32_t>(batch)};
  hipLaunchKernelGGL(
      (radix::RadixBucketSortK<uint32_t, uint64_t, StreamSink>),
      dim3(buckets), dim3(radix::kBucketBlock), 0, stream, b.keys_alt,
      b.pay_alt, sink, hist, tiles, buckets, total, lb, n, true, try_unique);
  SCEMB_LAUNCH_CHECK();
  return 0;
}

int GroupByRow(const scemb_csr_t* csr, const Geometry& geo, int64_t batch,
               const SortBuffers& b, Arena& ws, uint32_t* status,
               hipStream_t stream) {
  using radix::kSortBlock;
  using radix::kSortTile;
  using Arr = radix::ArraySource<uint32_t, uint64_t>;
  const int64_t n = geo.n;
  // With one segment, no entry lies at or past the largest of the segment's
  // row pointers (the last one, unless they decrease): the passes over the
  // CSR read those words and bound their positions by the largest, so a
  // buffer sized for more ids than the batch holds is not walked to its end.
  // The backward's walk (PartitionOf over every position) takes the same
  // entries, whatever the row pointers' order.
  const bool one_segment = csr->num_segments == 1 && csr->num_minibatches == 0;
  const uint32_t* csr_end =
      one_segment ? reinterpret_cast<const uint32_t*>(csr->row_pointers)
                  : nullptr;
  const int csr_end_words = one_segment ? csr->num_partitions : 0;
  const int bits = batch > 1 ? BitWidth(static_cast<uint64_t>(batch - 1)) : 1;
  if (bits > radix::kMaxDigitBits &&
      bits <= radix::kMaxDigitBits + radix::kBucketMaxBits) {
    const CsrRowSource src{MakeCsr(csr), geo.bps, geo.rows_per_partition,
                           status};
    // No more entries than activation rows: the buckets first try to place
    // entries by key (RadixBucketSortK), which needs no ranking when no key
    // repeats.
    const int64_t entries =
        csr->num_entries > 0 && csr->num_entries < n ? csr->num_entries : n;
    return GroupByRowInBuckets(src, n, csr_end, csr_end_words, bits, batch,
                               entries <= batch, b, ws, stream);
  }
  const radix::DigitPlan plan = radix::PlanDigits(bits);
  const int64_t tiles = CeilDiv(n, kSortTile);
  uint32_t* hist = ws.Take<uint32_t>(tiles * (int64_t{1} << plan.digit));
  uint32_t* totals = ws.Take<uint32_t>(plan.passes);
  const bool measuring = ws.measuring();
  if (!measuring && ws.overflow()) {
    return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  }
  const CsrRowSource csr_src{MakeCsr(csr), geo.bps, geo.rows_per_partition,
                             status};
  const uint32_t* taken = totals;  // entries kept by the first pass
  const uint32_t* in_keys = nullptr;
  const uint64_t* in_pay = nullptr;
  for (int pass = 0; pass < plan.passes; ++pass) {
    const int shift = pass * plan.digit;
    const int pbits = bits - shift < plan.digit ? bits - shift : plan.digit;
    const uint32_t mask = (1u << pbits) - 1u;
    const int64_t cells = tiles * (int64_t{1} << pbits);
    const bool first = pass == 0;
    const bool last = pass == plan.passes - 1;
    // Passes alternate so that the last one writes (b.keys, b.pay).
    const bool to_final = (plan.passes - 1 - pass) % 2 == 0;
    const StreamSink sink{to_final ? b.keys : b.keys_alt,
                          to_final ? b.pay : b.pay_alt,
                          static_cast<uint32_t>(batch)};
    const Arr arr{in_keys, in_pay};
    if (!measuring) {
      if (first) {
        hipLaunchKernelGGL((radix::RadixHistogramK<uint32_t, CsrRowSource>),
                           dim3(tiles), dim3(kSortBlock), 0, stream, csr_src,
                           n, csr_end, csr_end_words, shift, mask, tiles,
                           hist);
      } else {
        hipLaunchKernelGGL((radix::RadixHistogramK<uint32_t, Arr>),
                           dim3(tiles), dim3(kSortBlock), 0, stream, arr, n,
                           taken, 1, shift, mask, tiles, hist);
      }
      SCEMB_LAUNCH_CHECK();
    }
    const int st = ExclusiveScan<uint32_t>(hist, hist, cells, totals + pass,
                                           ws, stream);
    if (st != 0) return st;
    if (!measuring) {
      if (first) {
        hipLaunchKernelGGL(
            (radix::RadixScatterK<uint32_t, uint64_t, CsrRowSource,
                                  StreamSink>),
            dim3(tiles), dim3(kSortBlock), 0, stream, csr_src, sink, n,
            csr_end, csr_end_words, shift, mask, pbits, tiles, hist,
            totals + pass, last);
      } else {
        hipLaunchKernelGGL(
            (radix::RadixScatterK<uint32_t, uint64_t, Arr, StreamSink>),
            dim3(tiles), dim3(kSortBlock), 0, stream, arr, sink, n, taken, 1,
            shift, mask, pbits, tiles, hist, totals + pass, last);
      }
      SCEMB_LAUNCH_CHECK();
    }
    in_keys = sink.keys;
    in_pay = sink.entries;
  }
  return 0;
}

// Sample-major stream of a CSR into (keys, entries). With at most one entry
// per activation row (SCEMB_CSR_ONE_ENTRY_PER_ROW) the entries are placed by
// row through a count / scan / compaction; otherwise GroupByRow sorts them.
// The result lands in (b.keys, b.pay) (*in_alt is false).
int BuildSampleStream(const scemb_csr_t* csr, const Geometry& geo,
                      int64_t batch, const SortBuffers& b, Arena& ws,
                      uint32_t* status, hipStream_t stream, bool* in_alt) {
  const int64_t n = geo.n;
  if ((csr->flags & SCEMB_CSR_ONE_ENTRY_PER_ROW) != 0) {
    *in_alt = false;
    uint32_t* pos = ws.Take<uint32_t>(batch + 1);
    uint64_t* slot = ws.Take<uint64_t>(batch);
    const bool measuring = ws.measuring();
    if (!measuring) {
      if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
      hipLaunchKernelGGL(FillU32, dim3(CeilDiv(batch + 1, 256)), dim3(256), 0,
                         stream, pos, batch + 1, 0u);
      SCEMB_LAUNCH_CHECK();
      if (n > 0) {
        hipLaunchKernelGGL(SlotByRow, dim3(CeilDiv(n, 256)), dim3(256), 0,
                           stream, MakeCsr(csr), geo.bps,
                           geo.rows_per_partition, pos, slot, status);
        SCEMB_LAUNCH_CHECK();
      }
    }
    const int st = ExclusiveScan<uint32_t>(pos, pos, batch + 1, nullptr, ws,
                                           stream);
    if (st != 0 || measuring) return st;
    if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
    const int64_t grid = batch > n ? batch : n;
    if (grid > 0) {
      hipLaunchKernelGGL(CompactSlots, dim3(CeilDiv(grid, 256)), dim3(256), 0,
                         stream, pos, slot, batch, n, b.keys, b.pay);
      SCEMB_LAUNCH_CHECK();
    }
    return 0;
  }
  *in_alt = false;
  if (n == 0) return 0;
  return GroupByRow(csr, geo, batch, b, ws, status, stream);
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
  // Keys that never repeat: a view that says so, or the placement of a
  // one-entry-per-row CSR.
  r.single_runs =
      view != nullptr
          ? (view->flags & SCEMB_VIEW_ONE_ENTRY_PER_KEY) != 0
          : (csr->flags & SCEMB_CSR_ONE_ENTRY_PER_ROW) != 0;
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

// Slot variables each optimizer kind updates.
int SlotsOf(const scemb_optimizer_t& o) {
  switch (o.kind) {
    case SCEMB_OPTIMIZER_SGD:
      return 0;
    case SCEMB_OPTIMIZER_ADAGRAD:
      return 1;
    case SCEMB_OPTIMIZER_CUSTOM:
      return o.program != nullptr ? o.program->num_slots : 0;
    default:
      return 2;
  }
}

// A custom update program that the interpreter can run: counts and register
// indices in range, every register read before it is written holds an
// input, the outputs are set.
int CheckProgram(const scemb_update_program_t* p) {
  if (p == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "custom optimizer without program");
  }
  if (p->num_ops < 0 || p->num_ops > SCEMB_PROGRAM_MAX_OPS ||
      p->num_slots < 0 || p->num_slots > 2 || p->num_hyperparameters < 0 ||
      p->num_hyperparameters > kMaxHyper) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "custom optimizer program: at most " +
                    std::to_string(SCEMB_PROGRAM_MAX_OPS) +
                    " operations, 2 slot variables and " +
                    std::to_string(kMaxHyper) + " hyperparameters");
  }
  const int inputs = 2 + p->num_slots + p->num_hyperparameters;
  if (inputs > SCEMB_PROGRAM_MAX_REGISTERS) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "too many program inputs");
  }
  bool set[SCEMB_PROGRAM_MAX_REGISTERS] = {};
  for (int r = 0; r < inputs; ++r) set[r] = true;
  for (int i = 0; i < p->num_ops; ++i) {
    const int op = p->op[i];
    if (op >= SCEMB_OP_COUNT || p->dst[i] >= SCEMB_PROGRAM_MAX_REGISTERS ||
        p->a[i] >= SCEMB_PROGRAM_MAX_REGISTERS ||
        p->b[i] >= SCEMB_PROGRAM_MAX_REGISTERS ||
        p->c[i] >= SCEMB_PROGRAM_MAX_REGISTERS) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "custom optimizer program: bad opcode or register");
    }
    const int reads = ProgReads(op);
    const uint8_t src[3] = {p->a[i], p->b[i], p->c[i]};
    for (int k = 0; k < reads; ++k) {
      if (!set[src[k]]) {
        return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                    "custom optimizer program reads a register before "
                    "setting it");
      }
    }
    set[p->dst[i]] = true;
  }
  for (int k = 0; k <= p->num_slots; ++k) {
    if (p->out[k] >= SCEMB_PROGRAM_MAX_REGISTERS || !set[p->out[k]]) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "custom optimizer program: bad output register");
    }
  }
  return 0;
}

int GradEntry(const scemb_csr_t* csr, const float* activations_grad,
              const scemb_row_block_t* blocks, int32_t num_blocks,
              bool mapped, int64_t batch, float* table, int64_t table_rows,
              int32_t dim, const scemb_optimizer_t* opt, void* workspace,
              size_t workspace_bytes, uint32_t* device_status, void* stream) {
  if (workspace == nullptr) return Fail(SCEMB_ERR_WORKSPACE, "no workspace");
  if (opt == nullptr || opt->kind < SCEMB_OPTIMIZER_SGD ||
      opt->kind > SCEMB_OPTIMIZER_CUSTOM) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unknown optimizer");
  }
  if (opt->kind == SCEMB_OPTIMIZER_CUSTOM) {
    const int rc = CheckProgram(opt->program);
    if (rc != 0) return rc;
  }
  if ((opt->flags & ~SCEMB_OPTIMIZER_FLAG_MULTIPLY_LINEAR_BY_LR) != 0 ||
      (opt->flags != 0 && opt->kind != SCEMB_OPTIMIZER_FTRL)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "unknown optimizer flags");
  }
  const int nslots = SlotsOf(*opt);
  if (table == nullptr || (nslots >= 1 && opt->slots[0] == nullptr) ||
      (nslots >= 2 && opt->slots[1] == nullptr) ||
      (!mapped && activations_grad == nullptr)) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "null table, slot variable or gradient");
  }
  if ((opt->clip_mask & 3) == 3 && opt->min_value > opt->max_value) {
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
  GradCall c{};
  c.csr = csr;
  c.act_grad = activations_grad;
  c.map = mapped ? &map : nullptr;
  c.map_vec4 = vec4;
  c.batch = batch;
  c.table = table;
  c.slot0 = nslots >= 1 ? opt->slots[0] : nullptr;
  c.slot1 = nslots >= 2 ? opt->slots[1] : nullptr;
  c.table_rows = table_rows;
  c.dim = dim;
  for (int i = 0; i < kMaxHyper; ++i) {
    c.opt.ptr[i] = opt->hyperparameter_ptrs[i];
    c.opt.value[i] = opt->hyperparameters[i];
  }
  c.opt.clip_mask = opt->clip_mask;
  c.opt.min_value = opt->min_value;
  c.opt.max_value = opt->max_value;
  c.opt.flags = opt->flags;
  if (opt->kind == SCEMB_OPTIMIZER_CUSTOM) {
    c.opt.prog = EncodeProgram(*opt->program);
  }
  c.ws = &ws;
  c.status = device_status;
  c.stream = static_cast<hipStream_t>(stream);
  const int prof = ProfileBegin("bwd_call", c.stream);
  int rc;
  switch (opt->kind) {
    case SCEMB_OPTIMIZER_SGD:
      rc = GradImpl<kEpiSgd>(c);
      break;
    case SCEMB_OPTIMIZER_ADAGRAD:
      rc = GradImpl<kEpiAdagrad>(c);
      break;
    case SCEMB_OPTIMIZER_ADAM:
      rc = GradWithAdam(c);
      break;
    case SCEMB_OPTIMIZER_ADAGRAD_MOMENTUM:
      rc = GradWithAdagradMomentum(c);
      break;
    case SCEMB_OPTIMIZER_FTRL:
      rc = GradWithFtrl(c);
      break;
    case SCEMB_OPTIMIZER_LAPROP:
      rc = GradWithLaprop(c);
      break;
    case SCEMB_OPTIMIZER_CUSTOM:
      rc = GradWithCustom(c);
      break;
    default:
      rc = GradWithF2a(c);
      break;
  }
  ProfileEnd(prof, c.stream);
  return rc;
}

// The SGD / Adagrad entry points: one learning rate, at most one slot.
scemb_optimizer_t LrOptimizer(int32_t kind, float* accumulator,
                              const float* learning_rate,
                              float learning_rate_value, int32_t clip_mask,
                              float min_value, float max_value) {
  scemb_optimizer_t o{};
  o.kind = kind;
  o.slots[0] = accumulator;
  o.hyperparameter_ptrs[0] = learning_rate;
  o.hyperparameters[0] = learning_rate_value;
  o.clip_mask = clip_mask;
  o.min_value = min_value;
  o.max_value = max_value;
  return o;
}

}  // namespace
}  // namespace scemb

// ---------------------------------------------------------------------------
// The allocation-free forward (scemb_sparse_dense_matmul_no_alloc): the same
// call as scemb_sparse_dense_matmul, with its workspace in a file-scope
// device array instead of caller memory. Each GPU holds its own copy of the
// array, at its own address, for the life of the process; every call on a
// GPU uses that GPU's copy, so calls that overlap on one GPU race. Nothing
// in it must start at zero: every kernel writes what it later reads.
// ---------------------------------------------------------------------------

#include <mutex>
#include <vector>

namespace scemb {
namespace {

constexpr size_t kNoAllocScratchBytes = SCEMB_NO_ALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device, from hipGetSymbolAddress

// The device address of the current device's scratch array, looked up once
// per device with that device current. In host code `scratch` names a
// host-side stand-in, never the device memory.
int ScratchAddress(void** out) {
  int dev = 0;
  SCEMB_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (dev >= static_cast<int>(g_scratch_ptr.size())) {
    g_scratch_ptr.resize(dev + 1, nullptr);
  }
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    SCEMB_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) {
      return Fail(SCEMB_ERR_DEVICE, "no device address for the scratch array");
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace scemb

using namespace scemb;

extern "C" {

int scemb_sparse_dense_matmul_no_alloc(const scemb_csr_t* csr,
                                       const scemb_sample_view_t* view,
                                       const float* table, int64_t table_rows,
                                       int32_t dim, float* activations,
                                       int64_t device_batch_size,
                                       uint32_t* device_status,
                                       void* stream) {
  // The sizing pass of the workspace entry point: host arithmetic only.
  Arena sizing(nullptr, 0);
  int rc = ForwardImpl(csr, view, nullptr, table_rows, dim, nullptr, nullptr,
                       false, device_batch_size, sizing, nullptr, nullptr);
  if (rc != 0) return rc;
  const size_t need = sizing.used();
  if (need > kNoAllocScratchBytes) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "this lookup needs " + std::to_string(need) +
                    " bytes of scratch; the allocation-free entry point has " +
                    std::to_string(kNoAllocScratchBytes) +
                    " (use scemb_sparse_dense_matmul with a workspace)");
  }
  void* ws = nullptr;
  rc = ScratchAddress(&ws);
  if (rc != 0) return rc;
  return ForwardEntry(csr, view, table, table_rows, dim, activations, nullptr,
                      0, false, device_batch_size, ws, kNoAllocScratchBytes,
                      device_status, stream);
}

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
  GradCall c{};
  c.csr = csr;
  c.batch = device_batch_size;
  c.table_rows = table_rows;
  c.dim = dim;
  c.ws = &ws;
  if (GradImpl<kEpiSgd>(c) != 0) return 0;
  return ws.used() + 256;
}

int scemb_sparse_dense_matmul_grad_with_sgd(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  const scemb_optimizer_t o =
      LrOptimizer(SCEMB_OPTIMIZER_SGD, nullptr, learning_rate,
                  learning_rate_value, clip_mask, min_value, max_value);
  return GradEntry(csr, activations_grad, nullptr, 0, false,
                   device_batch_size, table, table_rows, dim, &o, workspace,
                   workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_sgd_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  const scemb_optimizer_t o =
      LrOptimizer(SCEMB_OPTIMIZER_SGD, nullptr, learning_rate,
                  learning_rate_value, clip_mask, min_value, max_value);
  return GradEntry(csr, nullptr, activation_grads, num_blocks, true,
                   device_batch_size, table, table_rows, dim, &o, workspace,
                   workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_adagrad(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, float* accumulator,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  const scemb_optimizer_t o =
      LrOptimizer(SCEMB_OPTIMIZER_ADAGRAD, accumulator, learning_rate,
                  learning_rate_value, clip_mask, min_value, max_value);
  return GradEntry(csr, activations_grad, nullptr, 0, false,
                   device_batch_size, table, table_rows, dim, &o, workspace,
                   workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    float* accumulator, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream) {
  const scemb_optimizer_t o =
      LrOptimizer(SCEMB_OPTIMIZER_ADAGRAD, accumulator, learning_rate,
                  learning_rate_value, clip_mask, min_value, max_value);
  return GradEntry(csr, nullptr, activation_grads, num_blocks, true,
                   device_batch_size, table, table_rows, dim, &o, workspace,
                   workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_optimizer(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, int64_t table_rows, int32_t dim,
    const scemb_optimizer_t* optimizer, void* workspace,
    size_t workspace_bytes, uint32_t* device_status, void* stream) {
  return GradEntry(csr, activations_grad, nullptr, 0, false,
                   device_batch_size, table, table_rows, dim, optimizer,
                   workspace, workspace_bytes, device_status, stream);
}

int scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    int64_t table_rows, int32_t dim, const scemb_optimizer_t* optimizer,
    void* workspace, size_t workspace_bytes, uint32_t* device_status,
    void* stream) {
  return GradEntry(csr, nullptr, activation_grads, num_blocks, true,
                   device_batch_size, table, table_rows, dim, optimizer,
                   workspace, workspace_bytes, device_status, stream);
}

}  // extern "C"
