// Segmented reduction kernels shared by the forward lookup and every fused
// backward + optimizer update (one translation unit per optimizer), for the
// SparseDenseMatmulOp and SparseDenseMatmulGradOpWithOptimizerUpdate custom
// calls of jax_tpu_embedding/sparsecore/lib/core/primitives/.
//
// Both directions are one segmented reduction over a stream of entries
// (key, row, gain) sorted by key:
//   forward   key = activation row, gathered row = table row
//             epilogue: store the activation row (rows without entries are
//             zero-filled)
//   backward  key = table row, gathered row = activation-gradient row
//             epilogue: optimizer update of the table row and its slot rows
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
#pragma once

#include "../../include/scemb.h"
#include "common.h"
#ifndef __HIPCC_RTC__
#include "scan.h"
#endif

namespace scemb {

// Which update the backward epilogue applies (the forward stores instead).
enum {
  kEpiFwd = 0,
  kEpiSgd = 1,
  kEpiAdagrad = 2,
  kEpiAdam = 3,
  kEpiAdagradMomentum = 4,
  kEpiFtrl = 5,
  kEpiLaprop = 6,
  kEpiF2a = 7,
  kEpiCustom = 8,       // a CustomOptimizerSpec update, run as a program
  kEpiCustomArith = 9,  // the same without exp/log/pow/tanh/log1p/expm1
  kEpiRtc = 10,         // a custom update compiled for its program (rtc.hip)
};

// The interpreted forms of custom update. Kept apart because the
// transcendental operations (double precision, inlined) take about 90 VGPRs:
// the kernels of programs without them stay small enough for the 16-byte
// layout, and those of programs with them run the 4-byte layout only.
template <int EPI>
__host__ __device__ constexpr bool IsInterpreted() {
  return EPI == kEpiCustom || EPI == kEpiCustomArith;
}
// Custom updates, interpreted or compiled: slots and hyperparameters as the
// program declares them.
template <int EPI>
__host__ __device__ constexpr bool IsCustom() {
  return IsInterpreted<EPI>() || EPI == kEpiRtc;
}

// The update of a custom program compiled at run time: the source rtc.hip
// generates for the program defines it for kEpiRtc, and only kernels
// compiled from that source call it. Returns the new table value and updates
// the slot values s0, s1 in place; h holds the hyperparameters.
template <int EPI>
__device__ float RtcUpdate(float g, float t, float& s0, float& s1,
                           const float* h);

constexpr int kMaxHyper = SCEMB_MAX_HYPERPARAMETERS;

// A custom update program (scemb_update_program_t) as the kernels read it:
// one 32-bit word per instruction, opcode in bits 0-7, then 5 bits each for
// the registers dst, a, b and c (operands the opcode does not read are 0).
// Each instruction is one scalar load from the kernel arguments and its
// register indices are uniform across the wave; byte-sized fields would be
// fetched by per-lane loads, and a register index held per lane costs a
// loop over its distinct values at every access.
struct DevProgram {
  int32_t num_ops;
  int32_t num_slots;
  int32_t num_hyper;
  int32_t num_regs;  // 1 + the largest register the program names
  int32_t transcendental;  // uses exp, log, pow, tanh, log1p or expm1
  uint32_t out;      // output register k in bits 8k .. 8k + 4
  uint32_t code[SCEMB_PROGRAM_MAX_OPS];
  float imm[SCEMB_PROGRAM_MAX_OPS];
};

// Interpreter registers per vector component. The register file is one
// 32-float vector value held in VGPRs: the 16-byte layout (four components)
// takes programs of up to 8 registers, and the host gives larger programs
// the 4-byte layout.
template <int VEC>
__host__ __device__ constexpr int ProgRegs() {
  return VEC == 4 ? 8 : SCEMB_PROGRAM_MAX_REGISTERS;
}

// Register r's component k is element r * VEC + k. A vector value rather
// than an array: an element picked by a wave-uniform index is an indexed
// register move, while a private array may be placed in scratch memory.
typedef float ProgRegFile __attribute__((ext_vector_type(32)));
static_assert(ProgRegs<4>() * 4 <= 32 && ProgRegs<1>() <= 32,
              "register file size");

// Hyperparameters of the update: value i is *ptr[i] (a device scalar, read
// once per block) when ptr[i] is set, else value[i]. Clipping of the updated
// table values, then the optimizer's flags.
struct OptParams {
  const float* ptr[kMaxHyper];
  float value[kMaxHyper];
  int32_t clip_mask;  // bit 0: min_value, bit 1: max_value
  float min_value;
  float max_value;
  uint32_t flags;     // SCEMB_OPTIMIZER_FLAG_*
  DevProgram prog;    // custom updates only
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

#ifndef __HIPCC_RTC__
// One backward call: the CSR, the activation gradients (dense, or through
// `map` when it is set), the table and up to two slot variables updated in
// place, the hyperparameters, and where temporaries and problems go.
struct GradCall {
  const scemb_csr_t* csr;
  const float* act_grad;
  const RowMap* map;
  bool map_vec4;  // every block of `map` allows 16-byte accesses
  int64_t batch;
  float* table;
  float* slot0;
  float* slot1;
  int64_t table_rows;
  int32_t dim;
  OptParams opt;
  Arena* ws;  // sizing pass when ws->measuring()
  uint32_t* status;
  hipStream_t stream;
};

// Backward + optimizer for the optimizers with two slot variables, each in a
// translation unit of its own (optimizer_*.hip).
int GradWithAdam(const GradCall& c);
int GradWithAdagradMomentum(const GradCall& c);
int GradWithFtrl(const GradCall& c);
int GradWithLaprop(const GradCall& c);
int GradWithF2a(const GradCall& c);
int GradWithCustom(const GradCall& c);
int GradWithCustomTranscendental(const GradCall& c);


// A custom program's update kernels compiled at run time for one layout
// (rtc.hip): SegReduce and SegFinish instantiated for kEpiRtc.
struct RtcKernels {
  hipFunction_t reduce;
  hipFunction_t finish;
};

// The kernels of program p for layout (g, vec, src, unroll, mapped) on the
// current device, compiled at the first request and kept for the process.
// 0: *k is set. kRtcInterpret: interpret the program instead (compilation
// switched off, or unavailable or failed while not required). Otherwise an
// error code (SCEMB_ERR_*), message set: SCEMB_CUSTOM_UPDATE unknown, or
// compilation required (SCEMB_CUSTOM_UPDATE=compile) and failed.
constexpr int kRtcInterpret = -1;
int RtcKernelsFor(const DevProgram& p, int g, int vec, int src, int unroll,
                  bool mapped, RtcKernels* k);
#endif  // __HIPCC_RTC__

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

struct Csr {
  const int32_t* rp;
  const int32_t* eid;
  const int32_t* sid;
  const float* gains;
  int64_t per_segment;  // coo_size / num_segments
  int32_t num_segments;
  int32_t num_partitions;
  int32_t rp_per_segment;
  int32_t num_minibatches;  // 0: one block per segment, relative positions
  int64_t coo_size;
  int64_t positions;        // minibatching layout: positions holding entries
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
constexpr int kUniformPartitions = 16;
__device__ __forceinline__ int PartitionOf(const int32_t* rp, int nparts,
                                           int64_t per_segment, int64_t off) {
  if (nparts <= kUniformPartitions) {
    // The same answer from straight-line code (a fully unrolled walk with a
    // uniform guard): the row pointer loads are uniform (scalar), and with no
    // loop boundary a caller's own loads of several positions stay in
    // flight together.
    int part = -1;
    bool found = false;
    int64_t start = 0;
#pragma unroll
    for (int q = 0; q < kUniformPartitions; ++q) {
      if (q >= nparts) break;
      int64_t end = rp[q];
      if (end > per_segment) end = per_segment;
      if (!found && off < end) {
        part = off >= start ? q : -1;
        found = true;
      }
      start = (end + kAlign - 1) / kAlign * kAlign;
    }
    return part;
  }
  int64_t start = 0;
  for (int q = 0; q < nparts; ++q) {
    int64_t end = rp[q];
    if (end > per_segment) end = per_segment;
    if (off < end) return off >= start ? q : -1;
    start = (end + kAlign - 1) / kAlign * kAlign;
  }
  return -1;
}

// COO positions of a CSR (the whole buffer in the minibatching layout).
__device__ __forceinline__ int64_t CsrPositions(const Csr& csr) {
  return csr.num_minibatches > 0 ? csr.positions
                                 : csr.per_segment * csr.num_segments;
}

// Segment (local SparseCore) and partition of COO position j, partition -1
// for padding. In the minibatching layout the (segment, minibatch,
// partition) ranges follow each other through the buffer, each starting at
// the aligned end of the one before: the first whose end lies past j holds
// it, unless j falls in the alignment gap before that range.
__device__ __forceinline__ int LocateEntry(const Csr& csr, int64_t j,
                                           int* segment) {
  if (csr.num_minibatches == 0) {
    // Positions fit 32 bits (the row pointers are int32): a 32-bit divide.
    const int s = csr.num_segments == 1
                      ? 0
                      : static_cast<int>(static_cast<uint32_t>(j) /
                                         static_cast<uint32_t>(
                                             csr.per_segment));
    *segment = s;
    return PartitionOf(csr.rp + static_cast<int64_t>(s) * csr.rp_per_segment,
                       csr.num_partitions, csr.per_segment,
                       j - static_cast<int64_t>(s) * csr.per_segment);
  }
  const int ns = csr.num_partitions;
  const int total = csr.num_segments * csr.num_minibatches * ns;
  auto end_of = [&](int f) -> int64_t {
    const int64_t e = csr.rp[static_cast<int64_t>(f / ns) * csr.rp_per_segment +
                             f % ns];
    return e < csr.coo_size ? e : csr.coo_size;
  };
  int lo = 0, hi = total;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (end_of(mid) > j) hi = mid; else lo = mid + 1;
  }
  if (lo == total) return -1;
  const int64_t start =
      lo == 0 ? 0 : (end_of(lo - 1) + kAlign - 1) / kAlign * kAlign;
  if (j < start) return -1;
  *segment = lo / ns / csr.num_minibatches;
  return lo % ns;
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
  const int64_t n = CsrPositions(csr);
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n) return;
  int s = 0;
  const int p = LocateEntry(csr, j, &s);
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
  // acc + g * v with one rounding per component (the hot-run reduction).
  __device__ static T Fused(T acc, float g, T v) {
    acc.x = __builtin_fmaf(g, v.x, acc.x);
    acc.y = __builtin_fmaf(g, v.y, acc.y);
    acc.z = __builtin_fmaf(g, v.z, acc.z);
    acc.w = __builtin_fmaf(g, v.w, acc.w);
    return acc;
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
  __device__ static T Fused(T acc, float g, T v) {
    return __builtin_fmaf(g, v, acc);
  }
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
  // kSrcCsr: entries of hot runs, which the hot-run kernels reduce instead
  // (null: none). Per block of kBlock entries, hot_head holds the count of
  // leading entries that belong to a hot run and hot_tail the index from
  // which the trailing ones do, each with that run's index in the upper 16
  // bits; a run whose entries failed their check (run_bad) stays here.
  const uint32_t* hot_head;
  const uint32_t* hot_tail;
  const uint32_t* run_bad;
};

// The entries [0, *lead) and [*trail, kBlock) of block b belong to hot runs.
__device__ __forceinline__ void HotSpan(const StreamArgs& s, int64_t b,
                                        int* lead, int* trail) {
  const uint32_t h = s.hot_head[b];
  const uint32_t t = s.hot_tail[b];
  *lead = (h & 0xffffu) != 0 && s.run_bad[h >> 16] == 0
              ? static_cast<int>(h & 0xffffu) : 0;
  *trail = (t & 0xffffu) < kBlock && s.run_bad[t >> 16] == 0
               ? static_cast<int>(t & 0xffffu) : kBlock;
}

// What the reduction reads and writes.
struct RowArgs {
  const float* src;  // gathered rows
  float* dst;        // activations (forward) or table (backward)
  float* slot0;      // slot variables of the optimizer (backward)
  float* slot1;
  int64_t dim;
  int64_t batch;     // forward: rows of dst
  bool stream_src;   // gathered rows are read about once: nontemporal loads
  RowMap act;        // activation layout (dst forward, src backward)
  OptParams opt;
  float* partials;   // [2 * num_blocks, dim]
  uint32_t* block_flags;
  uint32_t* block_keys;
  uint32_t* status;
  // Every key has one entry: no run crosses a block, SegFinish is not
  // launched, and a block that finds one reports SCEMB_STATUS_SHARED_ROW.
  bool single_runs;
};

// Key of CSR position e (partition * rows_per_partition + embedding id) and
// its sample in *sample, or kSkip for padding and invalid entries (reported
// through `status` when it is set).
__device__ __forceinline__ uint32_t CsrKeySample(const StreamArgs& s,
                                                 int64_t e, int32_t* sample,
                                                 uint32_t* status) {
  *sample = 0;
  int seg = 0;
  const int p = s.csr.num_minibatches > 0
                    ? LocateEntry(s.csr, e, &seg)
                    : PartitionOf(s.csr.rp, s.csr.num_partitions,
                                  s.csr.per_segment, e);
  if (p < 0) return kSkip;
  const int32_t id = s.csr.eid[e];
  const int32_t sm = s.csr.sid[e];
  if (id < 0 || id >= s.rows_per_partition || sm < 0 || sm >= s.bps) {
    if (status != nullptr) atomicOr(status, SCEMB_STATUS_BAD_ENTRY);
    return kSkip;
  }
  *sample = sm;
  return static_cast<uint32_t>(p * s.rows_per_partition + id);
}

// The same with the sample and gain packed in *ent (0 for kSkip).
__device__ __forceinline__ uint32_t CsrKey(const StreamArgs& s, int64_t e,
                                           uint64_t* ent, uint32_t* status) {
  int32_t sm;
  const uint32_t k = CsrKeySample(s, e, &sm, status);
  *ent = k == kSkip ? 0 : Pack(static_cast<uint32_t>(sm), s.csr.gains[e]);
  return k;
}

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
    return CsrKey(s, e, ent, status);
  }
}

// Slot variables and hyperparameters per optimizer, in the order of the
// reference's *SlotVariables and get_hyperparameters()
// (lib/nn/embedding_spec.py:377-916).
// (A custom update has up to 2 slots and kMaxHyper hyperparameters; how
// many it uses is in its program: HasSlot.)
template <int EPI>
__host__ __device__ constexpr int NumSlots() {
  return EPI == kEpiFwd || EPI == kEpiSgd ? 0 : EPI == kEpiAdagrad ? 1 : 2;
}
template <int EPI>
__host__ __device__ constexpr int NumHyper() {
  return EPI == kEpiFwd                                 ? 0
         : EPI == kEpiSgd || EPI == kEpiAdagrad         ? 1
         : EPI == kEpiAdam || EPI == kEpiLaprop         ? 4
         : EPI == kEpiFtrl                              ? 5
         : IsCustom<EPI>()                              ? kMaxHyper
                                                        : 6;
}
// Whether slot k is read and written.
template <int EPI>
__device__ __forceinline__ bool HasSlot(const OptParams& o, int k) {
  return NumSlots<EPI>() > k && (!IsCustom<EPI>() || o.prog.num_slots > k);
}

// The hyperparameters as the update reads them, plus what is constant for
// the whole call.
struct Hyper {
  float h[kMaxHyper];
  float derived;
  int pow_kind;  // PowKindOf() of the optimizer's per-value exponent
};

// pow(x, e) for a per-call exponent e. The exponents the optimizers' defaults
// use (1/2 for FTRL and F2A, -1/2 for AdagradMomentum) and a few others have
// exact forms that replace the library pow, which costs tens of
// instructions per value: sqrt and division are correctly rounded, so these
// differ from pow by at most its own rounding. x + 0.0f maps -0 to +0, as
// pow(-0, +-1/2) = +0 / +inf requires.
enum { kPowGeneric = 0, kPowHalf, kPowMinusHalf, kPowOne, kPowMinusOne,
       kPowTwo, kPowZero };

__device__ __forceinline__ int PowKindOf(float e) {
  return e == 0.5f    ? kPowHalf
         : e == -0.5f ? kPowMinusHalf
         : e == 1.0f  ? kPowOne
         : e == -1.0f ? kPowMinusOne
         : e == 2.0f  ? kPowTwo
         : e == 0.0f  ? kPowZero
                      : kPowGeneric;
}

__device__ __forceinline__ float PowBy(float x, float e, int kind) {
  switch (kind) {
    case kPowHalf:
      return sqrtf(x + 0.0f);
    case kPowMinusHalf:
      return 1.0f / sqrtf(x + 0.0f);
    case kPowOne:
      return x;
    case kPowMinusOne:
      return 1.0f / x;
    case kPowTwo:
      return x * x;
    case kPowZero:
      return 1.0f;
    default:
      return powf(x, e);
  }
}

template <int EPI>
__device__ __forceinline__ Hyper LoadHyper(const OptParams& o) {
  Hyper H{};
#pragma unroll
  for (int i = 0; i < NumHyper<EPI>(); ++i) {
    H.h[i] = o.ptr[i] != nullptr ? *o.ptr[i] : o.value[i];
  }
  if (EPI == kEpiAdagradMomentum) {
    H.derived = -1.0f / H.h[4];  // the power applied to accumulator + eps
    H.pow_kind = PowKindOf(H.derived);
  } else if (EPI == kEpiFtrl) {
    H.derived = -H.h[1];  // the power applied to the accumulators
    H.pow_kind = PowKindOf(H.derived);
  } else if (EPI == kEpiF2a) {
    H.pow_kind = PowKindOf(H.h[1]);  // rho
  } else if (EPI == kEpiLaprop) {
    H.derived = powf(1.0f - powf(H.h[1], 2.0f), 0.5f);  // sqrt(1 - b1^2)
  }
  return H;
}

// Transcendentals of a custom update program, evaluated in double and
// rounded once: correctly rounded but for the rarest double-rounding ties,
// so the result matches a correctly rounded float library (glibc's powf,
// numpy's float32 power) rather than differing in the last bit. Inlined: a
// call would make the caller save its live registers to scratch memory
// around it.
__device__ __forceinline__ float ProgTranscendental(int op, float x, float y) {
  const double a = static_cast<double>(x);
  switch (op) {
    case SCEMB_OP_EXP: return static_cast<float>(exp(a));
    case SCEMB_OP_LOG: return static_cast<float>(log(a));
    case SCEMB_OP_POW: return static_cast<float>(pow(a, static_cast<double>(y)));
    case SCEMB_OP_TANH: return static_cast<float>(tanh(a));
    case SCEMB_OP_LOG1P: return static_cast<float>(log1p(a));
    default: return static_cast<float>(expm1(a));  // SCEMB_OP_EXPM1
  }
}

// The value instruction OP (not CONST) gives for operands x, y, z: the one
// definition of each operation, used by the interpreter and by the programs
// compiled at run time alike. maximum / minimum propagate NaN, as
// StableHLO's do; comparisons give 1 or 0; sign keeps zeros and NaN.
template <int OP>
__device__ __forceinline__ float ProgApply(float x, float y, float z) {
  if constexpr (OP == SCEMB_OP_ADD) return x + y;
  else if constexpr (OP == SCEMB_OP_SUB) return x - y;
  else if constexpr (OP == SCEMB_OP_MUL) return x * y;
  else if constexpr (OP == SCEMB_OP_DIV) return x / y;
  else if constexpr (OP == SCEMB_OP_NEG) return -x;
  else if constexpr (OP == SCEMB_OP_SQRT) return sqrtf(x);
  else if constexpr (OP == SCEMB_OP_RSQRT) return 1.0f / sqrtf(x);
  else if constexpr (OP == SCEMB_OP_ABS) return fabsf(x);
  else if constexpr (OP == SCEMB_OP_EXP || OP == SCEMB_OP_LOG ||
                     OP == SCEMB_OP_POW || OP == SCEMB_OP_TANH ||
                     OP == SCEMB_OP_LOG1P || OP == SCEMB_OP_EXPM1)
    return ProgTranscendental(OP, x, y);
  else if constexpr (OP == SCEMB_OP_MAX)
    return (x != x || y != y) ? x + y : fmaxf(x, y);
  else if constexpr (OP == SCEMB_OP_MIN)
    return (x != x || y != y) ? x + y : fminf(x, y);
  else if constexpr (OP == SCEMB_OP_SIGN)
    return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x);
  else if constexpr (OP == SCEMB_OP_FLOOR) return floorf(x);
  else if constexpr (OP == SCEMB_OP_CEIL) return ceilf(x);
  else if constexpr (OP == SCEMB_OP_SELECT) return x != 0.0f ? y : z;
  else if constexpr (OP == SCEMB_OP_CMP_EQ) return x == y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CMP_NE) return x != y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CMP_LT) return x < y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CMP_LE) return x <= y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CMP_GT) return x > y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CMP_GE) return x >= y ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_CLAMP) return fminf(fmaxf(y, x), z);
  else if constexpr (OP == SCEMB_OP_AND)
    return (x != 0.0f && y != 0.0f) ? 1.0f : 0.0f;
  else if constexpr (OP == SCEMB_OP_OR)
    return (x != 0.0f || y != 0.0f) ? 1.0f : 0.0f;
  else {
    static_assert(OP == SCEMB_OP_NOT, "opcode");
    return x == 0.0f ? 1.0f : 0.0f;
  }
}

// o[k] = ProgApply<OP>(x[k], y[k], z[k]) for every vector component.
template <int OP, int VEC>
__device__ __forceinline__ void ApplyAll(float (&o)[VEC], const float (&x)[VEC],
                                         const float (&y)[VEC],
                                         const float (&z)[VEC]) {
#pragma unroll
  for (int k = 0; k < VEC; ++k) o[k] = ProgApply<OP>(x[k], y[k], z[k]);
}

// Register index field of an instruction word, kept inside the register
// file whatever the word holds (the host has checked it already).
template <int NR>
__device__ __forceinline__ int ProgReg(uint32_t field) {
  const int r = static_cast<int>(field & 31u);
  return r < NR ? r : NR - 1;
}

// Hyperparameters into registers B.. (constant indices). Registers past the
// program's inputs get values too: the program sets every register before
// reading it, so they are never read.
template <int B, int NR, int VEC>
__device__ __forceinline__ void SetHyperRegs(ProgRegFile& R, const float* h) {
#pragma unroll
  for (int i = 0; i < kMaxHyper; ++i) {
    if (B + i < NR) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) R[(B + i) * VEC + k] = h[i];
    }
  }
}

// A custom update (scemb_update_program_t) on VEC table values at once
// (kTranscendentals: the program may use the transcendental operations;
// without, those opcodes give NaN -- the host never sends them there):
// registers 0, 1 hold the summed gradient and the table value, then the slot
// values, then the hyperparameters; each instruction sets one register. The
// program is the same for every thread (kernel arguments), so each
// instruction is decoded and dispatched once per wave and applied to every
// component, and its register indices are uniform.
template <int VEC, bool kTranscendentals>
__device__ __forceinline__ void RunProgram(const DevProgram& p,
                                           const float (&g)[VEC],
                                           float (&t)[VEC], float (&s0)[VEC],
                                           float (&s1)[VEC], const float* h) {
  constexpr int NR = ProgRegs<VEC>();
  ProgRegFile R = {};
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    R[k] = g[k];
    R[VEC + k] = t[k];
  }
  // Each slot count is its own (uniform) branch, so every input lands at a
  // constant index.
  const int ns = p.num_slots;
  if (ns == 0) {
    SetHyperRegs<2, NR, VEC>(R, h);
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) R[2 * VEC + k] = s0[k];
    if (ns == 1) {
      SetHyperRegs<3, NR, VEC>(R, h);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k) R[3 * VEC + k] = s1[k];
      SetHyperRegs<4, NR, VEC>(R, h);
    }
  }
  const int n = p.num_ops;
  for (int i = 0; i < n; ++i) {
    const uint32_t w = __builtin_amdgcn_readfirstlane(p.code[i]);
    const int op = static_cast<int>(w & 0xffu);
    const int d = ProgReg<NR>(w >> 8) * VEC;
    const int a = ProgReg<NR>(w >> 13) * VEC;
    const int b = ProgReg<NR>(w >> 18) * VEC;
    float x[VEC], y[VEC], z[VEC], o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      x[k] = R[a + k];
      y[k] = R[b + k];
      z[k] = 0.0f;
    }
    switch (op) {
      case SCEMB_OP_CONST: {
        const float imm = __builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(
                       __builtin_bit_cast(uint32_t, p.imm[i])));
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = imm;
        break;
      }
      case SCEMB_OP_ADD: ApplyAll<SCEMB_OP_ADD>(o, x, y, z); break;
      case SCEMB_OP_SUB: ApplyAll<SCEMB_OP_SUB>(o, x, y, z); break;
      case SCEMB_OP_MUL: ApplyAll<SCEMB_OP_MUL>(o, x, y, z); break;
      case SCEMB_OP_DIV: ApplyAll<SCEMB_OP_DIV>(o, x, y, z); break;
      case SCEMB_OP_NEG: ApplyAll<SCEMB_OP_NEG>(o, x, y, z); break;
      case SCEMB_OP_SQRT: ApplyAll<SCEMB_OP_SQRT>(o, x, y, z); break;
      case SCEMB_OP_RSQRT: ApplyAll<SCEMB_OP_RSQRT>(o, x, y, z); break;
      case SCEMB_OP_ABS: ApplyAll<SCEMB_OP_ABS>(o, x, y, z); break;
      case SCEMB_OP_EXP:
      case SCEMB_OP_LOG:
      case SCEMB_OP_POW:
      case SCEMB_OP_TANH:
      case SCEMB_OP_LOG1P:
      case SCEMB_OP_EXPM1:
        if constexpr (kTranscendentals) {
          // One inlined copy: each pass takes component 0 and shifts the
          // operands down and the results up (constant indices throughout).
#pragma unroll 1
          for (int k = 0; k < VEC; ++k) {
            const float v = ProgTranscendental(op, x[0], y[0]);
#pragma unroll
            for (int j = 0; j + 1 < VEC; ++j) {
              x[j] = x[j + 1];
              y[j] = y[j + 1];
              o[j] = o[j + 1];
            }
            o[VEC - 1] = v;
          }
        } else {
#pragma unroll
          for (int k = 0; k < VEC; ++k) o[k] = __builtin_nanf("");
        }
        break;
      case SCEMB_OP_MAX: ApplyAll<SCEMB_OP_MAX>(o, x, y, z); break;
      case SCEMB_OP_MIN: ApplyAll<SCEMB_OP_MIN>(o, x, y, z); break;
      case SCEMB_OP_SIGN: ApplyAll<SCEMB_OP_SIGN>(o, x, y, z); break;
      case SCEMB_OP_FLOOR: ApplyAll<SCEMB_OP_FLOOR>(o, x, y, z); break;
      case SCEMB_OP_CEIL: ApplyAll<SCEMB_OP_CEIL>(o, x, y, z); break;
      case SCEMB_OP_SELECT:
      case SCEMB_OP_CLAMP: {
        const int c = ProgReg<NR>(w >> 23) * VEC;
#pragma unroll
        for (int k = 0; k < VEC; ++k) z[k] = R[c + k];
        if (op == SCEMB_OP_SELECT) {
          ApplyAll<SCEMB_OP_SELECT>(o, x, y, z);
        } else {
          ApplyAll<SCEMB_OP_CLAMP>(o, x, y, z);
        }
        break;
      }
      case SCEMB_OP_CMP_EQ: ApplyAll<SCEMB_OP_CMP_EQ>(o, x, y, z); break;
      case SCEMB_OP_CMP_NE: ApplyAll<SCEMB_OP_CMP_NE>(o, x, y, z); break;
      case SCEMB_OP_CMP_LT: ApplyAll<SCEMB_OP_CMP_LT>(o, x, y, z); break;
      case SCEMB_OP_CMP_LE: ApplyAll<SCEMB_OP_CMP_LE>(o, x, y, z); break;
      case SCEMB_OP_CMP_GT: ApplyAll<SCEMB_OP_CMP_GT>(o, x, y, z); break;
      case SCEMB_OP_CMP_GE: ApplyAll<SCEMB_OP_CMP_GE>(o, x, y, z); break;
      case SCEMB_OP_AND: ApplyAll<SCEMB_OP_AND>(o, x, y, z); break;
      case SCEMB_OP_OR: ApplyAll<SCEMB_OP_OR>(o, x, y, z); break;
      default: ApplyAll<SCEMB_OP_NOT>(o, x, y, z); break;
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) R[d + k] = o[k];
  }
  const uint32_t out = __builtin_amdgcn_readfirstlane(p.out);
  const int o0 = ProgReg<NR>(out) * VEC;
  const int o1 = ProgReg<NR>(out >> 8) * VEC;
  const int o2 = ProgReg<NR>(out >> 16) * VEC;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    t[k] = R[o0 + k];
    if (ns >= 1) s0[k] = R[o1 + k];
    if (ns >= 2) s1[k] = R[o2 + k];
  }
}

// The optimizer's clipping of an updated table value
// (primitives/utils.py:24-59).
__device__ __forceinline__ float ClipValue(const OptParams& o, float v) {
  if (o.clip_mask & 1) v = fmaxf(o.min_value, v);
  if (o.clip_mask & 2) v = fminf(o.max_value, v);
  return v;
}

// Update of one table value t with its summed gradient g and slot values
// s0, s1 (updated in place), followed by the optional clipping of the new
// table value (primitives/utils.py:24-59). Each form follows the row-wise
// update function the reference lowers (lib/core/primitives/, the update
// body of each file):
//   SGD              optimizers_computation.py:22-69
//   Adagrad          sparse_dense_matmul_grad_with_adagrad.py:205-233
//   Adam             sparse_dense_matmul_grad_with_adam.py:283-338
//   AdagradMomentum  sparse_dense_matmul_grad_with_adagrad_momentum.py:256-311
//   FTRL             sparse_dense_matmul_grad_with_ftrl.py:260-335
//   LaProp           sparse_dense_matmul_grad_with_laprop.py:282-340
//   F2A              sparse_dense_matmul_grad_with_f2a.py:244-290
// with the operations in the same order and association, so that only the
// rounding of pow (PowBy) can differ.
template <int EPI>
__device__ __forceinline__ float UpdateOne(float t, float& s0, float& s1,
                                           float g, const Hyper& H,
                                           const OptParams& o) {
  static_assert(!IsInterpreted<EPI>(), "these run through RunProgram");
  if constexpr (EPI == kEpiRtc) {
    return ClipValue(o, RtcUpdate<EPI>(g, t, s0, s1, H.h));
  }
  float v;
  if (EPI == kEpiSgd) {
    v = t - g * H.h[0];
  } else if (EPI == kEpiAdagrad) {
    const float acc = s0 + g * g;
    s0 = acc;
    v = t - (H.h[0] * g) / sqrtf(acc);
  } else if (EPI == kEpiAdam) {
    // (alpha_t, beta_1, beta_2, epsilon_hat); slots (momentum, velocity).
    const float m = s0 + (1.0f - H.h[1]) * (g - s0);
    const float vel = s1 + (1.0f - H.h[2]) * (g * g - s1);
    s0 = m;
    s1 = vel;
    v = t - (H.h[0] * m) / (sqrtf(vel) + H.h[3]);
  } else if (EPI == kEpiAdagradMomentum) {
    // (lr, momentum, beta2, epsilon, exponent, use_nesterov); slots
    // (accumulator, momentum).
    const float g2 = g * g;
    const float a = H.h[2] == 1.0f ? s0 + g2
                                   : H.h[2] * s0 + (1.0f - H.h[2]) * g2;
    const float sg = PowBy(a + H.h[3], H.derived, H.pow_kind) * g;
    const float m = H.h[1] * s1 + sg;
    const float upd = H.h[5] != 0.0f ? H.h[1] * m + sg : m;
    s0 = a;
    s1 = m;
    v = t - H.h[0] * upd;
  } else if (EPI == kEpiFtrl) {
    // (lr, lr_power, l1, l2, beta); slots (accumulator, linear).
    const float lr = H.h[0];
    const float a = s0 + g * g;
    const float p_old = PowBy(s0, H.derived, H.pow_kind);
    const float p_new = PowBy(a, H.derived, H.pow_kind);
    const float dp = p_new - p_old;
    const bool by_lr =
        (o.flags & SCEMB_OPTIMIZER_FLAG_MULTIPLY_LINEAR_BY_LR) != 0;
    const float lin = by_lr ? (s1 + lr * g) - dp * t
                            : (s1 + g) - (dp / lr) * t;
    const float l1s = H.h[2] * (by_lr ? lr : 1.0f);
    const float num =
        H.h[2] == 0.0f ? -lin : fminf(fmaxf(lin, -l1s), l1s) - lin;
    const float den = by_lr ? (p_new + 2.0f * (lr * H.h[3])) + H.h[4]
                            : (p_new + H.h[4]) / lr + 2.0f * H.h[3];
    s0 = a;
    s1 = lin;
    v = num / den;
  } else if (EPI == kEpiLaprop) {
    // (lr, b1, decay_rate, eps); slots (mu, nu).
    const float gs = g * g + H.h[3];
    const float nu = s1 * H.h[2] + (1.0f - H.h[2]) * gs;
    const float u = H.h[1] * s0 + H.derived * (g / sqrtf(nu));
    s0 = u;
    s1 = nu;
    v = t - H.h[0] * u;
  } else {
    // F2A: (lr, rho, l1, l2, max_lr_multiplier, global_step); slots
    // (accumulator, local_step). sign() keeps zeros (and NaN) as they are.
    const float ls = s1 + 1.0f;
    const float ratio = fmaxf(H.h[5], 1.0f) / ls;
    const float fa = fminf(PowBy(ratio, H.h[1], H.pow_kind), H.h[4]);
    const float a = s0 + g * g;
    const float sgn = t > 0.0f ? 1.0f : (t < 0.0f ? -1.0f : t);
    const float upd = (g * fa) / sqrtf(a) + (H.h[2] * sgn + H.h[3] * t);
    s0 = a;
    s1 = ls;
    v = t - H.h[0] * upd;
  }
  return ClipValue(o, v);
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
// slot values already loaded (backward) -- or the store (forward).
template <int VEC, int EPI, bool kMapped>
__device__ __forceinline__ void Epilogue(const RowArgs& r,
                                         const RowMapLds& m, uint32_t key,
                                         int64_t col, typename Vec<VEC>::T g,
                                         typename Vec<VEC>::T t,
                                         typename Vec<VEC>::T a,
                                         typename Vec<VEC>::T b,
                                         const Hyper& H) {
  using V = Vec<VEC>;
  const int64_t off = static_cast<int64_t>(key) * r.dim + col;
  if (EPI == kEpiFwd) {
    float* p = ActAddr<kMapped>(m, r.dst, r.dim, key, col);
    if (p != nullptr) StoreRow<VEC, kNtAct>(p, g);
    return;
  }
  if constexpr (IsInterpreted<EPI>()) {
    float tv[VEC], av[VEC], bv[VEC], gv[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      tv[k] = V::Get(t, k);
      av[k] = V::Get(a, k);
      bv[k] = V::Get(b, k);
      gv[k] = V::Get(g, k);
    }
    RunProgram<VEC, EPI == kEpiCustom>(r.opt.prog, gv, tv, av, bv, H.h);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      V::Set(t, k, ClipValue(r.opt, tv[k]));
      V::Set(a, k, av[k]);
      V::Set(b, k, bv[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      float ak = V::Get(a, k);
      float bk = V::Get(b, k);
      V::Set(t, k, UpdateOne<EPI>(V::Get(t, k), ak, bk, V::Get(g, k), H,
                                  r.opt));
      V::Set(a, k, ak);
      V::Set(b, k, bk);
    }
  }
  StoreRow<VEC, kNtTable>(r.dst + off, t);
  if (HasSlot<EPI>(r.opt, 0)) StoreRow<VEC, kNtTable>(r.slot0 + off, a);
  if (HasSlot<EPI>(r.opt, 1)) StoreRow<VEC, kNtTable>(r.slot1 + off, b);
}

template <int VEC, int EPI, bool kMapped>
__device__ __forceinline__ void EpilogueLoad(const RowArgs& r,
                                             const RowMapLds& m, uint32_t key,
                                             int64_t col,
                                             typename Vec<VEC>::T g,
                                             const Hyper& H) {
  using V = Vec<VEC>;
  typename V::T t = V::Zero(), a = V::Zero(), b = V::Zero();
  const int64_t off = static_cast<int64_t>(key) * r.dim + col;
  if (EPI != kEpiFwd) t = V::Load(r.dst + off);
  if (HasSlot<EPI>(r.opt, 0)) a = V::Load(r.slot0 + off);
  if (HasSlot<EPI>(r.opt, 1)) b = V::Load(r.slot1 + off);
  Epilogue<VEC, EPI, kMapped>(r, m, key, col, g, t, a, b, H);
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
      if (st.csr.num_minibatches > 0) {
        end = n;  // entries may lie anywhere below the positions bound
      } else {
        for (int q = 0; q < st.csr.num_partitions; ++q) {
          end = st.csr.rp[q] > end ? st.csr.rp[q] : end;
        }
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
  // Entries of hot runs read as outside any run; a block of nothing else
  // has no work.
  const bool hot = SRC == kSrcCsr && st.hot_head != nullptr;
  int lead = 0, trail = kBlock;
  if (hot) {
    HotSpan(st, blk, &lead, &trail);
    if (lead >= trail) {
      if (tid == 0) r.block_flags[blk] = 0;
      return;
    }
  }
  if (kMapped) StageRowMap(r.act, &s_map);
  {
    uint64_t en = 0;
    uint32_t k = kSkip;
    if (cb + tid < n && tid >= lead && tid < trail) {
      k = FetchEntry<SRC>(st, cb + tid, &en, r.status);
    }
    s_key[tid + 1] = k;
    s_ent[tid] = en;
    if (tid == 0) {
      uint64_t d;
      bool skip = cb == 0;
      if (!skip && hot) {
        int l, t;
        HotSpan(st, blk - 1, &l, &t);
        skip = kBlock - 1 < l || kBlock - 1 >= t;
      }
      s_key[0] = skip ? kSkip : FetchEntry<SRC>(st, cb - 1, &d, nullptr);
    }
    if (tid == kBlock - 1) {
      uint64_t d;
      bool skip = cb + kBlock >= n;
      if (!skip && hot) {
        int l, t;
        HotSpan(st, blk + 1, &l, &t);
        skip = 0 < l || 0 >= t;
      }
      s_key[kBlock + 1] =
          skip ? kSkip : FetchEntry<SRC>(st, cb + kBlock, &d, nullptr);
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

  // A minibatched CSR is contiguous by row but not ascending (a minibatch's
  // buckets follow each other); that cannot be checked locally.
  if (r.status != nullptr && mine &&
      (SRC != kSrcCsr || st.csr.num_minibatches == 0)) {
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
    if (r.single_runs && f != 0 && r.status != nullptr) {
      atomicOr(r.status, SCEMB_STATUS_SHARED_ROW);
    }
  }

  const Hyper H = LoadHyper<EPI>(r.opt);
  const int64_t dim = r.dim;
  for (int64_t col0 = 0; col0 < dim; col0 += static_cast<int64_t>(G) * VEC) {
    const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
    const bool col_ok = col < dim;
    T acc = V::Zero();
    for (int q = 0; q < cnt; q += kUnroll) {
      T v[kUnroll];
      T tv[kUnroll];
      T av[kUnroll];
      T bv[kUnroll];
      T res[kUnroll];  // interpreted updates: finished rows' gradient sums
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
        bv[u] = V::Zero();
        res[u] = V::Zero();
        if (EPI != kEpiFwd && fin[u] && col_ok) {
          const int64_t off = static_cast<int64_t>(kk[u]) * dim + col;
          tv[u] = V::Load(r.dst + off);
          if (HasSlot<EPI>(r.opt, 0)) av[u] = V::Load(r.slot0 + off);
          if (HasSlot<EPI>(r.opt, 1)) bv[u] = V::Load(r.slot1 + off);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int idx = q + u;
        if (idx < cnt && ((valid_m >> idx) & 1)) {
          acc = V::Fma(acc, gn[u], v[u]);
          if ((end_m >> idx) & 1) {
            if (fin[u]) {
              if constexpr (IsInterpreted<EPI>()) {
                res[u] = acc;  // updated below
              } else if (col_ok) {
                Epilogue<VEC, EPI, kMapped>(r, s_map, kk[u], col, acc, tv[u],
                                            av[u], bv[u], H);
              }
            } else {
              const bool first = (start_m & ~1ull & LowBits(idx + 1)) == 0;
              s_part[head_cont && first ? 2 * sub : 2 * sub + 1][cl] = acc;
            }
            acc = V::Zero();
          }
        }
      }
      if constexpr (IsInterpreted<EPI>()) {
        // The finished rows' updates through one inlined copy of the
        // interpreter (its register file then stays in VGPRs, and the loop
        // body in the instruction cache): each pass updates entry 0 and
        // shifts the rest down, so every index stays constant.
#pragma unroll 1
        for (int u = 0; u < kUnroll; ++u) {
          if (fin[0] && col_ok) {
            Epilogue<VEC, EPI, kMapped>(r, s_map, kk[0], col, res[0], tv[0],
                                        av[0], bv[0], H);
          }
#pragma unroll
          for (int j = 0; j + 1 < kUnroll; ++j) {
            fin[j] = fin[j + 1];
            kk[j] = kk[j + 1];
            res[j] = res[j + 1];
            tv[j] = tv[j + 1];
            av[j] = av[j + 1];
            bv[j] = bv[j + 1];
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
        if (col_ok) EpilogueLoad<VEC, EPI, kMapped>(r, s_map, key, col, g, H);
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
  // Most such runs end in the next block: one uniform load settles it.
  if (blk + 1 < num_blocks && (r.block_flags[blk + 1] & kFlagHeadEnd)) {
    c1 = blk + 1;
  }
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
  const Hyper H = LoadHyper<EPI>(r.opt);
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
      // Sub-groups past the m-th took no partial row.
      const int used = m < P ? static_cast<int>(m) : P;
      T g = s_part[0][cl];
      for (int s = 1; s < used; ++s) g = V::Add(g, s_part[s][cl]);
      if (col_ok) EpilogueLoad<VEC, EPI, kMapped>(r, s_map, key, col, g, H);
    }
    __syncthreads();
  }
}

#ifndef __HIPCC_RTC__
// ---------------------------------------------------------------------------
// Hot runs of the backward: the CSR read in place (one segment, no
// minibatching) with several entries per activation row. SegReduce gathers
// one activation-gradient row per entry, and the long runs of the hottest
// table rows spread over every sample: together they sweep the whole
// gradient matrix many times, from beyond the L2. A run longer than about
// a few times the number of sample tiles is reduced per tile instead. A
// block stages one tile of gradient rows in LDS, then the CSR entries its
// group's runs hold in that tile, and adds the rows up from LDS: each
// gradient row is read from memory once per (tile, group) rather than once
// per entry, and the reduction waits on no global load.
//
// The CSR holds a run's entries contiguously and ascending by sample (the
// grouping key's low bits are the sample row, input_preprocessing_util.cc
// and coo_format.h GetGroupingKey), so a run's entries in one tile form a
// contiguous range. Every entry of a candidate run is checked; a run that
// fails stays with SegReduce.
//   HotPoints  the key of every q-th position; a run holding two such
//              positions is hot. Bit masks of each run's first and last
//              sampled position and counts per 256 positions; one thread
//              per SegReduce block clears its hot marks.
//   HotPlan    one block per run: which sampled positions are its first and
//              last, its exact bounds, the SegReduce blocks' hot marks.
//   HotCheck   one thread per marked entry: same key, samples strictly
//              ascending; the first entry of each tile.
//   HotTile    one block per (tile, group): a partial row per (run, tile),
//              its entries spread over kHotAcc chains joined by a tree.
//   HotCombine kHotCombineSplit blocks per run, each over a range of tiles
//              (strided over sub-groups, joined by a tree).
//   HotUpdate  one sub-group per run: the HotCombine rows in order, then the
//              optimizer update. (A ticket for the last HotCombine block of
//              a run needs device-scope fences, which write back and
//              invalidate the per-XCD L2s: a launch is cheaper.)
// Run-to-run identical: every sum has a fixed order and no float atomics.
// ---------------------------------------------------------------------------
constexpr int kHotPointBlock = 256;  // sampled positions per HotPoints block
constexpr int kHotPlanBlock = 256;
constexpr int kHotTileBlock = 512;
// LDS of a HotTile block: one tile of gradient rows, a pass's runs and the
// CSR entries staged per pass; two blocks fit a CU, so that one block's
// loads overlap the other's arithmetic.
constexpr int kHotTileBytes = 64 * 1024;
constexpr int kHotStage = 1408;
constexpr int kHotPassRuns = 256;
constexpr int kHotMaxPointBlocks = 4 * kHotPlanBlock;  // HotPlan's scan
constexpr int kHotMaxRuns = 1 << 16;  // run index in 16 bits of a mark
// Accumulators per sub-group in HotTile. A run has at most one entry per
// sample (checked) and a tile at most kHotChain * kHotAcc samples, so each
// chain adds at most kHotChain entries; HotCombine then adds at most
// tiles / (kHotCombineSplit * kHotCombineBlock / G) partial rows per chain,
// joins its sub-groups by a tree and its kHotCombineSplit blocks' rows in
// order, like the error bound of the other reductions.
constexpr int kHotAcc = 8;
constexpr int kHotChain = 64;
static_assert(kHotChain * kHotAcc <= kHotStage,
              "a pass must hold one run's entries in a full tile");
constexpr int kHotCombineBlock = 1024;
constexpr int kHotCombineSplit = 8;  // HotCombine blocks per run
constexpr int kHotLoadUnroll = 8;  // loads per thread issued together

struct HotArgs {
  int64_t q;           // spacing of the sampled positions (multiple of kBlock)
  int64_t points;      // sampled positions: ceil(n / q)
  int64_t seg_blocks;  // SegReduce blocks: ceil(n / kBlock)
  int32_t max_runs;
  int32_t tile_rows;   // activation rows per tile
  int32_t num_tiles;
  int32_t num_groups;  // runs r, r + num_groups, ... share a HotTile block
  uint64_t* first_mask;   // [4 * point blocks]
  uint64_t* last_mask;
  uint32_t* first_count;  // [point blocks]
  uint32_t* last_count;
  uint32_t* count;        // runs taken: min(found, max_runs)
  uint32_t* run_key;      // [max_runs]
  int32_t* run_start;
  int32_t* run_end;
  uint32_t* run_bad;
  uint32_t* hot_head;     // [seg_blocks], as StreamArgs
  uint32_t* hot_tail;
  int32_t* tile_off;      // [max_runs][num_tiles + 1]: first entry per tile
  float* partials;        // [max_runs][num_tiles][dim]
  float* partials2;       // [max_runs][kHotCombineSplit][dim]
};

__global__ __launch_bounds__(kHotPointBlock) void HotPoints(StreamArgs st,
                                                            HotArgs h) {
  __shared__ uint32_t s_k[kHotPointBlock + 2];
  __shared__ uint32_t s_cnt[2][kHotPointBlock / kWave];
  const int tid = threadIdx.x;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kHotPointBlock + tid;
  // One thread per SegReduce block clears its marks (the grid covers the
  // larger of the two counts); the first blocks also sample the keys.
  if (i < h.seg_blocks) {
    h.hot_head[i] = 0;
    h.hot_tail[i] = kBlock;
  }
  if (static_cast<int64_t>(blockIdx.x) * kHotPointBlock >= h.points) return;
  int32_t d;
  s_k[tid + 1] =
      i < h.points ? CsrKeySample(st, i * h.q, &d, nullptr) : kSkip;
  if (tid == 0) {
    s_k[0] = i > 0 ? CsrKeySample(st, (i - 1) * h.q, &d, nullptr) : kSkip;
  }
  if (tid == kHotPointBlock - 1) {
    s_k[kHotPointBlock + 1] =
        i + 1 < h.points ? CsrKeySample(st, (i + 1) * h.q, &d, nullptr)
                         : kSkip;
  }
  __syncthreads();
  const uint32_t k = s_k[tid + 1];
  const uint32_t kp = s_k[tid];
  const uint32_t kn = s_k[tid + 2];
  const uint64_t fm = __ballot(k != kSkip && k == kn && k != kp);
  const uint64_t lm = __ballot(k != kSkip && k == kp && k != kn);
  const int wave = tid / kWave;
  if (tid % kWave == 0) {
    h.first_mask[i / kWave] = fm;
    h.last_mask[i / kWave] = lm;
    s_cnt[0][wave] = static_cast<uint32_t>(__popcll(fm));
    s_cnt[1][wave] = static_cast<uint32_t>(__popcll(lm));
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t a = 0, b = 0;
    for (int w = 0; w < kHotPointBlock / kWave; ++w) {
      a += s_cnt[0][w];
      b += s_cnt[1][w];
    }
    h.first_count[blockIdx.x] = a;
    h.last_count[blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(kHotPlanBlock) void HotPlan(StreamArgs st,
                                                         HotArgs h,
                                                         int64_t point_blocks,
                                                         uint32_t* status) {
  constexpr int kWaves = kHotPlanBlock / kWave;
  __shared__ uint32_t s_scan[kWaves + 1];
  __shared__ int64_t s_point[2];
  __shared__ int32_t s_red[2];
  const int tid = threadIdx.x;
  const uint32_t r = blockIdx.x;
  if (tid == 0) {
    s_point[0] = -1;
    s_point[1] = -1;
  }
  uint32_t runs = 0;
  for (int which = 0; which < 2; ++which) {
    const uint32_t* cnt = which == 0 ? h.first_count : h.last_count;
    const uint64_t* mask = which == 0 ? h.first_mask : h.last_mask;
    uint32_t c[4];
    uint32_t sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t idx = static_cast<int64_t>(tid) * 4 + u;
      c[u] = idx < point_blocks ? cnt[idx] : 0u;
      sum += c[u];
    }
    uint32_t total;
    uint32_t base =
        BlockExclusiveScan<uint32_t, kHotPlanBlock>(sum, s_scan, &total);
    if (which == 0) runs = total;
    if (r >= base && r < base + sum) {
      int u = 0;
      while (r >= base + c[u]) base += c[u++];
      uint32_t rank = r - base;
      const int64_t pb = static_cast<int64_t>(tid) * 4 + u;
      for (int w = 0; w < kHotPointBlock / kWave; ++w) {
        uint64_t m = mask[pb * (kHotPointBlock / kWave) + w];
        const uint32_t pc = static_cast<uint32_t>(__popcll(m));
        if (rank < pc) {
          for (uint32_t q = 0; q < rank; ++q) m &= m - 1;
          s_point[which] = pb * kHotPointBlock + w * kWave +
                           (__ffsll(static_cast<long long>(m)) - 1);
          break;
        }
        rank -= pc;
      }
    }
    __syncthreads();
  }
  const uint32_t taken =
      runs < static_cast<uint32_t>(h.max_runs) ? runs : h.max_runs;
  if (r == 0 && tid == 0) *h.count = taken;
  if (r >= taken) return;
  if (s_point[0] < 0 || s_point[1] <= s_point[0]) {
    if (tid == 0) h.run_bad[r] = 1;  // no marks: the run stays with SegReduce
    return;
  }
  const int64_t pf = s_point[0] * h.q;
  const int64_t pl = s_point[1] * h.q;
  int32_t d;
  const uint32_t key = CsrKeySample(st, pf, &d, nullptr);
  // The run's first entry lies in (pf - q, pf], its end in [pl, pl + q).
  // Each is the first position of a window where a predicate turns true
  // (wave 0: key == K; wave 1: key != K, or the window's end): rounds of 64
  // probes, each narrowing the window 64-fold (two rounds for q <= 4096).
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  if (wave < 2) {
    int64_t lo = wave == 0 ? (pf - h.q + 1 > 0 ? pf - h.q + 1 : 0) : pl;
    int64_t hi = wave == 0 ? pf + 1 : (pl + h.q < st.n ? pl + h.q : st.n);
    while (lo < hi) {
      const int64_t step = (hi - lo + kWave - 1) / kWave;
      const int64_t p = lo + lane * step;
      bool pred = false;
      if (p < hi) {
        const uint32_t k = CsrKeySample(st, p, &d, nullptr);
        pred = wave == 0 ? k == key : k != key;
      }
      const uint64_t m = __ballot(pred);
      if (m != 0) {
        const int64_t l = __ffsll(static_cast<long long>(m)) - 1;
        hi = lo + l * step;
        lo = l > 0 ? lo + (l - 1) * step + 1 : lo;
      } else {
        lo = lo + (hi - 1 - lo) / step * step + 1;
      }
    }
    if (lane == 0) s_red[wave] = static_cast<int32_t>(hi);
  }
  __syncthreads();
  const int32_t s = s_red[0];
  const int32_t e = s_red[1];
  // A run holds two sampled positions, so it spans more than q entries and
  // at least two SegReduce blocks; anything else is not a sorted run.
  const bool ok = key != kSkip && s <= pf && e > pl &&
                  static_cast<int64_t>(e) - s > h.q;
  if (tid == 0) {
    h.run_key[r] = key;
    h.run_start[r] = s;
    h.run_end[r] = e;
    h.run_bad[r] = ok ? 0u : 1u;
    // SegReduce no longer compares the keys on either side of the run.
    if (ok && status != nullptr) {
      const uint32_t kb =
          s > 0 ? CsrKeySample(st, s - 1, &d, nullptr) : kSkip;
      const uint32_t ka =
          e < st.n ? CsrKeySample(st, e, &d, nullptr) : kSkip;
      if ((kb != kSkip && kb > key) || (ka != kSkip && ka < key)) {
        atomicOr(status, SCEMB_STATUS_UNSORTED);
      }
    }
  }
  if (!ok) return;
  const int64_t b0 = s / kBlock;
  const int64_t b1 = (e - 1) / kBlock;
  const uint32_t tag = r << 16;
  for (int64_t b = b0 + tid; b <= b1; b += kHotPlanBlock) {
    if (b == b0) {
      h.hot_tail[b] = static_cast<uint32_t>(s - b0 * kBlock) | tag;
    } else if (b == b1) {
      h.hot_head[b] = static_cast<uint32_t>(e - b1 * kBlock) | tag;
    } else {
      h.hot_head[b] = static_cast<uint32_t>(kBlock) | tag;
    }
  }
}

// Each thread checks kHotCheckPer consecutive positions of one SegReduce
// block, their ids and samples read as 16-byte vectors.
constexpr int kHotCheckPer = 8;
constexpr int kHotCheckSpan = kBlock * kHotCheckPer;  // positions per block

__global__ __launch_bounds__(kBlock) void HotCheck(StreamArgs st, HotArgs h) {
  constexpr int K = kHotCheckPer;
  const int tid = threadIdx.x;
  const int64_t j0 = static_cast<int64_t>(blockIdx.x) * kHotCheckSpan +
                     static_cast<int64_t>(tid) * K;
  const int64_t b = j0 / kBlock;
  if (b >= h.seg_blocks) return;
  const uint32_t hw = h.hot_head[b];
  const uint32_t tw = h.hot_tail[b];
  const int lead = static_cast<int>(hw & 0xffffu);
  const int trail = static_cast<int>(tw & 0xffffu);
  const int i0 = static_cast<int>(j0 - b * kBlock);
  if (i0 >= lead && i0 + K <= trail) return;  // no position in a hot range
  if (lead > trail && i0 < lead && i0 + K > trail) {
    h.run_bad[hw >> 16] = 1;  // marks of two runs overlap: not sorted runs
    h.run_bad[tw >> 16] = 1;
    return;
  }
  int32_t eid[K], sid[K];
  // Vector loads where both arrays are 16-byte aligned at j0 (the CSR may be
  // slices of one buffer at any 4-byte offset).
  const bool vec = j0 + K <= st.n &&
                   ((reinterpret_cast<uintptr_t>(st.csr.eid + j0) |
                     reinterpret_cast<uintptr_t>(st.csr.sid + j0)) & 15u) == 0;
  if (vec) {
    const int4* pe = reinterpret_cast<const int4*>(st.csr.eid + j0);
    const int4* ps = reinterpret_cast<const int4*>(st.csr.sid + j0);
#pragma unroll
    for (int v = 0; v < K / 4; ++v) {
      const int4 e4 = pe[v];
      const int4 s4 = ps[v];
      eid[4 * v] = e4.x;
      eid[4 * v + 1] = e4.y;
      eid[4 * v + 2] = e4.z;
      eid[4 * v + 3] = e4.w;
      sid[4 * v] = s4.x;
      sid[4 * v + 1] = s4.y;
      sid[4 * v + 2] = s4.z;
      sid[4 * v + 3] = s4.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      eid[k] = j0 + k < st.n ? st.csr.eid[j0 + k] : -1;
      sid[k] = j0 + k < st.n ? st.csr.sid[j0 + k] : -1;
    }
  }
  const int32_t before = j0 > 0 ? st.csr.sid[j0 - 1] : -1;
  const uint32_t rl = hw >> 16;
  const uint32_t rt = tw >> 16;
  const uint32_t key_l = h.run_key[rl];
  const int32_t s_l = h.run_start[rl];
  const int32_t e_l = h.run_end[rl];
  const uint32_t key_t = h.run_key[rt];
  const int32_t s_t = h.run_start[rt];
  const int32_t e_t = h.run_end[rt];
  const int32_t rows = h.tile_rows;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = i0 + k;
    const bool in_lead = i < lead;
    if (!in_lead && i < trail) continue;
    const uint32_t r = in_lead ? rl : rt;
    const uint32_t want = in_lead ? key_l : key_t;
    const int32_t s = in_lead ? s_l : s_t;
    const int32_t e = in_lead ? e_l : e_t;
    const int64_t j = j0 + k;
    // The key as CsrKeySample forms it (one segment, no minibatching).
    const int p = j < st.n ? PartitionOf(st.csr.rp, st.csr.num_partitions,
                                         st.csr.per_segment, j)
                           : -1;
    const int32_t sm = sid[k];
    const bool valid = p >= 0 && eid[k] >= 0 &&
                       eid[k] < st.rows_per_partition && sm >= 0 &&
                       sm < st.bps;
    const uint32_t key =
        valid ? static_cast<uint32_t>(p * st.rows_per_partition + eid[k])
              : kSkip;
    const int32_t sp = k == 0 ? before : sid[k - 1];
    // Strictly ascending: a run has at most one entry per sample, so at
    // most tile_rows per tile.
    const bool ok = key == want && j >= s && j < e &&
                    (j == s || (sp >= 0 && sp < sm));
    if (!ok) {
      h.run_bad[r] = 1;
      continue;
    }
    const int32_t tj = sm / rows;
    int32_t* off = h.tile_off + static_cast<int64_t>(r) * (h.num_tiles + 1);
    for (int32_t t = j == s ? 0 : sp / rows + 1; t <= tj; ++t) {
      off[t] = static_cast<int32_t>(j);
    }
    if (j == e - 1) {
      for (int32_t t = tj + 1; t <= h.num_tiles; ++t) off[t] = e;
    }
  }
}

template <int G, int VEC, bool kMapped>
__global__ __launch_bounds__(kHotTileBlock) void HotTile(StreamArgs st,
                                                         HotArgs h,
                                                         RowArgs r) {
  using V = Vec<VEC>;
  using T = typename V::T;
  constexpr int P = kHotTileBlock / G;
  constexpr int kWaves = kHotTileBlock / kWave;
  constexpr int U = kHotLoadUnroll;
  __shared__ float s_tile[kHotTileBytes / sizeof(float)];
  __shared__ int32_t s_j0[kHotPassRuns];       // a pass's runs: first entry,
  __shared__ int32_t s_len[kHotPassRuns];      // entries in the tile,
  __shared__ int32_t s_pos[kHotPassRuns + 1];  // staged at [pos, pos')
  // Staged entries: the entry's row in s_tile (as a float index) and its
  // gain. Each run's entries are padded to a multiple of kHotAcc with
  // (row 0, gain 0), which adds 0 to its sum.
  __shared__ __align__(16) uint32_t s_row[kHotStage];
  __shared__ __align__(16) float s_gain[kHotStage];
  __shared__ int32_t s_scan[kWaves + 1];
  __shared__ RowMapLds s_map;
  const int tid = threadIdx.x;
  const int32_t t = static_cast<int32_t>(blockIdx.x) / h.num_groups;
  const int32_t g = static_cast<int32_t>(blockIdx.x) % h.num_groups;
  const int32_t ng = h.num_groups;
  const int32_t runs = static_cast<int32_t>(*h.count);
  const int32_t mine = runs > g ? (runs - g + ng - 1) / ng : 0;
  const int64_t dim = r.dim;
  const int64_t row0 = static_cast<int64_t>(t) * h.tile_rows;
  const int32_t rows = static_cast<int32_t>(
      r.batch - row0 < h.tile_rows ? r.batch - row0 : h.tile_rows);
  const int64_t stride = h.num_tiles + 1;
  const int sub = tid / G;
  const int cl = tid % G;
  // Dense rows of 16-byte vectors: the tile is one contiguous range of the
  // gradient matrix, copied into LDS by DMA loads (global_load_lds, 16
  // bytes per lane to the wave's LDS base + 16 * lane) while the block
  // reads its runs' ranges; the copy is waited for before the reduction.
  const bool dma = !kMapped && VEC == 4 &&
                   (reinterpret_cast<uintptr_t>(r.src) & 15u) == 0;
  bool staged = dma;
  if (dma) {
    constexpr int kChunk = kWave * 16;  // bytes one wave copies at once
    const int64_t bytes = static_cast<int64_t>(rows) * dim * sizeof(float);
    const char* src = reinterpret_cast<const char*>(r.src + row0 * dim);
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    for (int64_t c = static_cast<int64_t>(wave) * kChunk; c < bytes;
         c += static_cast<int64_t>(kWaves) * kChunk) {
      if (c + lane * 16 < bytes) {
        __builtin_amdgcn_global_load_lds(
            src + c + lane * 16, reinterpret_cast<char*>(s_tile) + c, 16, 0,
            0);
      }
    }
  }
  // The group's runs (g, g + ng, ...), up to kHotTileBlock at a time, one
  // per thread (its entry range in this tile read once), in passes: each
  // pass takes the longest prefix of the remaining runs whose padded entries
  // fit the staging area (a run has at most one entry per sample, so at
  // most tile_rows, and kHotStage holds that padded: every pass takes one
  // run at least).
  for (int32_t chunk = 0; chunk < mine; chunk += kHotTileBlock) {
    const int32_t avail = mine - chunk < kHotTileBlock ? mine - chunk
                                                       : kHotTileBlock;
    int32_t j0 = 0, len = 0;
    if (tid < avail) {
      // The three loads together: a bad run's offsets are in the buffer
      // (possibly stale) and dropped after.
      const int32_t run = g + (chunk + tid) * ng;
      const int32_t* off = h.tile_off + run * stride;
      const uint32_t bad = h.run_bad[run];
      const int32_t a = off[t];
      const int32_t z = off[t + 1];
      j0 = bad == 0 ? a : 0;
      len = bad == 0 ? z - a : 0;
    }
  for (int32_t lo = 0; lo < avail;) {
    const int32_t mine_k = tid - lo;  // this thread's run within the pass
    const bool live = tid >= lo && tid < avail && mine_k < kHotPassRuns;
    const int32_t padded =
        live ? (len + kHotAcc - 1) / kHotAcc * kHotAcc : 0;
    int32_t total;
    const int32_t excl =
        BlockExclusiveScan<int32_t, kHotTileBlock>(padded, s_scan, &total);
    const int32_t nk = __syncthreads_count(live && excl + padded <= kHotStage);
    if (live && mine_k < nk) {
      s_pos[mine_k] = excl;
      if (mine_k == nk - 1) s_pos[nk] = excl + padded;  // the pass's end
      s_j0[mine_k] = j0;
      s_len[mine_k] = len;
    }
    __syncthreads();
    const int32_t base = chunk + lo;
    const int32_t staged_entries = s_pos[nk];
    if (staged_entries > 0) {
      if (!staged) {
        staged = true;
        if (kMapped) {
          StageRowMap(r.act, &s_map);
          __syncthreads();
        }
        // Every thread's loads of the tile are issued before its stores.
        const int32_t vecs = static_cast<int32_t>(dim / VEC);
        const int32_t cells = rows * vecs;
        for (int32_t x0 = 0; x0 < cells; x0 += U * kHotTileBlock) {
          T v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int32_t x = x0 + u * kHotTileBlock + tid;
            v[u] = V::Zero();
            if (x < cells) {
              const int32_t row = x / vecs;
              const float* p = ActAddr<kMapped>(
                  s_map, const_cast<float*>(r.src), dim, row0 + row,
                  static_cast<int64_t>(x - row * vecs) * VEC);
              if (p != nullptr) v[u] = V::Load(p);
            }
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int32_t x = x0 + u * kHotTileBlock + tid;
            if (x < cells) {
              V::Store(&s_tile[static_cast<int64_t>(x) * VEC], v[u]);
            }
          }
        }
      }
      // The pass's entries: staged position x belongs to the run k with
      // s_pos[k] <= x < s_pos[k + 1] (a search in LDS); all of a thread's
      // loads are issued before its stores.
      for (int32_t x0 = 0; x0 < staged_entries; x0 += U * kHotTileBlock) {
        int32_t sv[U];
        float gv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int32_t x = x0 + u * kHotTileBlock + tid;
          sv[u] = -1;
          gv[u] = 0.0f;
          if (x < staged_entries) {
            int32_t lo = 0, hi = nk;  // last k with s_pos[k] <= x
            while (hi - lo > 1) {
              const int32_t mid = (lo + hi) >> 1;
              if (s_pos[mid] <= x) lo = mid; else hi = mid;
            }
            const int32_t i = x - s_pos[lo];
            if (i < s_len[lo]) {
              const int64_t e = s_j0[lo] + i;
              sv[u] = st.csr.sid[e];
              gv[u] = st.csr.gains[e];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int32_t x = x0 + u * kHotTileBlock + tid;
          if (x < staged_entries) {
            // Checked entries lie in the tile; padding and anything else
            // add 0.
            const int64_t rel = sv[u] - row0;
            const bool in = sv[u] >= 0 && rel >= 0 && rel < rows;
            s_row[x] = in ? static_cast<uint32_t>(rel * dim) : 0u;
            s_gain[x] = in ? gv[u] : 0.0f;
          }
        }
      }
      if (dma) __builtin_amdgcn_s_waitcnt(0);  // this wave's tile copies
      __syncthreads();
      for (int64_t col0 = 0; col0 < dim;
           col0 += static_cast<int64_t>(G) * VEC) {
        const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
        const bool col_ok = col < dim;
        const float* tile_col = s_tile + (col_ok ? col : 0);
        for (int32_t kk = sub; kk < nk; kk += P) {
          const int32_t p0 = s_pos[kk];
          const int32_t p1 = s_pos[kk + 1];
          if (p1 <= p0) continue;
          // Entry i of the run goes to accumulator i % kHotAcc:
          // independent chains, joined by a tree at the end. An
          // accumulator starts at +0 and so is never -0: adding a padding
          // entry's 0 leaves it unchanged.
          T acc[kHotAcc];
#pragma unroll
          for (int u = 0; u < kHotAcc; ++u) acc[u] = V::Zero();
          for (int32_t q = p0; q < p1; q += kHotAcc) {
            uint32_t ro[kHotAcc];
            float gu[kHotAcc];
#pragma unroll
            for (int u = 0; u < kHotAcc; ++u) {
              ro[u] = s_row[q + u];
              gu[u] = s_gain[q + u];
            }
            T v[kHotAcc];
#pragma unroll
            for (int u = 0; u < kHotAcc; ++u) v[u] = V::Load(tile_col + ro[u]);
#pragma unroll
            for (int u = 0; u < kHotAcc; ++u) {
              acc[u] = V::Fused(acc[u], gu[u], v[u]);
            }
          }
#pragma unroll
          for (int w = kHotAcc / 2; w > 0; w /= 2) {
#pragma unroll
            for (int u = 0; u < w; ++u) acc[u] = V::Add(acc[u], acc[u + w]);
          }
          if (col_ok) {
            const int32_t run = g + (base + kk) * ng;
            V::Store(h.partials +
                         (static_cast<int64_t>(run) * h.num_tiles + t) * dim +
                         col,
                     acc[0]);
          }
        }
      }
    }
    __syncthreads();  // the next pass overwrites the staging area
    lo += nk;
  }
  }
  // A block with nothing to add still waits for its copies before it ends.
  if (dma) __builtin_amdgcn_s_waitcnt(0);
}

template <int G, int VEC>
__global__ __launch_bounds__(kHotCombineBlock) void HotCombine(HotArgs h,
                                                               RowArgs r) {
  using V = Vec<VEC>;
  using T = typename V::T;
  constexpr int P = kHotCombineBlock / G;
  __shared__ T s_part[P][G];
  const int32_t run = static_cast<int32_t>(blockIdx.x) / kHotCombineSplit;
  const int part = static_cast<int>(blockIdx.x) % kHotCombineSplit;
  if (run >= static_cast<int32_t>(*h.count) || h.run_bad[run] != 0) return;
  const int tid = threadIdx.x;
  const int sub = tid / G;
  const int cl = tid % G;
  const int32_t* off = h.tile_off + static_cast<int64_t>(run) *
                                        (h.num_tiles + 1);
  const int64_t dim = r.dim;
  const float* part_rows = h.partials + static_cast<int64_t>(run) *
                                            h.num_tiles * dim;
  const int32_t chunk = (h.num_tiles + kHotCombineSplit - 1) / kHotCombineSplit;
  const int32_t t0 = part * chunk;
  const int32_t t1 = t0 + chunk < h.num_tiles ? t0 + chunk : h.num_tiles;
  float* mid = h.partials2 + (static_cast<int64_t>(run) * kHotCombineSplit +
                              part) * dim;
  // This block's tiles: strided over the sub-groups (every partial row is
  // loaded, its offsets settle whether it is added, so a thread's loads
  // overlap), then the sub-groups joined by a tree.
  for (int64_t col0 = 0; col0 < dim; col0 += static_cast<int64_t>(G) * VEC) {
    const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
    const bool col_ok = col < dim;
    T acc = V::Zero();
    if (col_ok) {
#pragma unroll 4
      for (int32_t t = t0 + sub; t < t1; t += P) {
        const bool has = off[t + 1] > off[t];
        const T v = V::Load(part_rows + static_cast<int64_t>(t) * dim + col);
        acc = has ? V::Add(acc, v) : acc;
      }
    }
    s_part[sub][cl] = acc;
    __syncthreads();
#pragma unroll
    for (int w = P / 2; w > 0; w /= 2) {
      if (sub < w) {
        s_part[sub][cl] = V::Add(s_part[sub][cl], s_part[sub + w][cl]);
      }
      __syncthreads();
    }
    if (sub == 0 && col_ok) V::Store(mid + col, s_part[0][cl]);
    __syncthreads();
  }
}

// The kHotCombineSplit rows of each run in order, then the update.
template <int G, int VEC, int EPI>
__global__ __launch_bounds__(kBlock) void HotUpdate(HotArgs h, RowArgs r) {
  using V = Vec<VEC>;
  using T = typename V::T;
  constexpr int P = kBlock / G;
  __shared__ RowMapLds s_map;  // not read: the backward stores no activations
  const int32_t run = static_cast<int32_t>(blockIdx.x) * P +
                      static_cast<int32_t>(threadIdx.x) / G;
  if (run >= static_cast<int32_t>(*h.count) || h.run_bad[run] != 0) return;
  const int cl = threadIdx.x % G;
  const int64_t dim = r.dim;
  const uint32_t key = h.run_key[run];
  const Hyper H = LoadHyper<EPI>(r.opt);
  const float* rows = h.partials2 + static_cast<int64_t>(run) *
                                        kHotCombineSplit * dim;
  for (int64_t col0 = 0; col0 < dim; col0 += static_cast<int64_t>(G) * VEC) {
    const int64_t col = col0 + static_cast<int64_t>(cl) * VEC;
    if (col >= dim) continue;
    T gsum = V::Load(rows + col);
#pragma unroll
    for (int k = 1; k < kHotCombineSplit; ++k) {
      gsum = V::Add(gsum, V::Load(rows + k * dim + col));
    }
    EpilogueLoad<VEC, EPI, false>(r, s_map, key, col, gsum, H);
  }
}
#endif  // __HIPCC_RTC__

#ifndef __HIPCC_RTC__
// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

struct Geometry {
  int64_t n;  // COO positions
  int64_t bps;
  int64_t rows_per_partition;
};

int64_t MinibatchPositions(const scemb_csr_t& csr);

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
  if (csr->num_minibatches < 0 || csr->num_minibatches > kMaxMinibatches) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "num_minibatches must be in [0, 64]");
  }
  if (csr->positions_used < 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "positions_used is negative");
  }
  const int64_t per_seg = csr->coo_size / csr->num_segments;
  geo->n = csr->num_minibatches > 0 ? MinibatchPositions(*csr)
                                    : per_seg * csr->num_segments;
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

int64_t MinibatchPositions(const scemb_csr_t& csr) {
  return csr.positions_used > 0 && csr.positions_used < csr.coo_size
             ? csr.positions_used
             : csr.coo_size;
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
  c.num_minibatches = csr->num_minibatches;
  c.coo_size = csr->coo_size;
  c.positions = MinibatchPositions(*csr);
  return c;
}

// Lanes per row (>= 4) and vector width for a row of `dim` floats.
// Whether opcode op is one of the transcendental operations.
inline bool ProgTranscendentalOp(int op) {
  return op == SCEMB_OP_EXP || op == SCEMB_OP_LOG || op == SCEMB_OP_POW ||
         op == SCEMB_OP_TANH || op == SCEMB_OP_LOG1P || op == SCEMB_OP_EXPM1;
}

// Registers an instruction of opcode op reads: a, then b, then c.
inline int ProgReads(int op) {
  switch (op) {
    case SCEMB_OP_CONST:
      return 0;
    case SCEMB_OP_NEG: case SCEMB_OP_SQRT: case SCEMB_OP_RSQRT:
    case SCEMB_OP_ABS: case SCEMB_OP_EXP: case SCEMB_OP_LOG:
    case SCEMB_OP_SIGN: case SCEMB_OP_TANH: case SCEMB_OP_LOG1P:
    case SCEMB_OP_EXPM1: case SCEMB_OP_FLOOR: case SCEMB_OP_CEIL:
    case SCEMB_OP_NOT:
      return 1;
    case SCEMB_OP_SELECT: case SCEMB_OP_CLAMP:
      return 3;
    default:
      return 2;
  }
}

// The device form of a checked program: operands an opcode does not read
// become register 0, and num_regs covers the inputs and every register an
// instruction reads or sets.
inline DevProgram EncodeProgram(const scemb_update_program_t& p) {
  DevProgram d{};
  d.num_ops = p.num_ops;
  d.num_slots = p.num_slots;
  d.num_hyper = p.num_hyperparameters;
  int regs = 2 + p.num_slots + p.num_hyperparameters;
  for (int i = 0; i < p.num_ops; ++i) {
    const int reads = ProgReads(p.op[i]);
    const uint32_t src[3] = {p.a[i], p.b[i], p.c[i]};
    uint32_t w = static_cast<uint32_t>(p.op[i]) |
                 (static_cast<uint32_t>(p.dst[i]) << 8);
    regs = std::max(regs, p.dst[i] + 1);
    for (int k = 0; k < reads; ++k) {
      w |= src[k] << (13 + 5 * k);
      regs = std::max(regs, static_cast<int>(src[k]) + 1);
    }
    d.code[i] = w;
    d.imm[i] = p.op[i] == SCEMB_OP_CONST ? p.imm[i] : 0.0f;
    d.transcendental |= ProgTranscendentalOp(p.op[i]);
  }
  for (int k = 0; k <= p.num_slots; ++k) {
    d.out |= static_cast<uint32_t>(p.out[k]) << (8 * k);
    regs = std::max(regs, p.out[k] + 1);
  }
  d.num_regs = regs;
  return d;
}

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

// SegReduce + SegFinish compiled for a custom program (RtcKernelsFor), with
// the arguments of the library's own kernels.
int LaunchRtc(const RtcKernels& k, StreamArgs st, RowArgs r, int64_t num_blocks,
              const char* reduce_span, const char* finish_span,
              hipStream_t stream) {
  const uint32_t grid = static_cast<uint32_t>(num_blocks);
  void* reduce_args[] = {&st, &r};
  int prof = ProfileBegin(reduce_span, stream);
  SCEMB_HIP(hipModuleLaunchKernel(k.reduce, grid, 1, 1, kBlock, 1, 1, 0,
                                  stream, reduce_args, nullptr));
  ProfileEnd(prof, stream);
  if (r.single_runs) return 0;
  void* finish_args[] = {&num_blocks, &r};
  prof = ProfileBegin(finish_span, stream);
  SCEMB_HIP(hipModuleLaunchKernel(k.finish, grid, 1, 1, kBlock, 1, 1, 0,
                                  stream, finish_args, nullptr));
  ProfileEnd(prof, stream);
  return 0;
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
  if constexpr (IsInterpreted<EPI>()) {
    // A custom program runs compiled for itself when it can (the same
    // kernels with its update inlined), else through the interpreter.
    RtcKernels k{};
    const int rc = RtcKernelsFor(r.opt.prog, g, vec, SRC,
                                 one_hot ? kWide : kNarrow, kMapped, &k);
    if (rc == 0) {
      return LaunchRtc(k, st, r, sb.num_blocks, reduce_span, finish_span,
                       stream);
    }
    if (rc != kRtcInterpret) return rc;
  }
  const dim3 grid(static_cast<uint32_t>(sb.num_blocks));
#define SCEMB_SEG_CASE(GG, VV)                                                \
  if constexpr (VV == 1 || EPI != kEpiCustom)                                \
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
    if (r.single_runs) return 0;                                              \
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

// Hot-run reduction of a backward call (HotPoints ... HotCombine).
// SCEMB_HOT_RUNS=0 switches it off, =1 on for every call that qualifies;
// otherwise it runs when the activation gradients exceed kHotMinGradBytes
// (the gathers of smaller ones are mostly served by the caches: at c3's
// 33.5 MB per stack SegReduce saved 41 us for 102 us of hot-run kernels)
// and a tile holds kHotMinTileRows samples at least (fewer make a run's
// partial row per tile cost about what its gathers did).
constexpr int64_t kHotMinGradBytes = 64'000'000;
constexpr int64_t kHotMinTileRows = 128;
constexpr int64_t kHotPartialBudget = 128ll << 20;
constexpr int64_t kHotTargetBlocks = 1024;
constexpr int64_t kHotEntriesPerTile = 4;

struct HotBuffers {
  bool on = false;
  int64_t point_blocks = 0;
  HotArgs a{};
};

inline int HotRunsMode() {
  const char* e = std::getenv("SCEMB_HOT_RUNS");
  if (e == nullptr || *e == '\0') return -1;
  return e[0] == '0' ? 0 : 1;
}

// Decides whether the call reduces hot runs and carves their buffers.
// `eligible`: the CSR is read in place with one segment and no minibatching,
// about more than one entry per activation row, and a built-in update.
HotBuffers TakeHotBuffers(Arena& ws, bool eligible, int64_t n, int64_t batch,
                          int64_t dim) {
  HotBuffers hb;
  const int mode = HotRunsMode();
  const int64_t row_bytes = dim * static_cast<int64_t>(sizeof(float));
  if (!eligible || mode == 0 || n <= 0 || batch <= 0 ||
      row_bytes > kHotTileBytes ||
      (mode < 0 && batch * row_bytes < kHotMinGradBytes)) {
    return hb;
  }
  HotArgs& a = hb.a;
  const int64_t tile_rows = std::min<int64_t>(
      {batch, kHotTileBytes / row_bytes, kHotChain * kHotAcc});
  if (mode < 0 && tile_rows < kHotMinTileRows) return hb;
  const int64_t tiles = CeilDiv(batch, tile_rows);
  // A run's partial row per tile (written, then read) costs about what two
  // gathered rows do: runs of a few entries per tile on average pay off.
  const int64_t q = std::min<int64_t>(
      RoundUp(std::max<int64_t>(kHotEntriesPerTile * tiles, kBlock), kBlock),
      1 << 16);
  const int64_t points = CeilDiv(n, q);
  const int64_t point_blocks = CeilDiv(points, kHotPointBlock);
  // Each run holds two sampled positions.
  int64_t max_runs = std::min<int64_t>(
      {kHotMaxRuns - 1, kHotPartialBudget / (tiles * row_bytes),
       points / 2 + 1});
  // SCEMB_HOT_MAX_RUNS: fewer runs per call (the rest stay with SegReduce).
  if (const char* e = std::getenv("SCEMB_HOT_MAX_RUNS")) {
    if (*e != '\0') max_runs = std::min<int64_t>(max_runs, std::atoll(e));
  }
  if (point_blocks > kHotMaxPointBlocks || max_runs < 1 ||
      n >= (int64_t{1} << 31)) {
    return hb;
  }
  hb.on = true;
  hb.point_blocks = point_blocks;
  a.q = q;
  a.points = points;
  a.seg_blocks = CeilDiv(n, kBlock);
  a.max_runs = static_cast<int32_t>(max_runs);
  a.tile_rows = static_cast<int32_t>(tile_rows);
  a.num_tiles = static_cast<int32_t>(tiles);
  a.num_groups = static_cast<int32_t>(std::min<int64_t>(
      CeilDiv(kHotTargetBlocks, tiles), max_runs));
  const int64_t words = point_blocks * (kHotPointBlock / kWave);
  a.first_mask = ws.Take<uint64_t>(words);
  a.last_mask = ws.Take<uint64_t>(words);
  a.first_count = ws.Take<uint32_t>(point_blocks);
  a.last_count = ws.Take<uint32_t>(point_blocks);
  a.count = ws.Take<uint32_t>(1);
  a.run_key = ws.Take<uint32_t>(max_runs);
  a.run_start = ws.Take<int32_t>(max_runs);
  a.run_end = ws.Take<int32_t>(max_runs);
  a.run_bad = ws.Take<uint32_t>(max_runs);
  a.hot_head = ws.Take<uint32_t>(a.seg_blocks);
  a.hot_tail = ws.Take<uint32_t>(a.seg_blocks);
  a.tile_off = ws.Take<int32_t>(max_runs * (tiles + 1));
  a.partials = ws.Take<float>(max_runs * tiles * dim);
  a.partials2 = ws.Take<float>(max_runs * kHotCombineSplit * dim);
  return hb;
}

// Finds the hot runs and marks their entries for SegReduce (before it).
inline int LaunchHotPlan(StreamArgs* st, const HotBuffers& hb, uint32_t* status,
                         hipStream_t stream) {
  const HotArgs& a = hb.a;
  int prof = ProfileBegin("bwd_hot_plan", stream);
  const int64_t point_grid =
      std::max<int64_t>(hb.point_blocks, CeilDiv(a.seg_blocks, kHotPointBlock));
  hipLaunchKernelGGL(HotPoints, dim3(static_cast<uint32_t>(point_grid)),
                     dim3(kHotPointBlock), 0, stream, *st, a);
  SCEMB_LAUNCH_CHECK();
  hipLaunchKernelGGL(HotPlan, dim3(static_cast<uint32_t>(a.max_runs)),
                     dim3(kHotPlanBlock), 0, stream, *st, a, hb.point_blocks,
                     status);
  SCEMB_LAUNCH_CHECK();
  const int64_t check_blocks = CeilDiv(a.seg_blocks * kBlock, kHotCheckSpan);
  hipLaunchKernelGGL(HotCheck, dim3(static_cast<uint32_t>(check_blocks)),
                     dim3(kBlock), 0, stream, *st, a);
  SCEMB_LAUNCH_CHECK();
  ProfileEnd(prof, stream);
  st->hot_head = a.hot_head;
  st->hot_tail = a.hot_tail;
  st->run_bad = a.run_bad;
  return 0;
}

// Reduces the hot runs and updates their rows (after SegReduce, or before:
// the two touch disjoint table rows).
template <int EPI>
int LaunchHotReduce(const StreamArgs& st, const RowArgs& r,
                    const HotBuffers& hb, int g, int vec, bool mapped,
                    hipStream_t stream) {
  const HotArgs& a = hb.a;
  const dim3 tiles(static_cast<uint32_t>(a.num_tiles * a.num_groups));
  const dim3 runs(static_cast<uint32_t>(a.max_runs * kHotCombineSplit));
  const dim3 updates(static_cast<uint32_t>(CeilDiv(a.max_runs, kBlock / g)));
  int prof = ProfileBegin("bwd_hot_reduce", stream);
#define SCEMB_HOT_CASE(GG, VV)                                              \
  if (g == GG && vec == VV) {                                               \
    if (mapped) {                                                           \
      hipLaunchKernelGGL((HotTile<GG, VV, true>), tiles, dim3(kHotTileBlock), \
                         0, stream, st, a, r);                              \
    } else {                                                                \
      hipLaunchKernelGGL((HotTile<GG, VV, false>), tiles,                   \
                         dim3(kHotTileBlock), 0, stream, st, a, r);         \
    }                                                                       \
    SCEMB_LAUNCH_CHECK();                                                   \
    hipLaunchKernelGGL((HotCombine<GG, VV>), runs, dim3(kHotCombineBlock),  \
                       0, stream, a, r);                                    \
    SCEMB_LAUNCH_CHECK();                                                   \
    hipLaunchKernelGGL((HotUpdate<GG, VV, EPI>), updates, dim3(kBlock), 0,  \
                       stream, a, r);                                       \
    SCEMB_LAUNCH_CHECK();                                                   \
    ProfileEnd(prof, stream);                                               \
    return 0;                                                               \
  }
  if constexpr (!IsCustom<EPI>()) {
    SCEMB_HOT_CASE(4, 1) SCEMB_HOT_CASE(8, 1) SCEMB_HOT_CASE(16, 1)
    SCEMB_HOT_CASE(32, 1) SCEMB_HOT_CASE(64, 1) SCEMB_HOT_CASE(4, 4)
    SCEMB_HOT_CASE(8, 4) SCEMB_HOT_CASE(16, 4) SCEMB_HOT_CASE(32, 4)
    SCEMB_HOT_CASE(64, 4)
  }
#undef SCEMB_HOT_CASE
  ProfileEnd(prof, stream);
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

// Backward + optimizer update for one call; with ws->measuring() it only
// sizes the workspace. `c.map` (may be null): the activation gradients as
// per-feature row blocks instead of the dense `c.act_grad`.
template <int EPI>
int GradImpl(const GradCall& c) {
  const scemb_csr_t* csr = c.csr;
  const int64_t batch = c.batch;
  const int64_t table_rows = c.table_rows;
  const int32_t dim = c.dim;
  Arena& ws = *c.ws;
  hipStream_t stream = c.stream;
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
                           c.status);
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
  // Entries per activation row: how often each gradient row is gathered.
  const int64_t entries =
      csr->num_entries > 0 && csr->num_entries < n ? csr->num_entries : n;
  const bool one_hot = entries <= kOneHotMaxEntriesPerRow * batch;
  const HotBuffers hb = TakeHotBuffers(
      ws, direct && csr->num_minibatches == 0 && !one_hot && !IsCustom<EPI>(),
      n, batch, dim);
  if (ws.measuring()) return 0;
  if (ws.overflow()) return Fail(SCEMB_ERR_WORKSPACE, "workspace too small");
  if (n == 0 || batch == 0) return 0;
  RowArgs r{};
  r.src = c.act_grad;
  r.dst = c.table;
  r.slot0 = c.slot0;
  r.slot1 = c.slot1;
  r.dim = dim;
  r.batch = batch;
  r.opt = c.opt;
  r.status = c.status;
  if (c.map != nullptr) r.act = *c.map;
  r.stream_src = one_hot;
  int g, vec;
  PickLayout(dim,
             Aligned16(c.table) &&
                 (c.map != nullptr ? c.map_vec4 : Aligned16(c.act_grad)) &&
                 (c.slot0 == nullptr || Aligned16(c.slot0)) &&
                 (c.slot1 == nullptr || Aligned16(c.slot1)) &&
                 EPI != kEpiCustom &&
                 (EPI != kEpiCustomArith ||
                  c.opt.prog.num_regs <= ProgRegs<4>()),
             &g, &vec);
  const bool mapped = c.map != nullptr;
  if (direct) {
    if (!hb.on) {
      return LaunchSeg<kSrcCsr, EPI>(st, r, sb, g, vec, one_hot, mapped,
                                     "bwd_reduce", "bwd_finish", stream);
    }
    rc = LaunchHotPlan(&st, hb, c.status, stream);
    if (rc != 0) return rc;
    // The hot runs and the cold entries update disjoint table rows: the
    // hot-run reduction (LDS and ALU bound) runs beside SegReduce (memory
    // bound) on a side stream, joined before the call returns.
    hipStream_t side = nullptr;
    rc = ForkSide(stream, &side);
    if (rc != 0) return rc;
    const int rc_seg = LaunchSeg<kSrcCsr, EPI>(
        st, r, sb, g, vec, one_hot, mapped, "bwd_reduce", "bwd_finish", stream);
    rc = LaunchHotReduce<EPI>(st, r, hb, g, vec, mapped, side);
    const int rc_join = JoinSide(stream);
    return rc != 0 ? rc : rc_seg != 0 ? rc_seg : rc_join;
  }
  return LaunchSeg<kSrcSorted, EPI>(st, r, sb, g, vec, one_hot, mapped,
                                    "bwd_reduce", "bwd_finish", stream);
}

#endif  // __HIPCC_RTC__

}  // namespace
}  // namespace scemb
