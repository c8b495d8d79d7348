// Shared device helpers for libscemb (gfx950, wave64). The host-side parts
// are left out when the header is compiled at run time (__HIPCC_RTC__: the
// kernels of a custom update program, rtc.hip).
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <string>
#endif

namespace scemb {

constexpr int kWave = 64;
constexpr int kAlign = 8;  // CSR partition alignment (8 elements).
// Minibatching buckets per SparseCore, and so the most minibatches
// (coo_format.h:52-53).
constexpr int kMaxMinibatches = 64;
constexpr int32_t kPadInt = 0x7fffffff;
constexpr uint32_t kNanBits = 0x7fc00000u;  // std::nanf("")

#ifndef __HIPCC_RTC__
// Status plumbing: every entry point returns a code and leaves a message in a
// thread-local buffer (scemb_last_error).
void SetError(const std::string& msg);
int Fail(int code, const std::string& msg);

// Optional launch timing (scemb_profile_enable): records a pair of HIP events
// around a span of launches on `stream`. Returns -1 when disabled.
int ProfileBegin(const char* name, hipStream_t stream);
void ProfileEnd(int token, hipStream_t stream);

// Runs work beside `stream`: *side (a stream of the current device, created
// once, default priority) first waits for what `stream` has enqueued so far.
// After enqueueing on *side, call JoinSide(stream) so that `stream` waits for
// it. Returns 0 or an error code. One side stream per device: the calls that
// fork from several streams share it and run one after another on it.
int ForkSide(hipStream_t stream, hipStream_t* side);
int JoinSide(hipStream_t stream);

#define SCEMB_HIP(expr)                                                     \
  do {                                                                      \
    hipError_t e_ = (expr);                                                 \
    if (e_ != hipSuccess) {                                                 \
      return ::scemb::Fail(4, std::string(#expr ": ") + hipGetErrorString(e_)); \
    }                                                                       \
  } while (0)

#define SCEMB_LAUNCH_CHECK()                                                 \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      return ::scemb::Fail(4, std::string("kernel launch: ") +              \
                                  hipGetErrorString(e_));                    \
    }                                                                        \
  } while (0)

inline int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t RoundUp(int64_t a, int64_t b) { return CeilDiv(a, b) * b; }
inline int BitWidth(uint64_t v) {
  int b = 0;
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

// Simple bump allocator over a caller-provided workspace. All carve-outs are
// 256-byte aligned. In "measure" mode (base == nullptr) it only sums sizes.
class Arena {
 public:
  Arena(void* base, size_t bytes) : base_(static_cast<char*>(base)), cap_(bytes) {}
  template <typename T>
  T* Take(int64_t count) {
    const size_t bytes = RoundUp(static_cast<int64_t>(sizeof(T)) *
                                     (count > 0 ? count : 1), 256);
    T* p = base_ ? reinterpret_cast<T*>(base_ + used_) : nullptr;
    used_ += bytes;
    return p;
  }
  size_t used() const { return used_; }
  bool measuring() const { return base_ == nullptr; }
  bool overflow() const { return base_ != nullptr && used_ > cap_; }

 private:
  char* base_;
  size_t cap_;
  size_t used_ = 0;
};
#endif  // __HIPCC_RTC__

// ---------------------------------------------------------------------------
// Device-side helpers.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int LaneId() { return __lane_id(); }

__device__ __forceinline__ uint64_t LaneMaskLt() {
  const int lane = __lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

template <typename T>
__device__ __forceinline__ T WaveInclusiveScan(T v) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const T o = __shfl_up(v, d, kWave);
    if (__lane_id() >= d) v += o;
  }
  return v;
}

// Exclusive block scan of one value per thread; returns the exclusive prefix
// and the block total. BLOCK must be a multiple of 64; `smem` holds
// BLOCK / 64 + 1 entries.
template <typename T, int BLOCK>
__device__ __forceinline__ T BlockExclusiveScan(T v, T* smem, T* total) {
  constexpr int kWaves = BLOCK / kWave;
  const int lane = __lane_id();
  const int wave = threadIdx.x / kWave;
  const T inc = WaveInclusiveScan(v);
  if (lane == kWave - 1) smem[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    T run = 0;
    for (int w = 0; w < kWaves; ++w) {
      const T t = smem[w];
      smem[w] = run;
      run += t;
    }
    smem[kWaves] = run;
  }
  __syncthreads();
  const T res = smem[wave] + inc - v;
  *total = smem[kWaves];
  __syncthreads();
  return res;
}

// ---------------------------------------------------------------------------
// Grouped launches: one kernel over several independent problems (the
// stacked tables of one call). Every problem's arguments A travel in the
// kernel argument block; problem p owns work-groups [first[p], first[p + 1]),
// and A::Run(args, block, blocks) runs one of them with its index within the
// problem. A kernel body written against (block, blocks) instead of
// (blockIdx.x, gridDim.x) serves single and grouped launches alike.
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 8;

template <typename A>
struct Group {
  int32_t n;
  uint32_t first[kMaxGroup + 1];
  A a[kMaxGroup];
};

template <typename A>
__global__ __launch_bounds__(A::kBlock) void GroupedKernel(Group<A> g) {
  int p = 0;
  while (p + 1 < g.n && blockIdx.x >= g.first[p + 1]) ++p;
  A::Run(g.a[p], blockIdx.x - g.first[p], g.first[p + 1] - g.first[p]);
}

#ifndef __HIPCC_RTC__
// Enqueues GroupedKernel<A> over problems i with args[i] and blocks[i]
// work-groups, at most kMaxGroup per launch; problems of no blocks are left
// out.
template <typename A>
int LaunchGrouped(const A* args, const int64_t* blocks, int n,
                  hipStream_t stream) {
  static_assert(sizeof(Group<A>) <= 3584,
                "grouped arguments must fit the kernel argument block");
  Group<A> g;
  g.n = 0;
  int64_t total = 0;
  for (int i = 0; i <= n; ++i) {
    const bool last = i == n;
    const int64_t b = last ? 0 : blocks[i];
    if (!last && b <= 0) continue;
    if (g.n > 0 && (last || g.n == kMaxGroup || total + b > 0xffffffffll)) {
      g.first[g.n] = static_cast<uint32_t>(total);
      hipLaunchKernelGGL(GroupedKernel<A>, dim3(static_cast<uint32_t>(total)),
                         dim3(A::kBlock), 0, stream, g);
      SCEMB_LAUNCH_CHECK();
      g.n = 0;
      total = 0;
    }
    if (last) break;
    g.first[g.n] = static_cast<uint32_t>(total);
    g.a[g.n] = args[i];
    ++g.n;
    total += b;
  }
  return 0;
}
#endif  // __HIPCC_RTC__

// Non-coherent-free load of data written by other work-groups of the same
// kernel after an acquire fence.
__device__ __forceinline__ void AcquireFence() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}
__device__ __forceinline__ void ReleaseFence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

}  // namespace scemb
