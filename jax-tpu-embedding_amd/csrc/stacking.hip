// Activation unstacking and gradient stacking as standalone device copies:
// the custom calls SparseActivationsUnstackInterleaved and
// SparseGradientsStackInterleaved of the reference's
// lib/core/primitives/sparse_dense_matmul_activation_unstack.py:83 and
// sparse_dense_matmul_gradient_stack.py:73.
//
// Both move rows between one stacked [rows, dim] matrix and per-feature row
// blocks (scemb_row_block_t, the descriptor the row-mapped lookup kernels
// take). Each launch takes up to kChunk blocks by value; a work-group copies
// consecutive rows of one block, about kUnitsPerGroup 16-byte units (4-byte
// ones where a row start is not 16-byte aligned). The work is HBM-bound:
// 4 * width bytes read and written per row (unstack), 4 * width read and
// 4 * dim written (stack, padding columns zeroed).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "../../include/scemb.h"
#include "common.h"

namespace scemb {
namespace {

constexpr int kChunk = 32;
constexpr int kThreads = 256;
constexpr int kUnitsPerGroup = 4096;  // (row, column unit) pairs

struct BlockChunk {
  int64_t first[kChunk];
  int64_t rows[kChunk];
  int64_t stride[kChunk];
  const float* src[kChunk];  // stack: the block's rows (nullptr: zeros)
  float* dst[kChunk];        // unstack: the block's rows
  int32_t width[kChunk];
};

// blockIdx.y = block of the chunk, blockIdx.x = a group of `rpg`
// consecutive rows of it, whose (row, column unit) pairs the threads take in
// order. kToBlocks: stacked -> blocks (columns [0, width)); otherwise
// blocks -> stacked (columns [0, width) copied, [width, dim) zero). VEC: 4
// when every row start and width is a multiple of 4 floats with 16-byte
// aligned bases.
template <bool kToBlocks, int VEC>
__global__ __launch_bounds__(kThreads) void CopyRowsK(BlockChunk c,
                                                      float* stacked_out,
                                                      const float* stacked_in,
                                                      int32_t dim, int rpg) {
  using V = typename std::conditional<VEC == 4, float4, float>::type;
  const int b = blockIdx.y;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rpg;
  const int64_t nrows = c.rows[b];
  if (r0 >= nrows) return;  // uniform: the whole work-group
  const int64_t rend = r0 + rpg < nrows ? r0 + rpg : nrows;
  const int width = c.width[b];
  const int units = (kToBlocks ? width : dim) / VEC;  // written per row
  const int64_t total = (rend - r0) * units;
  const int64_t first = c.first[b];
  const int64_t stride = c.stride[b];
  for (int64_t i = threadIdx.x; i < total; i += kThreads) {
    const int64_t r = r0 + i / units;
    const int col = static_cast<int>(i % units) * VEC;
    const int64_t at = (first + r) * static_cast<int64_t>(dim) + col;
    if constexpr (kToBlocks) {
      *reinterpret_cast<V*>(c.dst[b] + r * stride + col) =
          *reinterpret_cast<const V*>(stacked_in + at);
    } else {
      V v;
      if constexpr (VEC == 4) {
        v = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        v = 0.f;
      }
      if (c.src[b] != nullptr && col < width) {
        v = *reinterpret_cast<const V*>(c.src[b] + r * stride + col);
      }
      *reinterpret_cast<V*>(stacked_out + at) = v;
    }
  }
}

bool Aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int CheckBlocks(const scemb_row_block_t* blocks, int32_t num_blocks,
                int64_t rows, int32_t dim, bool writes_blocks) {
  if (num_blocks < 0 || (num_blocks > 0 && blocks == nullptr) || rows < 0 ||
      dim <= 0) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "row blocks: bad block count, matrix rows or dim");
  }
  for (int i = 0; i < num_blocks; ++i) {
    const scemb_row_block_t& b = blocks[i];
    if (b.first_row < 0 || b.num_rows < 0 || b.first_row + b.num_rows > rows ||
        b.width < 0 || b.width > dim ||
        (b.num_rows > 0 && b.row_stride < b.width) ||
        (b.num_rows > 0 && b.width > 0 && b.data == nullptr)) {
      return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                  "row block " + std::to_string(i) +
                      ": rows outside the stacked matrix, width above dim, "
                      "stride below width or no data");
    }
  }
  if (!writes_blocks) {
    // Stacked rows are written once: blocks must not overlap.
    std::vector<std::pair<int64_t, int64_t>> r;
    for (int i = 0; i < num_blocks; ++i) {
      if (blocks[i].num_rows > 0) {
        r.emplace_back(blocks[i].first_row,
                       blocks[i].first_row + blocks[i].num_rows);
      }
    }
    std::sort(r.begin(), r.end());
    for (size_t i = 1; i < r.size(); ++i) {
      if (r[i].first < r[i - 1].second) {
        return Fail(SCEMB_ERR_INVALID_ARGUMENT, "row blocks overlap");
      }
    }
  }
  return 0;
}

// One launch per chunk of kChunk blocks.
template <bool kToBlocks>
int Launch(const std::vector<scemb_row_block_t>& blocks, float* stacked_out,
           const float* stacked_in, int32_t dim, hipStream_t stream) {
  bool vec = dim % 4 == 0 &&
             Aligned16(kToBlocks ? static_cast<const void*>(stacked_in)
                                 : static_cast<const void*>(stacked_out));
  for (const auto& b : blocks) {
    if (b.num_rows == 0) continue;
    if (b.width % 4 != 0 || b.row_stride % 4 != 0 ||
        (b.data != nullptr && !Aligned16(b.data))) {
      vec = false;
    }
  }
  for (size_t at = 0; at < blocks.size(); at += kChunk) {
    BlockChunk c{};
    const int n = static_cast<int>(
        std::min<size_t>(kChunk, blocks.size() - at));
    int64_t most = 0;
    for (int i = 0; i < n; ++i) {
      const scemb_row_block_t& b = blocks[at + i];
      c.first[i] = b.first_row;
      c.rows[i] = b.num_rows;
      c.stride[i] = b.row_stride;
      c.width[i] = b.width;
      c.src[i] = b.data;
      c.dst[i] = b.data;
      most = std::max(most, b.num_rows);
    }
    if (most == 0) continue;
    const int units = (vec ? dim / 4 : dim);
    const int rpg = std::max(1, kUnitsPerGroup / std::max(1, units));
    const dim3 grid(static_cast<unsigned>(CeilDiv(most, rpg)), n);
    if (vec) {
      hipLaunchKernelGGL((CopyRowsK<kToBlocks, 4>), grid, dim3(kThreads), 0,
                         stream, c, stacked_out, stacked_in, dim, rpg);
    } else {
      hipLaunchKernelGGL((CopyRowsK<kToBlocks, 1>), grid, dim3(kThreads), 0,
                         stream, c, stacked_out, stacked_in, dim, rpg);
    }
    SCEMB_LAUNCH_CHECK();
  }
  return 0;
}

}  // namespace
}  // namespace scemb

extern "C" {

int scemb_activation_unstack(const float* stacked, int64_t rows, int32_t dim,
                             const scemb_row_block_t* blocks,
                             int32_t num_blocks, void* stream) {
  using namespace scemb;
  const int st = CheckBlocks(blocks, num_blocks, rows, dim, true);
  if (st != 0) return st;
  if (rows > 0 && stacked == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "stacked activations missing");
  }
  std::vector<scemb_row_block_t> list;
  for (int i = 0; i < num_blocks; ++i) {
    if (blocks[i].num_rows > 0 && blocks[i].width > 0) {
      list.push_back(blocks[i]);
    }
  }
  return Launch<true>(list, nullptr, stacked, dim,
                      static_cast<hipStream_t>(stream));
}

int scemb_gradient_stack(const scemb_row_block_t* blocks, int32_t num_blocks,
                         float* stacked, int64_t rows, int32_t dim,
                         void* stream) {
  using namespace scemb;
  const int st = CheckBlocks(blocks, num_blocks, rows, dim, false);
  if (st != 0) return st;
  if (rows > 0 && stacked == nullptr) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT, "stacked gradient missing");
  }
  // Rows in no block become zero rows: the gaps go in as blocks without
  // data, so every stacked row is written exactly once.
  std::vector<scemb_row_block_t> list;
  for (int i = 0; i < num_blocks; ++i) {
    if (blocks[i].num_rows > 0) list.push_back(blocks[i]);
  }
  std::sort(list.begin(), list.end(),
            [](const scemb_row_block_t& a, const scemb_row_block_t& b) {
              return a.first_row < b.first_row;
            });
  std::vector<scemb_row_block_t> all;
  int64_t next = 0;
  for (const auto& b : list) {
    if (b.first_row > next) {
      all.push_back(scemb_row_block_t{next, b.first_row - next, nullptr, 0, 0,
                                      0});
    }
    scemb_row_block_t c = b;
    if (c.width == 0) c.data = nullptr;
    all.push_back(c);
    next = b.first_row + b.num_rows;
  }
  if (next < rows) {
    all.push_back(scemb_row_block_t{next, rows - next, nullptr, 0, 0, 0});
  }
  return Launch<false>(all, stacked, nullptr, dim,
                       static_cast<hipStream_t>(stream));
}

}  // extern "C"
