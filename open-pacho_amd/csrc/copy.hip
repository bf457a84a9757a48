// Fill, strided gather and batched pad/crop copies (bit copies of raw words).
#include "common.h"

namespace {

// 16-byte stores of a replicated pattern, then the sub-16-byte tail.
template <typename T>
__global__ void fill_kernel(T* __restrict__ dst, int64_t count, T value, uint4 pattern) {
  const int64_t total_bytes = count * int64_t(sizeof(T));
  const int64_t n16 = total_bytes / 16;
  uint4* d16 = reinterpret_cast<uint4*>(dst);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) d16[i] = pattern;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    for (int64_t e = n16 * 16 / int64_t(sizeof(T)); e < count; ++e) dst[e] = value;
  }
}

struct Strided {
  int64_t shape[8];
  int64_t strides[8];
};

template <typename T>
__global__ void gather_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t count, int64_t offset,
                              int rank, Strided layout) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    int64_t rest = i, at = offset;
    for (int d = rank - 1; d >= 0; --d) {
      const int64_t extent = layout.shape[d];
      const int64_t q = rest / extent;
      at += (rest - q * extent) * layout.strides[d];
      rest = q;
    }
    dst[i] = src[at];
  }
}

// One workgroup per destination row (grid-stride over rows); lanes walk
// columns. Each lane issues kPadUnroll loads before its stores, so a row of a
// few thousand elements is one or two rounds of independent loads rather than
// a chain of load-store pairs. Rows of padded operands are rarely 16-byte
// aligned on both sides, so accesses stay element-wide (coalesced per wave).
constexpr int kPadUnroll = 8;

template <typename T>
__global__ void pad_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t rows_total, int64_t src_rows,
                           int64_t src_cols, int64_t dst_rows, int64_t dst_cols) {
  for (int64_t row = blockIdx.x; row < rows_total; row += gridDim.x) {
    const int64_t b = row / dst_rows;
    const int64_t r = row - b * dst_rows;
    T* out = dst + row * dst_cols;
    const bool from_src = r < src_rows;
    const T* in = src + (from_src ? (b * src_rows + r) * src_cols : 0);
    const int64_t copy_cols = from_src ? (src_cols < dst_cols ? src_cols : dst_cols) : 0;
    const int64_t step = int64_t(blockDim.x) * kPadUnroll;
    for (int64_t base = threadIdx.x; base < dst_cols; base += step) {
      T v[kPadUnroll];
#pragma unroll
      for (int j = 0; j < kPadUnroll; ++j) {
        const int64_t c = base + int64_t(j) * blockDim.x;
        v[j] = c < copy_cols ? in[c] : T(0);
      }
#pragma unroll
      for (int j = 0; j < kPadUnroll; ++j) {
        const int64_t c = base + int64_t(j) * blockDim.x;
        if (c < dst_cols) out[c] = v[j];
      }
    }
  }
}

int64_t grid_for(int64_t work, int64_t per_block) {
  int64_t g = hp::ceil_div(work, per_block);
  if (g < 1) g = 1;
  return g > 65536 * 16 ? 65536 * 16 : g;
}

uint4 replicate(uint64_t bits, int elem_bytes) {
  uint64_t word = 0;
  switch (elem_bytes) {
    case 1: word = (bits & 0xFF) * 0x0101010101010101ull; break;
    case 2: word = (bits & 0xFFFF) * 0x0001000100010001ull; break;
    case 4: word = (bits & 0xFFFFFFFFull) * 0x0000000100000001ull; break;
    default: word = bits; break;
  }
  uint4 p;
  p.x = uint32_t(word);
  p.y = uint32_t(word >> 32);
  p.z = p.x;
  p.w = p.y;
  return p;
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

int hp_fill(hp_ctx* ctx, void* dst, int64_t count, int elem_bytes, uint64_t bits) {
  return guarded([&] {
    hp::enter(ctx);
    require(count >= 0, "negative count");
    require(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
            "elem_bytes must be 1, 2, 4 or 8");
    if (count == 0) return;
    require(dst != nullptr, "null destination");
    require(reinterpret_cast<uintptr_t>(dst) % 16 == 0, "fill destination must be 16-byte aligned");
    const uint4 pattern = replicate(bits, elem_bytes);
    const int64_t grid = grid_for(count * elem_bytes / 16 + 1, 256 * 4);
    switch (elem_bytes) {
      case 1: fill_kernel<uint8_t><<<grid, 256, 0, ctx->stream>>>((uint8_t*)dst, count, uint8_t(bits), pattern); break;
      case 2: fill_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>((uint16_t*)dst, count, uint16_t(bits), pattern); break;
      case 4: fill_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>((uint32_t*)dst, count, uint32_t(bits), pattern); break;
      default: fill_kernel<uint64_t><<<grid, 256, 0, ctx->stream>>>((uint64_t*)dst, count, uint64_t(bits), pattern); break;
    }
    hp::check_launch("fill");
  });
}

int hp_gather(hp_ctx* ctx, int elem_bytes, const void* src, void* dst, int64_t offset, int rank,
              const int64_t* shape, const int64_t* strides) {
  return guarded([&] {
    hp::enter(ctx);
    require(rank >= 0 && rank <= 8, "gather rank must be <= 8");
    require(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
            "elem_bytes must be 1, 2, 4 or 8");
    Strided layout{};
    int64_t count = 1;
    for (int d = 0; d < rank; ++d) {
      require(shape[d] >= 0, "negative extent");
      layout.shape[d] = shape[d];
      layout.strides[d] = strides[d];
      count *= shape[d];
    }
    if (count == 0) return;
    require(src != nullptr && dst != nullptr, "null pointer");
    for (int d = 0; d < rank; ++d) require(layout.shape[d] > 0, "empty extent");
    const int64_t grid = grid_for(count, 256 * 4);
    switch (elem_bytes) {
      case 1: gather_kernel<uint8_t><<<grid, 256, 0, ctx->stream>>>((const uint8_t*)src, (uint8_t*)dst, count, offset, rank, layout); break;
      case 2: gather_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>((const uint16_t*)src, (uint16_t*)dst, count, offset, rank, layout); break;
      case 4: gather_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>((const uint32_t*)src, (uint32_t*)dst, count, offset, rank, layout); break;
      default: gather_kernel<uint64_t><<<grid, 256, 0, ctx->stream>>>((const uint64_t*)src, (uint64_t*)dst, count, offset, rank, layout); break;
    }
    hp::check_launch("gather");
  });
}

int hp_pad_copy(hp_ctx* ctx, int elem_bytes, const void* src, void* dst, int64_t batch, int64_t src_rows,
                int64_t src_cols, int64_t dst_rows, int64_t dst_cols) {
  return guarded([&] {
    hp::enter(ctx);
    require(elem_bytes == 4 || elem_bytes == 8, "pad copies move 4- or 8-byte words");
    require(batch >= 0 && src_rows >= 0 && src_cols >= 0 && dst_rows >= 0 && dst_cols >= 0,
            "negative extent");
    const int64_t rows_total = batch * dst_rows;
    if (rows_total == 0 || dst_cols == 0) return;
    require(dst != nullptr, "null destination");
    require(src != nullptr || src_rows == 0 || src_cols == 0, "null source");
    // A source with no rows or no columns contributes only zeros.
    int64_t sr = src_rows, sc = src_cols;
    if (sr == 0 || sc == 0) sr = 0;
    const int64_t grid = rows_total < 65536 * 4 ? rows_total : 65536 * 4;
    const int block = dst_cols >= 256 ? 256 : 64;
    if (elem_bytes == 4) {
      pad_kernel<uint32_t><<<grid, block, 0, ctx->stream>>>((const uint32_t*)src, (uint32_t*)dst, rows_total, sr,
                                                           sc, dst_rows, dst_cols);
    } else {
      pad_kernel<uint64_t><<<grid, block, 0, ctx->stream>>>((const uint64_t*)src, (uint64_t*)dst, rows_total, sr,
                                                           sc, dst_rows, dst_cols);
    }
    hp::check_launch("pad_copy");
  });
}

}  // extern "C"
