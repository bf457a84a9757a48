// Sum / min / max over the middle axis of an (outer, reduced, inner) view.
//
// Contract (reference _reductions.py:91-146, _cuda.py:449-491): extrema
// propagate NaN; on a zero tie min returns -0 if any operand is -0 and max
// returns +0 if any operand is +0; integers compare in their own type; bool
// min/max are logical and/or. The sum of an empty axis is 0.
//
// Contiguous rows are reduced by one 256-thread workgroup per (row, chunk of
// kChunk elements): lane-strided accumulation, a 64-lane butterfly and a
// fixed-order merge of the four wave results. Rows longer than kChunk leave
// one partial per chunk and are reduced again. Strided axes (inner > 1) go
// through the chunked column engine of strided.h.
//
// Signed integer sums add as the matching unsigned type (wrapping modulo
// 2^bits, as NumPy does) so that overflow is never undefined behaviour.
#include <limits>
#include <type_traits>

#include "common.h"
#include "strided.h"

namespace {

constexpr int kBlock = 256;
constexpr int64_t kChunk = 8192;

template <typename T, int OP>
struct Combine;

template <typename T>
struct Combine<T, HP_SUM> {
  __device__ static T identity() { return T(0); }
  __device__ static T apply(T a, T b) {
    if constexpr (std::is_integral<T>::value && std::is_signed<T>::value) {
      using U = typename std::make_unsigned<T>::type;
      return T(U(a) + U(b));
    } else {
      return a + b;
    }
  }
};

// IEEE 754-2019 minimum/maximum: NaN if either operand is NaN, -0 < +0.
// That is the extrema contract above; gfx950 has them as instructions
// (v_minimum3_f32 / v_maximum3_f32 take three operands, so the compiler
// folds two elements per instruction).
template <typename T>
__device__ __forceinline__ T float_min(T a, T b) {
  return __builtin_elementwise_minimum(a, b);
}
template <typename T>
__device__ __forceinline__ T float_max(T a, T b) {
  return __builtin_elementwise_maximum(a, b);
}

template <typename T>
struct Combine<T, HP_MIN> {
  __device__ static T identity() { return std::numeric_limits<T>::max(); }
  __device__ static T apply(T a, T b) { return a < b ? a : b; }
};
template <typename T>
struct Combine<T, HP_MAX> {
  __device__ static T identity() { return std::numeric_limits<T>::lowest(); }
  __device__ static T apply(T a, T b) { return a > b ? a : b; }
};
template <>
struct Combine<float, HP_MIN> {
  __device__ static float identity() { return INFINITY; }
  __device__ static float apply(float a, float b) { return float_min(a, b); }
};
template <>
struct Combine<float, HP_MAX> {
  __device__ static float identity() { return -INFINITY; }
  __device__ static float apply(float a, float b) { return float_max(a, b); }
};
template <>
struct Combine<double, HP_MIN> {
  __device__ static double identity() { return INFINITY; }
  __device__ static double apply(double a, double b) { return float_min(a, b); }
};
template <>
struct Combine<double, HP_MAX> {
  __device__ static double identity() { return -INFINITY; }
  __device__ static double apply(double a, double b) { return float_max(a, b); }
};
// bool is stored as one byte holding 0 or 1.
template <>
struct Combine<uint8_t, HP_MIN> {
  __device__ static uint8_t identity() { return 1; }
  __device__ static uint8_t apply(uint8_t a, uint8_t b) { return uint8_t(a != 0 && b != 0); }
};
template <>
struct Combine<uint8_t, HP_MAX> {
  __device__ static uint8_t identity() { return 0; }
  __device__ static uint8_t apply(uint8_t a, uint8_t b) { return uint8_t(a != 0 || b != 0); }
};

template <typename T>
__device__ __forceinline__ T shfl_xor_any(T v, int offset) {
  if constexpr (sizeof(T) == 8) {
    int64_t bits;
    __builtin_memcpy(&bits, &v, 8);
    bits = __shfl_xor(bits, offset, 64);
    __builtin_memcpy(&v, &bits, 8);
    return v;
  } else if constexpr (sizeof(T) == 4) {
    int bits;
    __builtin_memcpy(&bits, &v, 4);
    bits = __shfl_xor(bits, offset, 64);
    __builtin_memcpy(&v, &bits, 4);
    return v;
  } else {
    int bits = int(v);
    bits = __shfl_xor(bits, offset, 64);
    return T(bits);
  }
}

template <typename T, int OP>
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                             int64_t outer, int64_t reduced, int64_t chunks) {
  using C = Combine<T, OP>;
  __shared__ T partial[kBlock / 64];
  const int64_t g = blockIdx.x;
  const int64_t o = g / chunks, ch = g - o * chunks;
  const int64_t begin = ch * kChunk;
  const int64_t end = begin + kChunk < reduced ? begin + kChunk : reduced;
  const T* row = x + o * reduced;
  T acc = C::identity();
  for (int64_t r = begin + threadIdx.x; r < end; r += kBlock) acc = C::apply(acc, row[r]);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) acc = C::apply(acc, shfl_xor_any(acc, off));
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    T total = partial[0];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) total = C::apply(total, partial[w]);
    out[g] = total;
  }
}

// Strided-axis op for the column engine: rows fold in ascending order.
template <typename T, int OP>
struct ColumnOp {
  using In = T;
  using Acc = T;
  using Out = T;
  using C = Combine<T, OP>;
  static constexpr int kBatch = 8;
  __device__ static T identity_in() { return C::identity(); }
  __device__ static T identity() { return C::identity(); }
  __device__ static T fold(T acc, const T (&v)[kBatch]) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) acc = C::apply(acc, v[j]);
    return acc;
  }
  __device__ static T combine(T a, T b) { return C::apply(a, b); }
  __device__ static T finish(T a) { return a; }
};

template <typename T>
constexpr int vector_max() {
  return sizeof(T) == 4 ? 4 : (sizeof(T) == 8 ? 2 : 1);
}

template <typename T, int OP>
void run_cols(hp_ctx* ctx, const T* x, T* out, int64_t outer, int64_t reduced, int64_t inner) {
  const int v_in = hps::vector_width(x, inner, sizeof(T));
  const int v_acc = hps::vector_width(reinterpret_cast<const void*>(256), inner, sizeof(T));
  // 2 workgroups per compute unit for every operation: with 16 loads in
  // flight per lane the extrema's folds (two elements per v_maximum3_f32)
  // hide behind them too (1 GiB float32 axis 0, one MI355X: max 84.3% of HBM
  // at 2 against 81.3% at 4; sum 84.2%).
  const int64_t groups_per_cu = 2;
  const hps::Plan plan = hps::plan(outer, reduced, inner, v_in, v_acc, sizeof(T), ctx->compute_units, groups_per_cu);
  void* buffers[2] = {nullptr, nullptr};
  for (int i = 0; i < 2; ++i)
    if (plan.bytes[i] > 0) buffers[i] = hp::scratch_alloc(ctx, plan.bytes[i]);
  using Op = ColumnOp<T, OP>;
  hps::execute<Op, Op, vector_max<T>(), vector_max<T>()>(ctx->stream, plan, x, out, outer, reduced, inner, buffers);
  for (int i = 0; i < 2; ++i)
    if (buffers[i]) hp::scratch_free(ctx, buffers[i]);
}

template <typename T, int OP>
void run(hp_ctx* ctx, const T* x, T* out, int64_t outer, int64_t reduced, int64_t inner) {
  if (inner > 1) return run_cols<T, OP>(ctx, x, out, outer, reduced, inner);
  const int64_t chunks = hp::ceil_div(reduced, kChunk);
  const int64_t grid = outer * chunks;
  hp::require(grid <= hp::kMaxGrid, "reduction too large for one launch");
  if (chunks == 1) {
    reduce_rows_kernel<T, OP><<<grid, kBlock, 0, ctx->stream>>>(x, out, outer, reduced, 1);
    hp::check_launch("reduce_rows");
    return;
  }
  T* partial = static_cast<T*>(hp::scratch_alloc(ctx, size_t(grid) * sizeof(T)));
  reduce_rows_kernel<T, OP><<<grid, kBlock, 0, ctx->stream>>>(x, partial, outer, reduced, chunks);
  hp::check_launch("reduce_rows");
  run<T, OP>(ctx, partial, out, outer, chunks, 1);
  hp::scratch_free(ctx, partial);
}

template <typename T>
void dispatch_op(hp_ctx* ctx, int op, const void* x, void* out, int64_t outer, int64_t reduced, int64_t inner) {
  switch (op) {
    case HP_SUM: run<T, HP_SUM>(ctx, (const T*)x, (T*)out, outer, reduced, inner); break;
    case HP_MIN: run<T, HP_MIN>(ctx, (const T*)x, (T*)out, outer, reduced, inner); break;
    case HP_MAX: run<T, HP_MAX>(ctx, (const T*)x, (T*)out, outer, reduced, inner); break;
    default: hp::fail(HP_E_INVALID, "unknown reduction operation");
  }
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

int hp_reduce(hp_ctx* ctx, int dtype, int op, const void* x, void* out, int64_t outer, int64_t reduced,
              int64_t inner) {
  return guarded([&] {
    hp::enter(ctx);
    require(op == HP_SUM || op == HP_MIN || op == HP_MAX, "unknown reduction operation");
    require(outer >= 0 && reduced >= 0 && inner >= 0, "negative extent");
    require(!(dtype == HP_BOOL && op == HP_SUM), "boolean sum requires a numeric accumulator");
    const size_t size = hp::dtype_size(dtype);
    const int64_t count = outer * inner;
    if (count == 0) return;
    require(out != nullptr, "null output");
    if (reduced == 0) {
      require(op == HP_SUM, "zero-size reduction has no identity for min/max");
      HP_CHECK(hipMemsetAsync(out, 0, size_t(count) * size, ctx->stream));
      return;
    }
    require(x != nullptr, "null input");
    switch (dtype) {
      case HP_BOOL: dispatch_op<uint8_t>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_I32: dispatch_op<int32_t>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_I64: dispatch_op<int64_t>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_U32: dispatch_op<uint32_t>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_U64: dispatch_op<uint64_t>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_F32: dispatch_op<float>(ctx, op, x, out, outer, reduced, inner); break;
      case HP_F64: dispatch_op<double>(ctx, op, x, out, outer, reduced, inner); break;
      default: hp::fail(HP_E_INVALID, "unknown dtype code");
    }
  });
}

}  // extern "C"
