// Matrix-vector product and dot product (fp32/fp64), HBM-streaming.
//
// GEMV: one 256-thread workgroup owns kRows consecutive rows, i.e. one
// contiguous span of kRows*inner elements of A. Every lane loads 16-byte
// vectors with the nontemporal hint (A is streamed exactly once), keeps
// kRows*kUnroll loads in flight, and reuses each x vector across the kRows
// rows, so x is read from L2 once per workgroup instead of once per row.
// Accumulation: per lane a fused multiply-add chain over its strided vectors,
// then a 64-lane butterfly and a fixed-order sum of the four wave partials.
// Reference semantics: _cuda_gemv.py:20-95 (rows flattened, one output per
// row, zero-length rows give zeros). With `rhs` the kernels store the residual
// rhs[r] - y[r] instead: the same product, rounded to T, then one subtraction
// (the eager b - A @ x boundary of _gemv.py:10-75, fused).
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kRows = 4;
constexpr int kUnroll = 2;

template <typename T>
struct Vec;
template <>
struct Vec<float> {
  using type = hpd::f32x4;
  static constexpr int width = 4;
};
template <>
struct Vec<double> {
  using type = hpd::f64x2;
  static constexpr int width = 2;
};

__device__ __forceinline__ float dfma(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ double dfma(double a, double b, double c) { return fma(a, b, c); }

template <typename V, typename T>
__device__ __forceinline__ T dot_vec(const V& a, const V& x, T acc) {
#pragma unroll
  for (int i = 0; i < int(sizeof(V) / sizeof(T)); ++i) acc = dfma(a[i], x[i], acc);
  return acc;
}

// Sums `acc[r]` over the workgroup; lane r < kRows of wave 0 gets row r's total.
template <typename T, int R>
__device__ __forceinline__ void block_reduce_store(T (&acc)[R], T* y, int64_t r0, int64_t rows,
                                                   const T* rhs = nullptr) {
  __shared__ T partial[kBlock / 64][R];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const T s = hpd::wave_sum(acc[r]);
    if (lane == 0) partial[wave][r] = s;
  }
  __syncthreads();
  if (threadIdx.x < R && r0 + threadIdx.x < rows) {
    T total = partial[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) total += partial[w][threadIdx.x];
    y[r0 + threadIdx.x] = rhs ? rhs[r0 + threadIdx.x] - total : total;
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void gemv_vec_kernel(const T* __restrict__ a, const T* __restrict__ x,
                                                          const T* __restrict__ rhs, T* __restrict__ y, int64_t rows,
                                                          int64_t inner) {
  using V = typename Vec<T>::type;
  const int64_t r0 = int64_t(blockIdx.x) * kRows;
  const int64_t nv = inner / Vec<T>::width;
  const V* xv = reinterpret_cast<const V*>(x);
  const V* av[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r < rows ? r0 + r : rows - 1;  // clamp: duplicates are discarded
    av[r] = reinterpret_cast<const V*>(a + row * inner);
  }
  T acc[kRows] = {};
  int64_t j = threadIdx.x;
  for (; j + (kUnroll - 1) * kBlock < nv; j += kUnroll * kBlock) {
    V xs[kUnroll];
    V as[kUnroll][kRows];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) as[u][r] = __builtin_nontemporal_load(av[r] + j + u * kBlock);
      xs[u] = xv[j + u * kBlock];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r] = dot_vec(as[u][r], xs[u], acc[r]);
  }
  for (; j < nv; j += kBlock) {
    const V xs = xv[j];
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = dot_vec(__builtin_nontemporal_load(av[r] + j), xs, acc[r]);
  }
  block_reduce_store<T, kRows>(acc, y, r0, rows, rhs);
}

// Scalar loads for rows whose length is not a multiple of the vector width.
template <typename T>
__global__ __launch_bounds__(kBlock) void gemv_scalar_kernel(const T* __restrict__ a, const T* __restrict__ x,
                                                             const T* __restrict__ rhs, T* __restrict__ y,
                                                             int64_t rows, int64_t inner) {
  const int64_t r0 = int64_t(blockIdx.x) * kRows;
  const T* ar[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) ar[r] = a + (r0 + r < rows ? r0 + r : rows - 1) * inner;
  T acc[kRows] = {};
  for (int64_t j = threadIdx.x; j < inner; j += kBlock) {
    const T xs = x[j];
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = dfma(ar[r][j], xs, acc[r]);
  }
  block_reduce_store<T, kRows>(acc, y, r0, rows, rhs);
}

// Short rows: one wave per row, four rows per workgroup.
template <typename T>
__global__ __launch_bounds__(kBlock) void gemv_short_kernel(const T* __restrict__ a, const T* __restrict__ x,
                                                            const T* __restrict__ rhs, T* __restrict__ y,
                                                            int64_t rows, int64_t inner) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* ar = a + row * inner;
  T acc = T(0);
  for (int64_t j = lane; j < inner; j += 64) acc = dfma(ar[j], x[j], acc);
  acc = hpd::wave_sum(acc);
  if (lane == 0) y[row] = rhs ? rhs[row] - acc : acc;
}

// Dot product: each 1024-thread workgroup reduces one chunk of kDotChunk
// elements; partials are summed by a single workgroup in index order
// (deterministic). A full, aligned chunk is read with all of its 16-byte loads
// in flight at once (one memory round trip), so a 16384-element dot is one
// short launch.
constexpr int kDotThreads = 1024;
constexpr int64_t kDotChunk = 16384;

template <typename T>
__global__ __launch_bounds__(kDotThreads) void dot_kernel(const T* __restrict__ x, const T* __restrict__ z,
                                                         T* __restrict__ out, int64_t n, bool aligned) {
  using V = typename Vec<T>::type;
  constexpr int W = Vec<T>::width;
  constexpr int kPer = int(kDotChunk / W / kDotThreads);
  const int64_t begin = int64_t(blockIdx.x) * kDotChunk;
  const int64_t len = n - begin < kDotChunk ? n - begin : kDotChunk;
  T acc = T(0);
  if (aligned && len == kDotChunk) {
    const V* xv = reinterpret_cast<const V*>(x + begin);
    const V* zv = reinterpret_cast<const V*>(z + begin);
    V xs[kPer], zs[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      xs[j] = xv[threadIdx.x + j * kDotThreads];
      zs[j] = zv[threadIdx.x + j * kDotThreads];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) acc = dot_vec(xs[j], zs[j], acc);
  } else {
    for (int64_t i = threadIdx.x; i < len; i += kDotThreads) acc = dfma(x[begin + i], z[begin + i], acc);
  }
  __shared__ T partial[kDotThreads / 64];
  const T s = hpd::wave_sum(acc);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    T total = partial[0];
#pragma unroll
    for (int w = 1; w < kDotThreads / 64; ++w) total += partial[w];
    out[blockIdx.x] = total;
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void sum_partials_kernel(const T* __restrict__ partial, T* __restrict__ out,
                                                              int64_t count) {
  T acc[1] = {T(0)};
  for (int64_t i = threadIdx.x; i < count; i += kBlock) acc[0] += partial[i];
  block_reduce_store<T, 1>(acc, out, 0, 1);
}

template <typename T>
void run_gemv(hp_ctx* ctx, const T* a, const T* x, const T* rhs, T* y, int64_t rows, int64_t inner) {
  const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (inner < 1024) {
    const int64_t grid = hp::ceil_div(rows, 4);
    hp::require(grid <= hp::kMaxGrid, "too many rows for one launch");
    gemv_short_kernel<T><<<grid, kBlock, 0, ctx->stream>>>(a, x, rhs, y, rows, inner);
  } else {
    const int64_t grid = hp::ceil_div(rows, kRows);
    hp::require(grid <= hp::kMaxGrid, "too many rows for one launch");
    if (aligned && inner % Vec<T>::width == 0) {
      gemv_vec_kernel<T><<<grid, kBlock, 0, ctx->stream>>>(a, x, rhs, y, rows, inner);
    } else {
      gemv_scalar_kernel<T><<<grid, kBlock, 0, ctx->stream>>>(a, x, rhs, y, rows, inner);
    }
  }
  hp::check_launch("gemv");
}

template <typename T>
void run_dot(hp_ctx* ctx, const T* x, const T* z, T* out, int64_t n) {
  const int64_t chunks = hp::ceil_div(n, kDotChunk);
  hp::require(chunks <= hp::kMaxGrid, "dot too long for one launch");
  const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(z) % 16 == 0;
  if (chunks == 1) {
    dot_kernel<T><<<1, kDotThreads, 0, ctx->stream>>>(x, z, out, n, aligned);
    hp::check_launch("dot");
    return;
  }
  T* partial = static_cast<T*>(hp::scratch_alloc(ctx, size_t(chunks) * sizeof(T)));
  dot_kernel<T><<<chunks, kDotThreads, 0, ctx->stream>>>(x, z, partial, n, aligned);
  hp::check_launch("dot");
  sum_partials_kernel<T><<<1, kBlock, 0, ctx->stream>>>(partial, out, chunks);
  hp::check_launch("dot partials");
  hp::scratch_free(ctx, partial);
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

// Shared by hp_gemv (rhs == nullptr) and hp_gemv_residual.
static void gemv_entry(hp_ctx* ctx, int dtype, const void* a, const void* x, const void* rhs, void* y, int64_t rows,
                       int64_t inner) {
  hp::enter(ctx);
  require(dtype == HP_F32 || dtype == HP_F64, "gemv supports float32 and float64");
  require(rows >= 0 && inner >= 0, "negative extent");
  if (rows == 0) return;
  require(y != nullptr, "null output");
  if (inner == 0 && rhs == nullptr) {
    HP_CHECK(hipMemsetAsync(y, 0, size_t(rows) * hp::dtype_size(dtype), ctx->stream));
    return;
  }
  if (inner == 0) {
    // The product is empty: the residual is rhs itself, bit for bit.
    HP_CHECK(hipMemcpyAsync(y, rhs, size_t(rows) * hp::dtype_size(dtype), hipMemcpyDeviceToDevice, ctx->stream));
    return;
  }
  require(a != nullptr && x != nullptr, "null input");
  if (dtype == HP_F32) {
    run_gemv<float>(ctx, (const float*)a, (const float*)x, (const float*)rhs, (float*)y, rows, inner);
  } else {
    run_gemv<double>(ctx, (const double*)a, (const double*)x, (const double*)rhs, (double*)y, rows, inner);
  }
}

int hp_gemv(hp_ctx* ctx, int dtype, const void* a, const void* x, void* y, int64_t rows, int64_t inner) {
  return guarded([&] { gemv_entry(ctx, dtype, a, x, nullptr, y, rows, inner); });
}

int hp_gemv_residual(hp_ctx* ctx, int dtype, const void* a, const void* x, const void* rhs, void* y, int64_t rows,
                     int64_t inner) {
  return guarded([&] {
    require(rows == 0 || rhs != nullptr, "null right-hand side");
    gemv_entry(ctx, dtype, a, x, rhs, y, rows, inner);
  });
}

static void dot_entry(hp_ctx* ctx, int dtype, const void* x, const void* y, void* out, int64_t n) {
  require(out != nullptr, "null output");
  if (n == 0) {
    HP_CHECK(hipMemsetAsync(out, 0, hp::dtype_size(dtype), ctx->stream));
    return;
  }
  require(x != nullptr && y != nullptr, "null input");
  if (dtype == HP_F32) {
    run_dot<float>(ctx, (const float*)x, (const float*)y, (float*)out, n);
  } else {
    run_dot<double>(ctx, (const double*)x, (const double*)y, (double*)out, n);
  }
}

int hp_dot(hp_ctx* ctx, int dtype, const void* x, const void* y, void* out, int64_t n) {
  return guarded([&] {
    hp::enter(ctx);
    require(dtype == HP_F32 || dtype == HP_F64, "dot supports float32 and float64");
    require(n >= 0, "negative length");
    dot_entry(ctx, dtype, x, y, out, n);
  });
}

int hp_dot_new(hp_ctx* ctx, int dtype, const void* x, const void* y, int64_t n, void** out) {
  return guarded([&] {
    hp::enter(ctx);
    require(out != nullptr, "null output");
    require(dtype == HP_F32 || dtype == HP_F64, "dot supports float32 and float64");
    require(n >= 0, "negative length");
    void* block = hp::scratch_alloc(ctx, hp::dtype_size(dtype));
    try {
      dot_entry(ctx, dtype, x, y, block, n);
    } catch (...) {
      hp::scratch_free(ctx, block);
      throw;
    }
    *out = block;
  });
}

}  // extern "C"
