// GEMM entry points: C[b] = A[b'] @ B[b''] (hp_gemm) and the 2-D products
// with transposed operands (hp_gemm_layout). The kernels are described in
// gemm_kernels.h. Reference semantics: _gemm.py:24-137 (per-batch broadcast
// offsets _offset :13-21, never reads C), _cuda.py:493-518 and :619-636;
// transposed operands: _matmul_layout.py:9-48 (TransposedGemm.run).
#include <algorithm>

#include "gemm.h"

namespace {

template <typename T>
__global__ __launch_bounds__(256) void zero_kernel(T* __restrict__ out, int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < count; i += int64_t(gridDim.x) * 256) out[i] = T(0);
}

// Products of every layout: C[b] = op(A[b']) @ op(B[b'']).
void run(hp_ctx* ctx, int dtype, bool ta, bool tb, const void* a, const void* b, void* c, int64_t m, int64_t n,
         int64_t k, const hpgemm::BatchDesc& bd, int64_t batch) {
  static const hpgemm::Run table[2][4] = {
      {hpgemm::f32_nn, hpgemm::f32_tn, hpgemm::f32_nt, hpgemm::f32_tt},
      {hpgemm::f64_nn, hpgemm::f64_tn, hpgemm::f64_nt, hpgemm::f64_tt},
  };
  table[dtype == HP_F32 ? 0 : 1][(ta ? 1 : 0) + (tb ? 2 : 0)](ctx, a, b, c, m, n, k, bd, batch);
}

// Zero-fills C for k == 0 (no product launch).
void zero_output(hp_ctx* ctx, int dtype, void* c, int64_t outputs) {
  const int64_t grid = std::min<int64_t>(hp::ceil_div(outputs, 256), 65536);
  switch (dtype) {
    case HP_F32: zero_kernel<float><<<grid, 256, 0, ctx->stream>>>(static_cast<float*>(c), outputs); break;
    case HP_F64: zero_kernel<double><<<grid, 256, 0, ctx->stream>>>(static_cast<double*>(c), outputs); break;
    case HP_BOOL: zero_kernel<uint8_t><<<grid, 256, 0, ctx->stream>>>(static_cast<uint8_t*>(c), outputs); break;
    case HP_I32:
    case HP_U32: zero_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>(static_cast<uint32_t*>(c), outputs); break;
    default: zero_kernel<uint64_t><<<grid, 256, 0, ctx->stream>>>(static_cast<uint64_t*>(c), outputs); break;
  }
  hp::check_launch("gemm_zero");
}

// Integer and bool products, as NumPy computes them: sums of products in the
// operand type, wrapping modulo 2^bits (signed types are multiplied and added
// as unsigned words, whose two's-complement result is the same), and for bool
// the logical or of ands. Both are exact in any order, so this simple kernel
// is bit-identical to any other summation order (reference: the OpenCL
// backend's generic product, _opencl.py:386-420). One 256-thread workgroup
// per 16 x 16 output tile, 16-deep K slices staged in LDS.
template <typename W>
struct IntOps {
  static __device__ __forceinline__ W fma(W acc, W a, W b) { return acc + a * b; }
};
template <>
struct IntOps<uint8_t> {  // bool
  static __device__ __forceinline__ uint8_t fma(uint8_t acc, uint8_t a, uint8_t b) {
    return uint8_t(acc | ((a != 0) & (b != 0)));
  }
};

template <typename W>
__global__ __launch_bounds__(256) void int_gemm_kernel(const W* __restrict__ A, const W* __restrict__ B,
                                                       W* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                       hpgemm::BatchDesc bd, int64_t tiles_m, int64_t tiles_n) {
  __shared__ W As[16][17], Bs[16][17];
  const int64_t tile = blockIdx.x;
  const int64_t batch = tile / (tiles_m * tiles_n);
  const int64_t rest = tile - batch * tiles_m * tiles_n;
  const int64_t row = (rest / tiles_n) * 16 + (threadIdx.x >> 4);
  const int64_t col = (rest % tiles_n) * 16 + (threadIdx.x & 15);
  const int ty = threadIdx.x >> 4, tx = threadIdx.x & 15;
  int64_t a_off, b_off;
  hpgemm::batch_offsets(batch, bd, a_off, b_off);
  const W* a = A + a_off;
  const W* b = B + b_off;
  W acc = 0;
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    As[ty][tx] = row < M && k0 + tx < K ? a[row * K + k0 + tx] : W(0);
    Bs[ty][tx] = k0 + ty < K && col < N ? b[(k0 + ty) * N + col] : W(0);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc = IntOps<W>::fma(acc, As[ty][kk], Bs[kk][tx]);
    __syncthreads();
  }
  if (row < M && col < N) C[batch * M * N + row * N + col] = acc;
}

void run_int(hp_ctx* ctx, int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
             const hpgemm::BatchDesc& bd, int64_t batch) {
  const int64_t tiles_m = hp::ceil_div(m, 16), tiles_n = hp::ceil_div(n, 16);
  const int64_t grid = batch * tiles_m * tiles_n;
  hp::require(grid <= hp::kMaxGrid, "integer product has too many tiles for one launch");
#define PACHO_INT_GEMM(W)                                                                                   \
  int_gemm_kernel<W><<<grid, 256, 0, ctx->stream>>>(static_cast<const W*>(a), static_cast<const W*>(b),    \
                                                    static_cast<W*>(c), m, n, k, bd, tiles_m, tiles_n)
  switch (dtype) {
    case HP_BOOL: PACHO_INT_GEMM(uint8_t); break;
    case HP_I32:
    case HP_U32: PACHO_INT_GEMM(uint32_t); break;
    default: PACHO_INT_GEMM(uint64_t); break;
  }
#undef PACHO_INT_GEMM
  hp::check_launch("int_gemm");
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

int hp_gemm(hp_ctx* ctx, int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
            int batch_rank, const int64_t* batch_shape, const int64_t* a_batch_strides,
            const int64_t* b_batch_strides) {
  return guarded([&] {
    hp::enter(ctx);
    require(dtype >= HP_BOOL && dtype <= HP_F64, "unknown dtype code");
    require(m >= 0 && n >= 0 && k >= 0, "negative extent");
    require(batch_rank >= 0 && batch_rank <= 6, "batch rank must be <= 6");
    hpgemm::BatchDesc bd{};
    bd.rank = batch_rank;
    int64_t batch = 1;
    for (int d = 0; d < batch_rank; ++d) {
      require(batch_shape[d] >= 0, "negative batch extent");
      bd.shape[d] = batch_shape[d];
      bd.a_stride[d] = a_batch_strides[d];
      bd.b_stride[d] = b_batch_strides[d];
      batch *= batch_shape[d];
    }
    const int64_t outputs = batch * m * n;
    if (outputs == 0) return;
    require(c != nullptr, "null output");
    if (k == 0) {
      zero_output(ctx, dtype, c, outputs);
      return;
    }
    require(a != nullptr && b != nullptr, "null input");
    if (dtype == HP_F32 || dtype == HP_F64) {
      run(ctx, dtype, false, false, a, b, c, m, n, k, bd, batch);
    } else {
      run_int(ctx, dtype, a, b, c, m, n, k, bd, batch);
    }
  });
}

int hp_gemm_layout(hp_ctx* ctx, int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                   int transpose_a, int transpose_b) {
  return guarded([&] {
    hp::enter(ctx);
    require(dtype == HP_F32 || dtype == HP_F64, "gemm supports float32 and float64");
    require(m >= 0 && n >= 0 && k >= 0, "negative extent");
    if (m == 0 || n == 0) return;
    require(c != nullptr, "null output");
    if (k == 0) {
      zero_output(ctx, dtype, c, m * n);
      return;
    }
    require(a != nullptr && b != nullptr, "null input");
    hpgemm::BatchDesc bd{};
    run(ctx, dtype, transpose_a != 0, transpose_b != 0, a, b, c, m, n, k, bd, 1);
  });
}

}  // extern "C"
