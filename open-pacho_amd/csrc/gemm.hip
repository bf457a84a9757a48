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

// Zero-fills C for k == 0 (no MFMA launch).
void zero_output(hp_ctx* ctx, int dtype, void* c, int64_t outputs) {
  const int64_t grid = std::min<int64_t>(hp::ceil_div(outputs, 256), 65536);
  if (dtype == HP_F32) {
    zero_kernel<float><<<grid, 256, 0, ctx->stream>>>(static_cast<float*>(c), outputs);
  } else {
    zero_kernel<double><<<grid, 256, 0, ctx->stream>>>(static_cast<double*>(c), outputs);
  }
  hp::check_launch("gemm_zero");
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
    require(dtype == HP_F32 || dtype == HP_F64, "gemm supports float32 and float64");
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
    run(ctx, dtype, false, false, a, b, c, m, n, k, bd, batch);
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
