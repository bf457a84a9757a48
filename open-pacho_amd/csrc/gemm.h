// Shared declarations of the GEMM translation units (libpacho_hip.so
// internals). The kernels are compiled once per dtype and operand layout in
// gemm_<dtype>_<layout>.hip (n = stored as in the product, t = transposed)
// so that the variants build in parallel; gemm.hip holds the entry points.
#pragma once

#include <vector>

#include "common.h"

namespace hpgemm {

// Batch broadcast of a product: per batch axis its extent and the element
// strides of A and B (0 = broadcast), C batches being contiguous.
struct BatchDesc {
  int rank;
  int64_t shape[6];
  int64_t a_stride[6];
  int64_t b_stride[6];
};

// Element offsets of batch `batch`'s A and B matrices (row-major batch index).
__device__ __forceinline__ void batch_offsets(int64_t batch, const BatchDesc& bd, int64_t& a_off, int64_t& b_off) {
  a_off = 0;
  b_off = 0;
  int64_t rest = batch;
  for (int d = bd.rank - 1; d >= 0; --d) {
    const int64_t extent = bd.shape[d];
    const int64_t q = rest / extent;
    const int64_t idx = rest - q * extent;
    rest = q;
    a_off += idx * bd.a_stride[d];
    b_off += idx * bd.b_stride[d];
  }
}

// Edge strips of a 2-D fp32 product (gemm_edges.hip): the MFMA kernel takes
// the whole 256 x 256 tiles and these take strips of at most kEdgeMax rows or
// columns. a, b, c point at the strip's first element of op(A), op(B) and C;
// element (r, k) of op(A) is a[r * as_r + k * as_k], element (k, n) of op(B)
// is b[k * bs_k + n * bs_n]; C rows are ldc long.
constexpr int kEdgeMax = 8;
struct Strides {
  int64_t as_r, as_k, bs_k, bs_n;
};
// Their pool temporaries go to `deferred` (when given) for the caller to free
// once the strips' stream has been joined.
void edge_rows_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int rows, int64_t n, int64_t k,
                   const Strides& st, int64_t ldc, std::vector<void*>* deferred = nullptr);
void edge_cols_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int cols, int64_t k,
                   const Strides& st, int64_t ldc, std::vector<void*>* deferred = nullptr);

// C[b] = op(A[b']) @ op(B[b'']) for b < batch, m x n x k, row-major; op(A)
// is A stored [k][m] for layout t?, op(B) is B stored [n][k] for ?t.
using Run = void (*)(hp_ctx* ctx, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                     const BatchDesc& bd, int64_t batch);
void f32_nn(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f32_tn(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f32_nt(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f32_tt(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f64_nn(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f64_tn(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f64_nt(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);
void f64_tt(hp_ctx*, const void*, const void*, void*, int64_t, int64_t, int64_t, const BatchDesc&, int64_t);

}  // namespace hpgemm
