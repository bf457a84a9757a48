// Edge strips of an fp32 product C = A @ B (row-major, A [m][k], B [k][n]):
// the last few rows (all columns) and the last few columns (the other rows),
// when the MFMA kernel runs only on the whole 256 x 256 tiles of the rest.
// A strip one to kEdgeMax elements wide would otherwise cost a full tile row
// or column of MFMA work, nearly all of it on rows or columns that lie
// outside the matrix (4097 x 2049 x 3001: 16% of the product's MFMA work).
//
// Rows strip (r x n, r <= kEdgeMax): B is read once, coalesced: thread t of a
// workgroup owns column t of a 256-column block and keeps r accumulators; the
// r rows of A for the workgroup's K range are staged in LDS. The K axis is cut
// into chunks so that enough workgroups stream B; chunk partials are then
// added in chunk order by a second kernel.
//
// Columns strip (m x c, c <= kEdgeMax): the c columns of B are first packed
// into contiguous [c][k] rows; then one wave per row of A streams the row with
// 16-byte loads (any element alignment), keeps c accumulators and reduces
// them with a butterfly.
//
// Every sum has a fixed order, so results repeat bit for bit.
#include "gemm.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunkK = 256;  // K values per rows-strip workgroup (LDS staging)
constexpr int kUnroll = 16;  // B loads in flight per thread

typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));

// Element (r, k) of op(A) is A[r * as_r + k * as_k], element (k, n) of op(B)
// is B[k * bs_k + n * bs_n]: one kernel serves stored and transposed operands.
__global__ __launch_bounds__(kThreads) void rows_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ out, int rows, int64_t N, int64_t K,
                                                        int64_t as_r, int64_t as_k, int64_t bs_k, int64_t bs_n,
                                                        int64_t ldo, int64_t col_blocks, int64_t kchunk, int direct) {
  __shared__ float As[hpgemm::kEdgeMax][kChunkK];
  const int64_t cb = blockIdx.x % col_blocks, kc = blockIdx.x / col_blocks;
  const int64_t k0 = kc * kchunk;
  const int64_t klen = K - k0 < kchunk ? K - k0 : kchunk;
  for (int64_t i = threadIdx.x; i < rows * klen; i += kThreads) {
    const int64_t r = i / klen, k = i - r * klen;
    As[r][k] = A[r * as_r + (k0 + k) * as_k];
  }
  __syncthreads();
  const int64_t n = cb * kThreads + threadIdx.x;
  if (n >= N) return;
  float acc[hpgemm::kEdgeMax];
#pragma unroll
  for (int r = 0; r < hpgemm::kEdgeMax; ++r) acc[r] = 0.f;
  const float* b = B + k0 * bs_k + n * bs_n;
  int64_t k = 0;
  for (; k + kUnroll <= klen; k += kUnroll) {
    float v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = b[(k + u) * bs_k];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int r = 0; r < hpgemm::kEdgeMax; ++r)
        if (r < rows) acc[r] = fmaf(As[r][k + u], v[u], acc[r]);
  }
  for (; k < klen; ++k) {
    const float v = b[k * bs_k];
#pragma unroll
    for (int r = 0; r < hpgemm::kEdgeMax; ++r)
      if (r < rows) acc[r] = fmaf(As[r][k], v, acc[r]);
  }
  // direct: out is C (row stride ldo); else the partial array [chunk][row][N].
  float* dst = direct ? out + n : out + (kc * rows) * N + n;
  const int64_t stride = direct ? ldo : N;
#pragma unroll
  for (int r = 0; r < hpgemm::kEdgeMax; ++r)
    if (r < rows) dst[r * stride] = acc[r];
}

// C[r][n] = sum over chunks c (ascending) of partial[c][r][n].
__global__ __launch_bounds__(kThreads) void rows_merge_kernel(const float* __restrict__ partial, float* __restrict__ C,
                                                              int rows, int64_t N, int64_t chunks, int64_t ldc) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= rows * N) return;
  const int64_t r = i / N, n = i - r * N;
  // Loads in groups of 32 in flight (the merge is latency-bound: few
  // outputs, many chunks), added in chunk order.
  const int64_t step = rows * N;
  float sum = partial[i];
  int64_t c = 1;
  for (; c + 32 <= chunks; c += 32) {
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = partial[(c + u) * step + i];
#pragma unroll
    for (int u = 0; u < 32; ++u) sum += v[u];
  }
  for (; c + 8 <= chunks; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = partial[(c + u) * step + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += v[u];
  }
  for (; c < chunks; ++c) sum += partial[c * step + i];
  C[r * ldc + n] = sum;
}

// packed[j][k] = op(B)(k, j) for j < cols, k < K (B at the strip's first column).
__global__ __launch_bounds__(kThreads) void pack_columns_kernel(const float* __restrict__ B, float* __restrict__ packed,
                                                                int cols, int64_t K, int64_t bs_k, int64_t bs_n) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= cols * K) return;
  const int64_t j = i / K, k = i - j * K;
  packed[i] = B[k * bs_k + j * bs_n];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// C[m * ldc + j] = sum_k op(A)(m, k) * packed[j * K + k]: one wave per row.
// KCONTIG (as_k == 1): 16-byte loads along the row of A, any element
// alignment; otherwise one element per lane. Both walk k in the same order
// (lane l: 4-element groups 4l + 256t, then the tail one element at a time),
// so a stored and a transposed A give the same bits.
template <bool KCONTIG>
__global__ __launch_bounds__(kThreads) void cols_kernel(const float* __restrict__ A, const float* __restrict__ packed,
                                                        float* __restrict__ C, int64_t M, int cols, int64_t K,
                                                        int64_t as_r, int64_t as_k, int64_t ldc) {
  const int lane = threadIdx.x & 63;
  const int64_t m = int64_t(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (m >= M) return;  // no barriers below
  const float* a = A + m * as_r;
  float acc[hpgemm::kEdgeMax];
#pragma unroll
  for (int j = 0; j < hpgemm::kEdgeMax; ++j) acc[j] = 0.f;
  const int64_t whole = K / 256 * 256;
#pragma unroll 4
  for (int64_t k = 4 * lane; k < whole; k += 256) {
    f32x4u x;
    if (KCONTIG) {
      x = *reinterpret_cast<const f32x4u*>(a + k);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = a[(k + e) * as_k];
    }
#pragma unroll
    for (int j = 0; j < hpgemm::kEdgeMax; ++j) {
      if (j < cols) {
        const f32x4u y = *reinterpret_cast<const f32x4u*>(packed + j * K + k);
        acc[j] = fmaf(x[3], y[3], fmaf(x[2], y[2], fmaf(x[1], y[1], fmaf(x[0], y[0], acc[j]))));
      }
    }
  }
  for (int64_t k = whole + lane; k < K; k += 64) {
    const float x = a[k * as_k];
#pragma unroll
    for (int j = 0; j < hpgemm::kEdgeMax; ++j)
      if (j < cols) acc[j] = fmaf(x, packed[j * K + k], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < hpgemm::kEdgeMax; ++j) {
    if (j < cols) {
      const float total = wave_sum(acc[j]);
      if (lane == 0) C[m * ldc + j] = total;
    }
  }
}

}  // namespace

namespace hpgemm {

void edge_rows_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int rows, int64_t n, int64_t k,
                   const Strides& st, int64_t ldc, std::vector<void*>* deferred) {
  hp::require(rows >= 1 && rows <= kEdgeMax && n >= 1 && k >= 1, "internal: edge rows strip out of range");
  const int64_t col_blocks = hp::ceil_div(n, kThreads);
  // About 1,024 workgroups stream B (latency-bound loads: 4097 x 2049 x 3001
  // rows strip 10.9 us with 423 workgroups of 64 K values); chunks of 32 to
  // 256 K values.
  int64_t kchunk = hp::ceil_div(k, std::max<int64_t>(1, 1024 / col_blocks));
  kchunk = std::min<int64_t>(kChunkK, std::max<int64_t>(32, kchunk));
  const int64_t chunks = hp::ceil_div(k, kchunk);
  const int64_t grid = col_blocks * chunks;
  if (chunks == 1) {
    rows_kernel<<<grid, kThreads, 0, ctx->stream>>>(a, b, c, rows, n, k, st.as_r, st.as_k, st.bs_k, st.bs_n, ldc,
                                                    col_blocks, kchunk, 1);
    hp::check_launch("gemm_edge_rows");
    return;
  }
  float* partial = static_cast<float*>(hp::scratch_alloc(ctx, size_t(chunks) * rows * n * sizeof(float)));
  rows_kernel<<<grid, kThreads, 0, ctx->stream>>>(a, b, partial, rows, n, k, st.as_r, st.as_k, st.bs_k, st.bs_n, ldc,
                                                  col_blocks, kchunk, 0);
  hp::check_launch("gemm_edge_rows");
  rows_merge_kernel<<<hp::ceil_div(rows * n, kThreads), kThreads, 0, ctx->stream>>>(partial, c, rows, n, chunks, ldc);
  hp::check_launch("gemm_edge_rows_merge");
  if (deferred) deferred->push_back(partial);
  else hp::scratch_free(ctx, partial);
}

void edge_cols_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int cols, int64_t k,
                   const Strides& st, int64_t ldc, std::vector<void*>* deferred) {
  hp::require(cols >= 1 && cols <= kEdgeMax && m >= 1 && k >= 1, "internal: edge columns strip out of range");
  float* packed = static_cast<float*>(hp::scratch_alloc(ctx, size_t(cols) * k * sizeof(float)));
  pack_columns_kernel<<<hp::ceil_div(cols * k, kThreads), kThreads, 0, ctx->stream>>>(b, packed, cols, k, st.bs_k,
                                                                                     st.bs_n);
  hp::check_launch("gemm_edge_pack");
  const int64_t grid = hp::ceil_div(m, kThreads / 64);
  if (st.as_k == 1) {
    cols_kernel<true><<<grid, kThreads, 0, ctx->stream>>>(a, packed, c, m, cols, k, st.as_r, st.as_k, ldc);
  } else {
    cols_kernel<false><<<grid, kThreads, 0, ctx->stream>>>(a, packed, c, m, cols, k, st.as_r, st.as_k, ldc);
  }
  hp::check_launch("gemm_edge_cols");
  if (deferred) deferred->push_back(packed);
  else hp::scratch_free(ctx, packed);
}

}  // namespace hpgemm
