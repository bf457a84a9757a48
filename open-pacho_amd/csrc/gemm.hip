// MFMA GEMM for gfx950: C[b] = A[b'] @ B[b''] in fp32 and fp64.
//
// fp32: v_mfma_f32_16x16x4_f32 (measured 155 TFLOP/s peak on MI355X, against
// 137 for the 32x32x2 form). Workgroup tile 256x128x16, four waves in a 2x2
// grid, each wave 128x64 (8x4 MFMA blocks, 128 accumulators per lane).
// fp64: v_mfma_f64_16x16x4_f64, workgroup tile 128x128x16, each wave 64x64.
//
// Data path per K slice: global -> registers (prefetch of slice s+1 while
// slice s is multiplied) -> LDS (double-buffered, one barrier per slice) ->
// 16-byte LDS reads -> MFMA. LDS holds both operands k-contiguous: A as
// [m][k] (a copy of a row-major tile) and B as [n][k] (each lane loads one
// column's k values as scalars, so the transposition costs no shuffles). A
// lane of MFMA lane group g = lane/16 then reads four consecutive k values with one ds_read_b128 and feeds them to four
// MFMAs, i.e. MFMA number q contracts k = {q, 4+q, 8+q, 12+q}; A and B use
// the same permutation, so every product of the slice is summed exactly once.
//
// Tile order: workgroup ids are renumbered so each XCD (ids i % 8) owns a
// contiguous range of tiles, and tiles are visited in groups of kGroupM tile
// rows, so the workgroups resident on one XCD share A and B panels in its L2.
//
// Modes: 0 = interior (no guards; M, N, K multiples of the tile and 16-byte
// aligned rows), 1 = guarded vector loads of A (K % 4 == 0 for fp32, K even
// for fp64), 2 = guarded scalar loads (any shape). Guarded loads fill zeros, so edge
// tiles contract against +0 padding, and stores are masked.
//
// Reference semantics: _gemm.py:24-137 (per-batch broadcast offsets
// _offset :13-21, never reads C), _cuda.py:493-518 and :619-636.
#include "common.h"

namespace {

struct BatchDesc {
  int rank;
  int64_t shape[6];
  int64_t a_stride[6];
  int64_t b_stride[6];
};

struct TileMap {
  int64_t tiles_m, tiles_n, tiles_per_batch, total;
};

constexpr int64_t kGroupM = 8;

__device__ __forceinline__ void map_tile(int64_t bid, const TileMap& tm, int64_t& batch, int64_t& ti, int64_t& tj) {
  int64_t t = bid;
  const int64_t full = (tm.total / 8) * 8;
  if (bid < full) t = (bid % 8) * (full / 8) + bid / 8;
  batch = t / tm.tiles_per_batch;
  t -= batch * tm.tiles_per_batch;
  const int64_t group = t / (kGroupM * tm.tiles_n);
  const int64_t first = group * kGroupM;
  const int64_t gm = tm.tiles_m - first < kGroupM ? tm.tiles_m - first : kGroupM;
  const int64_t r = t - group * kGroupM * tm.tiles_n;
  ti = first + r % gm;
  tj = r / gm;
}

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

// ------------------------------------------------------------------ fp32 ----

namespace f32 {

constexpr int BM = 256, BN = 128, BK = 16;
constexpr int S = BK;  // LDS row stride (floats): 16-float rows, swizzled quads
constexpr int kThreads = 256;

// LDS rows hold 4 quads of 4 consecutive k values; quad q of row r is stored
// at slot q ^ ((r >> 1) & 3). Rows are 16 floats (64 B), so a ds_read_b128 by
// lanes reading rows r0..r0+15 at one logical quad, a ds_write_b128 of 4 rows x
// 4 quads, and the B writes of 16 consecutive n at one quad all land on
// distinct banks (measured: removes the LDS bank conflicts of padded rows).
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 3; }

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                      BatchDesc bd, TileMap tmap) {
  __shared__ __attribute__((aligned(16))) float As[2][BM * S];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * S];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int64_t batch, ti, tj;
  map_tile(blockIdx.x, tmap, batch, ti, tj);
  int64_t a_off, b_off;
  batch_offsets(batch, bd, a_off, b_off);
  const float* Ab = A + a_off;
  const float* Bb = B + b_off;
  float* Cb = C + batch * M * N;
  const int64_t m0 = ti * BM, n0 = tj * BN;

  // Global -> register assignment. A: 4 float4 per thread (rows tid/4 + 64i,
  // k quad tid%4). B: column n = tid%128, k quads 2*(tid/128) + {0, 1}
  // (8 scalar loads; 64 lanes read 256 contiguous bytes of one B row).
  int a_row[4], a_lds[4];
  const int a_kq = tid & 3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a_row[i] = (tid >> 2) + 64 * i;
    a_lds[i] = a_row[i] * S + 4 * (a_kq ^ swizzle(a_row[i]));
  }
  const int b_n = tid & (BN - 1);
  const int b_q = (tid / BN) * 2;
  const int b_lds0 = b_n * S + 4 * (b_q ^ swizzle(b_n));
  const int b_lds1 = b_n * S + 4 * ((b_q + 1) ^ swizzle(b_n));

  hpd::f32x4 ra[4];
  float rb[2][4];

  auto load_slice = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = m0 + a_row[i];
      const int64_t kk = k0 + 4 * a_kq;
      const float* p = Ab + row * K + kk;
      if (MODE == 0) {
        ra[i] = *reinterpret_cast<const hpd::f32x4*>(p);
      } else if (MODE == 1) {
        const bool ok = row < M && kk < K;
        ra[i] = ok ? *reinterpret_cast<const hpd::f32x4*>(p) : hpd::f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[i][e] = (row < M && kk + e < K) ? p[e] : 0.f;
      }
    }
    const int64_t col = n0 + b_n;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t kr = k0 + 4 * (b_q + q) + e;
        if (MODE == 0) {
          rb[q][e] = Bb[kr * N + col];
        } else {
          rb[q][e] = (kr < K && col < N) ? Bb[kr * N + col] : 0.f;
        }
      }
    }
  };

  auto store_slice = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<hpd::f32x4*>(&As[buf][a_lds[i]]) = ra[i];
    *reinterpret_cast<hpd::f32x4*>(&Bs[buf][b_lds0]) = hpd::f32x4{rb[0][0], rb[0][1], rb[0][2], rb[0][3]};
    *reinterpret_cast<hpd::f32x4*>(&Bs[buf][b_lds1]) = hpd::f32x4{rb[1][0], rb[1][1], rb[1][2], rb[1][3]};
  };

  hpd::f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = hpd::f32x4{0.f, 0.f, 0.f, 0.f};

  // Rows read by a lane differ by multiples of 16, so the swizzle of every
  // row it reads equals that of (lane & 15).
  const int a_read = (wm * 128 + (lane & 15)) * S + 4 * ((lane >> 4) ^ swizzle(lane & 15));
  const int b_read = (wn * 64 + (lane & 15)) * S + 4 * ((lane >> 4) ^ swizzle(lane & 15));
  const int64_t slices = (K + BK - 1) / BK;

  load_slice(0);
  store_slice(0);
  __syncthreads();
  for (int64_t s = 0; s < slices; ++s) {
    const int cur = int(s & 1);
    if (s + 1 < slices) load_slice((s + 1) * BK);
    hpd::f32x4 a[8], b[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const hpd::f32x4*>(&As[cur][a_read + 16 * i * S]);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const hpd::f32x4*>(&Bs[cur][b_read + 16 * j * S]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
    if (s + 1 < slices) store_slice(cur ^ 1);
    __syncthreads();
  }

  // Accumulator layout: lane holds column lane%16, rows 4*(lane/16) + r.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn * 64 + 16 * j + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * 128 + 16 * i + 4 * (lane >> 4) + r;
        if (MODE == 0 || (row < M && col < N)) Cb[row * N + col] = acc[i][j][r];
      }
    }
  }
}

}  // namespace f32

// ------------------------------------------------------------------ fp64 ----

namespace f64 {

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int SA = BK + 2;  // LDS row stride in doubles
constexpr int SB = BK + 2;
constexpr int kThreads = 256;

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void kernel(const double* __restrict__ A, const double* __restrict__ B,
                                                      double* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                      BatchDesc bd, TileMap tmap) {
  __shared__ __attribute__((aligned(16))) double As[2][BM * SA];
  __shared__ __attribute__((aligned(16))) double Bs[2][BN * SB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int64_t batch, ti, tj;
  map_tile(blockIdx.x, tmap, batch, ti, tj);
  int64_t a_off, b_off;
  batch_offsets(batch, bd, a_off, b_off);
  const double* Ab = A + a_off;
  const double* Bb = B + b_off;
  double* Cb = C + batch * M * N;
  const int64_t m0 = ti * BM, n0 = tj * BN;

  // A: 4 double2 per thread (rows tid/8 + 32i, k pair tid%8).
  // B: column n = tid%128, k rows 8*(tid/128) + {0..7} (8 scalar loads).
  int a_row[4];
  const int a_k = (tid & 7) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) a_row[i] = (tid >> 3) + 32 * i;
  const int b_n = tid & 127;
  const int b_k = (tid >> 7) * 8;

  hpd::f64x2 ra[4];
  double rb[8];

  auto load_slice = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = m0 + a_row[i];
      const int64_t kk = k0 + a_k;
      const double* p = Ab + row * K + kk;
      if (MODE == 0) {
        ra[i] = *reinterpret_cast<const hpd::f64x2*>(p);
      } else if (MODE == 1) {
        const bool ok = row < M && kk < K;
        ra[i] = ok ? *reinterpret_cast<const hpd::f64x2*>(p) : hpd::f64x2{0.0, 0.0};
      } else {
        ra[i][0] = (row < M && kk < K) ? p[0] : 0.0;
        ra[i][1] = (row < M && kk + 1 < K) ? p[1] : 0.0;
      }
    }
    const int64_t col = n0 + b_n;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int64_t kr = k0 + b_k + s;
      if (MODE == 0) {
        rb[s] = Bb[kr * N + col];
      } else {
        rb[s] = (kr < K && col < N) ? Bb[kr * N + col] : 0.0;
      }
    }
  };

  auto store_slice = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<hpd::f64x2*>(&As[buf][a_row[i] * SA + a_k]) = ra[i];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const hpd::f64x2 v = {rb[2 * s], rb[2 * s + 1]};
      *reinterpret_cast<hpd::f64x2*>(&Bs[buf][b_n * SB + b_k + 2 * s]) = v;
    }
  };

  f64x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

  // Lane group g = lane/16 reads k = 2g, 2g+1 (first half of the slice) and
  // 8 + 2g, 8 + 2g + 1 (second half): MFMA q in {0,1} per half.
  const int a_read = (wm * 64 + (lane & 15)) * SA + (lane >> 4) * 2;
  const int b_read = (wn * 64 + (lane & 15)) * SB + (lane >> 4) * 2;
  const int64_t slices = (K + BK - 1) / BK;

  load_slice(0);
  store_slice(0);
  __syncthreads();
  for (int64_t s = 0; s < slices; ++s) {
    const int cur = int(s & 1);
    if (s + 1 < slices) load_slice((s + 1) * BK);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      hpd::f64x2 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const hpd::f64x2*>(&As[cur][a_read + 16 * i * SA + 8 * half]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const hpd::f64x2*>(&Bs[cur][b_read + 16 * j * SB + 8 * half]);
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < slices) store_slice(cur ^ 1);
    __syncthreads();
  }

  // f64 accumulator layout: lane holds column lane%16, rows 4*r + lane/16.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn * 64 + 16 * j + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * 64 + 16 * i + 4 * r + (lane >> 4);
        if (MODE == 0 || (row < M && col < N)) Cb[row * N + col] = acc[i][j][r];
      }
    }
  }
}

}  // namespace f64

template <typename T>
bool aligned16(const T* p) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

void prepare(int64_t m, int64_t n, int64_t batch, int64_t bm, int64_t bn, TileMap& tm) {
  tm.tiles_m = hp::ceil_div(m, bm);
  tm.tiles_n = hp::ceil_div(n, bn);
  tm.tiles_per_batch = tm.tiles_m * tm.tiles_n;
  tm.total = tm.tiles_per_batch * batch;
  hp::require(tm.total <= hp::kMaxGrid, "GEMM has too many tiles for one launch");
}

bool a_strides_aligned(const BatchDesc& bd, int64_t elems_per_16b) {
  for (int d = 0; d < bd.rank; ++d) {
    if (bd.a_stride[d] % elems_per_16b) return false;
  }
  return true;
}

void run_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
             const BatchDesc& bd, int64_t batch) {
  using namespace f32;
  TileMap tm;
  prepare(m, n, batch, BM, BN, tm);
  const bool vec_ok = aligned16(a) && k % 4 == 0 && a_strides_aligned(bd, 4);
  const bool interior = vec_ok && m % BM == 0 && n % BN == 0 && k % BK == 0;
  if (interior) {
    kernel<0><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  } else if (vec_ok) {
    kernel<1><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  } else {
    kernel<2><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  }
  hp::check_launch("gemm_f32");
}

void run_f64(hp_ctx* ctx, const double* a, const double* b, double* c, int64_t m, int64_t n, int64_t k,
             const BatchDesc& bd, int64_t batch) {
  using namespace f64;
  TileMap tm;
  prepare(m, n, batch, BM, BN, tm);
  const bool vec_ok = aligned16(a) && k % 2 == 0 && a_strides_aligned(bd, 2);
  const bool interior = vec_ok && m % BM == 0 && n % BN == 0 && k % BK == 0;
  if (interior) {
    kernel<0><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  } else if (vec_ok) {
    kernel<1><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  } else {
    kernel<2><<<tm.total, kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  }
  hp::check_launch("gemm_f64");
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
    BatchDesc bd{};
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
      HP_CHECK(hipMemsetAsync(c, 0, size_t(outputs) * hp::dtype_size(dtype), ctx->stream));
      return;
    }
    require(a != nullptr && b != nullptr, "null input");
    if (dtype == HP_F32) {
      run_f32(ctx, (const float*)a, (const float*)b, (float*)c, m, n, k, bd, batch);
    } else {
      run_f64(ctx, (const double*)a, (const double*)b, (double*)c, m, n, k, bd, batch);
    }
  });
}

}  // extern "C"
