// Overflow/underflow-safe Euclidean norms (fp32/fp64) with one HBM read.
//
// Contiguous rows (inner == 1): one wave owns a chunk of kChunk<T> elements,
// loads it into registers with 16-byte nontemporal loads, then runs the two
// classic passes on the registers: (1) m = max|x| with NaN propagation, (2)
// t = sum (x * 2^-e)^2 where m = f * 2^e, f in [0.5, 1). Scaling by a power of
// two is exact, so the only roundings are the squares and the sum; t <= len.
// A chunk's result is the pair (e, t), i.e. norm^2 = 4^e * t. Pairs merge
// exactly by rescaling with powers of two, and the final value is
// ldexp(sqrt(t), e). Special pairs: NaN chunk -> (NaN, 0); Inf (no NaN) ->
// (+inf, 0); all-zero -> (-inf, 0).
//
// Reference semantics: _norm.py:28-36 (NaN beats Inf, Inf -> Inf, zeros -> +0),
// _norm.py:44-52 (two-pass max-scale closed form), linalg.py:8-35.
#include "common.h"
#include "strided.h"

namespace {

constexpr int kBlock = 256;
constexpr int kLoads = 16;  // 16-byte loads per lane per chunk
constexpr int kResidentGroupsPerCU = 16;

template <typename T>
struct Traits;
template <>
struct Traits<float> {
  using V = hpd::f32x4;
  static constexpr int width = 4;
};
template <>
struct Traits<double> {
  using V = hpd::f64x2;
  static constexpr int width = 2;
};

template <typename T>
constexpr int64_t chunk_len() {
  return int64_t(64) * kLoads * Traits<T>::width;
}

__device__ __forceinline__ float dabs(float x) { return fabsf(x); }
__device__ __forceinline__ double dabs(double x) { return fabs(x); }
__device__ __forceinline__ float dldexp(float x, int e) { return ldexpf(x, e); }
__device__ __forceinline__ double dldexp(double x, int e) { return ldexp(x, e); }
__device__ __forceinline__ int dexponent(float m) {
  int e;
  (void)frexpf(m, &e);
  return e;
}
__device__ __forceinline__ int dexponent(double m) {
  int e;
  (void)frexp(m, &e);
  return e;
}
__device__ __forceinline__ float dsqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double dsqrt(double x) { return sqrt(x); }

// max|.| that propagates NaN from either side.
template <typename T>
__device__ __forceinline__ T nan_max(T a, T b) {
  return (isnan(a) || a > b) ? a : b;
}

// Pair algebra on (k, t): norm^2 = 4^k * t for finite k; k = -inf means 0.
template <typename T>
struct Pair {
  T k, t;
};

// Without branches: k is the IEEE maximum of the exponents (NaN wins, then
// +inf, and -inf, the zero pair, is its identity); a side whose exponent
// difference is not finite (the zero pair, or any side once k is +inf or
// NaN) adds nothing, and a non-finite k keeps t = 0. For finite pairs this is
// k = max(ka, kb), t = ta 4^(ka-k) + tb 4^(kb-k), added in that order.
template <typename T>
__device__ __forceinline__ Pair<T> merge(Pair<T> a, Pair<T> b) {
  const T k = __builtin_elementwise_maximum(a.k, b.k);
  const T da = a.k - k, db = b.k - k;
  const T ta = isfinite(da) ? dldexp(a.t, 2 * int(da)) : T(0);
  const T tb = isfinite(db) ? dldexp(b.t, 2 * int(db)) : T(0);
  return {k, isfinite(k) ? ta + tb : T(0)};
}

template <typename T>
__device__ __forceinline__ T finish(Pair<T> p) {
  if (isnan(p.k)) return T(NAN);
  if (isinf(p.k)) return p.k > 0 ? T(INFINITY) : T(0);
  return dldexp(dsqrt(p.t), int(p.k));
}

template <typename T>
__device__ __forceinline__ Pair<T> wave_merge(Pair<T> p) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Pair<T> q = {__shfl_xor(p.k, o, 64), __shfl_xor(p.t, o, 64)};
    p = merge(p, q);
  }
  return p;
}

__device__ __forceinline__ float dfma(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ double dfma(double a, double b, double c) { return fma(a, b, c); }
__device__ __forceinline__ float dmax(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ double dmax(double a, double b) { return fmax(a, b); }

// Reduce registers `v[0..n)` (zeros beyond the valid range) to a wave pair.
// The max pass uses the NaN-dropping hardware max (one instruction per
// element): a NaN then reaches the sum of squares and makes t NaN. Only when
// the max is +inf or 0 (so no sum is formed) are the registers re-scanned for
// NaN, which keeps NaN ahead of Inf.
template <typename T, int N>
__device__ __forceinline__ Pair<T> registers_to_pair(const T (&v)[N]) {
  T m = T(0);
#pragma unroll
  for (int i = 0; i < N; ++i) m = dmax(m, dabs(v[i]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = dmax(m, __shfl_xor(m, o, 64));
  if (isinf(m) || m == T(0)) {
    bool nan = false;
#pragma unroll
    for (int i = 0; i < N; ++i) nan = nan || isnan(v[i]);
    nan = __any(nan);
    if (nan) return {T(NAN), T(0)};
    return isinf(m) ? Pair<T>{T(INFINITY), T(0)} : Pair<T>{T(-INFINITY), T(0)};
  }
  const int e = dexponent(m);
  T t = T(0);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const T s = dldexp(v[i], -e);
    t = dfma(s, s, t);
  }
  t = hpd::wave_sum(t);
  if (isnan(t)) return {T(NAN), T(0)};
  return {T(e), t};
}

// Contiguous rows, persistent: wave w of the grid handles units (row, chunk)
// w, w + W, w + 2W, ... (W waves in the grid), so each round of the grid reads
// one contiguous stretch of memory. Modes:
//   kFinal   one chunk per row: write the row's norm;
//   kPairs   several rows of several chunks: one pair per unit;
//   kRunning a single row: every wave folds its chunks into a running pair
//            and each workgroup writes one pair (few pairs left to merge).
constexpr int kFinal = 0, kPairs = 1, kRunning = 2;

template <typename T, bool kVector, int MODE>
__global__ __launch_bounds__(kBlock) void norm_rows_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                           int64_t outer, int64_t reduced, int64_t chunks) {
  using V = typename Traits<T>::V;
  constexpr int W = Traits<T>::width;
  constexpr int N = kLoads * W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t units = outer * chunks;
  const int64_t stride = int64_t(gridDim.x) * (kBlock / 64);
  Pair<T> running = {T(-INFINITY), T(0)};
  for (int64_t g = int64_t(blockIdx.x) * (kBlock / 64) + wave; g < units; g += stride) {
    const int64_t o = g / chunks, ch = g - o * chunks;
    const int64_t begin = ch * chunk_len<T>();
    const int64_t len = reduced - begin < chunk_len<T>() ? reduced - begin : chunk_len<T>();
    const T* base = x + o * reduced + begin;
    T v[N];
    if (kVector && len == chunk_len<T>()) {
      const V* bv = reinterpret_cast<const V*>(base);
      V q[kLoads];
#pragma unroll
      for (int i = 0; i < kLoads; ++i) q[i] = __builtin_nontemporal_load(bv + i * 64 + lane);
#pragma unroll
      for (int i = 0; i < kLoads; ++i)
#pragma unroll
        for (int w = 0; w < W; ++w) v[i * W + w] = q[i][w];
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int64_t e = int64_t(i) * 64 + lane;
        v[i] = e < len ? base[e] : T(0);
      }
    }
    const Pair<T> p = registers_to_pair<T, N>(v);
    if (MODE == kRunning) {
      running = merge(running, p);
    } else if (lane == 0) {
      if (MODE == kFinal) {
        out[o] = finish(p);
      } else {
        out[2 * g] = p.k;
        out[2 * g + 1] = p.t;
      }
    }
  }
  if (MODE == kRunning) {
    __shared__ T ks[kBlock / 64], ts[kBlock / 64];
    if (lane == 0) {
      ks[wave] = running.k;
      ts[wave] = running.t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      Pair<T> total = {ks[0], ts[0]};
      for (int w = 1; w < kBlock / 64; ++w) total = merge(total, Pair<T>{ks[w], ts[w]});
      out[2 * blockIdx.x] = total.k;
      out[2 * blockIdx.x + 1] = total.t;
    }
  }
}

// Pair merge pass: workgroup g merges pairs [c*kMerge, (c+1)*kMerge) of row
// o = g / groups_out (c = g % groups_out) into one pair, or, in the last pass,
// into the row's final norm. Passes repeat until one pair per row remains.
constexpr int64_t kMerge = 4096;

template <typename T>
__global__ __launch_bounds__(kBlock) void norm_merge_kernel(const T* __restrict__ pairs, T* __restrict__ out,
                                                            int64_t chunks, int64_t groups_out, bool final) {
  __shared__ T ks[kBlock / 64], ts[kBlock / 64];
  const int64_t g = blockIdx.x;
  const int64_t o = g / groups_out, c = g - o * groups_out;
  const int64_t begin = c * kMerge;
  const int64_t end = begin + kMerge < chunks ? begin + kMerge : chunks;
  const T* row = pairs + 2 * o * chunks;
  // All of a thread's pairs are loaded before any merge: one memory round
  // trip instead of one per pair (this kernel is latency-bound).
  constexpr int kPer = int(kMerge / kBlock);
  typedef T T2 __attribute__((ext_vector_type(2)));
  T2 q[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int64_t i = begin + threadIdx.x + int64_t(j) * kBlock;
    q[j] = i < end ? *reinterpret_cast<const T2*>(row + 2 * i) : T2{T(-INFINITY), T(0)};
  }
  Pair<T> p = {T(-INFINITY), T(0)};
#pragma unroll
  for (int j = 0; j < kPer; ++j) p = merge(p, Pair<T>{q[j][0], q[j][1]});
  p = wave_merge(p);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    ks[wave] = p.k;
    ts[wave] = p.t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Pair<T> total = {ks[0], ts[0]};
    for (int w = 1; w < kBlock / 64; ++w) total = merge(total, Pair<T>{ks[w], ts[w]});
    if (final) {
      out[o] = finish(total);
    } else {
      out[2 * g] = total.k;
      out[2 * g + 1] = total.t;
    }
  }
}

// Strided reduction axis (inner > 1): the column engine of strided.h with
// per-column pairs. A thread loads kBatch rows of its column into registers
// and forms their pair exactly as a wave does for a contiguous chunk (max,
// exponent, scaled sum of squares), so every element is read from HBM once;
// pairs then merge across batches, rows of a step, chunks and passes.
// Branch-free: the NaN-dropping max gives the scale; the scaled sum of
// squares is formed whatever the max, and a NaN anywhere makes it NaN (for a
// max of +inf the +inf squares stay +inf, for a max of 0 the other values are
// zeros), so a NaN sum marks NaN, then a max of +inf or 0 the infinite or the
// zero pair. frexp of +inf or 0 only feeds sums that these cases discard.
template <typename T>
__device__ __forceinline__ Pair<T> lane_pair(const T* v, int n) {
  T m = T(0);
  for (int i = 0; i < n; ++i) m = dmax(m, dabs(v[i]));
  const int e = dexponent(m);
  T t = T(0);
  for (int i = 0; i < n; ++i) {
    const T s = dldexp(v[i], -e);
    t = dfma(s, s, t);
  }
  if (isnan(t)) return {T(NAN), T(0)};
  if (isinf(m)) return {T(INFINITY), T(0)};
  return m == T(0) ? Pair<T>{T(-INFINITY), T(0)} : Pair<T>{T(e), t};
}

template <typename T>
struct NormColumns {
  using In = T;
  using Acc = Pair<T>;
  using Out = T;
  // Pairs of 8 rows: 1 GiB float32 axis 0 at 82% of HBM against 80% with 16
  // (the first pass streams from 2 workgroups per compute unit either way;
  // 3 or 4 measured 78% / 77%).
  static constexpr int kBatch = 8;
  __device__ static T identity_in() { return T(0); }  // a zero adds nothing to a pair
  __device__ static Pair<T> identity() { return {T(-INFINITY), T(0)}; }
  __device__ static Pair<T> fold(Pair<T> acc, const T (&v)[kBatch]) {
    return merge(acc, lane_pair<T>(v, kBatch));
  }
  __device__ static Pair<T> combine(Pair<T> a, Pair<T> b) { return merge(a, b); }
  __device__ static T finish(Pair<T> p) { return ::finish(p); }
};

template <typename T>
struct NormPairColumns {
  using In = Pair<T>;
  using Acc = Pair<T>;
  using Out = T;
  static constexpr int kBatch = 8;
  __device__ static Pair<T> identity_in() { return {T(-INFINITY), T(0)}; }
  __device__ static Pair<T> identity() { return {T(-INFINITY), T(0)}; }
  __device__ static Pair<T> fold(Pair<T> acc, const Pair<T> (&v)[kBatch]) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) acc = merge(acc, v[j]);
    return acc;
  }
  __device__ static Pair<T> combine(Pair<T> a, Pair<T> b) { return merge(a, b); }
  __device__ static T finish(Pair<T> p) { return ::finish(p); }
};

template <typename T>
hps::Plan plan_cols(hp_ctx* ctx, const T* x, int64_t outer, int64_t reduced, int64_t inner) {
  const int v_in = hps::vector_width(x, inner, sizeof(T));
  const int v_acc = hps::vector_width(reinterpret_cast<const void*>(256), inner, sizeof(Pair<T>));
  // 2 workgroups per compute unit: 1 GiB float32 axis 0 at 68% of HBM against
  // 64% at 4 (one MI355X).
  return hps::plan(outer, reduced, inner, v_in, v_acc, sizeof(Pair<T>), ctx->compute_units, 2);
}

template <typename T>
void run_cols(hp_ctx* ctx, const hps::Plan& plan, const T* x, T* out, int64_t outer, int64_t reduced,
              int64_t inner, void* const buffers[2]) {
  constexpr int v_in = sizeof(T) == 4 ? 4 : 2;
  constexpr int v_acc = sizeof(Pair<T>) == 8 ? 2 : 1;
  hps::execute<NormColumns<T>, NormPairColumns<T>, v_in, v_acc>(ctx->stream, plan, x, out, outer, reduced, inner,
                                                                 buffers);
}

// Temporary device memory of one norm call: the pair buffer the row pass
// writes (`first` bytes) and the output of the first of two or more merge
// passes (`second` bytes). Later merge passes alternate between the two: a
// pass only reads the buffer the previous pass wrote.
struct Workspace {
  void* first = nullptr;
  void* second = nullptr;
};

struct RowPlan {
  int mode = kFinal;
  bool vector = false;
  int64_t chunks = 0, grid = 0;
  int64_t pairs = 0;   // pairs the row pass writes (0 in kFinal mode)
  int64_t second = 0;  // pairs the first merge pass writes when it is not the last
};

template <typename T>
RowPlan plan_rows(hp_ctx* ctx, const T* x, int64_t outer, int64_t reduced) {
  RowPlan plan;
  plan.chunks = hp::ceil_div(reduced, chunk_len<T>());
  const int64_t units = outer * plan.chunks;
  plan.vector = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (reduced * int64_t(sizeof(T))) % 16 == 0;
  plan.mode = plan.chunks == 1 ? kFinal : (outer == 1 ? kRunning : kPairs);
  // Enough resident waves to keep HBM busy; the grid loops over the rest.
  const int64_t resident = int64_t(ctx->compute_units) * kResidentGroupsPerCU;
  plan.grid = hp::ceil_div(units, kBlock / 64);
  if (plan.grid > resident) plan.grid = resident;
  if (plan.mode != kFinal) {
    const int64_t per_row = plan.mode == kRunning ? plan.grid : plan.chunks;
    plan.pairs = plan.mode == kRunning ? plan.grid : units;
    const int64_t groups = hp::ceil_div(per_row, kMerge);
    plan.second = groups > 1 ? outer * groups : 0;
  }
  return plan;
}

template <typename T>
void run_rows(hp_ctx* ctx, const RowPlan& plan, const T* x, T* out, int64_t outer, int64_t reduced,
              Workspace ws) {
  const int64_t grid = plan.grid, chunks = plan.chunks;
  T* target = plan.mode == kFinal ? out : static_cast<T*>(ws.first);
#define PACHO_NORM_LAUNCH(VEC, MODE_)                                                                           \
  norm_rows_kernel<T, VEC, MODE_><<<grid, kBlock, 0, ctx->stream>>>(x, target, outer, reduced, chunks)
  if (plan.vector) {
    if (plan.mode == kFinal) PACHO_NORM_LAUNCH(true, kFinal);
    else if (plan.mode == kRunning) PACHO_NORM_LAUNCH(true, kRunning);
    else PACHO_NORM_LAUNCH(true, kPairs);
  } else {
    if (plan.mode == kFinal) PACHO_NORM_LAUNCH(false, kFinal);
    else if (plan.mode == kRunning) PACHO_NORM_LAUNCH(false, kRunning);
    else PACHO_NORM_LAUNCH(false, kPairs);
  }
#undef PACHO_NORM_LAUNCH
  hp::check_launch("norm_rows");
  if (plan.mode == kFinal) return;
  // Pair modes always finish with at least one merge pass (it writes `out`).
  T* source = static_cast<T*>(ws.first);
  T* spare = static_cast<T*>(ws.second);
  int64_t remaining = plan.mode == kRunning ? grid : chunks;
  for (;;) {
    const int64_t groups = hp::ceil_div(remaining, kMerge);
    const bool last = groups == 1;
    T* next = last ? out : spare;
    hp::require(outer * groups <= hp::kMaxGrid, "too many rows for one launch");
    norm_merge_kernel<T><<<outer * groups, kBlock, 0, ctx->stream>>>(source, next, remaining, groups, last);
    hp::check_launch("norm_merge");
    if (last) return;
    spare = source;
    source = next;
    remaining = groups;
  }
}

// hp_norm: the workspace comes from the context's stream-ordered pool and goes
// back to it as soon as the launches that use it are queued.
template <typename T>
void run_norm(hp_ctx* ctx, const T* x, T* out, int64_t outer, int64_t reduced, int64_t inner) {
  if (inner > 1) {
    const hps::Plan plan = plan_cols<T>(ctx, x, outer, reduced, inner);
    void* buffers[2] = {nullptr, nullptr};
    for (int i = 0; i < 2; ++i)
      if (plan.bytes[i] > 0) buffers[i] = hp::scratch_alloc(ctx, plan.bytes[i]);
    run_cols<T>(ctx, plan, x, out, outer, reduced, inner, buffers);
    for (int i = 0; i < 2; ++i)
      if (buffers[i]) hp::scratch_free(ctx, buffers[i]);
    return;
  }
  const RowPlan plan = plan_rows<T>(ctx, x, outer, reduced);
  Workspace ws;
  if (plan.pairs > 0) ws.first = hp::scratch_alloc(ctx, size_t(plan.pairs) * 2 * sizeof(T));
  if (plan.second > 0) ws.second = hp::scratch_alloc(ctx, size_t(plan.second) * 2 * sizeof(T));
  run_rows<T>(ctx, plan, x, out, outer, reduced, ws);
  if (ws.second) hp::scratch_free(ctx, ws.second);
  if (ws.first) hp::scratch_free(ctx, ws.first);
}

// ---- allocation-free variant ---------------------------------------------
//
// hp_norm_noalloc keeps its workspace in `scratch`, a fixed device array that
// every GPU the library runs on holds until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for
// the symbol): the device address comes from hipGetSymbolAddress, looked up
// once per device with that device current, and only that address is used.

constexpr size_t kAlign = 256;
inline size_t align_up(size_t bytes) { return (bytes + kAlign - 1) / kAlign * kAlign; }

template <typename T>
__global__ __launch_bounds__(kBlock) void zero_kernel(T* __restrict__ out, int64_t count) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) out[i] = T(0);
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[HP_NORM_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mutex;
std::unordered_map<int, void*> g_scratch_address;  // device -> address of `scratch`

// Device address of `scratch` on ctx->device (current after hp::enter).
void* scratch_address(hp_ctx* ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  auto found = g_scratch_address.find(ctx->device);
  if (found != g_scratch_address.end()) return found->second;
  void* address = nullptr;
  HP_CHECK(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
  hp::require(address != nullptr && reinterpret_cast<uintptr_t>(address) % kAlign == 0,
              "scratch symbol has no aligned device address");
  g_scratch_address.emplace(ctx->device, address);
  return address;
}

// Both workspace halves inside the static array, or a clear error.
void check_scratch(size_t first, size_t second) {
  if (first + second > HP_NORM_NOALLOC_SCRATCH_BYTES) {
    hp::fail(HP_E_INVALID, "hp_norm_noalloc: this shape needs " + std::to_string(first + second) +
                               " bytes of workspace, more than the " +
                               std::to_string(HP_NORM_NOALLOC_SCRATCH_BYTES) +
                               "-byte static scratch; call hp_norm");
  }
}

template <typename T>
void run_norm_noalloc(hp_ctx* ctx, const T* x, T* out, int64_t outer, int64_t reduced, int64_t inner) {
  if (inner > 1) {
    const hps::Plan plan = plan_cols<T>(ctx, x, outer, reduced, inner);
    const size_t first = align_up(plan.bytes[0]);
    check_scratch(first, plan.bytes[1]);
    void* buffers[2] = {nullptr, nullptr};
    if (first + plan.bytes[1] > 0) {
      char* base = static_cast<char*>(scratch_address(ctx));
      buffers[0] = base;
      buffers[1] = base + first;
    }
    return run_cols<T>(ctx, plan, x, out, outer, reduced, inner, buffers);
  }
  const RowPlan plan = plan_rows<T>(ctx, x, outer, reduced);
  const size_t first = align_up(size_t(plan.pairs) * 2 * sizeof(T));
  const size_t second = size_t(plan.second) * 2 * sizeof(T);
  check_scratch(first, second);
  Workspace ws;
  if (first + second > 0) {
    char* base = static_cast<char*>(scratch_address(ctx));
    ws.first = base;
    ws.second = base + first;
  }
  run_rows<T>(ctx, plan, x, out, outer, reduced, ws);
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

int hp_norm(hp_ctx* ctx, int dtype, const void* x, void* out, int64_t outer, int64_t reduced, int64_t inner) {
  return guarded([&] {
    hp::enter(ctx);
    require(dtype == HP_F32 || dtype == HP_F64, "norm supports float32 and float64");
    require(outer >= 0 && reduced >= 0 && inner >= 0, "negative extent");
    const int64_t count = outer * inner;
    if (count == 0) return;
    require(out != nullptr, "null output");
    if (reduced == 0) {
      HP_CHECK(hipMemsetAsync(out, 0, size_t(count) * hp::dtype_size(dtype), ctx->stream));
      return;
    }
    require(x != nullptr, "null input");
    if (dtype == HP_F32) {
      run_norm<float>(ctx, (const float*)x, (float*)out, outer, reduced, inner);
    } else {
      run_norm<double>(ctx, (const double*)x, (double*)out, outer, reduced, inner);
    }
  });
}

int hp_norm_noalloc(hp_ctx* ctx, int dtype, const void* x, void* out, int64_t outer, int64_t reduced,
                    int64_t inner) {
  return guarded([&] {
    hp::enter(ctx);
    require(dtype == HP_F32 || dtype == HP_F64, "norm supports float32 and float64");
    require(outer >= 0 && reduced >= 0 && inner >= 0, "negative extent");
    const int64_t count = outer * inner;
    if (count == 0) return;
    require(out != nullptr, "null output");
    if (reduced == 0) {
      // A fill kernel rather than hipMemsetAsync, so the call can be captured.
      int64_t grid = hp::ceil_div(count, kBlock);
      if (grid > 65536) grid = 65536;
      if (dtype == HP_F32) zero_kernel<float><<<grid, kBlock, 0, ctx->stream>>>((float*)out, count);
      else zero_kernel<double><<<grid, kBlock, 0, ctx->stream>>>((double*)out, count);
      hp::check_launch("norm_zero");
      return;
    }
    require(x != nullptr, "null input");
    if (dtype == HP_F32) {
      run_norm_noalloc<float>(ctx, (const float*)x, (float*)out, outer, reduced, inner);
    } else {
      run_norm_noalloc<double>(ctx, (const double*)x, (double*)out, outer, reduced, inner);
    }
  });
}

}  // extern "C"
