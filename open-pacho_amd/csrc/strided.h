// Reductions over a strided axis: x viewed as (outer, reduced, inner) with
// inner > 1, out[o*inner + i] = op over r of x[(o*reduced + r)*inner + i].
//
// Work split (reference _cuda.py:449-491 splits any reduced axis into
// fixed-size chunks, one block each; this is the same idea laid out for
// lanes on adjacent columns):
//   - a workgroup of 256 threads owns a column block and a chunk of rows of
//     one outer index; thread t reads columns (cg*V .. cg*V+V-1) of the block
//     (cg = t % cw) in rows ro, ro + S, ro + 2S, ... of the chunk
//     (ro = t / cw, S = 256 / cw rows per step). A narrow axis (inner < 256*V)
//     packs S > 1 rows into one step, so each step of the workgroup reads one
//     contiguous run of S*inner elements; a wide axis reads one 256*V-column
//     stretch of a row per step. V = 16 bytes / element when rows are 16-byte
//     aligned, else 1;
//   - each thread folds its rows in ascending order, batches of kBatch rows
//     at a time (loads issued before the fold), then the S partials of one
//     column combine in LDS by a fixed pairwise tree over ro;
//   - a chunk's result per column goes to a partial array (outer, chunks,
//     inner) of accumulators, which the next pass reduces the same way, until
//     one chunk remains. Every order is fixed, so results repeat bit for bit.
// An axis too short to fill a workgroup's rows (reduced < S/2) is reduced by
// one thread per output instead.
#pragma once

#include "common.h"

namespace hps {

constexpr int kThreads = 256;

// Op contract (all __device__ static):
//   In identity_in()               value of a row past the end of the chunk
//   Acc identity()                 accumulator of no rows
//   Acc fold(Acc, const In (&)[B]) fold B rows of one column, ascending
//   Acc combine(Acc a, Acc b)      a then b (fixed order)
//   Out finish(Acc)                final value of a column
// with types In, Acc, Out and the batch size kBatch.

// STREAM: nontemporal loads (a first pass over HBM data read once). A
// compile-time choice: a runtime select between the two load forms compiled
// to plain loads.
template <typename In, int V, bool STREAM>
__device__ __forceinline__ void load_row(const In* p, In (&v)[V]) {
  if constexpr (V > 1) {
    static_assert(sizeof(In) * V == 16, "vector loads are 16 bytes");
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    U4 bits;
    if constexpr (STREAM) bits = __builtin_nontemporal_load(reinterpret_cast<const U4*>(p));
    else bits = *reinterpret_cast<const U4*>(p);
    __builtin_memcpy(&v[0], &bits, 16);
  } else if constexpr (STREAM) {
    v[0] = __builtin_nontemporal_load(p);
  } else {
    v[0] = *p;
  }
}

template <class Op, int V, bool STREAM>
__global__ __launch_bounds__(kThreads) void strided_kernel(const typename Op::In* __restrict__ x, void* __restrict__ out,
                                                           int64_t reduced, int64_t inner, int64_t col_blocks,
                                                           int64_t chunks, int64_t rows_per_chunk, int cw,
                                                           int final_pass) {
  using In = typename Op::In;
  using Acc = typename Op::Acc;
  constexpr int B = Op::kBatch;
  __shared__ Acc lds[kThreads * V];
  const int tid = threadIdx.x;
  const int step = kThreads / cw;
  const int ro = tid / cw, cg = tid - ro * cw;
  int64_t b = blockIdx.x;
  const int64_t ch = b % chunks;
  b /= chunks;
  const int64_t cb = b % col_blocks, o = b / col_blocks;
  const int64_t col = (cb * cw + cg) * V;
  const bool active = ro < step && col < inner;
  Acc acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = Op::identity();
  if (active) {
    const int64_t begin = ch * rows_per_chunk;
    const int64_t end = begin + rows_per_chunk < reduced ? begin + rows_per_chunk : reduced;
    const In* base = x + o * reduced * inner + col;
    int64_t r = begin + ro;
    // Full batches, in ascending order, two register sets that swap roles:
    // the next batch's loads are issued before this one is folded. No exit
    // branch sits between a load and its fold: the loop takes batches in
    // pairs with its test at the bottom, and an odd last batch is folded
    // after it. (With an exit between them the compiler sank the lookahead
    // loads below the fold, or waited for every load before each fold.)
    // The lookahead of the last pair reloads the last batch, unused.
    // The fence keeps the scheduler from spreading a batch's loads among
    // the fold's instructions, which left half as many loads in flight.
    auto load = [&](int64_t row, In (&vals)[B][V]) {
#pragma unroll
      for (int j = 0; j < B; ++j) load_row<In, V, STREAM>(base + (row + int64_t(j) * step) * inner, vals[j]);
      __builtin_amdgcn_sched_barrier(0);
    };
    auto fold = [&](const In (&vals)[B][V]) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        In column[B];
#pragma unroll
        for (int j = 0; j < B; ++j) column[j] = vals[j][v];
        acc[v] = Op::fold(acc[v], column);
      }
    };
    const int64_t rows = r < end ? (end - r + step - 1) / step : 0;
    const int64_t batches = rows / B, stride = int64_t(B) * step;
    if (batches > 0) {
      const int64_t last = r + (batches - 1) * stride;
      In set0[B][V], set1[B][V];
      load(r, set0);
      for (int64_t i = 0; i + 1 < batches; i += 2) {
        load(r + stride, set1);
        fold(set0);
        load(r + 2 * stride < last ? r + 2 * stride : last, set0);
        fold(set1);
        r += 2 * stride;
      }
      if (batches & 1) {
        fold(set0);
        r += stride;
      }
    }
    if (r < end) {  // last partial batch: rows past the end read as identity
      In vals[B][V];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int64_t row = r + int64_t(j) * step;
        if (row < end) {
          load_row<In, V, STREAM>(base + row * inner, vals[j]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) vals[j][v] = Op::identity_in();
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        In column[B];
#pragma unroll
        for (int j = 0; j < B; ++j) column[j] = vals[j][v];
        acc[v] = Op::fold(acc[v], column);
      }
    }
  }
  if (step > 1) {
    // Pairwise tree over the rows of one step, in a fixed order.
#pragma unroll
    for (int v = 0; v < V; ++v) lds[tid * V + v] = acc[v];
    __syncthreads();
    for (int n = step; n > 1;) {
      const int half = (n + 1) / 2;
      if (ro < n - half) {
#pragma unroll
        for (int v = 0; v < V; ++v)
          lds[tid * V + v] = Op::combine(lds[tid * V + v], lds[(tid + half * cw) * V + v]);
      }
      __syncthreads();
      n = half;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = lds[tid * V + v];
  }
  if (ro != 0 || col >= inner) return;
  if (final_pass) {
    typename Op::Out* dst = static_cast<typename Op::Out*>(out) + o * inner + col;
#pragma unroll
    for (int v = 0; v < V; ++v) dst[v] = Op::finish(acc[v]);
  } else {
    Acc* dst = static_cast<Acc*>(out) + (o * chunks + ch) * inner + col;
#pragma unroll
    for (int v = 0; v < V; ++v) dst[v] = acc[v];
  }
}

// Short axes: one thread per output, rows in ascending order.
template <class Op>
__global__ __launch_bounds__(kThreads) void per_output_kernel(const typename Op::In* __restrict__ x,
                                                              typename Op::Out* __restrict__ out, int64_t outer,
                                                              int64_t reduced, int64_t inner) {
  using In = typename Op::In;
  constexpr int B = Op::kBatch;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t g = int64_t(blockIdx.x) * kThreads + threadIdx.x; g < outer * inner; g += stride) {
    const int64_t o = g / inner, i = g - o * inner;
    const In* base = x + o * reduced * inner + i;
    typename Op::Acc acc = Op::identity();
    for (int64_t r = 0; r < reduced; r += B) {
      In column[B];
#pragma unroll
      for (int j = 0; j < B; ++j) column[j] = r + j < reduced ? base[(r + j) * inner] : Op::identity_in();
      acc = Op::fold(acc, column);
    }
    out[g] = Op::finish(acc);
  }
}

struct Pass {
  int V = 1, cw = 1;
  int64_t reduced = 0, col_blocks = 0, chunks = 1, rows_per_chunk = 0;
};

struct Plan {
  bool per_output = false;
  int count = 0;
  Pass passes[12];
  size_t bytes[2] = {0, 0};  // partial buffers: even passes write [0], odd [1]
};

// Rows per thread of a chunk: the first pass reads HBM once, so each thread
// gets at least kFirstRows rows to keep loads in flight; merge passes read
// small partial arrays and take long chunks, so that few passes remain.
constexpr int64_t kFirstRows = 16;
constexpr int64_t kMergeRows = 32;
// Workgroups the merge passes aim for per compute unit; the first pass takes
// its own figure from the caller (the op's fold cost decides: a cheap fold
// runs best with few long chunks, an expensive one with more, shorter ones).
constexpr int64_t kGroupsPerCU = 4;
// The first pass's partial array is kept below this size by using fewer,
// longer chunks; this also bounds the static workspace of allocation-free
// callers.
constexpr int64_t kMaxPartialBytes = int64_t(8) << 20;

// A merge pass over at most kThreads * kOnePassRows rows finishes in one
// launch: its column blocks narrow (cw threads across, kThreads / cw rows per
// step) until each thread folds at most kOnePassRows rows, and the rows of
// one step meet in the LDS tree. Two launches of full-width blocks took 9-11
// us after a 1 GiB axis-0 pass, one narrow launch about half of that (16
// rows per thread against 32: the norm's pair merges +0.5% of HBM).
constexpr int64_t kOnePassRows = 16;

inline Pass plan_pass(int64_t outer, int64_t reduced, int64_t inner, int V, int64_t groups_wanted,
                      int64_t min_rows, int64_t acc_bytes, bool cap_partials, bool one_pass = false) {
  Pass p;
  p.V = V;
  p.reduced = reduced;
  const int64_t groups = hp::ceil_div(inner, V);
  int64_t cw = groups < kThreads ? groups : kThreads;
  if (one_pass) {
    const int64_t cap = kThreads / hp::ceil_div(reduced, kOnePassRows);  // >= 1 by the caller's bound
    while (cw > cap) cw = (cw + 1) / 2;
  }
  p.cw = int(cw);
  p.col_blocks = hp::ceil_div(groups, p.cw);
  const int64_t step = kThreads / p.cw;
  if (one_pass) {
    p.rows_per_chunk = hp::ceil_div(reduced, step) * step;
    p.chunks = 1;
    return p;
  }
  const int64_t blocks = outer * p.col_blocks;
  int64_t chunks = groups_wanted / blocks;
  if (chunks < 1) chunks = 1;
  int64_t rows = hp::ceil_div(reduced, chunks);
  if (rows < step * min_rows) rows = step * min_rows;
  if (cap_partials) {
    const int64_t per_chunk = outer * inner * acc_bytes;
    const int64_t max_chunks = kMaxPartialBytes / per_chunk > 1 ? kMaxPartialBytes / per_chunk : 1;
    const int64_t min_rows_cap = hp::ceil_div(reduced, max_chunks);
    if (rows < min_rows_cap) rows = min_rows_cap;
  }
  rows = hp::ceil_div(rows, step) * step;
  p.rows_per_chunk = rows;
  p.chunks = hp::ceil_div(reduced, rows);
  return p;
}

// Plans every pass of one strided reduction. `in_bytes`, `acc_bytes`: element
// sizes of the input and of the accumulator; V_in / V_acc: vector widths the
// first and the merge passes may use (1 if the rows are not 16-byte aligned).
inline Plan plan(int64_t outer, int64_t reduced, int64_t inner, int V_in, int V_acc, int64_t acc_bytes,
                 int64_t compute_units, int64_t first_groups_per_cu) {
  Plan plan;
  const int64_t cw0 = hp::ceil_div(inner, V_in) < kThreads ? hp::ceil_div(inner, V_in) : kThreads;
  if (reduced * 2 < kThreads / cw0) {
    plan.per_output = true;
    return plan;
  }
  int64_t rows = reduced;
  for (;;) {
    const bool first = plan.count == 0;
    const bool one_pass = !first && rows <= kThreads * kOnePassRows;
    Pass p = plan_pass(outer, rows, inner, first ? V_in : V_acc,
                       compute_units * (first ? first_groups_per_cu : kGroupsPerCU), first ? kFirstRows : kMergeRows,
                       acc_bytes, first, one_pass);
    hp::require(plan.count < 12, "strided reduction needs too many passes");
    hp::require(outer * p.col_blocks * p.chunks <= hp::kMaxGrid, "strided reduction too large for one launch");
    plan.passes[plan.count] = p;
    if (p.chunks > 1) {
      const size_t bytes = size_t(outer) * size_t(p.chunks) * size_t(inner) * size_t(acc_bytes);
      size_t& slot = plan.bytes[plan.count % 2];
      if (bytes > slot) slot = bytes;
    }
    ++plan.count;
    if (p.chunks == 1) return plan;
    rows = p.chunks;
  }
}

// Vector width for 16-byte loads of `elem`-byte elements (4 or 8 bytes; other
// sizes load one element per thread) from rows of `inner` elements starting at
// `base`.
inline int vector_width(const void* base, int64_t inner, int64_t elem) {
  if (elem != 4 && elem != 8) return 1;
  const int V = int(16 / elem);
  if (inner % V != 0 || reinterpret_cast<uintptr_t>(base) % 16 != 0) return 1;
  return V;
}

template <class Op, int V, bool STREAM>
void launch_pass(hipStream_t stream, const Pass& p, const void* in, void* out, int64_t outer, int64_t inner,
                 bool final_pass) {
  const int64_t grid = outer * p.col_blocks * p.chunks;
  strided_kernel<Op, V, STREAM><<<grid, kThreads, 0, stream>>>(static_cast<const typename Op::In*>(in), out,
                                                               p.reduced, inner, p.col_blocks, p.chunks,
                                                               p.rows_per_chunk, p.cw, final_pass ? 1 : 0);
  hp::check_launch("strided_reduce");
}

// Runs a plan: pass 0 reads x with FirstOp (vector width V_first), later
// passes read the previous partial array with MergeOp. buffers[0]/[1] hold
// at least plan.bytes[0]/[1].
template <class FirstOp, class MergeOp, int V_first, int V_merge>
void execute(hipStream_t stream, const Plan& plan, const typename FirstOp::In* x, typename FirstOp::Out* out,
             int64_t outer, int64_t reduced, int64_t inner, void* const buffers[2]) {
  static_assert(sizeof(typename FirstOp::Acc) == sizeof(typename MergeOp::In), "partials feed the merge op");
  if (plan.per_output) {
    int64_t grid = hp::ceil_div(outer * inner, kThreads);
    if (grid > 65536 * 4) grid = 65536 * 4;
    per_output_kernel<FirstOp><<<grid, kThreads, 0, stream>>>(x, out, outer, reduced, inner);
    hp::check_launch("strided_per_output");
    return;
  }
  const void* source = x;
  for (int i = 0; i < plan.count; ++i) {
    const Pass& p = plan.passes[i];
    const bool final_pass = i == plan.count - 1;
    void* target = final_pass ? static_cast<void*>(out) : buffers[i % 2];
    if (i == 0) {
      if (p.V == V_first && V_first > 1) launch_pass<FirstOp, V_first, true>(stream, p, source, target, outer, inner, final_pass);
      else launch_pass<FirstOp, 1, true>(stream, p, source, target, outer, inner, final_pass);
    } else {
      if (p.V == V_merge && V_merge > 1) launch_pass<MergeOp, V_merge, false>(stream, p, source, target, outer, inner, final_pass);
      else launch_pass<MergeOp, 1, false>(stream, p, source, target, outer, inner, final_pass);
    }
    source = target;
  }
}

}  // namespace hps
