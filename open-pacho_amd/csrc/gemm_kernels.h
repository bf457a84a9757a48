// MFMA GEMM for gfx950: C[b] = A[b'] @ B[b''] in fp32 and fp64.
//
// fp32: v_mfma_f32_16x16x4_f32 (measured 155 TFLOP/s peak on MI355X, against
// 137 for the 32x32x2 form). Workgroup tile 256x256x16, eight waves in a 2x4
// grid, each wave 128x64 (8x4 MFMA blocks, 128 accumulators per lane); one
// workgroup per compute unit. Against a 256x128 tile at two workgroups per CU
// this halves the global/L2 -> LDS traffic per flop (measured +4% of peak).
// fp64: v_mfma_f64_16x16x4_f64, workgroup tile 256x128x16, eight waves in a
// 4x2 grid of 64x64 wave tiles, one workgroup per compute unit.
//
// Data path per K slice: global -> registers (prefetched ahead) -> LDS
// (double-buffered, one barrier per slice) -> 16-byte LDS reads -> MFMA. LDS
// holds both operands k-contiguous: A as [m][k] (a copy of a row-major tile)
// and B as [n][k] (each lane loads one column's k values as scalars, so the
// transposition costs no shuffles). A lane of MFMA lane group g = lane/16
// then reads four consecutive k values with one ds_read_b128 and feeds them to
// four MFMAs, i.e. MFMA number q contracts k = {q, 4+q, 8+q, 12+q}; A and B
// use the same permutation, so every product of the slice is summed exactly
// once.
//
// Schedule. Tiles are numbered batch-major and, inside a batch, in groups of
// kGroupM tile rows, so neighbouring tiles share A and B panels. Whole rounds
// of resident workgroups (compute units x workgroups per CU) each take one
// tile and its full K range; workgroup ids are renumbered so each XCD (ids
// i % 8) owns a contiguous range of tiles and its L2 sees shared panels. The
// tiles of a last, partly filled round are instead cut into equal runs of K
// slices over every resident slot (stream-K): a worker's run covers the end
// of one tile and the start of the next, and every cut piece goes to a
// workspace. A second kernel adds the pieces of each cut tile in K order, so
// results are deterministic. Without this, e.g. 153 tiles on 256 compute units
// leave 103 of them idle for the whole product.
//
// Modes: 0 = interior (no guards; M, N, K multiples of the tile), 1 = M/N
// edges (K a multiple of 16): edge rows and columns load clamped addresses
// and only the stores are masked, since they feed no stored output; 2 = any
// K: as 1, plus the one slice holding the K edge takes scalar loads that
// zero-fill past K, so it contracts against +0 padding. A rows are read as
// 16-byte vectors at element alignment (odd K included).
//
// Reference semantics: _gemm.py:24-137 (per-batch broadcast offsets
// _offset :13-21, never reads C), _cuda.py:493-518 and :619-636.
// (Device code and host launch templates; included by the gemm_<dtype>_<layout>
// translation units only.)
#pragma once

#include <algorithm>
#include <type_traits>

#include "gemm.h"

#include <vector>

namespace {

using hpgemm::BatchDesc;

struct TileMap {
  int64_t tiles_m, tiles_n, tiles_per_batch, total;
  // Leading dimensions (elements) of A's and B's storage and of C. A product
  // over a sub-block of larger matrices (the edge split of run_f32) reads and
  // writes with the full matrices' row lengths; otherwise lda = K or M,
  // ldb = N or K and ldc = N.
  int64_t lda, ldb, ldc;
};

// Division of the tile space between whole-tile workgroups and stream-K
// workers. Logical tiles [0, dp_tiles) run whole; the K slices of tiles
// [dp_tiles, total) are dealt out in consecutive runs, worker w owning
// base + (w < extra) slices starting at sk_begin(w).
struct Split {
  int64_t dp_tiles;
  int64_t workers;
  int64_t base, extra;
  int64_t slices;  // K slices per tile
  void* partial;   // [workers][2][tile elements]: a worker's first and last cut piece
  int moved;       // edge tiles were computed at tile_origin() (the fixup stores alike)
};

// Tile rows per group. An XCD's 32 compute units run 32 consecutive tiles
// at a time: a 4 x 8 block of tiles, whose A and B panels per K slice its L2
// fetches once. For the 2:1 tiles (256 x 128, fp64's 256 x 128) that is 20%
// fewer bytes than an 8 x 4 block (4097 x 3001 x 2049: 251 -> 201 MB of
// fetches per product), the same for square tiles, and batches of grids four
// tiles tall or less are whole groups either way; times unchanged.
constexpr int64_t kGroupM = 4;

// 16-byte operand loads that need only element alignment (rows of an odd K
// or a view at any element offset): one global_load_dwordx4 all the same.
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));
typedef double f64x2u __attribute__((ext_vector_type(2), aligned(8)));
constexpr int64_t kShortRun = 8;   // shortest stream-K run
constexpr int64_t kLongRun = 16;   // run length once every compute unit has one

__device__ __forceinline__ void logical_tile(int64_t t, const TileMap& tm, int64_t& batch, int64_t& ti,
                                             int64_t& tj) {
  batch = t / tm.tiles_per_batch;
  t -= batch * tm.tiles_per_batch;
  const int64_t group = t / (kGroupM * tm.tiles_n);
  const int64_t first = group * kGroupM;
  const int64_t gm = tm.tiles_m - first < kGroupM ? tm.tiles_m - first : kGroupM;
  const int64_t r = t - group * kGroupM * tm.tiles_n;
  ti = first + r % gm;
  tj = r / gm;
}

// Origin of the tile computed for the tile owning [t0, t0 + tile) of an
// axis of `extent`. Edge tiles move back to end at the extent, so every row
// they read is in bounds and the interior loaders serve them; their first
// t0 - origin rows belong to the previous tile and are not stored. Only an
// axis shorter than one tile keeps origin 0 and reads clamped rows.
__device__ __forceinline__ int64_t tile_origin(int64_t t0, int64_t extent, int tile) {
  const int64_t last = extent > tile ? extent - tile : 0;
  return t0 < last ? t0 : last;
}

// Consecutive ids of a count-long range, renumbered so that ids landing on one
// XCD (ids i % 8) get a contiguous block of the range.
__device__ __forceinline__ int64_t xcd_major(int64_t id, int64_t count) {
  const int64_t full = (count / 8) * 8;
  return id < full ? (id % 8) * (full / 8) + id / 8 : id;
}

__host__ __device__ __forceinline__ int64_t sk_begin(const Split& sp, int64_t w) {
  return w * sp.base + (w < sp.extra ? w : sp.extra);
}

__device__ __forceinline__ int64_t sk_worker(const Split& sp, int64_t g) {
  const int64_t long_runs = sp.extra * (sp.base + 1);
  return g < long_runs ? g / (sp.base + 1) : sp.extra + (g - long_runs) / sp.base;
}

using hpgemm::batch_offsets;

// ---------------------------------------------------------------- loaders ----

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  using type = hpd::f32x4;
  using loose = f32x4u;
};
template <>
struct Vec16<double> {
  using type = hpd::f64x2;
  using loose = f64x2u;
};

// One operand's K slice: ROWS tile rows x 16 k values, global -> registers
// -> LDS rows [row][16 k] in 16-byte groups, group g of row r stored at slot
// g ^ ((r >> 1) & (G - 1)) (G groups per row; conflict-free fragment reads,
// see the kernels).
//   KM = false: stored k-contiguous, element (r, k) at p[r * ld + k] (A, or
//     B transposed). Each thread loads whole 16-byte groups.
//   KM = true: stored row-contiguous, element (r, k) at p[k * ld + r] (B, or
//     A transposed). Each thread owns one row and loads NE consecutive k as
//     scalars; 64 lanes read 64 consecutive rows of one k.
// Rows past `rows` load clamped addresses (their outputs are never stored);
// in mode 2 the slice holding the K edge zero-fills past kp.
template <typename T, int ROWS, bool KM, int MODE, int THREADS>
struct SliceLoader {
  using V = typename Vec16<T>::type;
  using VL = typename Vec16<T>::loose;
  static constexpr int W = 16 / sizeof(T);         // elements per group
  static constexpr int G = 16 / W;                 // groups per LDS row
  static constexpr int NV = ROWS * G / THREADS;    // groups per thread (KM = false)
  static constexpr int NE = 16 * ROWS / THREADS;   // elements per thread (KM = true)
  static constexpr int NR = KM ? NE / W : NV;      // register groups per thread
  static_assert(NV >= 1 && NE % W == 0, "tile does not divide over the workgroup");

  V reg[NR];
  int lds[NR];  // LDS element offsets of the register groups
  int row0;     // KM = false: first row of this thread; true: its row
  int kbase;    // KM = true: first k of this thread in the slice

  __device__ __forceinline__ static int swz(int row) { return (row >> 1) & (G - 1); }

  __device__ __forceinline__ void init(int tid) {
    if (!KM) {
      const int g = tid % G;
      row0 = tid / G;
      kbase = g * W;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int r = row0 + (THREADS / G) * i;
        lds[i] = r * 16 + W * (g ^ swz(r));
      }
    } else {
      row0 = tid % ROWS;
      kbase = (tid / ROWS) * NE;
#pragma unroll
      for (int j = 0; j < NR; ++j) lds[j] = row0 * 16 + W * ((kbase / W + j) ^ swz(row0));
    }
  }

  // p: operand origin at this piece's first k; r0: first tile row; rows:
  // operand rows; ld: leading dimension; kp: valid k from the origin. Rows
  // past `rows` load clamped addresses (their outputs are never stored); in
  // mode 2 the slice holding the K edge zero-fills past kp.
  //
  // fp32 (kUniformCheck): a workgroup-uniform test sends only the K-edge
  // slice, or a tile that an operand shorter than one tile leaves partly
  // empty, to the checked path, and other slices load without clamps
  // (4097x2049x3001: 54.6% -> 58% of peak). The fp64 kernels run at the
  // 256-VGPR limit, where that split spills (4096^2 x 4095: 76% -> 64%), so
  // they clamp rows on every slice and check K in the K-edge slice.
  static constexpr bool kUniformCheck = sizeof(T) == 4;

  __device__ __forceinline__ void load(const T* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp, int64_t k0) {
    constexpr bool kClamp = MODE != 0 && !kUniformCheck;
    if (kUniformCheck && MODE == 2 && (k0 + 16 > kp || r0 + ROWS > rows)) {
      load_checked(p, r0, rows, ld, kp, k0);
      return;
    }
    if (!KM) {
      if (!kUniformCheck && MODE == 2 && k0 + 16 > kp) {
        load_checked(p, r0, rows, ld, kp, k0);
        return;
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int64_t r = r0 + row0 + (THREADS / G) * i;
        reg[i] = *reinterpret_cast<const VL*>(p + (!kClamp || r < rows ? r : rows - 1) * ld + k0 + kbase);
      }
    } else {
      const int64_t r = !kClamp || r0 + row0 < rows ? r0 + row0 : rows - 1;
      if (!kUniformCheck && MODE == 2 && k0 + 16 > kp) {
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          const int64_t k = k0 + kbase + e;
          reg[e / W][e % W] = k < kp ? p[k * ld + r] : T(0);
        }
        return;
      }
#pragma unroll
      for (int e = 0; e < NE; ++e) reg[e / W][e % W] = p[(k0 + kbase + e) * ld + r];
    }
  }

  // Rows past `rows` read clamped addresses (their outputs are never
  // stored); k at or past kp reads as +0.
  __device__ __forceinline__ void load_checked(const T* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp,
                                               int64_t k0) {
    if (!KM) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int64_t r = r0 + row0 + (THREADS / G) * i;
        const T* q = p + (r < rows ? r : rows - 1) * ld;
#pragma unroll
        for (int e = 0; e < W; ++e) reg[i][e] = k0 + kbase + e < kp ? q[k0 + kbase + e] : T(0);
      }
    } else {
      const int64_t r = r0 + row0 < rows ? r0 + row0 : rows - 1;
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int64_t k = k0 + kbase + e;
        reg[e / W][e % W] = k < kp ? p[k * ld + r] : T(0);
      }
    }
  }

  __device__ __forceinline__ void store(T* buf) const {
#pragma unroll
    for (int j = 0; j < NR; ++j) *reinterpret_cast<V*>(buf + lds[j]) = reg[j];
  }

  // Element offset of the operand origin for a piece starting at slice s0.
  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t ld) { return KM ? s0 * 16 * ld : s0 * 16; }
};

// LDS-DMA through a buffer resource: 16 bytes per lane from base + voffset +
// soffset into LDS at `lds` (the wave's base; lane l lands at lds + 16 l).
// The MUBUF form, unlike global_load_lds, is not taken by the compiler for
// an access to both memory and LDS: after a global_load_lds it waits for
// every pending LDS read (lgkmcnt(0)) at the next use of any of them, the
// buffer form leaves its in-order lgkmcnt counts intact. Offsets are 32-bit:
// hosts route operands whose tile spans reach 2^31 bytes elsewhere. Third
// descriptor dword 0x00020000: 32-bit data format (gfx9).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, void* lds, unsigned voffset, unsigned soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0,
                                           0);
}

// s_waitcnt vmcnt(0) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8 left at their maxima).
constexpr unsigned kWaitVmcnt0 = 0x0F70;

// s_waitcnt vmcnt(N), the other counters at their maxima.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | N);
}

// Workgroup barrier without any wait: neither the wave's LDS reads nor its
// LDS-DMA (callers wait for what the barrier publishes themselves).
__device__ __forceinline__ void dma_barrier() { __builtin_amdgcn_s_barrier(); }

// Workgroup barrier for LDS that leaves LDS-DMA in flight: every LDS read
// and write of this wave completes (lgkmcnt(0)), then s_barrier. A
// __syncthreads() fence also waits for vmcnt(0), since the DMA writes LDS,
// which would drain the loads of the slice after next. Callers wait for the
// DMA that the barrier publishes themselves (wait_vmcnt). The loops that use
// it keep every LDS access that must not cross it on its own side through
// data dependences: fragment reads feed the next iteration's MFMAs, DMA
// destinations rotate through buffers that the reads cannot prove distinct.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

// ------------------------------------------------------------------ fp32 ----

namespace f32 {

constexpr int BK = 16;
constexpr int S = BK;  // LDS row stride (floats): 16-float rows, swizzled quads

// A workgroup tile configuration: BM x BN tile, waves in a WAVES_M x WAVES_N
// grid of WM x WN wave tiles (FM x FN MFMA blocks of 16 x 16 per wave),
// MIN_BLOCKS workgroups resident per compute unit.
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int MIN_BLOCKS_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int kThreads = 64 * WAVES_M * WAVES_N;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int FM = WM / 16, FN = WN / 16;
  static constexpr int kMinBlocks = MIN_BLOCKS_;
  // The staged slice goes to LDS after the MFMAs of this A fragment.
  static constexpr int kCommitAfter = FM - 3;
  static_assert(FM >= 4 && FN <= FM, "B refills ride on the first FN A fragments");
};
// 256 x 256, 8 waves of 128 x 64, one workgroup per compute unit: the
// headline tile (fewest operand loads per flop).
using Big = Tile<256, 256, 2, 4, 1>;
// 128 x 128, 4 waves of 64 x 64, two workgroups per compute unit: four times
// the tiles of Big, for products whose Big tiles do not fill the chip.
using Small = Tile<128, 128, 2, 2, 2>;
// 256 x 192, 8 waves of 128 x 48, one workgroup per compute unit: a third
// more tiles than Big, for products whose Big tiles would fill part of a
// round (stream-K and a fixup) while these fill it whole. Both operands by
// 4-byte LDS-DMA (mode 2 kernels only: 192-row slices are not whole 16-byte
// DMA chunks per wave).
using Wide = Tile<256, 192, 2, 4, 1>;
// 256 x 128, 8 waves of 64 x 64, one workgroup per compute unit: twice the
// tiles of Big, for products whose Big tiles would fill part of one round
// while these fill it whole.
using Half = Tile<256, 128, 4, 2, 1>;

// gfx950 LDS banks, measured with SQ_LDS_BANK_CONFLICT on probe kernels: a
// ds_read_b128 serves its 64 lanes in four groups of 16 (lane bit 5 and the
// parity of lane bits 2-4), ds_read_b64 in two groups of 32 consecutive
// lanes, ds_write_b64 in groups of 16 and ds_write_b128 in groups of 8; a
// group takes as many cycles as the most distinct addresses that fall on one
// bank set (16 bytes, 256 bytes of banks), and lanes at one address share.
//
// LDS rows hold 4 quads of 4 consecutive k values; quad q of row r is stored
// at slot q ^ ((r >> 1) & 3). Rows are 16 floats (64 B); the fragment reads
// (rows r0..r0+15, quad lane / 16) are conflict-free.
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 3; }

// An operand whose K axis is strided in memory (B stored [k][n], or A stored
// [k][m] when transposed) is read as 16-byte vectors along its tile rows:
// each thread loads a 2 (k) x 4 (row) block, k = 2 kh + {0, 1} (kh = t % 8),
// rows 4 b .. 4 b + 3 (b = t / 8), two global_load_dwordx4 instead of eight
// scalar loads, and writes it transposed, 8 bytes per row, into LDS rows of
// 16 k values padded to PS floats (8192^3: 85.6% -> 89.0% of peak against
// scalar loads). With the 80-byte row stride the commit's ds_write2_b64 (rows
// e, e + 1) is conflict-free and each fragment read costs 4 conflict cycles;
// no padded stride frees both (the reads need a stride of 2 mod 4 16-byte
// units, the paired writes an odd one). Where the operand's rows are 16-byte
// aligned, the 256-wide tiles take RowDmaLoader instead (no conflicts).
constexpr int PS = 20;

template <int ROWS, int THREADS, int MODE>
struct PairLoader {
  static_assert(MODE != 1, "mode 1 moves edge tiles inside the operands and uses the interior loader");
  static_assert(ROWS == THREADS / 2, "8 k pairs x THREADS / 8 row blocks of 4 per slice");
  hpd::f32x4 v[2];
  int kh, b;

  __device__ __forceinline__ void init(int tid) {
    kh = tid & 7;
    b = tid >> 3;
  }

  // Same contract as SliceLoader::load with KM = true: element (r, k) at
  // p[k * ld + r]; in mode 2 the K-edge slice and tiles of operands shorter
  // than one tile take a checked path (uniform test): rows past `rows` read
  // clamped addresses (outputs never stored), k at or past kp reads as +0.
  __device__ __forceinline__ void load(const float* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp,
                                       int64_t k0) {
    const int64_t c = r0 + 4 * b;
    if (MODE == 2 && (k0 + 16 > kp || r0 + ROWS > rows)) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int64_t k = k0 + 2 * kh + r;
        const float* q = p + (k < kp ? k : kp - 1) * ld;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = q[c + e < rows ? c + e : rows - 1];
          v[r][e] = k < kp ? x : 0.f;
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) v[r] = *reinterpret_cast<const f32x4u*>(p + (k0 + 2 * kh + r) * ld + c);
  }

  __device__ __forceinline__ void store(float* buf) const {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 4; ++e) *reinterpret_cast<f32x2*>(buf + (4 * b + e) * PS + 2 * kh) = f32x2{v[0][e], v[1][e]};
  }

  // Pipeline interface: issue the global loads of a slice, commit it to LDS.
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp, int64_t k0,
                                        float*) {
    load(p, r0, rows, ld, kp, k0);
  }
  __device__ __forceinline__ void commit(float* buf) const { store(buf); }
  static constexpr bool kDirect = false;

  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t ld) { return s0 * 16 * ld; }
};

// A k-contiguous operand in modes 0 and 1 (and the whole K slices of mode
// 2): its K slice goes from global memory straight into LDS with 16-byte
// LDS-DMA, without registers or ds_write. LDS-DMA writes 16 bytes per lane
// at consecutive addresses, so a wave fills whole 16-row chunks (1 KB each;
// kChunks per wave, the last waves fewer when the chunks do not divide
// evenly) and lane l fetches the global group that the swizzle places at its
// position: row 16c + l / 4, k group (l % 4) ^ swizzle(row). Completion is
// tracked by vmcnt; kernels wait for vmcnt(0) before the barrier that
// publishes a slice. Every row read is in bounds.
template <int ROWS, int THREADS, int MODE>
struct DmaLoader {
  static_assert(MODE == 0, "in-bounds rows only: mode 1 moves edge tiles inside, mode 2 stages");
  static constexpr int kRowChunks = ROWS / 16;
  static_assert(kRowChunks * 16 == ROWS, "whole 16-row chunks");
  static constexpr int kChunks = (kRowChunks + THREADS / 64 - 1) / (THREADS / 64);  // per wave, at most
  int chunk0, lane;

  __device__ __forceinline__ void init(int tid) {
    chunk0 = kChunks * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }

  // Element (r, k) of the tile at p[(r0 + r) * ld + k]; byte offsets from
  // the tile's first row: ROWS * ld * 4 < 2^31 (host check).
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t, int64_t ld, int64_t, int64_t k0,
                                        float* buf) const {
    issue(buffer_rsrc(p + r0 * ld), ld, k0, buf);
  }
  // The same from a descriptor whose base is the tile's first row.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, int64_t ld, int64_t k0, float* buf) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = chunk0 + i;
      if (kRowChunks % (THREADS / 64) != 0 && c >= kRowChunks) break;  // wave-uniform
      const unsigned row = 16 * c + (lane >> 2);
      const unsigned element = row * unsigned(ld) + 4 * ((lane & 3) ^ swizzle(row));
      dma16(rsrc, buf + 256 * c, 4 * element, 4 * unsigned(k0));
    }
  }
  __device__ __forceinline__ void commit(float*) const {}
  static constexpr bool kDirect = true;
  static constexpr int kLoads = kChunks;  // LDS-DMA instructions per wave and slice

  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t) { return s0 * 16; }
};

// Register-staged k-contiguous loads (mode 2: the K-edge slice zero-fills).
template <int ROWS, int THREADS, int MODE>
struct StagedLoader : SliceLoader<float, ROWS, false, MODE, THREADS> {
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp, int64_t k0,
                                        float*) {
    this->load(p, r0, rows, ld, kp, k0);
  }
  __device__ __forceinline__ void commit(float* buf) const { this->store(buf); }
  static constexpr bool kDirect = false;
};

// A K-strided operand ([k][rows] in memory: B, or A transposed) in modes 0
// and 1 (and the whole K slices of mode 2): one 16-byte LDS-DMA per k row
// moves the tile's ROWS floats (1 KB for 256 rows; narrower tiles leave the
// lanes past ROWS / 4 idle) into LDS, stored [k][row] at a row stride of RS
// floats. No registers, no ds_write and no wait in the middle of the slice,
// against the register-staged pair loader (8192^3: the staged B path costs
// 3.7% of peak, its DMA 1%). A fragment is then four 4-byte reads, rows 4
// (lane / 16) + q: the 16-byte pad puts the four lane groups on disjoint
// bank sets (4 RS = 16 mod 64 dwords for RS = 132, 196, 260).
template <int ROWS, int THREADS>
struct RowDmaLoader {
  static_assert(ROWS % 64 == 0 && ROWS <= 256, "16-byte lanes of one LDS-DMA per k row");
  static constexpr int kLanes = ROWS / 4;
  static constexpr int kRowsPerWave = 16 / (THREADS / 64);
  static_assert(kRowsPerWave * (THREADS / 64) == 16, "whole k rows per wave");
  static constexpr int RS = ROWS + 4;
  static constexpr int kBufFloats = 16 * RS;
  int k0w, lane;

  __device__ __forceinline__ void init(int tid) {
    k0w = kRowsPerWave * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }

  // Element (r, k) at p[k * ld + r0 + r]; byte offsets from the tile's
  // first column: (K * ld + ROWS) * 4 < 2^31 (host check).
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t, int64_t ld, int64_t, int64_t k0,
                                        float* buf) const {
    issue(buffer_rsrc(p + r0), ld, k0, buf);
  }
  // The same from a descriptor whose base is the tile's first column.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, int64_t ld, int64_t k0, float* buf) const {
    if (kLanes < 64 && lane >= kLanes) return;
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
      const unsigned k = k0w + i;
      dma16(rsrc, buf + k * RS, 4 * (k * unsigned(ld) + 4 * lane), 4 * unsigned(k0 * ld));
    }
  }
  __device__ __forceinline__ void commit(float*) const {}
  static constexpr bool kDirect = true;
  static constexpr int kLoads = kRowsPerWave;  // LDS-DMA instructions per wave and slice

  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t ld) { return s0 * 16 * ld; }
  // Fragment base of lane `lane` for tile rows row0 + (lane & 15).
  __device__ __forceinline__ static int read_offset(int row0, int lane) {
    return 4 * (lane >> 4) * RS + row0 + (lane & 15);
  }
  // Fragment `f` (rows 16 f on): k values 4 (lane / 16) + q, q = 0..3.
  __device__ __forceinline__ static hpd::f32x4 read(const float* base, int f) {
    return hpd::f32x4{base[16 * f], base[16 * f + RS], base[16 * f + 2 * RS], base[16 * f + 3 * RS]};
  }
};

// 4-byte LDS-DMA: any operand alignment (rows of odd K, views at any element
// offset) and the edges of mode 2. One instruction fills 64 consecutive
// dwords of LDS, a quarter of what the 16-byte form moves, so a slice takes
// four times the instructions (16 per wave for a 256 x 256 tile, against 128
// MFMAs); their offsets are formed once per slice, so each costs an M0 write
// and a scalar add. The descriptor's range ends at the operand's last valid
// element: anything past it loads +0 and nothing outside the operand is read.
// Rows (columns) past the operand's extent that still lie inside that range
// hold other data, which reaches only outputs that are never stored; k past
// the K edge must load +0, which the range gives K-strided operands (their
// rows past K lie beyond the last valid element) and k-contiguous ones get
// from lanes that take an offset outside every range in the K-edge slice.
constexpr unsigned kOutOfRange = 0x80000000u;
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc, void* lds, unsigned voffset, unsigned soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 4, voffset, soffset, 0,
                                           0);
}

// A k-contiguous operand by 4-byte LDS-DMA into DmaLoader's swizzled
// [row][16 k] layout: instruction i of a wave fills rows 4 g .. 4 g + 3
// (g = the wave's first group + i); lane l writes row 4 g + l / 16 at slot
// (l % 16) / 4, element l % 4, so it fetches k = 4 ((l % 16) / 4 ^
// swizzle(row)) + l % 4. swizzle(row) = ((4 g + l / 16) >> 1) & 3 depends on
// g only through its parity: two offsets per lane serve every instruction.
template <int ROWS, int THREADS>
struct DmaLoader4 {
  static constexpr int kWaves = THREADS / 64;
  static constexpr int kLoads = ROWS / 4 / kWaves;  // per wave and slice
  static_assert(kLoads * 4 * kWaves == ROWS && kLoads % 2 == 0, "whole pairs of 4-row groups per wave");
  int g0, lane;

  __device__ __forceinline__ void init(int tid) {
    g0 = kLoads * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }
  // This lane's k within a slice for row groups of parity `odd`.
  __device__ __forceinline__ unsigned k_of(int odd) const {
    const unsigned row = 4 * (g0 + odd) + (lane >> 4), d = lane & 15;
    return 4 * ((d >> 2) ^ swizzle(row)) + (d & 3);
  }

  // Element (r, k) of the tile at p[(r0 + r) * ld + k], valid for r0 + r <
  // rows and k < kp; byte offsets from the tile's first row below 2^31 (host
  // check).
  // Descriptor from the tile's first row through the last valid element of
  // the tile's own rows: (ROWS - 1) * ld + kp elements at most, which the
  // host's span check keeps below 2^31 bytes. A range through the end of the
  // whole operand would wrap its 32 bits for operands of 2^29 floats or
  // more and could exceed kOutOfRange, which must stay outside every range.
  __device__ __forceinline__ static __amdgpu_buffer_rsrc_t rsrc_of(const float* p, int64_t r0, int64_t rows,
                                                                   int64_t ld, int64_t kp) {
    const int64_t own = rows - r0 < ROWS ? rows - r0 : ROWS;
    const int64_t extent = (own - 1) * ld + kp;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p + r0 * ld), 0, int(4 * extent), 0x00020000);
  }
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp, int64_t k0,
                                        float* buf) const {
    const __amdgpu_buffer_rsrc_t rsrc = rsrc_of(p, r0, rows, ld, kp);
    const unsigned rl = lane >> 4;
    const unsigned k_even = k_of(0), k_odd = k_of(1);
    // k at or past kp - k0 (the K-edge slice only) loads +0.
    const int64_t left = kp - k0;
    const unsigned kk = left < 16 ? unsigned(left) : 16u;
    const unsigned v_even = k_even < kk ? 4 * (rl * unsigned(ld) + k_even) : kOutOfRange;
    const unsigned v_odd = k_odd < kk ? 4 * (rl * unsigned(ld) + k_odd) : kOutOfRange;
    // A running scalar offset: one register, one add per instruction.
    unsigned soffset = 4 * (4 * unsigned(g0) * unsigned(ld) + unsigned(k0));
    const unsigned group = 16 * unsigned(ld);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      dma4(rsrc, buf + 64 * (g0 + i), i % 2 ? v_odd : v_even, soffset);
      soffset += group;
    }
  }
  __device__ __forceinline__ void commit(float*) const {}
  static constexpr bool kDirect = true;
  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t) { return s0 * 16; }
};

// A K-strided operand by 4-byte LDS-DMA into RowDmaLoader's [k][row] layout
// (row stride ROWS + 4): instruction (k, c) fills tile rows 64 c .. 64 c + 63
// of k row k, lane l fetching row 64 c + l. No lane takes a special offset:
// k rows past kp lie beyond the descriptor's range.
template <int ROWS, int THREADS>
struct RowDma4 {
  static constexpr int kPerRow = ROWS / 64;  // instructions per k row
  static constexpr int kWaves = THREADS / 64;
  static constexpr int kLoads = 16 * kPerRow / kWaves;
  static_assert(kLoads * kWaves == 16 * kPerRow, "whole k rows per wave");
  static constexpr int RS = ROWS + 4;
  static constexpr int kBufFloats = 16 * RS;
  int t0, lane;

  __device__ __forceinline__ void init(int tid) {
    t0 = kLoads * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }

  // Element (r, k) at p[k * ld + r0 + r], valid for r0 + r < rows and
  // k < kp; byte offsets from the tile's first column below 2^31 (host
  // check).
  // Descriptor from the tile's first column through the last valid element.
  __device__ __forceinline__ static __amdgpu_buffer_rsrc_t rsrc_of(const float* p, int64_t r0, int64_t rows,
                                                                   int64_t ld, int64_t kp) {
    const int64_t extent = (kp - 1) * ld + rows - r0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p + r0), 0, int(4 * extent), 0x00020000);
  }
  __device__ __forceinline__ void issue(const float* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp, int64_t k0,
                                        float* buf) const {
    const __amdgpu_buffer_rsrc_t rsrc = rsrc_of(p, r0, rows, ld, kp);
    // A running scalar offset (t0 is a multiple of kPerRow: the wave's rows
    // start at column 0): one register, one add per instruction.
    static_assert(kLoads % kPerRow == 0, "whole k rows per wave");
    unsigned soffset = 4 * ((unsigned(k0) + unsigned(t0) / kPerRow) * unsigned(ld));
    const unsigned next_row = 4 * unsigned(ld) - 256 * (kPerRow - 1);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const unsigned t = t0 + i, k = t / kPerRow, c = t % kPerRow;
      dma4(rsrc, buf + k * RS + 64 * c, 4 * lane, soffset);
      soffset += c == kPerRow - 1 ? next_row : 256u;
    }
  }
  __device__ __forceinline__ void commit(float*) const {}
  static constexpr bool kDirect = true;
  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t ld) { return s0 * 16 * ld; }
  __device__ __forceinline__ static int read_offset(int row0, int lane) {
    return 4 * (lane >> 4) * RS + row0 + (lane & 15);
  }
  __device__ __forceinline__ static hpd::f32x4 read(const float* base, int f) {
    return hpd::f32x4{base[16 * f], base[16 * f + RS], base[16 * f + 2 * RS], base[16 * f + 3 * RS]};
  }
};

// LDS floats per buffer: the row-DMA layout's, else ROWS x the row stride.
template <class L, bool ROW, int FALLBACK>
constexpr int buf_floats() {
  if constexpr (ROW) return L::kBufFloats;
  else return FALLBACK;
}

// LDS row stride of an operand and its loader: k-contiguous operands use the
// swizzled 16-float rows of SliceLoader, K-strided ones the padded pair rows.
template <bool KM>
constexpr int lds_stride() {
  return KM ? PS : S;
}
// Modes 0 and 1 share the interior loaders: mode 1 (M, N >= one tile) moves
// edge tiles inside the operands instead of clamping their rows.
template <bool KM, int MODE, int ROWS, int THREADS>
using Loader = typename std::conditional<
    KM, PairLoader<ROWS, THREADS, MODE == 1 ? 0 : MODE>,
    typename std::conditional<MODE == 2, StagedLoader<ROWS, THREADS, MODE>,
                              DmaLoader<ROWS, THREADS, MODE == 1 ? 0 : MODE>>::type>::type;

// Loaders of the kernel's operands: K-strided operands by row LDS-DMA (the
// 4-byte form when DWORD), other operands by Loader, or DmaLoader4 when
// DWORD.
template <bool DWORD, int ROWS, int THREADS>
using RowLoader =
    typename std::conditional<DWORD, RowDma4<ROWS, THREADS>, RowDmaLoader<ROWS, THREADS>>::type;
template <bool DWORD, bool KM, int MODE, int ROWS, int THREADS>
using FlatLoader =
    typename std::conditional<DWORD, DmaLoader4<ROWS, THREADS>, Loader<KM, MODE, ROWS, THREADS>>::type;

// Fragment read offset of lane `lane` for tile row `row0 + (lane & 15)`.
template <bool KM>
__device__ __forceinline__ int fragment_offset(int row0, int lane) {
  const int row = row0 + (lane & 15);
  return KM ? row * PS + 4 * (lane >> 4) : row * S + 4 * ((lane >> 4) ^ swizzle(lane & 15));
}

// Waves in a WAVES_M x WAVES_N grid of wave tiles. Accumulator layout: lane
// holds column lane%16, rows 4*(lane/16) + r.
template <class T>
struct Layout {
  static constexpr int kBM = T::BM, kBN = T::BN, kFM = T::FM, kFN = T::FN;
  static __device__ __forceinline__ int row(int wave, int i, int lane, int r) {
    return (wave / T::WAVES_N) * T::WM + 16 * i + 4 * (lane >> 4) + r;
  }
  static __device__ __forceinline__ int col(int wave, int j, int lane) {
    return (wave % T::WAVES_N) * T::WN + 16 * j + (lane & 15);
  }
};

// Big: one workgroup per compute unit (64-72 KB of LDS, 2 waves per SIMD);
// Small: two (two waves per SIMD as well). The pipeline per K slice s:
//   - global loads of slice s+2 into registers, issued first;
//   - FM x FN x 4 MFMAs per wave on the fragments of slice s, already in
//     registers;
//     after the 16 MFMAs of A fragment i, that register is refilled with
//     fragment i of slice s+1 from LDS (B fragments are double-buffered and
//     refilled after A fragments 0-3), so LDS reads overlap the matrix pipe
//     instead of stalling each slice start;
//   - after the MFMAs of fragment FM - 3, slice s+2 goes from registers to the
//     LDS buffer that held slice s (all waves read it during slice s-1);
//   - one barrier.
// STREAM_K = false: workgroup b computes whole tile xcd_major(b). true:
// workgroup b is stream-K worker xcd_major(b) and computes its run, at most
// the end of one tile and the start of the next (kept out of the whole-tile
// kernel: the second inlined piece measurably slows the main loop).
template <class CFG, int MODE, bool STREAM_K, bool TA, bool TB, bool ROWDMA>
__global__ __launch_bounds__(CFG::kThreads, CFG::kMinBlocks) void kernel(const float* __restrict__ A,
                                                                         const float* __restrict__ B,
                                                                         float* __restrict__ C, int64_t M, int64_t N,
                                                                         int64_t K, BatchDesc bd, TileMap tmap,
                                                                         Split sp) {
  constexpr int BM = CFG::BM, BN = CFG::BN, WM = CFG::WM, WN = CFG::WN, FM = CFG::FM, FN = CFG::FN;
  constexpr int kThreads = CFG::kThreads;
  using L = Layout<CFG>;
  constexpr int SA = lds_stride<TA>(), SB = lds_stride<!TB>();
  // ROWDMA in modes 0 and 1: K-strided operands (A if TA, B unless TB) arrive
  // by RowDmaLoader (16-byte rows). In mode 2 both operands arrive by 4-byte
  // LDS-DMA (RowDma4 for K-strided ones, DmaLoader4 for k-contiguous ones),
  // else register-staged. K-strided operands by DMA take the [k][row] layout.
  constexpr bool kDword = ROWDMA && MODE == 2;
  constexpr bool kRowA = TA && ROWDMA, kRowB = !TB && ROWDMA;
  using LA = typename std::conditional<kRowA, RowLoader<kDword, BM, kThreads>,
                                       FlatLoader<kDword, TA, MODE, BM, kThreads>>::type;
  using LB = typename std::conditional<kRowB, RowLoader<kDword, BN, kThreads>,
                                       FlatLoader<kDword, !TB, MODE, BN, kThreads>>::type;
  constexpr int kBufA = buf_floats<LA, kRowA, BM * SA>(), kBufB = buf_floats<LB, kRowB, BN * SB>();
  // Mode 2 by LDS-DMA: the K slices inside K of a product whose tiles all lie
  // inside M and N (M >= BM, N >= BN; edge tiles are moved inside) go by the
  // 16-byte forms, which write the same LDS layouts as the 4-byte ones and
  // read only elements of the operands; the 16-byte loads need 4-byte
  // aligned addresses only. The K-edge slice and other products take the
  // 4-byte forms. Measured against the 4-byte forms throughout, TFLOP/s:
  // 8192 x 8192 x 8191 139.8 -> 147.9, 4096 x 4096 x 2047 136.2 -> 143.6,
  // 4097 x 2049 x 3001 (edge strips beside) 123.8 -> 128.9.
  constexpr bool kWhole16 = kDword && (kRowA ? BM % 64 == 0 : BM % 16 == 0) && (kRowB ? BN % 64 == 0 : BN % 16 == 0);
  using LA16 = typename std::conditional<
      kWhole16, typename std::conditional<kRowA, RowDmaLoader<BM, kThreads>, DmaLoader<BM, kThreads, 0>>::type,
      LA>::type;
  using LB16 = typename std::conditional<
      kWhole16, typename std::conditional<kRowB, RowDmaLoader<BN, kThreads>, DmaLoader<BN, kThreads, 0>>::type,
      LB>::type;
  // Slices in LDS, one variable per buffer and operand: three buffers when
  // both operands arrive by LDS-DMA (loads run two slices ahead), else two.
  constexpr int kStages = LA::kDirect && LB::kDirect ? 3 : 2;
  __shared__ __attribute__((aligned(16))) float As0[kBufA];
  __shared__ __attribute__((aligned(16))) float As1[kBufA];
  __shared__ __attribute__((aligned(16))) float As2[kStages == 3 ? kBufA : 4];
  __shared__ __attribute__((aligned(16))) float Bs0[kBufB];
  __shared__ __attribute__((aligned(16))) float Bs1[kBufB];
  __shared__ __attribute__((aligned(16))) float Bs2[kStages == 3 ? kBufB : 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / CFG::WAVES_N, wn = wave % CFG::WAVES_N;

  // Global -> register -> LDS operand slices. A is k-contiguous ([m][k])
  // unless TA ([k][m]); B is row-contiguous ([k][n]) unless TB ([n][k]).
  // k-contiguous operands go straight to LDS (DmaLoader; register-staged in
  // mode 2), K-strided ones as 2 float4 row vectors per thread (PairLoader).
  LA la;
  LB lb;
  LA16 la16;
  LB16 lb16;
  constexpr bool kDirect = decltype(la)::kDirect || decltype(lb)::kDirect;
  la.init(tid);
  lb.init(tid);
  la16.init(tid);
  lb16.init(tid);
  const bool inside = M >= BM && N >= BN;
  const int64_t lda = tmap.lda, ldb = tmap.ldb;
  // Rows read by a lane differ by multiples of 16, so the swizzle of every
  // row it reads equals that of (lane & 15).
  int a_read, b_read;
  if constexpr (kRowA) a_read = LA::read_offset(wm * WM, lane);
  else a_read = fragment_offset<TA>(wm * WM, lane);
  if constexpr (kRowB) b_read = LB::read_offset(wn * WN, lane);
  else b_read = fragment_offset<!TB>(wn * WN, lane);
  // Fragment f of A (B) at base = buffer + a_read (b_read).
  auto frag_a = [&](const float* base, int f) {
    if constexpr (kRowA) return LA::read(base, f);
    else return *reinterpret_cast<const hpd::f32x4*>(base + 16 * f * SA);
  };
  auto frag_b = [&](const float* base, int f) {
    if constexpr (kRowB) return LB::read(base, f);
    else return *reinterpret_cast<const hpd::f32x4*>(base + 16 * f * SB);
  };

  // Tile `tile` over K slices [s0, s1). slot < 0: the piece is the whole K
  // range and is stored to C; else it goes to workspace slot `slot`.
  auto piece = [&](int64_t tile, int64_t s0, int64_t s1, int64_t slot) {
    int64_t batch, ti, tj;
    logical_tile(tile, tmap, batch, ti, tj);
    int64_t a_off, b_off;
    batch_offsets(batch, bd, a_off, b_off);
    // Owned tile [m0, m0 + BM) x [n0, n0 + BN), computed at (ms, ns).
    const int64_t m0 = ti * BM, n0 = tj * BN;
    const int64_t ms = MODE == 0 ? m0 : tile_origin(m0, M, BM), ns = MODE == 0 ? n0 : tile_origin(n0, N, BN);
    // Operand origins at the piece's first k; kp = valid k extent from there.
    const float* Ap = A + a_off + decltype(la)::origin(s0, lda);
    const float* Bp = B + b_off + decltype(lb)::origin(s0, ldb);
    const int64_t kp = K - s0 * BK;
    const int64_t slices = s1 - s0;
    // Slice k0 into LDS buffer `buf`: issue() starts the global reads (direct
    // loads land in LDS by themselves), commit() writes staged registers.
    // Direct loads go first. The compiler waits for vmcnt(0) before any
    // ds_write while an LDS-DMA is in flight (it cannot tell the buffers
    // apart), so the staged commit waits for them anyway; issued first they
    // have the most time. Same-box A/B at 8192^3: direct first 89.8-90.1% of
    // peak, staged first 84.6%, no direct loads 88.6-89.2%.
    auto load_slice = [&](int64_t k0, float* as, float* bs) {
      if constexpr (kWhole16) {
        if (inside && k0 + BK <= kp) {
          // The 4-byte loaders' descriptors (one pair of registers for both).
          la16.issue(LA::rsrc_of(Ap, ms, M, lda, kp), lda, k0, as);
          lb16.issue(LB::rsrc_of(Bp, ns, N, ldb, kp), ldb, k0, bs);
          return;
        }
      }
      if (decltype(la)::kDirect) la.issue(Ap, ms, M, lda, kp, k0, as);
      if (decltype(lb)::kDirect) lb.issue(Bp, ns, N, ldb, kp, k0, bs);
      if (!decltype(la)::kDirect) la.issue(Ap, ms, M, lda, kp, k0, as);
      if (!decltype(lb)::kDirect) lb.issue(Bp, ns, N, ldb, kp, k0, bs);
    };
    auto store_slice = [&](float* as, float* bs) {
      la.commit(as);
      lb.commit(bs);
    };
    auto publish = [&] {
      if (kDirect) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
    };

    hpd::f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = hpd::f32x4{0.f, 0.f, 0.f, 0.f};

    if constexpr (kStages == 3) {
      load_slice(0, As0, Bs0);
      if (slices > 1) load_slice(BK, As1, Bs1);
      publish();
    } else {
      load_slice(0, As0, Bs0);
      store_slice(As0, Bs0);
      if (slices > 1) {
        load_slice(BK, As1, Bs1);
        store_slice(As1, Bs1);
      }
      publish();
    }
    hpd::f32x4 a[FM], b[FN], b_next[FN];
    // B first: the loop's first MFMAs then wait on the same in-order LDS
    // counts as after a slice of the loop, whose last reads are A's.
#pragma unroll
    for (int j = 0; j < FN; ++j) b[j] = frag_b(Bs0 + b_read, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FM; ++i) a[i] = frag_a(As0 + a_read, i);
    __builtin_amdgcn_sched_barrier(0);
    // Slice s: slice s+2 goes into the buffers (as, bs) that held slice s,
    // fragments of slice s+1 come from an, bn (buffer plus this lane's
    // fragment offset).
    auto slice = [&](int64_t s, float* as, float* bs, const float* an, const float* bn) {
      const bool more = s + 1 < slices;
      if (s + 2 < slices) load_slice((s + 2) * BK, as, bs);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
        if (more) {
          a[i] = frag_a(an, i);
          // B refills ride on the first FN A fragments, so only A refills
          // are in flight at the barrier (same-box A/B: +0.3-0.6% of peak).
          if (i < FN) b_next[i] = frag_b(bn, i);
        }
        if (i == CFG::kCommitAfter && s + 2 < slices) store_slice(as, bs);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) b[j] = b_next[j];
      publish();
    };
    // Every wave has read buffer 0 before slice 0 refills it. This barrier
    // sits under the loop's own guard (slices > 0 always holds). Before the
    // guard, the compiler sank the reads above to their first use, past the
    // barrier, where a late wave could read slice 2's data after a faster
    // wave's LDS-DMA refilled buffer 0 (one wrong 16 x 64 fragment block,
    // with several workgroups per compute unit). Other ways of holding the
    // reads above the barrier (an asm memory clobber, an asm use of the
    // fragments, buffer arrays indexed at run time) led the compiler to wait
    // for vmcnt(0) before every fragment read of the loop (8192^3: -4% of
    // peak), and so did unrolling two slices per iteration over fixed
    // buffers (-2.5%). The assembly is checked for both in the CPU tests.
    if (kStages == 2 && slices > 0) __syncthreads();
    // The next slice's fragment addresses are carried across iterations:
    // picking them per slice lets the compiler rematerialize the address
    // into each fragment register, and that write has to wait for the MFMAs
    // still reading the register (measured: -3% of peak).
    const float* an = As1 + a_read;
    const float* bn = Bs1 + b_read;
    if constexpr (kStages == 3) {
      // Slice s: slice s+2 goes into the third buffer (the one that held
      // slice s-1), fragments of slice s+1 come from an, bn. Every wave read
      // slice s-1's fragments before slice s-2's barrier and used them before
      // slice s-1's, so the barrier that publishes a slice need not wait for
      // the wave's own LDS reads: only the LDS-DMA it publishes. Refills are
      // unconditional (past the last slice they read stale LDS and go unused)
      // and the two B fragment sets swap roles every slice, so the next
      // slice's first MFMAs wait only for reads issued early in this one.
      auto slice3 = [&](int64_t s, float* as, float* bs, const float* an, const float* bn, hpd::f32x4* bc,
                        hpd::f32x4* bx) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][q], bc[j][q], acc[i][j], 0, 0, 0);
          // The compiler orders LDS reads and LDS-DMA with one counter and
          // waits for every LDS read before the first fragment use after an
          // LDS-DMA issue. Issued after fragment 0's MFMAs, with that
          // fragment's refill held back to fragment 1, the DMA is followed by
          // no read younger than the previous slice's last one.
          if (i == 0) {
            if (s + 2 < slices) load_slice((s + 2) * BK, as, bs);
          } else {
            if (i == 1) {
              a[0] = frag_a(an, 0);
              bx[0] = frag_b(bn, 0);
            }
            a[i] = frag_a(an, i);
            if (i < FN) bx[i] = frag_b(bn, i);
          }
          // Keep the refills behind their fragment's MFMAs: without branches
          // the scheduler otherwise interleaves the whole slice and renames
          // accumulators.
          __builtin_amdgcn_sched_barrier(0);
        }
        wait_vmcnt<0>();
        dma_barrier();
      };
      float *a1 = As1, *a2 = As2, *a0 = As0, *b1 = Bs1, *b2 = Bs2, *b0 = Bs0;
      auto rotate = [&] {
        an = a2 + a_read;
        bn = b2 + b_read;
        float* t = a0;
        a0 = a1;
        a1 = a2;
        a2 = t;
        t = b0;
        b0 = b1;
        b1 = b2;
        b2 = t;
      };
      int64_t s = 0;
      for (; s + 1 < slices; s += 2) {
        slice3(s, a2, b2, an, bn, b, b_next);
        rotate();
        slice3(s + 1, a2, b2, an, bn, b_next, b);
        rotate();
      }
      if (s < slices) slice3(s, a2, b2, an, bn, b, b_next);
    } else {
      for (int64_t s = 0; s < slices; ++s) {
        const bool odd = s & 1;
        slice(s, odd ? As1 : As0, odd ? Bs1 : Bs0, an, bn);
        an = (odd ? As1 : As0) + a_read;
        bn = (odd ? Bs1 : Bs0) + b_read;
      }
    }

    if (slot < 0) {
      float* Cb = C + batch * M * tmap.ldc;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t col = ns + L::col(wave, j, lane);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = ms + L::row(wave, i, lane, r);
            if (MODE == 0 || (row >= m0 && row < M && col >= n0 && col < N)) Cb[row * tmap.ldc + col] = acc[i][j][r];
          }
        }
      }
    } else {
      // Cut piece: whole accumulator tile to the workspace slot, in register
      // order (16 contiguous bytes per lane).
      hpd::f32x4* out = static_cast<hpd::f32x4*>(sp.partial) + slot * (BM * BN / 4);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) out[((wave * FM + i) * FN + j) * 64 + lane] = acc[i][j];
    }
  };

  if (!STREAM_K) {
    piece(xcd_major(blockIdx.x, sp.dp_tiles), 0, sp.slices, -1);
  } else {
    const int64_t worker = xcd_major(blockIdx.x, sp.workers);
    const int64_t g = sk_begin(sp, worker), g_end = sk_begin(sp, worker + 1);
    // A run is at most one tile long: the end of one tile and the start of
    // the next at most. The start of the next tile goes first: every worker
    // then sits at K slice tau (first piece) or slices - run + tau (second
    // piece) at time tau, so workers sharing an XCD read the same A and B
    // slices together and its L2 serves them, as in the whole-tile kernel
    // (in run order the K positions of neighbouring workers all differ).
    const int64_t t0 = g / sp.slices;
    const int64_t s0 = g - t0 * sp.slices;
    const int64_t s1 = g_end - t0 * sp.slices < sp.slices ? g_end - t0 * sp.slices : sp.slices;
    const int64_t rest = g_end - (t0 + 1) * sp.slices;
    if (rest > 0) piece(sp.dp_tiles + t0 + 1, 0, rest, rest == sp.slices ? -1 : worker * 2 + 1);
    piece(sp.dp_tiles + t0, s0, s1, s0 == 0 && s1 == sp.slices ? -1 : worker * 2);
  }
}

}  // namespace f32

// ---------------------------------------------------------- fp32 narrow ----

// 64 x 64 output tiles, one workgroup each, for products whose 256 x 256 and
// 128 x 128 tiles leave compute units idle or need stream-K (1024^3: 16 and
// 64 tiles, against 256 here). Each of the workgroup's KW waves computes the
// whole tile (4 x 4 MFMA blocks) over every KW-th K slice, from LDS buffers
// of its own: no barrier in the K loop, no partial tiles in global memory and
// no second kernel. At the end the KW accumulator tiles are added in wave
// order through LDS, so results are deterministic. Interior products only:
// M and N multiples of 64, K of 16, operand rows 16-byte aligned.
namespace narrow {

constexpr int T = 64;
// LDS per slice and operand. A k-contiguous operand keeps rows of 16 k in
// swizzled quads (fragment reads as in the tiled kernel). A K-strided one
// ([k][rows] in memory) arrives as 4 k rows (1 KB) per LDS-DMA; 16 floats of
// padding between those groups put the four lane groups of a fragment read
// (k = 4 g + q) on disjoint banks (272 = 16 mod 64).
constexpr int kGroup = 4 * T + 16;
constexpr int kOperand = 4 * kGroup;  // >= T * 16, the k-contiguous size
constexpr int kSlice = 2 * kOperand;  // A then B

template <bool KM>
struct Operand {
  // Issue the LDS-DMA of one slice (16 k from k0) of a 64-row operand whose
  // tile origin is p: KM = false, element (r, k) at p[r * ld + k]; KM = true,
  // at p[k * ld + r]. Four 1 KB transfers per wave, all in bounds, through a
  // buffer descriptor (byte offsets from p below 2^31, host check).
  __device__ __forceinline__ static void issue(const float* p, int64_t ld, int64_t k0, float* buf, int lane) {
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(p);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if constexpr (KM) {
        const unsigned element = (4 * c + (lane >> 4)) * unsigned(ld) + 4 * (lane & 15);
        dma16(rsrc, buf + c * kGroup, 4 * element, 4 * unsigned(k0 * ld));
      } else {
        const int row = 16 * c + (lane >> 2);
        const unsigned element = row * unsigned(ld) + 4 * ((lane & 3) ^ f32::swizzle(row));
        dma16(rsrc, buf + 256 * c, 4 * element, 4 * unsigned(k0));
      }
    }
  }
  // Fragment f (tile rows 16 f + lane % 16): k = 4 (lane / 16) + q in
  // element q, the k order of the tiled kernel's fragments.
  __device__ __forceinline__ static hpd::f32x4 frag(const float* buf, int f, int lane) {
    if constexpr (KM) {
      const float* base = buf + (lane >> 4) * kGroup + 16 * f + (lane & 15);
      return hpd::f32x4{base[0], base[T], base[2 * T], base[3 * T]};
    } else {
      const int row = 16 * f + (lane & 15);
      return *reinterpret_cast<const hpd::f32x4*>(buf + row * 16 + 4 * ((lane >> 4) ^ f32::swizzle(row)));
    }
  }
};

// s_waitcnt vmcnt(n), other counters at their maxima (gfx9: vmcnt bits 3:0
// and 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((kWaitVmcnt0 & ~0xC00Fu) | (N & 15) | ((N >> 4) << 14));
}

// KW waves per 64 x 64 tile take every KW-th K slice. Two LDS buffers per
// wave: slice t + 2 goes into slice t's buffer once its fragments are read.
template <bool TA, bool TB, int KW>
__global__ __launch_bounds__(64 * KW) void kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                  BatchDesc bd, TileMap tmap) {
  static_assert(KW == 4 || KW == 8, "four or eight waves per tile");
  // Buffers of every wave: [KW][A slice, B slice].
  __shared__ __attribute__((aligned(16))) float L0[KW * kSlice];
  __shared__ __attribute__((aligned(16))) float L1[KW * kSlice];
  using OA = Operand<TA>;   // A is K-strided when transposed
  using OB = Operand<!TB>;  // B is K-strided unless transposed
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int64_t tile = xcd_major(blockIdx.x, tmap.total);
  int64_t batch, ti, tj;
  logical_tile(tile, tmap, batch, ti, tj);
  int64_t a_off, b_off;
  batch_offsets(batch, bd, a_off, b_off);
  const int64_t m0 = ti * T, n0 = tj * T;
  const float* Ap = A + a_off + (TA ? m0 : m0 * tmap.lda);
  const float* Bp = B + b_off + (TB ? n0 * tmap.ldb : n0);

  // This wave's slices: wave, wave + KW, ...
  const int64_t slices = K / 16;
  const int64_t count = slices > wave ? (slices - wave + KW - 1) / KW : 0;
  float* const b0 = L0 + wave * kSlice;
  float* const b1 = L1 + wave * kSlice;
  auto issue = [&](int64_t t, float* buf) {
    const int64_t k0 = (wave + t * KW) * 16;
    OA::issue(Ap, tmap.lda, k0, buf, lane);
    OB::issue(Bp, tmap.ldb, k0, buf + kOperand, lane);
  };

  hpd::f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = hpd::f32x4{0.f, 0.f, 0.f, 0.f};
  // Fragments of the current slice and of the next one; the two sets swap
  // roles every slice (the loop body covers two).
  hpd::f32x4 a0[4], b0f[4], a1[4], b1f[4];
  auto read = [&](const float* buf, hpd::f32x4* fa, hpd::f32x4* fb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = OA::frag(buf, i, lane);
      fb[i] = OB::frag(buf + kOperand, i, lane);
    }
  };

  if (count > 0) issue(0, b0);
  if (count > 1) issue(1, b1);
  wait_vm<0>();
  read(b0, a0, b0f);
  // Slice t (fragments in fa, fb): once every LDS-DMA has landed (only slice
  // t + 1's can be in flight), read slice t + 1 into na, nb, then issue slice
  // t + 2's LDS-DMA into `cur` (slice t was read from it: lgkmcnt(0)), then
  // the MFMAs. No LDS read follows an LDS-DMA still in flight, so none waits
  // for one. Reads past the last slice return stale LDS and go unused; they
  // are unconditional so that the fragments stay in fixed registers.
  auto slice = [&](int64_t t, float* cur, const float* nxt, const hpd::f32x4* fa, const hpd::f32x4* fb,
                   hpd::f32x4* na, hpd::f32x4* nb) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    wait_vm<0>();
    read(nxt, na, nb);
    if (t + 2 < count) issue(t + 2, cur);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][q], fb[j][q], acc[i][j], 0, 0, 0);
  };
  int64_t t = 0;
  for (; t + 1 < count; t += 2) {
    slice(t, b0, b1, a0, b0f, a1, b1f);
    slice(t + 1, b1, b0, a1, b1f, a0, b0f);
  }
  if (t < count) slice(t, b0, b1, a0, b0f, a1, b1f);

  // Sum the KW accumulator tiles in wave order: waves [0, KW/2) stage theirs
  // in L0, the rest in L1 (16 KB each), then every thread adds whole
  // accumulator groups and stores them.
  __syncthreads();
  constexpr int kHalf = KW / 2 > 0 ? KW / 2 : 1;
  static_assert(kHalf * 16 * 64 * 4 <= KW * kSlice, "accumulators fit the slice buffers");
  auto stage = [&](int w) -> hpd::f32x4* {
    return reinterpret_cast<hpd::f32x4*>(w < kHalf ? L0 : L1) + (w % kHalf) * 16 * 64;
  };
  hpd::f32x4* mine = stage(wave);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) mine[(i * 4 + j) * 64 + lane] = acc[i][j];
  __syncthreads();
  float* Cb = C + batch * M * tmap.ldc;
  for (int e = threadIdx.x; e < 16 * 64; e += 64 * KW) {
    hpd::f32x4 sum = stage(0)[e];
#pragma unroll
    for (int w = 1; w < KW; ++w) sum += stage(w)[e];
    const int blk = e >> 6, l = e & 63;
    const int i = blk >> 2, j = blk & 3;
    const int64_t col = n0 + 16 * j + (l & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) Cb[(m0 + 16 * i + 4 * (l >> 4) + r) * tmap.ldc + col] = sum[r];
  }
}

}  // namespace narrow

// ------------------------------------------------------------------ fp64 ----

namespace f64 {

constexpr int BM = 256, BN = 128, BK = 16;
constexpr int S = BK;  // LDS row stride (doubles): 8 swizzled k pairs of 16 bytes
constexpr int kThreads = 512;
constexpr int FM = 4, FN = 4;
constexpr int WM = 64, WN = 64;

typedef double f64x4 __attribute__((ext_vector_type(4)));

// LDS rows hold 8 pairs of consecutive k values; pair p of row r is stored at
// slot p ^ ((r >> 1) & 7). Rows are 128 bytes, so 16 lanes reading one pair of
// rows r0..r0+15 (fragment reads), writing 8 pairs of 2 rows (A stores) or one
// pair of 16 rows (B stores) touch 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

// Eight waves in a 4x2 grid of 64x64 wave tiles. f64 accumulator layout: lane
// holds column lane%16, rows 4*r + lane/16.
struct Layout {
  static constexpr int kBM = BM, kBN = BN, kFM = FM, kFN = FN;
  static __device__ __forceinline__ int row(int wave, int i, int lane, int r) {
    return (wave >> 1) * WM + 16 * i + 4 * r + (lane >> 4);
  }
  static __device__ __forceinline__ int col(int wave, int j, int lane) { return (wave & 1) * WN + 16 * j + (lane & 15); }
};

// A k-contiguous fp64 operand in modes 0 and 1 (rows 16-byte aligned, host
// check): its K slice goes from global memory straight into LDS by LDS-DMA
// (dma16), as in the fp32 kernel. One instruction fills a 1 KB chunk of 8
// rows; lane l writes row 8c + l / 8 at slot l % 8, so it fetches the k pair
// that the swizzle stores there: (l % 8) ^ swizzle(row). Rows past `rows`
// read clamped addresses (mode 1; outputs never stored).
template <int ROWS, int MODE>
struct DmaLoader64 {
  static_assert(MODE != 2, "the K-edge slice needs zero fill: staged loads only");
  static_assert(kThreads == 512 && ROWS % 64 == 0, "ROWS / 64 chunks of 8 rows per wave");
  static constexpr int kChunks = ROWS / 64;  // per wave
  static constexpr int kLoads = kChunks;     // LDS-DMA instructions per wave and slice
  int chunk0, lane;

  __device__ __forceinline__ void init(int tid) {
    chunk0 = kChunks * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }

  // Byte offsets from the tile's first row: ROWS * ld * 8 < 2^31 (host check).
  __device__ __forceinline__ void issue(const double* p, int64_t r0, int64_t rows, int64_t ld, int64_t, int64_t k0,
                                        double* buf) const {
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(p + r0 * ld);
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = chunk0 + i;
      const unsigned row = 8 * c + (lane >> 3);
      const unsigned r = MODE == 0 || r0 + row < rows ? row : unsigned(rows - 1 - r0);
      const unsigned element = r * unsigned(ld) + 2 * ((lane & 7) ^ swizzle(row));
      dma16(rsrc, buf + 128 * c, 8 * element, 8 * unsigned(k0));
    }
  }
  __device__ __forceinline__ void commit(double*) const {}
  static constexpr bool kDirect = true;
  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t) { return s0 * 16; }
};

// A K-strided fp64 operand ([k][rows] in memory: B, or A transposed) in
// modes 0 and 1, k rows 16-byte aligned (host check): each k row of the tile
// (ROWS doubles, 1 KB per LDS-DMA) lands in LDS as [k][row] at a row stride
// of RS doubles. A fragment (k pair 8h + 2g + {0, 1}, row r) is two 8-byte
// reads RS apart, one ds_read2_b64 for 128-wide tiles. The 8-double pad
// puts lane groups g and g + 1 (one 32-lane serving group) 128 bytes apart
// in the banks, for both reads. Columns past the operand's end (mode 1 edge
// tiles) read as 0 through the descriptor's range check; columns past `rows`
// inside it feed outputs that are never stored.
template <int ROWS>
struct RowDma64 {
  static constexpr int kPerRow = ROWS * 8 / 1024;  // LDS-DMA instructions per k row
  static constexpr int kLoads = 16 * kPerRow / (kThreads / 64);
  static_assert(kLoads * (kThreads / 64) == 16 * kPerRow, "whole k rows per wave");
  static constexpr int RS = ROWS + 8;
  static constexpr int kBufDoubles = 16 * RS;
  int first, lane;

  __device__ __forceinline__ void init(int tid) {
    first = kLoads * __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
  }

  // Element (r, k) at p[k * ld + r0 + r]; `extent` elements from p + r0 are
  // in bounds. Byte offsets: (K * ld + ROWS) * 8 < 2^31 (host check).
  __device__ __forceinline__ void issue(const double* p, int64_t r0, int64_t extent, int64_t ld, int64_t,
                                        int64_t k0, double* buf) const {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(p + r0), 0, int(8 * extent), 0x00020000);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const unsigned t = first + i;
      const unsigned k = t / kPerRow, c = t % kPerRow;
      dma16(rsrc, buf + k * RS + 128 * c, 8 * (k * unsigned(ld) + 128 * c + 2 * lane), 8 * unsigned(k0 * ld));
    }
  }
  __device__ __forceinline__ void commit(double*) const {}
  static constexpr bool kDirect = true;
  __device__ __forceinline__ static int64_t origin(int64_t s0, int64_t ld) { return s0 * 16 * ld; }
};

// Register-staged fp64 operand slices behind the same issue/commit interface.
template <int ROWS, bool KM, int MODE>
struct Staged64 : SliceLoader<double, ROWS, KM, MODE, kThreads> {
  __device__ __forceinline__ void issue(const double* p, int64_t r0, int64_t rows, int64_t ld, int64_t kp,
                                        int64_t k0, double*) {
    this->load(p, r0, rows, ld, kp, k0);
  }
  __device__ __forceinline__ void commit(double* buf) const { this->store(buf); }
  static constexpr bool kDirect = false;
};

template <int ROWS, bool KM, int MODE>
using Loader = typename std::conditional<!KM && MODE != 2, DmaLoader64<ROWS, MODE>, Staged64<ROWS, KM, MODE>>::type;

// One workgroup per compute unit, the pipeline of the fp32 kernel: per slice,
// global loads of slice s+2 first; MFMAs of slice s in two k halves of 8,
// each A fragment refilled from LDS with slice s+1 right after its MFMAs and
// the B fragments of a half after that half; slice s+2 to LDS after half 0;
// one barrier. A lane of MFMA lane group g = lane/16 reads the k pair
// {2g, 2g+1} (half 0) or {8+2g, 9+2g} (half 1) with one ds_read_b128 and
// feeds it to two MFMAs (k-permutation shared by A and B).
template <int MODE, bool STREAM_K, bool TA, bool TB, bool ROWDMA>
__global__ __launch_bounds__(kThreads, 1) void kernel(const double* __restrict__ A, const double* __restrict__ B,
                                                      double* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                      BatchDesc bd, TileMap tmap, Split sp) {
  // ROWDMA: K-strided operands (A if TA, B unless TB) arrive by RowDma64.
  constexpr bool kRowA = TA && ROWDMA && MODE != 2, kRowB = !TB && ROWDMA && MODE != 2;
  using LA = typename std::conditional<kRowA, RowDma64<BM>, Loader<BM, TA, MODE>>::type;
  using LB = typename std::conditional<kRowB, RowDma64<BN>, Loader<BN, !TB, MODE>>::type;
  constexpr int kBufA = kRowA ? RowDma64<BM>::kBufDoubles : BM * S;
  constexpr int kBufB = kRowB ? RowDma64<BN>::kBufDoubles : BN * S;
  // Three LDS stages when both operands arrive by LDS-DMA, else two.
  constexpr int kStages = LA::kDirect && LB::kDirect ? 3 : 2;
  __shared__ __attribute__((aligned(16))) double As0[kBufA];
  __shared__ __attribute__((aligned(16))) double As1[kBufA];
  __shared__ __attribute__((aligned(16))) double As2[kStages == 3 ? kBufA : 2];
  __shared__ __attribute__((aligned(16))) double Bs0[kBufB];
  __shared__ __attribute__((aligned(16))) double Bs1[kBufB];
  __shared__ __attribute__((aligned(16))) double Bs2[kStages == 3 ? kBufB : 2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Operand slices as in the fp32 kernel. Untransposed: A as 4 double2 per
  // thread (rows tid/8 + 64i, k pair tid%8), B as 4 scalars per thread
  // (column tid%128, k rows 4*(tid/128) + {0..3}; 64 lanes read 512
  // contiguous bytes of one B row), stored as 2 pairs.
  // Edge tiles stay at their own origin and load clamped rows (modes 1, 2):
  // moving them inside, as the fp32 kernel does, measured no faster here.
  LA la;
  LB lb;
  constexpr bool kDirect = decltype(la)::kDirect || decltype(lb)::kDirect;
  la.init(tid);
  lb.init(tid);
  const int64_t lda = tmap.lda, ldb = tmap.ldb;
  // Fragment rows differ from (lane & 15) by multiples of 16: same swizzle.
  const int sw = swizzle(lane & 15), g = lane >> 4;
  // Fragment offsets per k half: swizzled k-contiguous rows, or for a row-DMA
  // operand ([k][row], stride RS) row 8h + 2g of the tile column.
  auto read_offset = [&](bool rowdma, int rs, int row0, int h) {
    return rowdma ? (8 * h + 2 * g) * rs + row0 + (lane & 15) : (row0 + (lane & 15)) * S + 2 * ((4 * h + g) ^ sw);
  };
  constexpr int kRsA = kRowA ? RowDma64<BM>::RS : S, kRsB = kRowB ? RowDma64<BN>::RS : S;
  const int a_read0 = read_offset(kRowA, kRsA, wm * WM, 0), a_read1 = read_offset(kRowA, kRsA, wm * WM, 1);
  const int b_read0 = read_offset(kRowB, kRsB, wn * WN, 0), b_read1 = read_offset(kRowB, kRsB, wn * WN, 1);
  // Fragment f of half h: a k pair of tile rows 16 f + lane % 16.
  auto frag_a = [&](const double* buf, int h, int f) {
    const double* q = buf + (h ? a_read1 : a_read0);
    if constexpr (kRowA) return hpd::f64x2{q[16 * f], q[16 * f + kRsA]};
    else return *reinterpret_cast<const hpd::f64x2*>(q + 16 * f * S);
  };
  auto frag_b = [&](const double* buf, int h, int f) {
    const double* q = buf + (h ? b_read1 : b_read0);
    if constexpr (kRowB) return hpd::f64x2{q[16 * f], q[16 * f + kRsB]};
    else return *reinterpret_cast<const hpd::f64x2*>(q + 16 * f * S);
  };

  auto piece = [&](int64_t tile, int64_t s0, int64_t s1, int64_t slot) {
    int64_t batch, ti, tj;
    logical_tile(tile, tmap, batch, ti, tj);
    int64_t a_off, b_off;
    batch_offsets(batch, bd, a_off, b_off);
    const int64_t m0 = ti * BM, n0 = tj * BN;
    const double* Ap = A + a_off + decltype(la)::origin(s0, lda);
    const double* Bp = B + b_off + decltype(lb)::origin(s0, ldb);
    const int64_t kp = K - s0 * BK;
    const int64_t slices = s1 - s0;
    // Direct (LDS-DMA) loads first, as in the fp32 kernel. Staged loaders are
    // called through SliceLoader::load itself: at the 256-VGPR limit of the
    // all-staged mode-2 kernels, one more inlined wrapper level reshuffled
    // registers into spills (transposed A: 23 -> 209 spilled VGPRs).
    auto load_slice = [&](int64_t k0, double* as, double* bs) {
      // A row-DMA operand takes its in-bounds extent from the tile's first
      // column: through the last valid element, row kp - 1, column M (N) - 1.
      if constexpr (kRowA) la.issue(Ap, m0, (kp - 1) * lda + M - m0, lda, kp, k0, as);
      else if constexpr (decltype(la)::kDirect) la.issue(Ap, m0, M, lda, kp, k0, as);
      if constexpr (kRowB) lb.issue(Bp, n0, (kp - 1) * ldb + N - n0, ldb, kp, k0, bs);
      else if constexpr (decltype(lb)::kDirect) lb.issue(Bp, n0, N, ldb, kp, k0, bs);
      if constexpr (!decltype(la)::kDirect) la.load(Ap, m0, M, lda, kp, k0);
      if constexpr (!decltype(lb)::kDirect) lb.load(Bp, n0, N, ldb, kp, k0);
    };
    auto store_slice = [&](double* as, double* bs) {
      la.commit(as);
      lb.commit(bs);
    };
    auto publish = [&] {
      if (kDirect) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
    };

    f64x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

    load_slice(0, As0, Bs0);
    store_slice(As0, Bs0);
    if (slices > 1) {
      load_slice(BK, As1, Bs1);
      store_slice(As1, Bs1);
    }
    publish();
    hpd::f64x2 a[2][FM], b[2][FN];
    // B of half 0 first: the loop's first MFMAs then wait on the same
    // in-order LDS counts as after a slice of the three-stage loop.
#pragma unroll
    for (int j = 0; j < FN; ++j) b[0][j] = frag_b(Bs0, 0, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FM; ++i) a[0][i] = frag_a(As0, 0, i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FM; ++i) a[1][i] = frag_a(As0, 1, i);
#pragma unroll
    for (int j = 0; j < FN; ++j) b[1][j] = frag_b(Bs0, 1, j);
    __builtin_amdgcn_sched_barrier(0);
    auto mfmas = [&](int h, int i) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[h][i][q], b[h][j][q], acc[i][j], 0, 0, 0);
    };
    const double* an = As1;
    const double* bn = Bs1;
    if constexpr (kStages == 3) {
      // The fp32 kernel's three-stage slice: slice s+2 goes into the third
      // buffer, issued after the first fragment's MFMAs (that fragment's
      // refill held back one fragment), unconditional refills, and a barrier
      // that waits only for the LDS-DMA it publishes.
      auto slice3 = [&](int64_t s, double* as, double* bs, const double* an, const double* bn) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            mfmas(h, i);
            if (h == 0 && i == 0) {
              if (s + 2 < slices) load_slice((s + 2) * BK, as, bs);
            } else {
              if (h == 0 && i == 1) a[0][0] = frag_a(an, 0, 0);
              a[h][i] = frag_a(an, h, i);
            }
            if (i == FM - 1) {
#pragma unroll
              for (int j = 0; j < FN; ++j) b[h][j] = frag_b(bn, h, j);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        wait_vmcnt<0>();
        dma_barrier();
      };
      double *a0 = As0, *a1 = As1, *a2 = As2, *b0 = Bs0, *b1 = Bs1, *b2 = Bs2;
      for (int64_t s = 0; s < slices; ++s) {
        slice3(s, a2, b2, an, bn);
        an = a2;
        bn = b2;
        double* t = a0;
        a0 = a1;
        a1 = a2;
        a2 = t;
        t = b0;
        b0 = b1;
        b1 = b2;
        b2 = t;
      }
    } else {
      // Slice s as in the fp32 kernel: into (as, bs), fragments from (an, bn).
      auto slice = [&](int64_t s, double* as, double* bs, const double* an, const double* bn) {
        const bool more = s + 1 < slices;
        if (s + 2 < slices) load_slice((s + 2) * BK, as, bs);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            mfmas(h, i);
            if (more) a[h][i] = frag_a(an, h, i);
          }
          if (more) {
#pragma unroll
            for (int j = 0; j < FN; ++j) b[h][j] = frag_b(bn, h, j);
          }
          if (h == 0 && s + 2 < slices) store_slice(as, bs);
        }
        publish();
      };
      // Every wave has read buffer 0 before slice 0 refills it: the barrier
      // under the loop's guard, and the carried buffers, as in the fp32
      // kernel.
      if (slices > 0) __syncthreads();
      for (int64_t s = 0; s < slices; ++s) {
        const bool odd = s & 1;
        slice(s, odd ? As1 : As0, odd ? Bs1 : Bs0, an, bn);
        an = odd ? As1 : As0;
        bn = odd ? Bs1 : Bs0;
      }
    }

    if (slot < 0) {
      double* Cb = C + batch * M * tmap.ldc;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t col = n0 + Layout::col(wave, j, lane);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + Layout::row(wave, i, lane, r);
            if (MODE == 0 || (row < M && col < N)) Cb[row * tmap.ldc + col] = acc[i][j][r];
          }
        }
      }
    } else {
      f64x4* out = static_cast<f64x4*>(sp.partial) + slot * (BM * BN / 4);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) out[((wave * FM + i) * FN + j) * 64 + lane] = acc[i][j];
    }
  };

  if (!STREAM_K) {
    piece(xcd_major(blockIdx.x, sp.dp_tiles), 0, sp.slices, -1);
  } else {
    const int64_t worker = xcd_major(blockIdx.x, sp.workers);
    const int64_t g0 = sk_begin(sp, worker), g_end = sk_begin(sp, worker + 1);
    const int64_t t0 = g0 / sp.slices;
    const int64_t s0 = g0 - t0 * sp.slices;
    const int64_t s1 = g_end - t0 * sp.slices < sp.slices ? g_end - t0 * sp.slices : sp.slices;
    // Start of the next tile first, as in the f32 kernel (L2 sharing).
    const int64_t rest = g_end - (t0 + 1) * sp.slices;
    if (rest > 0) piece(sp.dp_tiles + t0 + 1, 0, rest, rest == sp.slices ? -1 : worker * 2 + 1);
    piece(sp.dp_tiles + t0, s0, s1, s0 == 0 && s1 == sp.slices ? -1 : worker * 2);
  }
}

}  // namespace f64

// Adds the cut pieces of each stream-K tile in K order (workers in increasing
// order own increasing K ranges) and stores the tile. Tiles that one worker
// covered whole were stored by it. A thread handles kFixupVectors
// accumulator 4-vectors kFixupThreads apart (loads of all its pieces issued
// before the adds); a workgroup covers kFixupThreads * kFixupVectors vectors
// of one tile.
constexpr int kFixupThreads = 256;
constexpr int kFixupVectors = 4;

template <typename T, typename V, typename L>
__global__ __launch_bounds__(kFixupThreads) void fixup_kernel(T* __restrict__ C, int64_t M, int64_t N, TileMap tmap,
                                                              Split sp) {
  constexpr int BM = L::kBM, BN = L::kBN, FM = L::kFM, FN = L::kFN;
  constexpr int kVectors = BM * BN / 4;
  constexpr int kBlocksPerTile = kVectors / (kFixupThreads * kFixupVectors);
  static_assert(kBlocksPerTile * kFixupThreads * kFixupVectors == kVectors, "whole blocks per tile");
  const int64_t tl = blockIdx.x / kBlocksPerTile;
  const int v0 = (blockIdx.x % kBlocksPerTile) * (kFixupThreads * kFixupVectors) + threadIdx.x;
  const int64_t g0 = tl * sp.slices;
  const int64_t w0 = sk_worker(sp, g0), w1 = sk_worker(sp, g0 + sp.slices - 1);
  if (w0 == w1) return;
  const V* partial = static_cast<const V*>(sp.partial);
  // w0 holds the tile's K start: as its first piece when its run starts
  // there, else as its last. Later workers start inside the tile.
  const int64_t first = (w0 * 2 + (sk_begin(sp, w0) == g0 ? 0 : 1)) * kVectors;
  V sum[kFixupVectors];
#pragma unroll
  for (int q = 0; q < kFixupVectors; ++q) sum[q] = partial[first + v0 + q * kFixupThreads];
  for (int64_t w = w0 + 1; w <= w1; ++w) {
    V part[kFixupVectors];
#pragma unroll
    for (int q = 0; q < kFixupVectors; ++q) part[q] = partial[w * 2 * kVectors + v0 + q * kFixupThreads];
#pragma unroll
    for (int q = 0; q < kFixupVectors; ++q) sum[q] = sum[q] + part[q];
  }
  int64_t batch, ti, tj;
  logical_tile(sp.dp_tiles + tl, tmap, batch, ti, tj);
  T* Cb = C + batch * M * tmap.ldc;
  // The tile was computed at its (possibly moved) origin, as in the kernels.
  const int64_t m0 = ti * BM, n0 = tj * BN;
  const int64_t mo = sp.moved ? tile_origin(m0, M, BM) : m0, no = sp.moved ? tile_origin(n0, N, BN) : n0;
#pragma unroll
  for (int q = 0; q < kFixupVectors; ++q) {
    const int v = v0 + q * kFixupThreads;
    const int lane = v & 63;
    const int block = v >> 6;
    const int wave = block / (FM * FN);
    const int i = (block / FN) % FM;
    const int j = block % FN;
    const int64_t col = no + L::col(wave, j, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = mo + L::row(wave, i, lane, r);
      if (row >= m0 && row < M && col >= n0 && col < N) Cb[row * tmap.ldc + col] = sum[q][r];
    }
  }
}


void prepare(int64_t m, int64_t n, int64_t batch, int64_t bm, int64_t bn, TileMap& tm, int64_t lda, int64_t ldb,
             int64_t ldc) {
  tm.lda = lda;
  tm.ldb = ldb;
  tm.ldc = ldc;
  tm.tiles_m = hp::ceil_div(m, bm);
  tm.tiles_n = hp::ceil_div(n, bn);
  tm.tiles_per_batch = tm.tiles_m * tm.tiles_n;
  tm.total = tm.tiles_per_batch * batch;
  hp::require(tm.total <= hp::kMaxGrid, "GEMM has too many tiles for one launch");
}

// Workgroups of `kernel` resident per compute unit, queried once per kernel.
template <typename F>
int resident_per_cu(F kernel, int threads) {
  static std::mutex mutex;
  static std::unordered_map<const void*, int> known;
  const void* key = reinterpret_cast<const void*>(kernel);
  std::lock_guard<std::mutex> lock(mutex);
  auto it = known.find(key);
  if (it != known.end()) return it->second;
  int blocks = 0;
  HP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, 0));
  hp::require(blocks > 0, "GEMM kernel does not fit on a compute unit");
  known.emplace(key, blocks);
  return blocks;
}

// Whole tiles for every complete round of cus * per_cu resident workgroups;
// the tiles of an incomplete last round go to stream-K unless that round is
// nearly full or K is too short to cut. Every stream-K run writes two
// partial tiles that the fixup reads back, so fewer, longer runs can win
// over filling every slot: runs of kLongRun slices, but each compute unit
// one run of at least kShortRun, and at most two runs per compute unit (or
// one per cut tile, if more). Measured on one MI355X, TFLOP/s: 128 x 128
// tiles of 1024^3 62 / 66 / 46 with runs of 8 / 16 / 32 slices (512 / 256 /
// 128 workers); 1024 x 1024 x 4096 96 with three workers per compute unit,
// 104 with two; 256 x 256 tiles of 512 x 512 x 8192 56 with 256 runs of 8,
// 52 with 128 of 16.
Split plan_split(int64_t total, int64_t slices, int64_t cus, int64_t per_cu) {
  Split sp{};
  sp.dp_tiles = total;
  sp.slices = slices;
  const int64_t slots = cus * per_cu;
  const int64_t rem = total % slots;
  if (rem == 0 || 8 * rem >= 7 * slots || slices < 2 * kShortRun) return sp;
  sp.dp_tiles = total - rem;
  const int64_t work = rem * slices;
  const int64_t cap = std::max(cus * std::min<int64_t>(per_cu, 2), rem);
  const int64_t want = std::max(work / kLongRun, std::min(cus, work / kShortRun));
  sp.workers = std::min(cap, std::max<int64_t>(1, want));
  // One worker per cut tile runs whole tiles: no pieces, no fixup.
  if (sp.workers == rem) {
    sp.dp_tiles = total;
    sp.workers = 0;
    return sp;
  }
  sp.base = work / sp.workers;
  sp.extra = work % sp.workers;
  // The kernels handle runs of at most one tile (two pieces). Both cap and
  // want are at least rem (slices >= kLongRun), and workers > rem here, so
  // base < slices.
  if (sp.base + (sp.extra > 0 ? 1 : 0) > slices) hp::fail(HP_E_HIP, "internal: stream-K run longer than a tile");
  return sp;
}

// Points ctx->stream at the side stream for the lifetime of the object (the
// launch helpers enqueue on ctx->stream), restoring the main stream after.
struct SideStream {
  hp_ctx* ctx;
  hipStream_t main;
  explicit SideStream(hp_ctx* c) : ctx(c), main(c->stream) { ctx->stream = ctx->side; }
  ~SideStream() { ctx->stream = main; }
};

// Joins the side stream back into the main one when it leaves scope (work
// queued on the main stream afterwards waits for the side stream's), then
// frees the side stream's pool temporaries, whose frees are ordered on the
// main stream. Errors while joining are not thrown from the destructor: a
// failed event call leaves the HIP error for the next checked call.
struct SideJoin {
  hp_ctx* ctx;
  std::vector<void*> deferred;
  explicit SideJoin(hp_ctx* c) : ctx(c) {}
  ~SideJoin() {
    if (hipEventRecord(ctx->join, ctx->side) != hipSuccess || hipStreamWaitEvent(ctx->stream, ctx->join, 0) != hipSuccess)
      (void)hipStreamSynchronize(ctx->side);
    for (void* p : deferred) {
      try {
        hp::scratch_free(ctx, p);
      } catch (...) {
      }
    }
  }
};

// Launches the whole-tile kernel over the complete rounds and, if tiles are
// cut, the stream-K kernel and the fixup over a pooled workspace.
template <typename T, int BM, int BN, typename Whole, typename Cut, typename Fix>
void launch_split(hp_ctx* ctx, Whole whole, Cut cut, Fix fixup, int threads, const T* a, const T* b, T* c,
                  int64_t m, int64_t n, int64_t k, const BatchDesc& bd, const TileMap& tm, int64_t bk,
                  const char* name, bool moved) {
  const int per_cu = std::min(resident_per_cu(whole, threads), resident_per_cu(cut, threads));
  Split sp = plan_split(tm.total, hp::ceil_div(k, bk), ctx->compute_units, per_cu);
  sp.moved = moved;
  if (sp.dp_tiles > 0) {
    whole<<<sp.dp_tiles, threads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm, sp);
    hp::check_launch(name);
  }
  if (sp.workers > 0) {
    sp.partial = hp::scratch_alloc(ctx, size_t(sp.workers) * 2 * BM * BN * sizeof(T));
    cut<<<sp.workers, threads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm, sp);
    hp::check_launch(name);
    fixup<<<(tm.total - sp.dp_tiles) * (BM * BN / 4 / (kFixupThreads * kFixupVectors)), kFixupThreads, 0, ctx->stream>>>(
        c, m, n, tm, sp);
    hp::check_launch(name);
    hp::scratch_free(ctx, sp.partial);
  }
}

// Mode of a product: 0 interior, 1 M/N edges, 2 any K (see the kernels).
// 0: whole tiles; 1: K whole, edge tiles moved inside M, N >= one tile;
// 2: a K edge (zero fill) or an axis shorter than a tile (clamped rows).
int mode_of(int64_t m, int64_t n, int64_t k, int64_t bm, int64_t bn, int64_t bk) {
  if (k % bk != 0 || m < bm || n < bn) return 2;
  return m % bm == 0 && n % bn == 0 ? 0 : 1;
}

// The fp64 kernels' modes 0 and 1 and the narrow fp32 kernel load the
// k-contiguous operands (A unless TA, B if TB) with 16-byte LDS-DMA under a
// 16-byte row alignment contract. K % 16 == 0 in those modes, so rows inside
// a matrix follow from its origin: the base pointer and each batch stride
// must be multiples of 16 bytes. (The fp32 tiled kernels' 16-byte LDS-DMA
// runs at any element alignment: the memory path takes 4-byte aligned
// addresses, as the unaligned-operand tests check.)
template <typename T, bool TA, bool TB>
bool dma_aligned(const T* a, const T* b, const BatchDesc& bd) {
  auto aligned = [&](const T* p, const int64_t* strides) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    for (int d = 0; d < bd.rank; ++d)
      if ((strides[d] * int64_t(sizeof(T))) % 16 != 0) return false;
    return true;
  };
  return (TA || aligned(a, bd.a_stride)) && (!TB || aligned(b, bd.b_stride));
}

// The buffer-form LDS-DMA addresses an operand with 32-bit byte offsets
// from its tile origin: a k-contiguous operand (A unless TA, B if TB) spans
// rows * ld + k elements from there, a K-strided one k * ld + rows. Both
// below 2^31 bytes, else the register-staged mode-2 loads serve the product.
template <bool TA, bool TB>
bool dma_offsets_fit(int64_t k, int64_t lda, int64_t ldb, int64_t bm, int64_t bn, int64_t size = 4) {
  auto fits = [&](int64_t elements) { return elements < (int64_t(1) << 31) / size; };
  const int64_t a_span = TA ? k * lda + bm : bm * lda + k;
  const int64_t b_span = TB ? bn * ldb + k : k * ldb + bn;
  return fits(a_span) && fits(b_span);
}

// The narrow kernel's row LDS-DMA contract: every k row of the K-strided
// operand (A if TA, B unless TB) 16-byte aligned: the base pointer and each
// batch stride, the leading dimension, and the tile origins along the rows.
template <bool TA, bool TB>
bool rows_aligned(const float* a, const float* b, const BatchDesc& bd, int64_t m, int64_t n, int64_t lda,
                  int64_t ldb) {
  auto aligned = [&](const float* p, const int64_t* strides, int64_t ld, int64_t extent) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0 || ld % 4 != 0 || extent % 4 != 0) return false;
    for (int d = 0; d < bd.rank; ++d)
      if (strides[d] % 4 != 0) return false;
    return true;
  };
  return (!TA || aligned(a, bd.a_stride, lda, m)) && (TB || aligned(b, bd.b_stride, ldb, n));
}

// The tiled MFMA product over an m x n block with one tile configuration.
template <class CFG, bool TA, bool TB>
void run_f32_config(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                    const BatchDesc& bd, int64_t batch, int64_t lda, int64_t ldb, int64_t ldc) {
  using namespace f32;
  constexpr int BM = CFG::BM, BN = CFG::BN, T = CFG::kThreads;
  // A K-strided operand (A if TA, B unless TB) goes by 16-byte row LDS-DMA
  // in modes 0 and 1; both operands by LDS-DMA in mode 2 when the 32-bit
  // offsets fit. The 16-byte LDS-DMA needs 4-byte aligned addresses only.
  constexpr bool kRows = TA || !TB;
  TileMap tm;
  prepare(m, n, batch, BM, BN, tm, lda, ldb, ldc);
  auto fix = fixup_kernel<float, hpd::f32x4, Layout<CFG>>;
  int mode = mode_of(m, n, k, BM, BN, BK);
  const bool fits = dma_offsets_fit<TA, TB>(k, lda, ldb, BM, BN);
  if (!fits) mode = 2;
  const bool rows = kRows && mode != 2;
  auto run = [&](auto whole, auto cut, bool moved) {
    launch_split<float, BM, BN>(ctx, whole, cut, fix, T, a, b, c, m, n, k, bd, tm, BK, "gemm_f32", moved);
  };
  // The register-staged loaders (K-strided operands without row DMA, mode 2
  // operands past the 32-bit DMA offsets) take tiles of THREADS / 2 rows;
  // other configurations run only where the DMA loaders serve both operands
  // (callers check the offsets).
  constexpr bool kStaged = 2 * BM == T && 2 * BN == T;
  if (mode == 0 && rows) {
    run(kernel<CFG, 0, false, TA, TB, kRows>, kernel<CFG, 0, true, TA, TB, kRows>, false);
  } else if (mode == 1 && rows) {
    run(kernel<CFG, 1, false, TA, TB, kRows>, kernel<CFG, 1, true, TA, TB, kRows>, true);
  } else if (mode == 2 && fits) {
    // 4-byte LDS-DMA of both operands at any alignment, edges loading +0.
    run(kernel<CFG, 2, false, TA, TB, true>, kernel<CFG, 2, true, TA, TB, true>, true);
  } else if constexpr (kStaged || !kRows) {
    if (mode == 0) {
      run(kernel<CFG, 0, false, TA, TB, false>, kernel<CFG, 0, true, TA, TB, false>, false);
    } else if (mode == 1) {
      run(kernel<CFG, 1, false, TA, TB, false>, kernel<CFG, 1, true, TA, TB, false>, true);
    } else if constexpr (kStaged) {
      run(kernel<CFG, 2, false, TA, TB, false>, kernel<CFG, 2, true, TA, TB, false>, true);
    } else {
      hp::fail(HP_E_HIP, "internal: tile configuration without staged loaders");
    }
  } else {
    hp::fail(HP_E_HIP, "internal: tile configuration without staged loaders");
  }
}

// Tile choice. Big unless its tiles fill less than two rounds of the chip,
// leave the last one partly filled (stream-K then cuts them) and the product
// is short: at most 64 K slices, or at most a quarter round of tiles and 256
// slices. Small has four times the tiles at three workgroups per compute
// unit but moves twice the operand bytes per flop, so it loses where Big
// runs whole rounds (4096 x 4096 x 1024: 114 against 133 TFLOP/s) and where
// stream-K runs are long. Measured on one MI355X, TFLOP/s Big / Small:
//   1536^3 86 / 94, 1024 x 1024 x 4096 96 / 105, 2048^3 113 / 116,
//   64 x (512 x 1024 @ 1024 x 768) 126 / 128, 6144 x 4096 x 1024 126 / 128;
//   2048 x 2048 x 4096 127 / 124, 3072^2 x 1024 110 / 92,
//   4097 x 3001 x 2049 116 / 111, 8192 x 1024 x 4096 134 / 130.
inline bool small_tiles(hp_ctx* ctx, int64_t m, int64_t n, int64_t k, int64_t batch) {
  using f32::Big;
  using f32::Small;
  const int64_t tiles = hp::ceil_div(m, Big::BM) * hp::ceil_div(n, Big::BN) * batch;
  const int64_t cus = ctx->compute_units, slices = hp::ceil_div(k, f32::BK);
  if (tiles >= 2 * cus || tiles % cus == 0) return false;
  // Small runs three workgroups per compute unit; a partly filled round of
  // more than two per compute unit runs whole tiles unevenly (3072^2 x 1024:
  // 95 against Big's 110 TFLOP/s).
  const int64_t small = hp::ceil_div(m, Small::BM) * hp::ceil_div(n, Small::BN) * batch;
  if (small > 2 * cus && small % (3 * cus) != 0) return false;
  return slices <= 64 || (4 * tiles <= cus && slices <= 256);
}

// The narrow kernel's interior contract: M and N multiples of 64, K of 16,
// every operand row 16-byte aligned (LDS-DMA of both operands).
template <bool TA, bool TB>
bool narrow_fits(const float* a, const float* b, const BatchDesc& bd, int64_t m, int64_t n, int64_t k, int64_t lda,
                 int64_t ldb) {
  return m % narrow::T == 0 && n % narrow::T == 0 && k % 16 == 0 && k > 0 && lda % 4 == 0 && ldb % 4 == 0 &&
         dma_aligned<float, TA, TB>(a, b, bd) && rows_aligned<TA, TB>(a, b, bd, m, n, lda, ldb) &&
         dma_offsets_fit<TA, TB>(k, lda, ldb, narrow::T, narrow::T);
}

// Narrow tiles for short products that the 64 x 64 tiles spread over the
// chip: one to four tiles per compute unit and at most 2^23 multiply-adds
// per compute unit. There the narrow kernel's missing stream-K and fixup
// launch outweigh its lower MFMA rate; on longer products the 256 x 256 and
// 128 x 128 kernels win. Measured on one MI355X, TFLOP/s narrow / otherwise:
//   1024^3 90 / 67, 1024 x 1024 x 2048 97 / 86, 2048 x 2048 x 512 90 / 82;
//   1024 x 1024 x 4096 105 / 105, 2048 x 2048 x 1024 101 / 103,
//   1536^3 78 / 95, 512 x 512 x 8192 27 / 55, 8 x 1024^3 106 / 119.
// Waves per tile: eight (two per SIMD; their 136 KiB of LDS leave room for
// one workgroup per compute unit) where there is one tile per compute unit,
// else four (two workgroups per compute unit). Against four waves, us per
// product: 1024^3 20.8 -> 20.3 and 1024 x 1024 x 2048 37.3 -> 36.3 with
// eight; 2048 x 2048 x 512 (four tiles per compute unit) 39.7 against 47.0.

inline bool narrow_tiles(hp_ctx* ctx, int64_t m, int64_t n, int64_t k, int64_t batch) {
  const int64_t cus = ctx->compute_units;
  const int64_t tiles = hp::ceil_div(m, narrow::T) * hp::ceil_div(n, narrow::T) * batch;
  if (tiles < cus || tiles > 4 * cus) return false;
  // m n k batch <= 2^23 cus, without overflow (each factor < 2^31 here).
  const double work = double(m) * double(n) * double(k) * double(batch);
  return work <= double(cus) * double(int64_t(1) << 23);
}

template <bool TA, bool TB>
void run_f32_narrow(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                    const BatchDesc& bd, int64_t batch, int64_t lda, int64_t ldb, int64_t ldc) {
  TileMap tm;
  prepare(m, n, batch, narrow::T, narrow::T, tm, lda, ldb, ldc);
  if (tm.total <= ctx->compute_units)
    narrow::kernel<TA, TB, 8><<<tm.total, 64 * 8, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  else
    narrow::kernel<TA, TB, 4><<<tm.total, 64 * 4, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm);
  hp::check_launch("gemm_f32");
}

// Wide tiles where Big's fill part of one round (all of them then cut into
// stream-K runs and summed by a fixup launch) while Wide's fill 7/8 of one
// round or more, whole. Measured on one MI355X, TFLOP/s Wide / Big:
//   4096 x 3001 x 2049 128.9 / 121.0, 2048 x 6000 x 1024 126.6 / 118.5,
//   4000 x 2900 x 3001 123.3 / 119.7, 4096 x 3072 x 2048 133.3 / 133.6;
// where Big's tiles span more than one round only the last is cut and the
// whole-tile Wide product loses (4096 x 6000 x 1024, two Wide rounds:
// 127.5 / 129.2), and so do 256 x 128 tiles against Big's cut ones (4096 x
// 2048 x 3008: 129.3 / 136.5).
inline bool wide_tiles(hp_ctx* ctx, int64_t m, int64_t n, int64_t batch) {
  using f32::Big;
  using f32::Wide;
  const int64_t cus = ctx->compute_units;
  const int64_t big = hp::ceil_div(m, Big::BM) * hp::ceil_div(n, Big::BN) * batch;
  const int64_t wide = hp::ceil_div(m, Wide::BM) * hp::ceil_div(n, Wide::BN) * batch;
  return big < cus && wide <= cus && 8 * wide >= 7 * cus;
}

// Whole Wide tiles, one launch: 4-byte LDS-DMA at any alignment, edges load
// +0 (the mode 2 kernel), no stream-K.
template <bool TA, bool TB>
void run_f32_wide(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                  const BatchDesc& bd, int64_t batch, int64_t lda, int64_t ldb, int64_t ldc) {
  using namespace f32;
  TileMap tm;
  prepare(m, n, batch, Wide::BM, Wide::BN, tm, lda, ldb, ldc);
  Split sp{};
  sp.dp_tiles = tm.total;
  sp.slices = hp::ceil_div(k, BK);
  kernel<Wide, 2, false, TA, TB, true><<<tm.total, Wide::kThreads, 0, ctx->stream>>>(a, b, c, m, n, k, bd, tm, sp);
  hp::check_launch("gemm_f32");
}

// Half tiles where Big's fill part of one round (all of them cut into
// stream-K runs and summed by a fixup launch) while Half's fill 7/8 of one
// round or more, whole, and K holds more than 64 slices. Measured on one
// MI355X, microseconds Half / before (Big cut by stream-K, or Small):
//   4096 x 3001 x 2048 367.8 / 381.3, 4097 x 3001 x 2049 385.5 / 406.2,
//   8192 x 4096 x 1024 477.8 / 493.2, 2048 x 4096 x 4096 477.6 / 491.4,
//   4096 x 2048 x 1920 244.5 / 261.4, 3840 x 2048 x 2048 250.9 / 257.7;
// with 64 slices or fewer they are even or behind (2048 x 1024 x 4096
// 138.0 / 136.0, 4096 x 1024 x 2048 135.3 / 134.0, 4096 x 256 x 2048
// 41.4 / 41.1).
inline bool half_tiles(hp_ctx* ctx, int64_t m, int64_t n, int64_t k, int64_t batch) {
  using f32::Big;
  using f32::Half;
  const int64_t cus = ctx->compute_units;
  const int64_t big = hp::ceil_div(m, Big::BM) * hp::ceil_div(n, Big::BN) * batch;
  const int64_t half = hp::ceil_div(m, Half::BM) * hp::ceil_div(n, Half::BN) * batch;
  return big < cus && half <= cus && 8 * half >= 7 * cus && hp::ceil_div(k, f32::BK) > 64;
}

template <bool TA, bool TB>
void run_f32_tiles(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                   const BatchDesc& bd, int64_t batch, int64_t lda, int64_t ldb, int64_t ldc) {
  if (narrow_tiles(ctx, m, n, k, batch) && narrow_fits<TA, TB>(a, b, bd, m, n, k, lda, ldb)) {
    run_f32_narrow<TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, ldc);
  } else if (wide_tiles(ctx, m, n, batch) &&
             dma_offsets_fit<TA, TB>(k, lda, ldb, f32::Wide::BM, f32::Wide::BN)) {
    run_f32_wide<TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, ldc);
  } else if (half_tiles(ctx, m, n, k, batch) &&
             dma_offsets_fit<TA, TB>(k, lda, ldb, f32::Half::BM, f32::Half::BN)) {
    run_f32_config<f32::Half, TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, ldc);
  } else if (small_tiles(ctx, m, n, k, batch)) {
    run_f32_config<f32::Small, TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, ldc);
  } else {
    run_f32_config<f32::Big, TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, ldc);
  }
}

// A 2-D product (any operand layout) whose last tile row (column) would hold
// at most kEdgeMax rows (columns) runs as three parts: the MFMA kernel on the
// whole tiles, the edge columns strip for the other rows, the edge rows strip
// for every column (gemm_edges.hip). The same split for every layout keeps a
// product of transposed operands bit-identical to the product of their
// materialized transposes. Otherwise the whole product is tiled, edge tiles
// included.
template <bool TA, bool TB>
void run_f32(hp_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
             const BatchDesc& bd, int64_t batch) {
  constexpr int64_t BM = f32::Big::BM, BN = f32::Big::BN;
  const int64_t lda = TA ? m : k, ldb = TB ? k : n;
  if (batch == 1) {
    const int64_t rows = m % BM, cols = n % BN;
    const bool split_rows = m > BM && rows > 0 && rows <= hpgemm::kEdgeMax;
    const bool split_cols = n > BN && cols > 0 && cols <= hpgemm::kEdgeMax;
    if (split_rows || split_cols) {
      const int64_t mt = split_rows ? m - rows : m, nt = split_cols ? n - cols : n;
      // op(A)(r, k) and op(B)(k, n) in the stored layouts.
      const hpgemm::Strides st{TA ? 1 : k, TA ? m : 1, TB ? 1 : n, TB ? k : 1};
      // The strips write outputs the tiles do not and read only A and B, so
      // they run on the side stream beside the tiled kernels: a few dozen
      // small workgroups among the tiles' one per compute unit cost the
      // tiles little, where run after them they and the launch gaps between
      // them added a tenth to the product. The main stream waits for them
      // before its next work; their pool temporaries are freed after that.
      HP_CHECK(hipEventRecord(ctx->fork, ctx->stream));
      HP_CHECK(hipStreamWaitEvent(ctx->side, ctx->fork, 0));
      SideJoin join(ctx);  // also on an error part way
      {
        SideStream on_side(ctx);
        if (split_cols) hpgemm::edge_cols_f32(ctx, a, b + nt * st.bs_n, c + nt, mt, int(cols), k, st, n, &join.deferred);
        if (split_rows) hpgemm::edge_rows_f32(ctx, a + mt * st.as_r, b, c + mt * n, int(rows), n, k, st, n, &join.deferred);
      }
      run_f32_tiles<TA, TB>(ctx, a, b, c, mt, nt, k, bd, 1, lda, ldb, n);
      return;
    }
  }
  run_f32_tiles<TA, TB>(ctx, a, b, c, m, n, k, bd, batch, lda, ldb, n);
}

template <bool TA, bool TB>
void run_f64(hp_ctx* ctx, const double* a, const double* b, double* c, int64_t m, int64_t n, int64_t k,
             const BatchDesc& bd, int64_t batch) {
  using namespace f64;
  TileMap tm;
  const int64_t lda = TA ? m : k, ldb = TB ? k : n;
  prepare(m, n, batch, BM, BN, tm, lda, ldb, n);
  auto fix = fixup_kernel<double, f64x4, Layout>;
  int mode = mode_of(m, n, k, BM, BN, BK);
  if (!dma_aligned<double, TA, TB>(a, b, bd) || !dma_offsets_fit<TA, TB>(k, lda, ldb, BM, BN, sizeof(double)))
    mode = 2;
  // RowDma64 takes the K-strided operands (A if TA, B unless TB) when each of
  // their k rows starts 16-byte aligned.
  auto rows_aligned = [&] {
    auto aligned = [&](const double* p, const int64_t* strides, int64_t ld) {
      if (reinterpret_cast<uintptr_t>(p) % 16 != 0 || ld % 2 != 0) return false;
      for (int d = 0; d < bd.rank; ++d)
        if (strides[d] % 2 != 0) return false;
      return true;
    };
    return (!TA || aligned(a, bd.a_stride, lda)) && (TB || aligned(b, bd.b_stride, ldb));
  };
  auto run = [&](auto whole, auto cut) {
    launch_split<double, BM, BN>(ctx, whole, cut, fix, kThreads, a, b, c, m, n, k, bd, tm, BK, "gemm_f64", false);
  };
  const bool rows = mode != 2 && rows_aligned();
  if (mode == 0 && rows) run(kernel<0, false, TA, TB, true>, kernel<0, true, TA, TB, true>);
  else if (mode == 0) run(kernel<0, false, TA, TB, false>, kernel<0, true, TA, TB, false>);
  else if (mode == 1 && rows) run(kernel<1, false, TA, TB, true>, kernel<1, true, TA, TB, true>);
  else if (mode == 1) run(kernel<1, false, TA, TB, false>, kernel<1, true, TA, TB, false>);
  else run(kernel<2, false, TA, TB, false>, kernel<2, true, TA, TB, false>);
}

}  // namespace
