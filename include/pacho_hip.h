/*
 * pacho_hip.h - C ABI of libpacho_hip.so, the MI355X (gfx950) engine behind
 * OpenPacho's `hip` backend.
 *
 * Conventions
 *   - Every entry point returns int: 0 on success, a nonzero HP_E_* code on
 *     failure. The message of the last failure on the calling thread is
 *     available from hp_last_error().
 *   - Sizes and element counts are int64_t; strides are in elements.
 *   - Device pointers are plain `void*` obtained from hp_alloc().
 *   - All device work of one context is ordered on that context's
 *     non-blocking stream. (A GEMM may run independent kernels on a second,
 *     context-owned stream; that stream is forked from and joined back into
 *     the main one inside the call, so ordering is as if on one stream.)
 *     Entry points that launch kernels return as soon as the work is
 *     enqueued; hp_d2h() and hp_sync() wait for it. A context is used from
 *     one host thread at a time.
 *   - No entry point reads an output buffer before writing it, and none writes
 *     to an input buffer.
 *
 * Each entry point names the reference interface it replaces. Reference
 * paths are relative to diegoxfx/open-pacho `src/openpacho/`.
 */
#ifndef PACHO_HIP_H
#define PACHO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define HP_OK 0
#define HP_E_INVALID 1     /* bad argument (shape, dtype, pointer, size cap) */
#define HP_E_HIP 2         /* HIP runtime failure (message holds the HIP error) */
#define HP_E_OOM 3         /* device allocation failed after releasing the cache */
#define HP_E_RTC 4         /* hipRTC compilation failure (message holds the log) */
#define HP_E_UNSUPPORTED 5 /* dtype/operation not provided by this library */
#define HP_E_INJECTED 6    /* failure forced by hp_debug_fail_next() */

/* Element types (values are stable ABI). */
#define HP_BOOL 0
#define HP_I32 1
#define HP_I64 2
#define HP_U32 3
#define HP_U64 4
#define HP_F32 5
#define HP_F64 6

/* Distributions of the counter-based generator. */
#define HP_RANDOM 0
#define HP_UNIFORM 1
#define HP_NORMAL 2
#define HP_EXPONENTIAL 3

/* Reduction operations. */
#define HP_SUM 0
#define HP_MIN 1
#define HP_MAX 2

typedef struct hp_ctx hp_ctx;
typedef struct hp_kernel hp_kernel;
typedef struct hp_event hp_event;

/* ---- errors and discovery ------------------------------------------------ */

/* Message of the last failed call on this thread ("" if none).
 * Replaces: _cuda.py:49-53 (_check -> RuntimeError text). */
const char* hp_last_error(void);

/* Library version string, e.g. "pacho_hip 0.1.0 gfx950". */
const char* hp_version(void);

/* Number of visible HIP devices. Replaces: _cuda.py:68-94 (cuda_devices). */
int hp_device_count(int* count);

/* Name, gfx architecture, memory, CU count and fp64 capability of a device.
 * Replaces: _cuda.py:68-94 (DeviceInfo fields). */
int hp_device_info(int device, char* name, int64_t name_len, char* arch, int64_t arch_len,
                   int64_t* total_bytes, int* compute_units, int* fp64);

/* ---- context, memory, transfers ------------------------------------------ */

/* Create a context on `device`: a non-blocking stream (and a second one for
 * work forked and joined inside a call), a stream-ordered caching pool and a
 * hipRTC module table.
 * Replaces: _cuda.py:138-199 (CUDABackend.__init__). */
int hp_init(int device, hp_ctx** out);

/* Wait for the stream, free every cached and live allocation and RTC module.
 * Replaces: _cuda.py:644-673 (close). */
int hp_destroy(hp_ctx* ctx);

/* Allocate `bytes` (>= 1) of device memory from the pool (256-byte aligned).
 * Replaces: _cuda.py:241-256 (empty). */
int hp_alloc(hp_ctx* ctx, int64_t bytes, void** out);

/* Return an allocation to the pool. Safe while kernels that use it are still
 * queued: every later use is ordered after them on the same stream.
 * Replaces: _cuda.py:258-278 (_recycle). */
int hp_free(hp_ctx* ctx, void* ptr);

/* Synchronize and free every cached (not live) block.
 * Replaces: _cuda.py:280-291 (release_cached_memory). */
int hp_release_cached(hp_ctx* ctx);

/* Upper bound on cached bytes; larger frees go straight back to HIP. */
int hp_set_pool_limit(hp_ctx* ctx, int64_t bytes);

/* Pool counters: cached bytes, cached blocks, live bytes, live blocks. */
int hp_pool_stats(hp_ctx* ctx, int64_t* cached_bytes, int64_t* cached_items, int64_t* live_bytes,
                  int64_t* live_items);

/* Host -> device copy, complete when the call returns (the host buffer may be
 * reused at once). Replaces: _cuda.py:293-303 (upload). */
int hp_h2d(hp_ctx* ctx, void* dst, const void* src, int64_t bytes);

/* Device -> host copy after all queued work. Replaces: _cuda.py:305-311. */
int hp_d2h(hp_ctx* ctx, void* dst, const void* src, int64_t bytes);

/* Device -> device copy, stream ordered. */
int hp_d2d(hp_ctx* ctx, void* dst, const void* src, int64_t bytes);

/* Wait for all queued work. Replaces: _cuda.py:232-235 (_synchronize). */
int hp_sync(hp_ctx* ctx);

/* ---- fills, copies, gathers ---------------------------------------------- */

/* dst[0..count) = the `elem_bytes`-wide little-endian pattern `bits`
 * (elem_bytes in {1,2,4,8}). Replaces: _cuda.py:404-414 (full). */
int hp_fill(hp_ctx* ctx, void* dst, int64_t count, int elem_bytes, uint64_t bits);

/* Strided gather: dst[i] = src[offset + sum_d idx_d(i) * strides[d]] with
 * idx the C-order coordinates of i in `shape` (rank <= 8, strides may be
 * negative). Bit copy of `elem_bytes`-wide words.
 * Replaces: _cuda.py:436-447 (gather). */
int hp_gather(hp_ctx* ctx, int elem_bytes, const void* src, void* dst, int64_t offset, int rank,
              const int64_t* shape, const int64_t* strides);

/* Batched rectangular pad/crop of `elem_bytes`-wide words:
 * dst[b][r][c] = (r < src_rows && c < src_cols) ? src[b][r][c] : 0 (all bits
 * zero), for r < dst_rows, c < dst_cols. Bit-preserving.
 * Replaces: _padding_copy.py:208-236 (_body) / :274-286 (cuda_copy). */
int hp_pad_copy(hp_ctx* ctx, int elem_bytes, const void* src, void* dst, int64_t batch,
                int64_t src_rows, int64_t src_cols, int64_t dst_rows, int64_t dst_cols);

/* ---- dense linear algebra ------------------------------------------------ */

/* C[b] = A[b'] @ B[b''] for row-major A (m x k), B (k x n), C (m x n),
 * dtype HP_F32 or HP_F64 on MFMA; the integer dtypes (wrapping modulo
 * 2^bits) and HP_BOOL (or of ands) on a tiled integer kernel, as the
 * reference OpenCL backend's generic product (_opencl.py:386-420); vector
 * operands are 1-row / 1-column matrices. The output batch is contiguous with
 * batch_rank dims `batch_shape`; operand batch offsets are
 * sum_d idx_d * a_batch_strides[d] (resp. b_...) elements, 0 = broadcast.
 * batch_rank <= 6. k == 0 writes zeros. C is never read.
 * Replaces: _gemm.py:102-137 (register_gemm_data) and _cuda.py:619-636
 * (direct fp64 kernel), reached from _cuda.py:493-518 (matmul routing). */
int hp_gemm(hp_ctx* ctx, int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
            int64_t k, int batch_rank, const int64_t* batch_shape, const int64_t* a_batch_strides,
            const int64_t* b_batch_strides);

/* C = op(A) @ op(B), 2-D, m x n x k, row-major C. op(A) = A stored (m, k), or
 * its transpose stored (k, m) when transpose_a; op(B) = B stored (k, n), or
 * stored (n, k) when transpose_b. Same kernels, accumulation and K order as
 * hp_gemm; k == 0 writes zeros; C is never read.
 * Replaces: _matmul_layout.py:19-31 (TransposedGemm.run, a CLBlast GEMM with
 * transpose flags), reached from _compiler.py:136-156 ("layout_matmul"). */
int hp_gemm_layout(hp_ctx* ctx, int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
                   int64_t k, int transpose_a, int transpose_b);

/* y[r] = sum_j a[r*inner + j] * x[j] for r < rows (HP_F32/HP_F64).
 * inner == 0 writes zeros. Replaces: _cuda_gemv.py:47-95 (matvec_data). */
int hp_gemv(hp_ctx* ctx, int dtype, const void* a, const void* x, void* y, int64_t rows,
            int64_t inner);

/* y[r] = rhs[r] - (a @ x)[r]: the hp_gemv product of row r, rounded to the
 * dtype, then one subtraction, in the same launch (the eager b - A @ x,
 * bit for bit). inner == 0 copies rhs. y must not alias rhs or a.
 * Replaces: _gemv.py:10-75 (residual_matvec_data), reached from
 * _compiler.py:157-176 ("residual_matvec" plan steps). */
int hp_gemv_residual(hp_ctx* ctx, int dtype, const void* a, const void* x, const void* rhs, void* y,
                     int64_t rows, int64_t inner);

/* out[0] = sum_i x[i] * y[i] (HP_F32/HP_F64); n == 0 writes 0.
 * Replaces: _cuda_gemv.py:47-95 with a 1-D left operand (DOT partials +
 * _cuda.py:449-491 reduce). */
int hp_dot(hp_ctx* ctx, int dtype, const void* x, const void* y, void* out, int64_t n);

/* hp_dot into a new pool block: *out = a fresh allocation of one element
 * (release it with hp_free) holding sum_i x[i] * y[i]. One call instead of
 * hp_alloc + hp_dot, for a host path whose cost is the calls themselves.
 * Replaces: _cuda.py:241-256 (empty of the 0-d result) with
 * _cuda_gemv.py:47-95 (the dot into it). */
int hp_dot_new(hp_ctx* ctx, int dtype, const void* x, const void* y, int64_t n, void** out);

/* ---- reductions ---------------------------------------------------------- */

/* Euclidean norm over the middle axis of x viewed as (outer, reduced, inner):
 * out[o*inner + i] = sqrt(sum_r x[(o*reduced + r)*inner + i]^2) computed
 * without overflow or underflow (power-of-two max scaling). NaN wins over
 * Inf; all-zero gives +0; reduced == 0 gives +0. HP_F32/HP_F64.
 * Replaces: _norm.py:39-118 (norm_data), reached from _cuda.py:639-642. */
int hp_norm(hp_ctx* ctx, int dtype, const void* x, void* out, int64_t outer, int64_t reduced,
            int64_t inner);

/* Size of the static device workspace of hp_norm_noalloc, per GPU. */
#define HP_NORM_NOALLOC_SCRATCH_BYTES (16 << 20)

/* hp_norm with the same kernels and results (bit for bit), but it allocates
 * nothing: no hipMalloc/hipFree, no pool block, no memset node. Its
 * temporaries (the per-chunk pairs and merge partials) live in a static
 * device array of HP_NORM_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends. A shape whose temporaries exceed it fails with HP_E_INVALID
 * before any launch (every contiguous f32 shape within the 2^31-element
 * array cap fits, and every strided shape: their first partial array is
 * planned below 8 MiB).
 * Every call on one GPU shares that GPU's array, so calls whose work overlaps
 * on one GPU (two contexts' streams, or threads without ordering) race; calls
 * on one context are ordered by its stream and do not.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
int hp_norm_noalloc(hp_ctx* ctx, int dtype, const void* x, void* out, int64_t outer, int64_t reduced,
                    int64_t inner);

/* out[o*inner + i] = op_r x[(o*reduced + r)*inner + i] for op in
 * {HP_SUM, HP_MIN, HP_MAX}. Sum: any numeric dtype except bool. Min/max:
 * NaN propagates, min prefers -0 and max prefers +0 on zero ties.
 * reduced == 0 writes the identity (sum) and is invalid for min/max.
 * Replaces: _cuda.py:449-491 (reduce) with _reductions.py:91-146. */
int hp_reduce(hp_ctx* ctx, int dtype, int op, const void* x, void* out, int64_t outer,
              int64_t reduced, int64_t inner);

/* ---- counter-based random numbers ---------------------------------------- */

/* out[i] for i < count from Philox4x32-10 block (counter = start + i as two
 * 32-bit words, key = seed as two 32-bit words), transformed to `dist` in
 * HP_F32/HP_F64. `first`, `second` are the distribution parameters (low/high,
 * loc/scale, or unused/scale) already rounded to the output dtype; `upper` is
 * nextafter(second, first) for HP_UNIFORM. start + count must not exceed 2^64.
 * Replaces: _random_cuda.py:31-41 (random_data) with _random.py:61-111. */
int hp_philox(hp_ctx* ctx, int dtype, int dist, void* out, int64_t count, uint64_t seed,
              uint64_t start, double first, double second, double upper);

/* Raw Philox4x32-10 words: out[4*i + w] = word w of the block for counter
 * start + i. Exposes the integer stream for bit-exact checks.
 * Replaces: _random.py:19-31 (_philox_numpy) on the device. */
int hp_philox_words(hp_ctx* ctx, uint32_t* out, int64_t count, uint64_t seed, uint64_t start);

/* ---- runtime compilation for fused elementwise / map-reduce kernels ------ */

/* Compile HIP source with hipRTC for gfx950 and load `name` from it.
 * Replaces: _cuda.py:313-351 (_compile: NVRTC + module cache). */
int hp_rtc_compile(hp_ctx* ctx, const char* source, const char* name, hp_kernel** out);

/* Launch a compiled kernel on the context stream with a 1-D grid; `args` is
 * the usual array of pointers to argument values.
 * Replaces: _cuda.py:359-374 (_run / cuLaunchKernel). */
int hp_rtc_launch(hp_ctx* ctx, hp_kernel* kernel, int64_t grid, int block, int shared_bytes,
                  void** args);

/* Unload a compiled module. */
int hp_rtc_release(hp_ctx* ctx, hp_kernel* kernel);

/* ---- timing and fault injection ------------------------------------------ */

/* Events recorded on the context stream (bench instrumentation).
 * Replaces: benchmarks/cuda_dispatch.py:62-110 (event-timed launches). */
int hp_event_create(hp_ctx* ctx, hp_event** out);
int hp_event_record(hp_ctx* ctx, hp_event* event);
int hp_event_elapsed_ms(hp_event* start, hp_event* stop, float* ms);
int hp_event_destroy(hp_event* event);

/* Make the next `count` entry points on this context fail with
 * HP_E_INJECTED before touching the device (host-side error-path tests).
 * Replaces: the fake driver failures of tests/test_cuda_arguments.py:123-183. */
int hp_debug_fail_next(hp_ctx* ctx, int count);

#ifdef __cplusplus
}
#endif

#endif /* PACHO_HIP_H */
