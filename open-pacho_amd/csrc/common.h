// Internal declarations shared by the libpacho_hip.so translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "pacho_hip.h"

namespace hp {

// Failure carried from deep inside an entry point to its C boundary.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(int code, const std::string& message) { throw Error(code, message); }

inline void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    fail(status == hipErrorOutOfMemory ? HP_E_OOM : HP_E_HIP,
         std::string(what) + " failed: " + hipGetErrorString(status) + " (" +
             std::to_string(static_cast<int>(status)) + ")");
  }
}

#define HP_CHECK(call) ::hp::check_hip((call), #call)

void set_last_error(const std::string& message);

// Runs `body` and converts exceptions into a status code + thread-local message.
template <typename F>
int guarded(F&& body) {
  try {
    body();
    set_last_error("");
    return HP_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return HP_E_OOM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return HP_E_HIP;
  }
}

}  // namespace hp

struct hp_kernel {
  hipModule_t module = nullptr;
  hipFunction_t function = nullptr;
};

struct hp_event {
  hipEvent_t event = nullptr;
  int device = 0;
};

struct hp_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // A second stream (default priority) for independent work that may overlap
  // the main stream's (the edge strips of a GEMM beside its tiled kernels),
  // forked and joined with these events; the main stream always waits for it
  // before its next work, so callers see one stream. A context's calls are
  // not to be made from several host threads at once (the GEMM points
  // `stream` at `side` while it queues the strips).
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  int compute_units = 0;
  std::recursive_mutex mutex;
  // Stream-ordered caching pool: size class -> free blocks.
  std::multimap<size_t, void*> free_blocks;
  std::unordered_map<void*, size_t> live;  // pointer -> capacity
  size_t cached_bytes = 0;
  size_t live_bytes = 0;
  size_t pool_limit = 0;
  int fail_next = 0;
};

namespace hp {

// Makes ctx->device current for the calling thread and validates the context.
void enter(hp_ctx* ctx);

// Pool allocation used by entry points for their own temporaries (stream
// ordered: the block may be freed right after the launches that use it).
void* scratch_alloc(hp_ctx* ctx, size_t bytes);
void scratch_free(hp_ctx* ctx, void* ptr);

inline void require(bool condition, const std::string& message) {
  if (!condition) fail(HP_E_INVALID, message);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline void check_launch(const char* name) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    fail(HP_E_HIP, std::string("launch of ") + name + " failed: " + hipGetErrorString(status));
  }
}

// Grid dimension cap of a 1-D launch; kernels use grid-stride loops beyond it.
constexpr int64_t kMaxGrid = int64_t(1) << 30;

inline size_t dtype_size(int dtype) {
  switch (dtype) {
    case HP_BOOL: return 1;
    case HP_I32: case HP_U32: case HP_F32: return 4;
    case HP_I64: case HP_U64: case HP_F64: return 8;
    default: fail(HP_E_INVALID, "unknown dtype code " + std::to_string(dtype));
  }
}

}  // namespace hp

// ---- device helpers shared by kernels ------------------------------------

namespace hpd {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

// Full-wave (64 lanes) butterfly reductions; every lane receives the result.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace hpd
