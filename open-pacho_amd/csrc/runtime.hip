// Context, stream-ordered caching pool, transfers, events and hipRTC modules.
//
// One context owns one non-blocking stream. Every kernel and copy of the
// context is issued on that stream, so a block returned to the pool can be
// handed to the next request immediately: any later use is queued behind the
// work that used it before. This replaces the reference's host-side retention
// list (_cuda.py:353-357) with stream ordering.
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdio>

#include "common.h"

namespace hp {

static thread_local std::string g_last_error;

void set_last_error(const std::string& message) { g_last_error = message; }

static size_t size_class(size_t bytes) {
  if (bytes <= 512) return 512;
  if (bytes <= (size_t(1) << 20)) {
    size_t c = 512;
    while (c < bytes) c <<= 1;
    return c;
  }
  const size_t granule = size_t(2) << 20;
  return (bytes + granule - 1) / granule * granule;
}

static void set_device(int device) {
  int current = -1;
  HP_CHECK(hipGetDevice(&current));
  if (current != device) HP_CHECK(hipSetDevice(device));
}

void enter(hp_ctx* ctx) {
  require(ctx != nullptr, "null context");
  if (ctx->fail_next > 0) {
    --ctx->fail_next;
    fail(HP_E_INJECTED, "injected failure (hp_debug_fail_next)");
  }
  set_device(ctx->device);
}

// Each block leaves the cache as soon as its free succeeds, so a failure part
// way through leaves only blocks that are still allocated: a freed pointer is
// never handed out again (reference test_cuda_lifetime.py:79-126).
static void release_cache_locked(hp_ctx* ctx) {
  if (ctx->free_blocks.empty()) return;
  HP_CHECK(hipStreamSynchronize(ctx->stream));
  for (auto it = ctx->free_blocks.begin(); it != ctx->free_blocks.end();) {
    HP_CHECK(hipFree(it->second));
    ctx->cached_bytes -= it->first;
    it = ctx->free_blocks.erase(it);
  }
}

static void* pool_alloc(hp_ctx* ctx, size_t bytes) {
  std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
  const size_t cls = size_class(std::max<size_t>(bytes, 1));
  auto it = ctx->free_blocks.find(cls);
  void* ptr = nullptr;
  if (it != ctx->free_blocks.end()) {
    ptr = it->second;
    ctx->free_blocks.erase(it);
    ctx->cached_bytes -= cls;
  } else {
    hipError_t status = hipMalloc(&ptr, cls);
    if (status != hipSuccess) {
      (void)hipGetLastError();
      release_cache_locked(ctx);
      status = hipMalloc(&ptr, cls);
      if (status != hipSuccess) {
        (void)hipGetLastError();
        fail(HP_E_OOM, "hipMalloc of " + std::to_string(cls) + " bytes failed: " +
                           hipGetErrorString(status));
      }
    }
  }
  ctx->live[ptr] = cls;
  ctx->live_bytes += cls;
  return ptr;
}

static void pool_free(hp_ctx* ctx, void* ptr) {
  std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
  auto it = ctx->live.find(ptr);
  require(it != ctx->live.end(), "pointer was not allocated by this context");
  const size_t cls = it->second;
  ctx->live.erase(it);
  ctx->live_bytes -= cls;
  if (cls > ctx->pool_limit) {
    HP_CHECK(hipStreamSynchronize(ctx->stream));
    HP_CHECK(hipFree(ptr));
    return;
  }
  if (ctx->cached_bytes + cls > ctx->pool_limit) {
    // Evict the largest cached blocks first until the new one fits.
    HP_CHECK(hipStreamSynchronize(ctx->stream));
    while (!ctx->free_blocks.empty() && ctx->cached_bytes + cls > ctx->pool_limit) {
      auto last = std::prev(ctx->free_blocks.end());
      HP_CHECK(hipFree(last->second));
      ctx->cached_bytes -= last->first;
      ctx->free_blocks.erase(last);
    }
  }
  ctx->free_blocks.emplace(cls, ptr);
  ctx->cached_bytes += cls;
}

void* scratch_alloc(hp_ctx* ctx, size_t bytes) { return pool_alloc(ctx, bytes); }
void scratch_free(hp_ctx* ctx, void* ptr) { pool_free(ctx, ptr); }

}  // namespace hp

using hp::guarded;
using hp::require;

extern "C" {

const char* hp_last_error(void) { return hp::g_last_error.c_str(); }

const char* hp_version(void) { return "pacho_hip 0.1.0 gfx950"; }

int hp_device_count(int* count) {
  return guarded([&] {
    require(count != nullptr, "null output");
    int n = 0;
    hipError_t status = hipGetDeviceCount(&n);
    if (status == hipErrorNoDevice || status == hipErrorInvalidDevice) {
      (void)hipGetLastError();
      n = 0;
    } else {
      HP_CHECK(status);
    }
    *count = n;
  });
}

int hp_device_info(int device, char* name, int64_t name_len, char* arch, int64_t arch_len,
                   int64_t* total_bytes, int* compute_units, int* fp64) {
  return guarded([&] {
    hipDeviceProp_t prop;
    HP_CHECK(hipGetDeviceProperties(&prop, device));
    if (name && name_len > 0) {
      std::snprintf(name, static_cast<size_t>(name_len), "%s",
                    prop.name[0] ? prop.name : "AMD Instinct GPU");
    }
    if (arch && arch_len > 0) std::snprintf(arch, static_cast<size_t>(arch_len), "%s", prop.gcnArchName);
    if (total_bytes) *total_bytes = static_cast<int64_t>(prop.totalGlobalMem);
    if (compute_units) *compute_units = prop.multiProcessorCount;
    if (fp64) *fp64 = 1;
  });
}

int hp_init(int device, hp_ctx** out) {
  hp_ctx* ctx = nullptr;
  int status = guarded([&] {
    require(out != nullptr, "null output");
    int n = 0;
    HP_CHECK(hipGetDeviceCount(&n));
    require(device >= 0 && device < n, "device " + std::to_string(device) + " not found");
    hipDeviceProp_t prop;
    HP_CHECK(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    require(arch.rfind("gfx950", 0) == 0,
            "libpacho_hip is built for gfx950 (MI355X); device reports " + arch);
    HP_CHECK(hipSetDevice(device));
    ctx = new hp_ctx();
    ctx->device = device;
    ctx->compute_units = prop.multiProcessorCount;
    ctx->pool_limit = static_cast<size_t>(prop.totalGlobalMem / 4);
    HP_CHECK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    HP_CHECK(hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking));
    HP_CHECK(hipEventCreateWithFlags(&ctx->fork, hipEventDisableTiming));
    HP_CHECK(hipEventCreateWithFlags(&ctx->join, hipEventDisableTiming));
    *out = ctx;
  });
  if (status != HP_OK && ctx != nullptr) {
    if (ctx->join) (void)hipEventDestroy(ctx->join);
    if (ctx->fork) (void)hipEventDestroy(ctx->fork);
    if (ctx->side) (void)hipStreamDestroy(ctx->side);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    if (out) *out = nullptr;
  }
  return status;
}

int hp_destroy(hp_ctx* ctx) {
  if (ctx == nullptr) return HP_OK;
  int status = guarded([&] {
    hp::set_device(ctx->device);
    std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
    HP_CHECK(hipStreamSynchronize(ctx->stream));
    HP_CHECK(hipStreamSynchronize(ctx->side));
    for (auto& entry : ctx->free_blocks) HP_CHECK(hipFree(entry.second));
    for (auto& entry : ctx->live) HP_CHECK(hipFree(entry.first));
    ctx->free_blocks.clear();
    ctx->live.clear();
    HP_CHECK(hipEventDestroy(ctx->join));
    HP_CHECK(hipEventDestroy(ctx->fork));
    HP_CHECK(hipStreamDestroy(ctx->side));
    HP_CHECK(hipStreamDestroy(ctx->stream));
    ctx->stream = nullptr;
  });
  delete ctx;
  return status;
}

int hp_alloc(hp_ctx* ctx, int64_t bytes, void** out) {
  return guarded([&] {
    hp::enter(ctx);
    require(out != nullptr, "null output");
    require(bytes >= 0, "negative allocation size");
    *out = hp::pool_alloc(ctx, static_cast<size_t>(bytes));
  });
}

int hp_free(hp_ctx* ctx, void* ptr) {
  return guarded([&] {
    require(ctx != nullptr, "null context");
    if (ptr == nullptr) return;
    hp::set_device(ctx->device);
    hp::pool_free(ctx, ptr);
  });
}

int hp_release_cached(hp_ctx* ctx) {
  return guarded([&] {
    hp::enter(ctx);
    std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
    HP_CHECK(hipStreamSynchronize(ctx->stream));
    hp::release_cache_locked(ctx);
  });
}

int hp_set_pool_limit(hp_ctx* ctx, int64_t bytes) {
  return guarded([&] {
    hp::enter(ctx);
    require(bytes >= 0, "negative pool limit");
    std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
    ctx->pool_limit = static_cast<size_t>(bytes);
    if (ctx->cached_bytes > ctx->pool_limit) hp::release_cache_locked(ctx);
  });
}

int hp_pool_stats(hp_ctx* ctx, int64_t* cached_bytes, int64_t* cached_items, int64_t* live_bytes,
                  int64_t* live_items) {
  return guarded([&] {
    require(ctx != nullptr, "null context");
    std::lock_guard<std::recursive_mutex> lock(ctx->mutex);
    if (cached_bytes) *cached_bytes = static_cast<int64_t>(ctx->cached_bytes);
    if (cached_items) *cached_items = static_cast<int64_t>(ctx->free_blocks.size());
    if (live_bytes) *live_bytes = static_cast<int64_t>(ctx->live_bytes);
    if (live_items) *live_items = static_cast<int64_t>(ctx->live.size());
  });
}

int hp_h2d(hp_ctx* ctx, void* dst, const void* src, int64_t bytes) {
  return guarded([&] {
    hp::enter(ctx);
    require(bytes >= 0, "negative copy size");
    if (bytes == 0) return;
    require(dst != nullptr && src != nullptr, "null pointer");
    HP_CHECK(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice, ctx->stream));
    HP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int hp_d2h(hp_ctx* ctx, void* dst, const void* src, int64_t bytes) {
  return guarded([&] {
    hp::enter(ctx);
    require(bytes >= 0, "negative copy size");
    if (bytes == 0) {
      HP_CHECK(hipStreamSynchronize(ctx->stream));
      return;
    }
    require(dst != nullptr && src != nullptr, "null pointer");
    HP_CHECK(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, ctx->stream));
    HP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int hp_d2d(hp_ctx* ctx, void* dst, const void* src, int64_t bytes) {
  return guarded([&] {
    hp::enter(ctx);
    require(bytes >= 0, "negative copy size");
    if (bytes == 0) return;
    require(dst != nullptr && src != nullptr, "null pointer");
    HP_CHECK(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice, ctx->stream));
  });
}

int hp_sync(hp_ctx* ctx) {
  return guarded([&] {
    hp::enter(ctx);
    HP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

// ---- hipRTC ----------------------------------------------------------------

int hp_rtc_compile(hp_ctx* ctx, const char* source, const char* name, hp_kernel** out) {
  return guarded([&] {
    hp::enter(ctx);
    require(source != nullptr && name != nullptr && out != nullptr, "null argument");
    hipDeviceProp_t prop;
    HP_CHECK(hipGetDeviceProperties(&prop, ctx->device));
    std::string arch = std::string("--offload-arch=") + prop.gcnArchName;
    // Same numerics policy as the precompiled kernels: no contraction, IEEE
    // denormals, correctly rounded fp32 division/sqrt, no packed fp32 math.
    const char* options[] = {arch.c_str(), "-O3", "-std=c++17", "-ffp-contract=off",
                             "-fhip-fp32-correctly-rounded-divide-sqrt",
                             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
    hiprtcProgram program;
    if (hiprtcCreateProgram(&program, source, "pacho_rtc.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
      hp::fail(HP_E_RTC, "hiprtcCreateProgram failed");
    }
    struct Destroy {
      hiprtcProgram* p;
      ~Destroy() { (void)hiprtcDestroyProgram(p); }
    } destroy{&program};
    hiprtcResult status = hiprtcCompileProgram(program, sizeof(options) / sizeof(options[0]), options);
    if (status != HIPRTC_SUCCESS) {
      size_t size = 0;
      (void)hiprtcGetProgramLogSize(program, &size);
      std::string log(size, '\0');
      if (size) (void)hiprtcGetProgramLog(program, &log[0]);
      hp::fail(HP_E_RTC, std::string("hipRTC compilation failed: ") + hiprtcGetErrorString(status) +
                             "\n" + log);
    }
    size_t code_size = 0;
    if (hiprtcGetCodeSize(program, &code_size) != HIPRTC_SUCCESS || code_size == 0) {
      hp::fail(HP_E_RTC, "hipRTC produced no code object");
    }
    std::vector<char> code(code_size);
    if (hiprtcGetCode(program, code.data()) != HIPRTC_SUCCESS) hp::fail(HP_E_RTC, "hiprtcGetCode failed");
    hp_kernel* kernel = new hp_kernel();
    hipError_t load = hipModuleLoadData(&kernel->module, code.data());
    if (load != hipSuccess) {
      delete kernel;
      HP_CHECK(load);
    }
    hipError_t get = hipModuleGetFunction(&kernel->function, kernel->module, name);
    if (get != hipSuccess) {
      (void)hipModuleUnload(kernel->module);
      delete kernel;
      HP_CHECK(get);
    }
    *out = kernel;
  });
}

int hp_rtc_launch(hp_ctx* ctx, hp_kernel* kernel, int64_t grid, int block, int shared_bytes,
                  void** args) {
  return guarded([&] {
    hp::enter(ctx);
    require(kernel != nullptr && kernel->function != nullptr, "null kernel");
    require(grid >= 0 && grid <= hp::kMaxGrid, "grid out of range");
    require(block > 0 && block <= 1024, "block out of range");
    if (grid == 0) return;
    HP_CHECK(hipModuleLaunchKernel(kernel->function, static_cast<unsigned>(grid), 1, 1,
                                   static_cast<unsigned>(block), 1, 1,
                                   static_cast<unsigned>(shared_bytes), ctx->stream, args, nullptr));
  });
}

int hp_rtc_release(hp_ctx* ctx, hp_kernel* kernel) {
  return guarded([&] {
    require(ctx != nullptr, "null context");
    if (kernel == nullptr) return;
    hp::set_device(ctx->device);
    HP_CHECK(hipStreamSynchronize(ctx->stream));
    if (kernel->module) HP_CHECK(hipModuleUnload(kernel->module));
    delete kernel;
  });
}

// ---- events ----------------------------------------------------------------

int hp_event_create(hp_ctx* ctx, hp_event** out) {
  return guarded([&] {
    hp::enter(ctx);
    require(out != nullptr, "null output");
    hp_event* event = new hp_event();
    event->device = ctx->device;
    hipError_t status = hipEventCreate(&event->event);
    if (status != hipSuccess) {
      delete event;
      HP_CHECK(status);
    }
    *out = event;
  });
}

int hp_event_record(hp_ctx* ctx, hp_event* event) {
  return guarded([&] {
    hp::enter(ctx);
    require(event != nullptr, "null event");
    HP_CHECK(hipEventRecord(event->event, ctx->stream));
  });
}

int hp_event_elapsed_ms(hp_event* start, hp_event* stop, float* ms) {
  return guarded([&] {
    require(start && stop && ms, "null argument");
    HP_CHECK(hipEventSynchronize(stop->event));
    HP_CHECK(hipEventElapsedTime(ms, start->event, stop->event));
  });
}

int hp_event_destroy(hp_event* event) {
  return guarded([&] {
    if (event == nullptr) return;
    if (event->event) HP_CHECK(hipEventDestroy(event->event));
    delete event;
  });
}

int hp_debug_fail_next(hp_ctx* ctx, int count) {
  return guarded([&] {
    require(ctx != nullptr, "null context");
    require(count >= 0, "negative count");
    ctx->fail_next = count;
  });
}

}  // extern "C"
