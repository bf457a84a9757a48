// fp32 GEMM kernels, A transposed, B transposed (see gemm_kernels.h).
#include "gemm_kernels.h"

void hpgemm::f32_tt(hp_ctx* ctx, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                    const BatchDesc& bd, int64_t batch) {
  run_f32<true, true>(ctx, static_cast<const float*>(a), static_cast<const float*>(b),
                                static_cast<float*>(c), m, n, k, bd, batch);
}
