// fp64 GEMM kernels, A transposed, B transposed (see gemm_kernels.h).
#include "gemm_kernels.h"

void hpgemm::f64_tt(hp_ctx* ctx, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                    const BatchDesc& bd, int64_t batch) {
  run_f64<true, true>(ctx, static_cast<const double*>(a), static_cast<const double*>(b),
                                static_cast<double*>(c), m, n, k, bd, batch);
}
