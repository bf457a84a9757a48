// Counter-based Philox4x32-10 generator (Salmon et al., SC11 "Parallel random
// numbers: as easy as 1, 2, 3"), one counter block per output element in C
// order, so the stream is independent of launch geometry and call splitting.
// Stream contract: reference _random.py:19-31 (rounds), :43-45 / :73-77 (unit
// conversion), :50-56 / :93-102 (transforms), _random_cuda.py:10-28.
//
// Throughput is bound by vector ALU issue, not HBM: per element about 17
// 32x32->64 multiplies (v_mad_u64_u32) and as many three-input XORs, each a
// full wave64 instruction. Each thread produces four consecutive elements for
// instruction-level parallelism and 16-byte stores. When a wave's 256 counters share their high
// 32-bit word, that word lives in a scalar register: round 1 then needs one
// vector multiply (its c2 input is zero) and round 2's c0 product is a scalar
// multiply, saving 2 of the 20 vector multiplies per element.
#include <cmath>

#include "common.h"

namespace {

constexpr uint32_t kM0 = 0xD2511F53u;
constexpr uint32_t kM1 = 0xCD9E8D57u;
constexpr uint32_t kW0 = 0x9E3779B9u;
constexpr uint32_t kW1 = 0xBB67AE85u;

struct Words {
  uint32_t x0, x1, x2, x3;
};

// a ^ b ^ c as one gfx950 v_bitop3_b32 (truth table 0x96 is the 3-input
// parity); the compiler otherwise emits two v_xor_b32, and the XORs then cost
// as many VALU cycles as the multiplies.
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ Words philox10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                          uint32_t k1) {
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    const uint64_t p0 = uint64_t(c0) * kM0;
    const uint64_t p1 = uint64_t(c2) * kM1;
    const uint32_t n0 = xor3(uint32_t(p1 >> 32), c1, k0);
    const uint32_t n2 = xor3(uint32_t(p0 >> 32), c3, k1);
    c0 = n0;
    c1 = uint32_t(p1);
    c2 = n2;
    c3 = uint32_t(p0);
    k0 += kW0;
    k1 += kW1;
  }
  return {c0, c1, c2, c3};
}

// The same ten rounds for a counter block (lo + J, hi, 0, 0) whose high word
// hi is wave-uniform and lo + J does not carry (the kernel's common path),
// arranged so that the wave-uniform values stay on the scalar unit:
// round 1's c2 product is zero and its new c0 = hi ^ k0 is uniform, so round
// 2's c0 product is a scalar multiply whose low word, c3 of round 3, is
// uniform too. Uniform XORs are written with ^ (a scalar instruction; the
// three-input builtin would force them onto the vector unit, and gfx9 vector
// instructions read one scalar register at most). J rides in round 1's
// multiply-add: (lo + J) M0 = lo M0 + J M0 with no carry out of 64 bits.
// m0 is M0 held in a vector register, so that the multiply-add's one scalar
// operand is the 64-bit addend J M0 (with M0 in a scalar register the
// compiler moved the addend into two vector registers per sample).
template <int J>
__device__ __forceinline__ Words philox10_uniform_hi(uint32_t lo, uint32_t m0, uint32_t hi, uint32_t k0,
                                                     uint32_t k1) {
  // Round 1.
  const uint64_t a0 = uint64_t(lo) * m0 + uint64_t(J) * kM0;
  uint32_t c0 = hi ^ k0;
  uint32_t c2 = uint32_t(a0 >> 32) ^ k1;
  uint32_t c3 = uint32_t(a0);
  k0 += kW0;
  k1 += kW1;
  // Round 2 (c1 = 0).
  const uint64_t p0 = uint64_t(c0) * kM0;
  const uint64_t p1 = uint64_t(c2) * kM1;
  c0 = uint32_t(p1 >> 32) ^ k0;
  c2 = (uint32_t(p0 >> 32) ^ k1) ^ c3;
  c3 = uint32_t(p0);
  uint32_t c1 = uint32_t(p1);
  k0 += kW0;
  k1 += kW1;
  // Round 3 (c3 uniform).
  const uint64_t q0 = uint64_t(c0) * kM0;
  const uint64_t q1 = uint64_t(c2) * kM1;
  c0 = xor3(uint32_t(q1 >> 32), c1, k0);
  c2 = uint32_t(q0 >> 32) ^ (c3 ^ k1);
  c1 = uint32_t(q1);
  c3 = uint32_t(q0);
  k0 += kW0;
  k1 += kW1;
  // Rounds 4-10.
#pragma unroll
  for (int round = 3; round < 10; ++round) {
    const uint64_t r0 = uint64_t(c0) * kM0;
    const uint64_t r1 = uint64_t(c2) * kM1;
    const uint32_t n0 = xor3(uint32_t(r1 >> 32), c1, k0);
    const uint32_t n2 = xor3(uint32_t(r0 >> 32), c3, k1);
    c0 = n0;
    c1 = uint32_t(r1);
    c2 = n2;
    c3 = uint32_t(r0);
    k0 += kW0;
    k1 += kW1;
  }
  return {c0, c1, c2, c3};
}

template <typename T>
__device__ __forceinline__ T unit(uint32_t a, uint32_t b);

template <>
__device__ __forceinline__ float unit<float>(uint32_t a, uint32_t) {
  return float(a >> 8) * 5.9604644775390625e-8f;  // 2^-24, exact
}

template <>
__device__ __forceinline__ double unit<double>(uint32_t a, uint32_t b) {
  return (double(a >> 5) * 67108864.0 + double(b >> 6)) * 1.1102230246251565404236316680908203125e-16;
}

__device__ __forceinline__ float neg_log1m(float u) { return -log1pf(-u); }
__device__ __forceinline__ double neg_log1m(double u) { return -log1p(-u); }
__device__ __forceinline__ float dsqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double dsqrt(double x) { return sqrt(x); }
__device__ __forceinline__ float dcos(float x) { return cosf(x); }
__device__ __forceinline__ double dcos(double x) { return cos(x); }

template <typename T, int DIST>
__device__ __forceinline__ T transform(const Words& w, T first, T second, T upper) {
  const T u = unit<T>(w.x0, w.x1);
  if (DIST == HP_RANDOM) return u;
  if (DIST == HP_UNIFORM) {
    const T value = first + (second - first) * u;
    return value < first ? first : (value > upper ? upper : value);
  }
  const T nl = neg_log1m(u);
  if (DIST == HP_EXPONENTIAL) return second * nl;
  const T v = unit<T>(w.x2, w.x3);
  const T two_pi = T(6.283185307179586476925286766559);
  return first + second * (dsqrt(T(2) * nl) * dcos(two_pi * v));
}

// float32 normal/exponential on the hardware transcendental units. On the
// unit grid u = k * 2^-24 the value 1 - u is exact, so -log(1 - u) =
// -log2(1 - u) * ln 2 with v_log_f32 (measured max relative error 1.2e-7 over
// all 2^24 grid points); cos(2*pi*v) is v_cos_f32, whose input is in
// revolutions (max abs error 1.3e-7 over the grid); v_sqrt_f32 has max
// relative error 9e-8. Against the reference's libm transforms this stays far
// inside the 3e-6 tolerance of the float32 stream contract, and replaces ~100
// instructions of log1pf/cosf/sqrtf per sample with ~6.
//
// log2(1 - u) <= 0 on the grid, so -log(1 - u) is written |log2(1 - u)| * ln 2.
// At u = 0 this is +0, as -log1p(-0) is; the form 0 - log2(1 - u) * ln 2 was
// turned into a negation by the code generator and gave -0 there.
__device__ __forceinline__ float neg_log1m_grid(float u) {
  return __builtin_fabsf(__builtin_amdgcn_logf(1.0f - u)) * 0.693147180559945309417f;
}

template <>
__device__ __forceinline__ float transform<float, HP_NORMAL>(const Words& w, float first, float second, float) {
  const float u = unit<float>(w.x0, w.x1);
  // 2 * (|log2(1 - u)| * ln2) == |log2(1 - u)| * (2 * ln2) exactly: doubling
  // commutes with rounding, so the factor 2 costs no instruction.
  const float two_nl = __builtin_fabsf(__builtin_amdgcn_logf(1.0f - u)) * (2.0f * 0.693147180559945309417f);
  const float v = unit<float>(w.x2, w.x3);
  return first + second * (__builtin_amdgcn_sqrtf(two_nl) * __builtin_amdgcn_cosf(v));
}

template <>
__device__ __forceinline__ float transform<float, HP_EXPONENTIAL>(const Words& w, float, float second, float) {
  const float u = unit<float>(w.x0, w.x1);
  const float nl = neg_log1m_grid(u);
  return second * nl;
}

// 1 - u on the float32 unit grid as one fused multiply-add: u = k 2^-24 and
// 1 - u are exact, so fma(k, -2^-24, 1) is the same value as 1 - (k 2^-24)
// in one instruction instead of two.
__device__ __forceinline__ float one_minus_unit(uint32_t a) {
  return __builtin_fmaf(float(a >> 8), -5.9604644775390625e-8f, 1.0f);
}

// float32 exponential and normal with their constant factors folded on the
// host into one normal-range float (one multiply per sample fewer; the
// result moves by at most ~2 ulp, inside the 3e-6 stream tolerance):
// exponential: scale * ln 2 * |log2(1 - u)|; normal: sqrt(2 ln 2 scale^2 *
// |log2(1 - u)|) * cos(2 pi v) + loc, for scale >= 0. At u = 0 both give +0
// (+ loc), as the unfolded forms do.
constexpr int kExponentialFolded = 6, kNormalFolded = 7;

template <>
__device__ __forceinline__ float transform<float, kExponentialFolded>(const Words& w, float, float folded, float) {
  return __builtin_fabsf(__builtin_amdgcn_logf(one_minus_unit(w.x0))) * folded;
}

// loc + radius * cos as one fused multiply-add: one rounding instead of two
// (within the stream tolerance; for loc = 0 the same value, and +0 where the
// radius is +0, as before).
template <>
__device__ __forceinline__ float transform<float, kNormalFolded>(const Words& w, float first, float folded, float) {
  const float radius2 = __builtin_fabsf(__builtin_amdgcn_logf(one_minus_unit(w.x0))) * folded;
  const float v = unit<float>(w.x2, w.x3);
  return __builtin_fmaf(__builtin_amdgcn_sqrtf(radius2), __builtin_amdgcn_cosf(v), first);
}

// Uniform with the width pre-scaled by the unit's power of two, selected by
// the host when that scaling is exact (see uniform_scaled). The unit numerator
// k (float32: word0 >> 8; float64: the 53-bit integer) is exact in T, so
// k * (width * 2^-b) and (k * 2^-b) * width are the same real product and
// round to the same value: one multiply per sample fewer, bit for bit.
constexpr int kUniformScaled = 4;

template <>
__device__ __forceinline__ float transform<float, kUniformScaled>(const Words& w, float first, float scaled,
                                                                  float upper) {
  const float value = first + float(w.x0 >> 8) * scaled;
  // first <= upper, value is finite and neither bound is -0 (host check), so
  // the median of three is the reference clamp to [first, upper].
  return __builtin_amdgcn_fmed3f(value, first, upper);
}

template <>
__device__ __forceinline__ double transform<double, kUniformScaled>(const Words& w, double first, double scaled,
                                                                    double upper) {
  const double k = double(w.x0 >> 5) * 67108864.0 + double(w.x1 >> 6);
  const double value = first + k * scaled;
  return value < first ? first : (value > upper ? upper : value);
}

// Pre-scaled uniform with first == 0 and a positive width w (the default
// uniform()): the reference value clip(0 + w * u, 0, nextafter(w, 0)) is
// k * scaled rounded once. The sum with 0 is exact, and the clip never
// binds: k <= 2^b - 1 gives k * scaled = w (1 - 2^-b) at most, whose
// distance below w is at least half an ulp of w, so it rounds to a float
// below w (a power-of-two w leaves it exactly representable).
constexpr int kUniformScaledZero = 5;

template <>
__device__ __forceinline__ float transform<float, kUniformScaledZero>(const Words& w, float, float scaled, float) {
  return float(w.x0 >> 8) * scaled;
}

template <>
__device__ __forceinline__ double transform<double, kUniformScaledZero>(const Words& w, double, double scaled,
                                                                        double) {
  return (double(w.x0 >> 5) * 67108864.0 + double(w.x1 >> 6)) * scaled;
}

constexpr int kBlock = 256;
// Samples per thread: eight consecutive counters, stored as 16-byte vectors;
// the per-thread work around the blocks (counter base, tail test, address)
// is then shared by eight samples (with four it added ~1.5 instructions per
// sample).
constexpr int kPerThread = 8;

// values[0 .. kPerThread) to out[e0 ..), vector stores when all are inside.
template <typename T>
__device__ __forceinline__ void store_run(T* out, int64_t e0, int64_t count, const T (&v)[kPerThread]) {
  if (e0 + kPerThread <= count) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int q = 0; q < kPerThread / 4; ++q)
        reinterpret_cast<hpd::f32x4*>(out + e0)[q] = hpd::f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
#pragma unroll
      for (int q = 0; q < kPerThread / 2; ++q) reinterpret_cast<hpd::f64x2*>(out + e0)[q] = hpd::f64x2{v[2 * q], v[2 * q + 1]};
    }
  } else {
    for (int j = 0; j < kPerThread; ++j)
      if (e0 + j < count) out[e0 + j] = v[j];
  }
}

// values[J ..) of a run whose counters (lo0 + j, hi) share the wave-uniform hi.
template <typename T, int DIST, int J = 0>
__device__ __forceinline__ void run_uniform_hi(T (&values)[kPerThread], uint32_t lo0, uint32_t m0, uint32_t hi,
                                               uint32_t k0, uint32_t k1, T first, T second, T upper) {
  if constexpr (J < kPerThread) {
    values[J] = transform<T, DIST>(philox10_uniform_hi<J>(lo0, m0, hi, k0, k1), first, second, upper);
    run_uniform_hi<T, DIST, J + 1>(values, lo0, m0, hi, k0, k1, first, second, upper);
  }
}

template <typename T, int DIST>
__global__ __launch_bounds__(kBlock) void philox_kernel(T* __restrict__ out, int64_t count, uint32_t k0,
                                                        uint32_t k1, uint64_t start, T first, T second,
                                                        T upper) {
  const int64_t block_first = int64_t(blockIdx.x) * (kBlock * kPerThread);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t wave_first = start + uint64_t(block_first) + uint64_t(wave) * (64 * kPerThread);
  const uint64_t wave_last = wave_first + (64 * kPerThread - 1);
  const int64_t e0 = block_first + int64_t(threadIdx.x) * kPerThread;
  if (e0 >= count) return;
  T values[kPerThread];
  if (uint32_t(wave_first >> 32) == uint32_t(wave_last >> 32)) {
    // Wave-uniform high word: no carry inside this wave's counters.
    uint32_t m0;
    asm("v_mov_b32 %0, 0xd2511f53" : "=v"(m0));  // kM0, in a vector register
    run_uniform_hi<T, DIST>(values, uint32_t(start) + uint32_t(e0), m0, uint32_t(wave_first >> 32), k0, k1, first,
                            second, upper);
  } else {
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const uint64_t counter = start + uint64_t(e0 + j);
      const Words w = philox10(uint32_t(counter), uint32_t(counter >> 32), 0u, 0u, k0, k1);
      values[j] = transform<T, DIST>(w, first, second, upper);
    }
  }
  store_run<T>(out, e0, count, values);
}

__global__ __launch_bounds__(kBlock) void philox_words_kernel(uint32_t* __restrict__ out, int64_t count,
                                                              uint32_t k0, uint32_t k1, uint64_t start) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= count) return;
  const uint64_t counter = start + uint64_t(i);
  const Words w = philox10(uint32_t(counter), uint32_t(counter >> 32), 0u, 0u, k0, k1);
  uint4 q;
  q.x = w.x0;
  q.y = w.x1;
  q.z = w.x2;
  q.w = w.x3;
  reinterpret_cast<uint4*>(out)[i] = q;
}

// The pre-scaled uniform applies when width * 2^-b is exact (no underflow)
// and, for the float32 median clamp, neither bound is -0: then the sample
// first + width * u is never -0 and med3 orders exactly like the comparisons.
template <typename T>
bool uniform_scaled(T first, T second, T upper, T* scaled) {
  const int bits = sizeof(T) == 4 ? 24 : 53;
  const T width = second - first;
  *scaled = std::ldexp(width, -bits);
  if (!std::isfinite(width) || std::ldexp(*scaled, bits) != width) return false;
  if (sizeof(T) == 4 && ((first == 0 && std::signbit(first)) || (upper == 0 && std::signbit(upper)))) return false;
  return true;
}

template <typename T>
void launch(hp_ctx* ctx, int dist, T* out, int64_t count, uint32_t k0, uint32_t k1, uint64_t start, T first,
            T second, T upper) {
  const int64_t grid = hp::ceil_div(count, kBlock * kPerThread);
  hp::require(grid <= hp::kMaxGrid, "random output too large for one launch");
  T scaled;
  if (dist == HP_UNIFORM && uniform_scaled(first, second, upper, &scaled)) {
    if (first == 0 && scaled > 0) {
      philox_kernel<T, kUniformScaledZero><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first,
                                                                             scaled, upper);
    } else {
      philox_kernel<T, kUniformScaled><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first, scaled,
                                                                         upper);
    }
    hp::check_launch("philox");
    return;
  }
  if (sizeof(T) == 4 && (dist == HP_EXPONENTIAL || dist == HP_NORMAL) && second >= 0) {
    const double ln2 = 0.69314718055994530942;
    const double scale = double(second);
    const float folded = float(dist == HP_EXPONENTIAL ? scale * ln2 : 2.0 * ln2 * scale * scale);
    if (std::isnormal(folded)) {
      if (dist == HP_EXPONENTIAL) {
        philox_kernel<float, kExponentialFolded><<<grid, kBlock, 0, ctx->stream>>>(
            reinterpret_cast<float*>(out), count, k0, k1, start, float(first), folded, float(upper));
      } else {
        philox_kernel<float, kNormalFolded><<<grid, kBlock, 0, ctx->stream>>>(
            reinterpret_cast<float*>(out), count, k0, k1, start, float(first), folded, float(upper));
      }
      hp::check_launch("philox");
      return;
    }
  }
  switch (dist) {
    case HP_RANDOM:
      philox_kernel<T, HP_RANDOM><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first, second, upper);
      break;
    case HP_UNIFORM:
      philox_kernel<T, HP_UNIFORM><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first, second, upper);
      break;
    case HP_NORMAL:
      philox_kernel<T, HP_NORMAL><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first, second, upper);
      break;
    case HP_EXPONENTIAL:
      philox_kernel<T, HP_EXPONENTIAL><<<grid, kBlock, 0, ctx->stream>>>(out, count, k0, k1, start, first, second, upper);
      break;
    default:
      hp::fail(HP_E_INVALID, "unknown distribution code " + std::to_string(dist));
  }
  hp::check_launch("philox");
}

}  // namespace

using hp::guarded;
using hp::require;

extern "C" {

int hp_philox(hp_ctx* ctx, int dtype, int dist, void* out, int64_t count, uint64_t seed, uint64_t start,
              double first, double second, double upper) {
  return guarded([&] {
    hp::enter(ctx);
    require(count >= 0, "negative count");
    require(dtype == HP_F32 || dtype == HP_F64, "random generation requires float32 or float64");
    require(dist >= HP_RANDOM && dist <= HP_EXPONENTIAL, "unknown distribution code");
    // The counter range [start, start + count) must fit in 64 bits.
    require(count == 0 || uint64_t(count) - 1 <= ~start, "Philox counter range exceeds 2^64");
    if (count == 0) return;
    require(out != nullptr && reinterpret_cast<uintptr_t>(out) % 16 == 0,
            "random output must be a 16-byte aligned device buffer");
    const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
    if (dtype == HP_F32) {
      launch<float>(ctx, dist, static_cast<float*>(out), count, k0, k1, start, float(first), float(second),
                    float(upper));
    } else {
      launch<double>(ctx, dist, static_cast<double*>(out), count, k0, k1, start, first, second, upper);
    }
  });
}

int hp_philox_words(hp_ctx* ctx, uint32_t* out, int64_t count, uint64_t seed, uint64_t start) {
  return guarded([&] {
    hp::enter(ctx);
    require(count >= 0, "negative count");
    require(count == 0 || uint64_t(count) - 1 <= ~start, "Philox counter range exceeds 2^64");
    if (count == 0) return;
    require(out != nullptr && reinterpret_cast<uintptr_t>(out) % 16 == 0, "output must be 16-byte aligned");
    const int64_t grid = hp::ceil_div(count, kBlock);
    require(grid <= hp::kMaxGrid, "output too large for one launch");
    philox_words_kernel<<<grid, kBlock, 0, ctx->stream>>>(out, count, uint32_t(seed), uint32_t(seed >> 32), start);
    hp::check_launch("philox_words");
  });
}

}  // extern "C"
