/*
 * TEST INFRASTRUCTURE ONLY - CPU restatement of the reference's Philox4x32-10
 * stream, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * as the checker. Never linked into libpacho_hip.so.
 *
 * Follows reference src/openpacho/_random.py:19-31 (rounds: multipliers
 * 0xD2511F53 / 0xCD9E8D57, key increments 0x9E3779B9 / 0xBB67AE85, word update
 * (hi(c2*M1)^c1^k0, lo(c2*M1), hi(c0*M0)^c3^k1, lo(c0*M0))), :34-45 (counter =
 * start + i split into (lo, hi, 0, 0); key = (lo(seed), hi(seed)); float32
 * unit (w0 >> 8) * 2^-24; float64 unit ((w0 >> 5) * 2^26 + (w1 >> 6)) * 2^-53),
 * :50-51 (uniform with clamp to [low, nextafter(high, low)]).
 * Build: oracle/Makefile -> oracle/_build/libphilox_oracle.so
 */
#include <stdint.h>

static void rounds(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)c[0] * 0xD2511F53u;
    uint64_t p1 = (uint64_t)c[2] * 0xCD9E8D57u;
    uint32_t w0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    uint32_t w1 = (uint32_t)p1;
    uint32_t w2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    uint32_t w3 = (uint32_t)p0;
    c[0] = w0;
    c[1] = w1;
    c[2] = w2;
    c[3] = w3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

/* General block function on four counter words (for published vectors). */
void oracle_philox_block(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c[4] = {counter[0], counter[1], counter[2], counter[3]};
  rounds(c, key[0], key[1]);
  for (int i = 0; i < 4; ++i) out[i] = c[i];
}

/* out[4*i + w] = word w of the block for counter start + i. */
void oracle_philox_words(uint32_t* out, int64_t count, uint64_t seed, uint64_t start) {
  for (int64_t i = 0; i < count; ++i) {
    uint64_t ctr = start + (uint64_t)i;
    uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u};
    rounds(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    for (int w = 0; w < 4; ++w) out[4 * i + w] = c[w];
  }
}

/* "random" (dist 0) and "uniform" (dist 1) samples, float32: the exact
 * (bit-for-bit) part of the stream contract. */
void oracle_uniform_f32(float* out, int64_t count, uint64_t seed, uint64_t start, int dist, float low,
                        float high, float upper) {
  for (int64_t i = 0; i < count; ++i) {
    uint64_t ctr = start + (uint64_t)i;
    uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u};
    rounds(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    volatile float u = (float)(c[0] >> 8) * 5.9604644775390625e-8f;
    if (dist == 0) {
      out[i] = u;
    } else {
      volatile float width = high - low;
      volatile float scaled = width * u;
      volatile float value = low + scaled;
      out[i] = value < low ? low : (value > upper ? upper : value);
    }
  }
}

void oracle_uniform_f64(double* out, int64_t count, uint64_t seed, uint64_t start, int dist, double low,
                        double high, double upper) {
  for (int64_t i = 0; i < count; ++i) {
    uint64_t ctr = start + (uint64_t)i;
    uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u};
    rounds(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    volatile double u = ((double)(c[0] >> 5) * 67108864.0 + (double)(c[1] >> 6)) *
                        1.1102230246251565404236316680908203125e-16;
    if (dist == 0) {
      out[i] = u;
    } else {
      volatile double width = high - low;
      volatile double scaled = width * u;
      volatile double value = low + scaled;
      out[i] = value < low ? low : (value > upper ? upper : value);
    }
  }
}
