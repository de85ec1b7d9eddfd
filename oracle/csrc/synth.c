/* Seeded synthetic generator, C statement of the spec in oracle/synth.py.
 *
 * ORACLE / TEST INFRASTRUCTURE ONLY: used to build golden fixtures and CPU
 * models quickly. It must equal oracle/synth.py bit for bit (checked by a CPU
 * test) and the product's HIP generator (checked by a GPU test).
 * Built with -ffp-contract=off so no multiply-add is fused.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ULL
#define STREAM_MUL 0xD1B54A32D192ED03ULL

static const double LN2 = 0.6931471805599453;
static const double SQRT2 = 1.4142135623730951;

static inline uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ULL;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t synth_stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed * GAMMA + stream * STREAM_MUL + 1ULL);
}

static inline uint64_t splitmix(uint64_t key, uint64_t ctr) { return mix64(key + ctr * GAMMA); }

double synth_det_log(double s) {
  uint64_t bits;
  memcpy(&bits, &s, 8);
  int64_t e = (int64_t)((bits >> 52) & 0x7FFULL) - 1023;
  uint64_t mb = (bits & 0x000FFFFFFFFFFFFFULL) | 0x3FF0000000000000ULL;
  double m;
  memcpy(&m, &mb, 8);
  if (m > SQRT2) {
    m = m * 0.5;
    e = e + 1;
  }
  double f = (m - 1.0) / (m + 1.0);
  double f2 = f * f;
  double p = 1.0 / 23.0;
  for (int k = 10; k >= 0; --k) p = p * f2 + 1.0 / (double)(2 * k + 1);
  return (double)e * LN2 + (2.0 * f) * p;
}

double synth_normal_one(uint64_t key, uint64_t i) {
  for (uint64_t j = 0; j < 64; ++j) {
    uint64_t c = i * 64ULL + j;
    uint64_t h1 = splitmix(key, 2ULL * c);
    uint64_t h2 = splitmix(key, 2ULL * c + 1ULL);
    double x = (double)(h1 >> 11) * 0x1p-53 * 2.0 - 1.0;
    double y = (double)(h2 >> 11) * 0x1p-53 * 2.0 - 1.0;
    double s = x * x + y * y;
    if (s > 0.0 && s < 1.0) return x * sqrt((-2.0 * synth_det_log(s)) / s);
  }
  return 0.0;
}

/* out[k] = float32(std * z(start + k)), k in [0, count). */
void synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t start, uint64_t count, double std,
                      float* out) {
  uint64_t key = synth_stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < (int64_t)count; ++k) out[k] = (float)(std * synth_normal_one(key, start + (uint64_t)k));
}

void synth_uniform_ids(uint64_t seed, uint64_t stream, uint64_t count, uint64_t vocab, int64_t* out) {
  uint64_t key = synth_stream_key(seed, stream);
  for (uint64_t k = 0; k < count; ++k) out[k] = (int64_t)(((splitmix(key, k) >> 32) * vocab) >> 32);
}
