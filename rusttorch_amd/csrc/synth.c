/* Seeded synthetic weights: SplitMix64 -> 53-bit uniforms -> Box-Muller in
 * double -> float32 (the generator specified in rusttorch_amd/synth.py).
 * Pair p of the stream uses outputs 2p and 2p+1; normal 2p is r*cos, 2p+1 is
 * r*sin. Multi-threaded over pairs; the result does not depend on threads. */
#include <math.h>
#include <stdint.h>

static inline uint64_t splitmix_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* out[j] = (float)(a + b * normal_{2*pair_start + j}) for j < n. */
void synth_normals(uint64_t seed, uint64_t pair_start, uint64_t n, double a, double b, float* out) {
  const uint64_t npairs = (n + 1) / 2;
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (long long q = 0; q < (long long)npairs; ++q) {
    const uint64_t p = pair_start + (uint64_t)q;
    const double u1 = (double)(splitmix_at(seed, 2 * p) >> 11) * 0x1.0p-53;
    const double u2 = (double)(splitmix_at(seed, 2 * p + 1) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log1p(-u1));
    const double th = two_pi * u2;
    const uint64_t j = 2 * (uint64_t)q;
    out[j] = (float)(a + b * (r * cos(th)));
    if (j + 1 < n) out[j + 1] = (float)(a + b * (r * sin(th)));
  }
}
